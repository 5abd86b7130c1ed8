"""GPU parity of the backward path (hif8_linear.py:88-111): the code and bf16 transposes, dgrad
grad_q @ w_q on the transposed codes, wgrad grad_q^T @ x_q on the decode-free GEMM over the
transposed operands, and HIF8Linear's gradients.

Oracle: the gradient quantisation is checked bit for bit against the CPU restatement;
products against fp32 torch on the same (bit-exact) quantised operands, with the
tolerance of the forward tests (max element error relative to max(|ref|, 1e-2 rms)
<= 1e-2, normwise <= 4e-3)."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_ELEM = 1e-2
TOL_NORM = 4e-3


def rel_errors(y, y_ref):
    y, y_ref = y.double(), y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


@pytest.mark.parametrize("R,C", [(1, 1), (17, 33), (64, 64), (100, 300), (513, 1024), (1536, 8960), (640, 48)])
def test_transpose_codes(pkg, R, C):
    g = torch.Generator(device="cpu").manual_seed(R * 7 + C)
    codes = torch.randint(0, 256, (R, C), generator=g, dtype=torch.int32).to(torch.uint8)
    out = pkg.transpose_codes(codes.to(DEV))
    assert out.shape == (C, R)
    assert torch.equal(out.cpu(), codes.t().contiguous())


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (300, 320, 264), (1000, 1536, 1536), (777, 5120, 1024),
                                   (129, 64, 8)])
def test_fused_dgrad_vs_fp32(pkg, R, M, N, K):
    """grad_q [M, N] @ w_q [N, K] on the fused GEMM (transposed codes, the weight's table)."""
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    assert pkg.dgrad_fused_ok(gq, packed)
    gx = pkg.linear_dgrad(gq, packed)
    ref = gq.float() @ packed.dequantize().float()
    elem, norm = rel_errors(gx, ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


def test_gradient_quant_is_bit_exact(pkg, R):
    """_quant(grad, 224) (hif8_linear.py:93) against the CPU restatement."""
    g = torch.Generator(device="cpu").manual_seed(3)
    gy = (torch.randn(333, 520, generator=g) * 1e-3).to(torch.bfloat16)
    gq, _ = pkg._quant(gy.to(DEV), 224.0)
    want, _ = R.quant_bf16(gy.view(torch.int16).numpy().view(np.uint16), 224.0, "npu")
    assert np.array_equal(gq.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("M,K,N,bias", [(384, 256, 320, True), (1000, 1536, 8960, False), (257, 512, 100, True)])
def test_hif8linear_backward(pkg, M, K, N, bias):
    """HIF8Linear gradients vs the reference formula in fp32 on the same quantised tensors.
    N = 100 takes the vendor-GEMM dgrad (N % 64 != 0); the others the fused dgrad."""
    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    shape = (2, M // 2, K) if M % 2 == 0 else (M, K)
    x = torch.randn(shape, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    lin = pkg.HIF8Linear(K, N, bias=bias, device=DEV, dtype=torch.bfloat16)
    y = lin(x)
    gy = torch.randn(y.shape, generator=g).to(torch.bfloat16).to(DEV)
    y.backward(gy)
    xq, _ = pkg._quant(x.detach(), 15.0)
    wq, _ = pkg._quant(lin.weight.detach(), 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    g2, x2 = gq.reshape(-1, N).float(), xq.reshape(-1, K).float()
    gx = (g2 @ wq.float()).view(x.shape)
    gw = g2.t() @ x2
    checks = [(x.grad, gx), (lin.weight.grad, gw)]
    if bias:
        checks.append((lin.bias.grad, g2.sum(0)))
    for got, want in checks:
        assert got.dtype == torch.bfloat16
        elem, norm = rel_errors(got, want)
        assert elem <= TOL_ELEM and norm <= TOL_NORM, (got.shape, elem, norm)


def test_fp32_input_gradients_promote_like_the_reference(pkg):
    """fp32 x (self-attention o) with a bf16 weight: dgrad in the promoted fp32, wgrad
    g^T @ x_q with x_q fp32 (hif8_linear.py:97,104), grads cast to the inputs' dtypes."""
    M, K, N = 300, 256, 192
    g = torch.Generator(device="cpu").manual_seed(11)
    x = torch.randn(M, K, generator=g).to(DEV).requires_grad_(True)
    lin = pkg.HIF8Linear(K, N, bias=False, device=DEV, dtype=torch.bfloat16)
    y = lin(x)
    gy = torch.randn(y.shape, generator=g).to(torch.bfloat16).to(DEV)
    y.backward(gy)
    assert x.grad.dtype == torch.float32 and lin.weight.grad.dtype == torch.bfloat16
    xq, _ = pkg._quant(x.detach(), 15.0)
    wq, _ = pkg._quant(lin.weight.detach(), 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    for got, want in ((x.grad, gq.float() @ wq.float()), (lin.weight.grad, gq.float().t() @ xq.float())):
        elem, norm = rel_errors(got, want)
        assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


def test_dgrad_config2_shape(pkg):
    """1.3B 480P FFN-down backward shape: grad [32760, 1536] @ w_q [1536, 8960], sampled rows."""
    M, N, K = 32760, 1536, 8960
    g = torch.Generator(device="cpu").manual_seed(4)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    gx = pkg.linear_dgrad(gq, packed)
    rows = torch.cat([torch.randint(0, M, (256,), generator=g), torch.arange(M - 40, M)]).to(DEV)
    ref = gq[rows].float() @ packed.dequantize().float()
    elem, norm = rel_errors(gx[rows], ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


@pytest.mark.parametrize("R,C,pad", [(1, 8, 0), (17, 33, 47), (64, 64, 0), (100, 300, 28), (513, 1024, 63),
                                     (75, 8, 5), (640, 48, 0)])
def test_transpose_bf16(pkg, R, C, pad):
    """[R, C] -> [C, R + pad] with zero columns past R; misaligned sizes take the scalar path."""
    g = torch.Generator(device="cpu").manual_seed(R + C + pad)
    x = torch.randn(R, C, generator=g).to(torch.bfloat16)
    out = pkg.transpose_bf16(x.to(DEV), R + pad)
    want = torch.zeros(C, R + pad, dtype=torch.bfloat16)
    want[:, :R] = x.t()
    assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))


def wgrad_bound(gq, xq, got):
    """Every element of grad_q^T @ x_q within one bf16 unit (2^-7 relative) plus 2^-16 of
    sum |g||x| of the fp64 product (fp32 accumulation over the tokens); a wrong row, column or
    token index gives errors of the order of the values themselves."""
    ref = gq.double().t() @ xq.double()
    tol = ref.abs() * 2.0 ** -7 + (gq.double().abs().t() @ xq.double().abs()) * 2.0 ** -16
    err = (got.double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


@pytest.mark.parametrize("M,N,K", [(64, 256, 256), (300, 320, 264), (1000, 1536, 1536), (4100, 520, 8),
                                   (65, 8, 64), (2049, 5120, 1024), (1, 16, 8), (130, 264, 1032)])
def test_wgrad_vs_fp64(pkg, M, N, K):
    """grad_q^T [N, M] @ x_q [M, K] read token-major (a last partial k-step of tokens, columns past
    a tile's end), bounded against fp64, and bit-identical to the transposed route (both operands
    transposed and zero-padded, then the row-major GEMM): the same MFMA products in the same
    order."""
    print(f"[wgrad] M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 3 + N + K)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    gq, _ = pkg._quant(gy, 224.0)
    xq, _ = pkg._quant(x, 15.0)
    assert pkg.wgrad_ok(gq, xq)
    gw = pkg.linear_wgrad(gq, xq)
    assert gw.shape == (N, K) and gw.dtype == torch.bfloat16
    wgrad_bound(gq, xq, gw)
    gw_t = pkg.linear_wgrad(gq, xq, transposed=True)
    assert torch.equal(gw.view(torch.int16), gw_t.view(torch.int16))


def test_wgrad_config3_full_size_rows(pkg):
    """Wan-14B 720P FFN up backward: grad [75600, 13824], x_q [75600, 5120] (1182 k-steps of 64
    tokens, the last one padded), sampled output rows against fp64."""
    M, N, K = 75600, 13824, 5120
    print(f"[wgrad] full size M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(8)
    gq, _ = pkg._quant(torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16), 224.0)
    xq, _ = pkg._quant(torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16), 15.0)
    gw = pkg.linear_wgrad(gq, xq)
    rows = torch.cat([torch.randint(0, N, (48,), generator=g, device=DEV), torch.arange(N - 16, N, device=DEV)])
    wgrad_bound(gq[:, rows], xq, gw[rows])
    gw_t = pkg.linear_wgrad(gq, xq, transposed=True)
    assert torch.equal(gw.view(torch.int16), gw_t.view(torch.int16))


def test_wgrad_split_tail(pkg):
    """A shape whose last wave of tiles is split: 17 x 16 = 272 tiles of 256 x 256 on 256 CUs
    leave 16 tail tiles, each computed as 8 token ranges whose fp32 sums the reduce kernel adds.
    The split result is bounded against fp64 like the rest, agrees with the unsplit GEMM to
    rounding (the sums only change order), and is the same on a second call."""
    M, N, K = 4100, 4352, 4096
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    L = pkg._lib.load()
    Mp = (M + 63) // 64 * 64
    tiles = (N // 256) * (K // 256)
    nbytes = int(L.hif8_linear_split_workspace_bytes(N, K, Mp))
    tail = tiles % cus
    if cus == 256:
        assert nbytes == tail * 8 * 256 * 256 * 4, nbytes
    print(f"[wgrad] split tail M={M} N={N} K={K} cus={cus} workspace={nbytes}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    gq, _ = pkg._quant(torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16), 224.0)
    xq, _ = pkg._quant(torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16), 15.0)
    split = pkg.linear_wgrad(gq, xq)
    whole = pkg.linear_wgrad(gq, xq, split_tail=False)
    again = pkg.linear_wgrad(gq, xq)
    assert torch.equal(split.view(torch.int16), again.view(torch.int16))
    # the transposed route splits the same tail the same way
    split_t = pkg.linear_wgrad(gq, xq, transposed=True)
    assert torch.equal(split.view(torch.int16), split_t.view(torch.int16))
    wgrad_bound(gq, xq, split)
    wgrad_bound(gq, xq, whole)
    # only the tail tiles' sums change order: about one bf16 rounding step apart at most
    a, b = split.double(), whole.double()
    diff = (a - b).abs()
    floor = b.square().mean().sqrt() * 2.0 ** -12
    assert bool((diff <= torch.maximum(a.abs(), b.abs()) * 2.0 ** -7 + floor).all())
    frac = float((diff > 0).double().mean())
    print(f"[wgrad] split vs whole: {frac:.4%} of outputs differ", flush=True)
    assert frac < 0.1


def test_wgrad_workspace_sizes(pkg):
    """No split for a grid that fills whole waves, runs 8 waves or more, or whose tail is over half
    the CUs, or whose reduction is too short to divide; the 14B FFN-up weight splits 56 tail tiles
    4 ways on 256 CUs."""
    L = pkg._lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert L.hif8_linear_split_workspace_bytes(4096, 4096, 75648) == 0     # 256 tiles: whole waves
    assert L.hif8_linear_split_workspace_bytes(256, 256, 75648) == 0       # fewer tiles than CUs
    assert L.hif8_linear_split_workspace_bytes(4352, 4096, 128) == 0       # 2 k-steps: nothing to split
    if cus == 256:
        assert L.hif8_linear_split_workspace_bytes(13824, 5120, 75648) == 56 * 4 * 256 * 256 * 4
        assert L.hif8_linear_split_workspace_bytes(75600, 5120, 13824) == 0     # 5920 tiles: 23 waves


def test_dgrad_full_size_rows(pkg):
    """Wan-14B 720P FFN-up dgrad on the decode-once route: grad_q [75600, 13824] @ w_q [13824, 5120]
    (216 k-steps).  Its 296 x 20 = 5920 tiles are 23 whole waves on 256 CUs, more than the split
    tail takes (no workspace).  Sampled rows, the last 40 included, against fp32 torch on the same
    operands; the plain decode-free GEMM agrees within one bf16 step."""
    M, N, K = 75600, 13824, 5120
    print(f"[dgrad] full size M={M} N={N} K={K}", flush=True)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert pkg._lib.load().hif8_linear_split_workspace_bytes(M, K, N) == 0
    g = torch.Generator(device=DEV).manual_seed(12)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    packed = pkg.PackedWeight(w, 15.0)
    gq, _ = pkg._quant(torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16), 224.0)
    gx = pkg.linear_dgrad(gq, packed)
    w_qt = pkg.decode(packed.codes_t(), packed.state, torch.bfloat16)
    whole = pkg.linear_fwd_wq(gq, w_qt, None)
    rows = torch.cat([torch.randint(0, M, (256,), generator=g, device=DEV), torch.arange(M - 40, M, device=DEV)])
    ref = gq[rows].float() @ packed.dequantize().float()
    elem, norm = rel_errors(gx[rows], ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)
    a, b = gx[rows].double(), whole[rows].double()
    floor = b.square().mean().sqrt() * 2.0 ** -12
    assert bool(((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * 2.0 ** -7 + floor).all())
