"""GPU parity of the fused HiF8 linear (hif8_linear_fwd, HIF8Linear) against the
reference fake-quant linear.

Tolerance (north star): max relative error 1e-2 with bf16 output and fp32
accumulation.  "Relative" is taken per element against a floor, so that outputs
near zero do not divide by ~0:
    err = max |y - y_ref| / max(|y_ref|, 1e-2 * rms(y_ref))   <= 1e-2
and the normwise error ||y - y_ref|| / ||y_ref|| is checked against 4e-3.  The
dequantised operands are bit-exact (checked separately), so the only sources of
difference are the fp32 accumulation order and the final bf16 rounding (2^-9).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_ELEM = 1e-2
TOL_NORM = 4e-3


def dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def rel_errors(y: torch.Tensor, y_ref: torch.Tensor):
    y = y.double()
    y_ref = y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    elem = float(((y - y_ref).abs() / floor).max())
    norm = float((y - y_ref).norm() / y_ref.norm())
    return elem, norm


def ref_linear_fp32(xq: torch.Tensor, wq: torch.Tensor, b):
    """Plain PyTorch fp32 reference of F.linear on the (bit-exact) dequantised operands."""
    y = xq.float() @ wq.float().t()
    if b is not None:
        y = y + b.float()
    return y


@pytest.mark.parametrize("M,N,K", [(1, 8, 64), (17, 24, 64), (256, 256, 64), (300, 264, 128),
                                   (513, 520, 192), (1000, 1536, 1536), (2048, 2048, 512)])
@pytest.mark.parametrize("a_fmt", ["bf16", "codes"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fused_linear_small_vs_oracle(pkg, R, M, N, K, a_fmt, with_bias):
    seed = M * 7 + N * 3 + K
    xb = R.activation_input(seed, M, K, n_outlier=min(8, K // 8))
    wb = R.weight_input(seed + 1, N, K)
    bb = R.weight_input(seed + 2, 1, N)[0] if with_bias else None
    x, w = dev_bf16(xb), dev_bf16(wb)
    b = dev_bf16(bb) if with_bias else None
    packed = pkg.PackedWeight(w, 15.0)
    a, fmt, st = pkg.quantize_activation(x, 15.0, a_fmt)
    y = pkg.linear_fwd(a, fmt, st, packed, b)
    torch.cuda.synchronize()
    # operands bit-exact with the oracle
    xq_ref, _ = R.quant_bf16(xb, 15.0, "npu")
    wq_ref, _ = R.quant_bf16(wb, 15.0, "npu")
    assert np.array_equal(packed.dequantize().view(torch.int16).cpu().numpy().view(np.uint16), wq_ref)
    # output vs exactly summed oracle (float64)
    y_ref, _, _ = R.linear(xb, wb, bb, 15.0, "npu", accumulate="f64")
    elem, norm = rel_errors(y.cpu(), torch.from_numpy(y_ref))
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)
    # also against the oracle's torch-semantics linear (the reference CPU path)
    y_ref_t, _, _ = R.linear(xb, wb, bb, 15.0, "torch", accumulate="f64")
    elem, norm = rel_errors(y.cpu(), torch.from_numpy(y_ref_t))
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)
    del xq_ref


def _c2_case(pkg, R, N, K, seed):
    M = 32760
    xb = R.activation_input(1, M, K, n_outlier=8)
    wb = R.weight_input(seed, N, K)
    x, w = dev_bf16(xb), dev_bf16(wb)
    b = torch.zeros(N, dtype=torch.bfloat16, device=DEV)
    return xb, wb, x, w, b


@pytest.mark.parametrize("N,K,seed", [(1536, 1536, 2), (8960, 1536, 3), (1536, 8960, 4)])
def test_config2_shapes(pkg, R, N, K, seed):
    """Wan-1.3B 480P shapes: operands bit-exact vs the oracle; product vs fp32 torch."""
    xb, wb, x, w, b = _c2_case(pkg, R, N, K, seed)
    packed = pkg.PackedWeight(w, 15.0)
    for a_fmt in ("bf16", "codes"):
        a, fmt, st = pkg.quantize_activation(x, 15.0, a_fmt)
        y = pkg.linear_fwd(a, fmt, st, packed, b)
        xq = a if fmt == pkg._lib.A_BF16 else pkg.decode(a, st)
        wq = packed.dequantize()
        y_ref = ref_linear_fp32(xq, wq, b)
        elem, norm = rel_errors(y, y_ref)
        assert elem <= TOL_ELEM and norm <= TOL_NORM, (a_fmt, elem, norm)
    xq_ref, _ = R.quant_bf16(xb, 15.0, "npu")
    wq_ref, _ = R.quant_bf16(wb, 15.0, "npu")
    assert np.array_equal(xq.view(torch.int16).cpu().numpy().view(np.uint16), xq_ref)
    assert np.array_equal(wq.view(torch.int16).cpu().numpy().view(np.uint16), wq_ref)


def test_config3_ffn_up_full_size_rows(pkg, R):
    """Wan-14B 720P FFN up (75600 x 5120 -> 13824), full size on the GPU; checked on
    a row sample against fp32 torch on the same bit-exact operands, plus M-tail rows."""
    M, K, N = 75600, 5120, 13824
    g = torch.Generator(device="cpu").manual_seed(21)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ch = torch.randperm(K, generator=g)[:16]
    x[:, ch] *= 20
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x, w = x.to(DEV), w.to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    y = pkg.linear_fwd(a, fmt, st, packed, None)
    rows = torch.cat([torch.randint(0, M, (384,), generator=g), torch.arange(M - 80, M)]).to(DEV)
    y_ref = a[rows].float() @ packed.dequantize().float().t()
    elem, norm = rel_errors(y[rows], y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)
    # the sampled activation rows are bit-exact vs the oracle's _quant with the full-tensor scale
    amax, scale = st.read()
    xs_rows = x[rows[:64]].cpu().view(torch.int16).numpy().view(np.uint16)
    sb = R.hif8_scale_bf16(amax, 15.0)
    assert R.bf16_to_f32(np.array([sb], np.uint16))[0] == np.float32(scale)
    sf = np.float32(scale)
    xs = R.f32_to_bf16(R.bf16_to_f32(xs_rows) * sf)
    q = R.f32_to_bf16(R.quant_hif8_npu(R.bf16_to_f32(xs)))
    xq_want = R.f32_to_bf16(R.bf16_to_f32(q) / sf)
    assert np.array_equal(a[rows[:64]].cpu().view(torch.int16).numpy().view(np.uint16), xq_want)


def test_hif8linear_module(pkg, R):
    torch.manual_seed(0)
    M, K, N = 777, 1024, 512
    xb = R.activation_input(31, M, K, n_outlier=8)
    x = dev_bf16(xb).view(3, 259, K)
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.bias.normal_(0, 0.1)
    y = lin(x)
    assert y.shape == (3, 259, N) and y.dtype == torch.bfloat16
    # reference composition: _quant(x), _quant(W), F.linear in fp32
    xq, _ = pkg._quant(x, 15.0)
    wq, _ = pkg._quant(lin.weight, 15.0)
    y_ref = ref_linear_fp32(xq.view(-1, K), wq, lin.bias).view(3, 259, N)
    elem, norm = rel_errors(y, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM
    # prepacked weights give the identical result; codes activations within tolerance
    y2 = lin.prepack()(x)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    lin.a_format = "codes"
    y3 = lin(x)
    elem, norm = rel_errors(y3, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM


def test_hif8linear_fp32_input_autocast_semantics(pkg, R):
    """Self-attention o gets fp32 input (osp_next.py:644,777): _quant in fp32, then
    the bf16 autocast cast of x_q; the fused path decodes codes to that bf16."""
    M, K, N = 640, 512, 256
    g = torch.Generator(device="cpu").manual_seed(5)
    xf = torch.randn(M, K, generator=g).to(DEV)
    lin = pkg.HIF8Linear(K, N, bias=False, device=DEV, dtype=torch.bfloat16)
    y = lin(xf)
    xq, _ = pkg._quant(xf, 15.0)                 # fp32 x_q
    xq_ref, s = R.quant_f32(xf.cpu().numpy(), 15.0, "npu")
    assert np.array_equal(xq.cpu().numpy().view(np.uint32), xq_ref.view(np.uint32))
    wq, _ = pkg._quant(lin.weight, 15.0)
    y_ref = ref_linear_fp32(xq.to(torch.bfloat16), wq, None)
    elem, norm = rel_errors(y, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM


def test_hif8linear_backward_matches_reference_formula(pkg):
    M, K, N = 384, 256, 320
    g = torch.Generator(device="cpu").manual_seed(9)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    y = lin(x)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    y.backward(gy)
    # hif8_linear.py:88-111 on the same quantised tensors, in fp32
    xq, _ = pkg._quant(x.detach(), 15.0)
    wq, _ = pkg._quant(lin.weight.detach(), 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    gx = gq.float() @ wq.float()
    gw = gq.float().t() @ xq.float()
    gb = gq.float().sum(0)
    for got, want in ((x.grad, gx), (lin.weight.grad, gw), (lin.bias.grad, gb)):
        elem, norm = rel_errors(got, want)
        assert elem <= TOL_ELEM and norm <= TOL_NORM, (got.shape, elem, norm)


@pytest.mark.parametrize("K,N", [(100, 36), (64, 100), (130, 257), (40, 8)])
def test_hif8linear_shapes_outside_the_fused_gemm(pkg, R, K, N):
    """in_features % 64 != 0 or out_features % 8 != 0: the layer still works (vendor bf16 GEMM
    on the same dequantised operands; none of the model's linears has such a shape)."""
    g = torch.Generator(device="cpu").manual_seed(K * 3 + N)
    x = torch.randn(3, 41, K, generator=g).to(torch.bfloat16).to(DEV)
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.bias.normal_(0, 0.1)
        y = lin(x)
    assert y.shape == (3, 41, N) and y.dtype == torch.bfloat16
    xq, _ = pkg._quant(x, 15.0)
    wq, _ = pkg._quant(lin.weight, 15.0)
    y_ref = ref_linear_fp32(xq.view(-1, K), wq, lin.bias).view(3, 41, N)
    elem, norm = rel_errors(y, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM
