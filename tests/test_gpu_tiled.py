"""GPU parity of the fast path: fake quant into the GEMM operand layout (XT),
weight-code tiling (WT) and the tiled fused linear.

Layout outputs are compared bit for bit (after undoing the tiling on the host);
the linear output uses the tolerance of test_gpu_linear (max element error
relative to max(|y_ref|, 1e-2 rms) <= 1e-2, normwise <= 4e-3)."""
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


def untile(buf: np.ndarray, rows_pad: int, K: int) -> np.ndarray:
    """XT/WT -> row-major: [rb][ks][kk][half][r][e] -> [rb*32 + r][64ks + 16kk + 8half + e]."""
    a = buf.reshape(rows_pad // 32, K // 64, 4, 2, 32, 8)
    return a.transpose(0, 4, 1, 2, 3, 5).reshape(rows_pad, K)


def rel_errors(y, y_ref):
    y, y_ref = y.double(), y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


@pytest.mark.parametrize("M,K", [(1, 64), (31, 128), (300, 512), (1000, 1536), (4101, 256)])
@pytest.mark.parametrize("sem", ["npu", "torch"])
def test_fake_quant_tiled_bf16(pkg, R, M, K, sem):
    xb = R.activation_input(M * 3 + K, M, K, n_outlier=min(8, K // 8))
    x = dev_bf16(xb)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    xt = pkg.fake_quant_tiled(x, st, pkg._lib.SEM_TORCH if sem == "torch" else pkg._lib.SEM_NPU)
    Mp = pkg.tiled_rows(M)
    assert xt.numel() == Mp * K
    got = untile(xt.view(torch.int16).cpu().numpy().view(np.uint16), Mp, K)
    want, _ = R.quant_bf16(xb, 15.0, sem)
    assert np.array_equal(got[:M], want)
    assert not got[M:].any()


def test_fake_quant_tiled_fp32_is_autocast_rounding(pkg, R):
    M, K = 333, 256
    g = torch.Generator(device="cpu").manual_seed(4)
    e = torch.randint(-30, 8, (M, K), generator=g).float()
    xf = (torch.rand(M, K, generator=g) + 1) * torch.exp2(e) * (torch.randint(0, 2, (M, K), generator=g) * 2 - 1)
    x = xf.to(DEV)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    xt = pkg.fake_quant_tiled(x, st)
    got = untile(xt.view(torch.int16).cpu().numpy().view(np.uint16), pkg.tiled_rows(M), K)[:M]
    xq, _ = R.quant_f32(xf.numpy(), 15.0, "npu")
    assert np.array_equal(got, R.f32_to_bf16(xq))


def test_tile_weight_codes(pkg, R):
    N, K = 520, 192
    wb = R.weight_input(77, N, K)
    packed = pkg.PackedWeight(dev_bf16(wb), 15.0)
    Np = pkg.tiled_rows(N)
    got = untile(packed.wt.cpu().numpy(), Np, K)
    assert np.array_equal(got[:N], packed.codes.cpu().numpy())
    assert not got[N:].any()
    codes, _ = R.codes_bf16(wb, 15.0)
    assert np.array_equal(packed.codes.cpu().numpy(), codes)


@pytest.mark.parametrize("M,N,K", [(1, 8, 64), (17, 24, 128), (256, 256, 64), (300, 264, 128), (513, 520, 192),
                                   (1000, 1536, 1536), (2048, 2048, 512), (777, 5120, 320)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_tiled_linear_vs_oracle(pkg, R, M, N, K, with_bias):
    seed = M * 11 + N * 5 + K
    xb = R.activation_input(seed, M, K, n_outlier=min(8, K // 8))
    wb = R.weight_input(seed + 1, N, K)
    bb = R.weight_input(seed + 2, 1, N)[0] if with_bias else None
    x, w = dev_bf16(xb), dev_bf16(wb)
    b = dev_bf16(bb) if with_bias else None
    packed = pkg.PackedWeight(w, 15.0)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    y = pkg.linear_fwd_tiled(pkg.fake_quant_tiled(x, st), M, packed, b)
    y_ref, _, _ = R.linear(xb, wb, bb, 15.0, "npu", accumulate="f64")
    elem, norm = rel_errors(y.cpu(), torch.from_numpy(y_ref))
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


@pytest.mark.parametrize("N,K,seed", [(1536, 1536, 2), (8960, 1536, 3), (1536, 8960, 4)])
def test_tiled_config2_shapes(pkg, R, N, K, seed):
    M = 32760
    xb = R.activation_input(1, M, K, n_outlier=8)
    wb = R.weight_input(seed, N, K)
    x, w = dev_bf16(xb), dev_bf16(wb)
    b = torch.zeros(N, dtype=torch.bfloat16, device=DEV)
    packed = pkg.PackedWeight(w, 15.0)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    y = pkg.linear_fwd_tiled(pkg.fake_quant_tiled(x, st), M, packed, b)
    xq = pkg.fake_quant(x, st)
    y_ref = xq.float() @ packed.dequantize().float().t()
    elem, norm = rel_errors(y, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


@pytest.mark.parametrize("N,K", [(13824, 5120), (5120, 13824), (5120, 5120)])
def test_tiled_config3_full_size_rows(pkg, N, K):
    """Wan-14B 720P shapes at full size; checked on sampled rows plus the M tail
    against fp32 torch on the same bit-exact operands."""
    M = 75600
    g = torch.Generator(device="cpu").manual_seed(N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[:, torch.randperm(K, generator=g)[:16]] *= 20
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x, w = x.to(DEV), w.to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    y = pkg.linear_fwd_tiled(pkg.fake_quant_tiled(x, st), M, packed, None)
    rows = torch.cat([torch.randint(0, M, (256,), generator=g), torch.arange(M - 80, M)]).to(DEV)
    xq = pkg.fake_quant(x[rows].contiguous(), st)
    y_ref = xq.float() @ packed.dequantize().float().t()
    elem, norm = rel_errors(y[rows], y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


def test_hif8linear_inference_uses_tiled_path(pkg, R):
    M, K, N = 1234, 1024, 768
    xb = R.activation_input(5, M, K, n_outlier=8)
    x = dev_bf16(xb).view(2, 617, K)
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    lin.a_format = "tiled"
    with torch.no_grad():
        lin.bias.normal_(0, 0.1)
        y_fast = lin(x)
    lin.a_format = "bf16"
    with torch.no_grad():
        y_rm = lin(x)
    elem, norm = rel_errors(y_fast, y_rm)
    assert elem <= TOL_ELEM and norm <= 1e-3
    xq, _ = pkg._quant(x, 15.0)
    wq, _ = pkg._quant(lin.weight, 15.0)
    y_ref = (xq.view(-1, K).float() @ wq.float().t() + lin.bias.float()).view(2, 617, N)
    elem, norm = rel_errors(y_fast, y_ref)
    assert elem <= TOL_ELEM and norm <= TOL_NORM
