"""GPU parity of the decode-once route (hif8_gemm_w16.hip): the weight decoded once to bf16
(hif8_decode) and the decode-free GEMM (hif8_linear_fwd_wq and its GELU + amax and grouped
forms) against the fused GEMM, which decodes the packed codes inside.

Both kernels issue the same v_mfma_f32_16x16x32_bf16 products on the same operand values in the
same k order, so their outputs are compared bit for bit.  Both are also checked against the fp64
product of the same operands: every output within one bf16 ulp (2^-7 |ref|) plus 2^-16 of
sum |x_q||w_q| (fp32 accumulation); a wrong row, column or k index gives errors of the order of
the output itself.  The fused GEMM is also checked against the oracle in test_gpu_linear.py.
Shapes cover ragged M and N, an odd k-step count and a single k-step."""
from __future__ import annotations

import ctypes

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
# K = 64, 128, 192, 256: one to four k-steps, the edges of both kernels' pipelines (the
# decode-free ring's prologue loads two k-steps; the fused kernel pads an odd count)
SHAPES = [(300, 256, 264), (777, 512, 1024), (256, 64, 256), (1000, 1536, 8960), (2048, 192, 520), (1, 64, 8),
          (4101, 5120, 5120), (513, 128, 776), (257, 128, 8), (64, 320, 264)]


def operands(pkg, M, K, N, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, :3] *= 20
    x = x.to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).to(DEV) if bias else None
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    return a, fmt, st, pkg.PackedWeight(w, 15.0), b


def bound(a, w_q, b, *ys):
    """Asserts every y within one bf16 ulp + 2^-16 sum|x||w| of the fp64 product, and the ys
    equal bit for bit."""
    ref = a.double() @ w_q.double().t()
    if b is not None:
        ref = ref + b.double()
    tol = ref.abs() * 2.0 ** -7 + (a.double().abs() @ w_q.double().abs().t()) * 2.0 ** -16
    for y in ys:
        err = (y.double() - ref).abs()
        assert bool((err <= tol).all()), float((err / tol).max())
    for y in ys[1:]:
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))


def fused(pkg, a, fmt, st, packed, b):
    old = pkg.hif8_linear.GEMM_ROUTE
    pkg.hif8_linear.GEMM_ROUTE = "fused"
    try:
        return pkg.linear_fwd(a, fmt, st, packed, b)
    finally:
        pkg.hif8_linear.GEMM_ROUTE = old


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("bias", [True, False])
def test_wq_matches_fused(pkg, M, K, N, bias):
    print(f"[w16] M={M} K={K} N={N} bias={bias}", flush=True)
    a, fmt, st, packed, b = operands(pkg, M, K, N, M + K + N, bias)
    want = fused(pkg, a, fmt, st, packed, b)
    w_q = packed.dequantize(torch.bfloat16)
    got = pkg.linear_fwd_wq(a, w_q, b)
    torch.cuda.synchronize()
    bound(a, w_q, b, want, got)


def _amax_bits(y):
    return int((y.view(torch.int16).int() & 0x7FFF).max())


@pytest.mark.parametrize("M,K,N", [(300, 256, 264), (2048, 1536, 8960)])
def test_wq_gelu_stat_matches_fused(pkg, M, K, N):
    """The GELU-statistic epilogue on both routes: the plain output, bit for bit, and the same
    settled state (amax of GELU(y) and its scale)."""
    a, fmt, st, packed, b = operands(pkg, M, K, N, 7 * M + N)
    s_f, s_w = pkg.QuantState(DEV), pkg.QuantState(DEV)
    old = pkg.hif8_linear.GEMM_ROUTE
    try:
        pkg.hif8_linear.GEMM_ROUTE = "fused"
        want = pkg.linear_fwd_gelu_stat(a, packed, b, s_f, 15.0)
        pkg.hif8_linear.GEMM_ROUTE = "decode_once"
        got = pkg.linear_fwd_gelu_stat(a, packed, b, s_w, 15.0)
        plain = pkg.linear_fwd(a, fmt, st, packed, b)
    finally:
        pkg.hif8_linear.GEMM_ROUTE = old
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got.view(torch.int16), plain.view(torch.int16))
    assert s_f.read() == s_w.read()
    # the amax the statistic settled is the one a full pass over GELU(y) finds
    s_p = pkg.gelu_absmax_scale(got, 15.0, pkg.QuantState(DEV))
    assert s_f.read() == s_p.read()


def test_wq_grouped_equals_single(pkg):
    M, K = 1000, 512
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    packs, biases = [], []
    for n in (512, 256, 264):
        w = (torch.randn(n, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
        packs.append(pkg.PackedWeight(w, 15.0))
        biases.append((torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(DEV))
    gw = pkg.GroupedWeight(packs, biases)
    old = pkg.hif8_linear.GEMM_ROUTE
    try:
        pkg.hif8_linear.GEMM_ROUTE = "decode_once"
        ys = pkg.linear_fwd_grouped(a, gw)
        pkg.hif8_linear.GEMM_ROUTE = "fused"
        for y, p, b in zip(ys, packs, biases):
            w_q = p.dequantize(torch.bfloat16)
            # a group's output equals the single-weight launch of the same kernel bit for bit
            assert torch.equal(y.view(torch.int16), pkg.linear_fwd_wq(a, w_q, b).view(torch.int16))
            bound(a, w_q, b, pkg.linear_fwd(a, fmt, st, p, b), y)
    finally:
        pkg.hif8_linear.GEMM_ROUTE = old


def test_module_routes_agree(pkg):
    """HIF8Linear gives the same bits on either route (bf16 and fp32 input)."""
    lin = pkg.HIF8Linear(512, 768, device=DEV, dtype=torch.bfloat16)
    x = torch.randn(3000, 512, device=DEV).to(torch.bfloat16)
    outs = {}
    old = pkg.hif8_linear.GEMM_ROUTE
    try:
        for route in ("fused", "decode_once"):
            pkg.hif8_linear.GEMM_ROUTE = route
            with torch.no_grad():
                outs[route] = (lin(x), lin(x.float()))
    finally:
        pkg.hif8_linear.GEMM_ROUTE = old
    for u, v in zip(outs["fused"], outs["decode_once"]):
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))


def test_wq_rejects_bad_shapes(pkg):
    L = pkg._lib.load()
    a = torch.zeros(64, 96, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 96, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(64, 64, dtype=torch.bfloat16, device=DEV)
    s = pkg._lib.stream_ptr(torch.device(DEV))
    assert L.hif8_linear_fwd_wq(a.data_ptr(), w.data_ptr(), None, y.data_ptr(), 64, 64, 96, s) != 0   # K % 64
    assert L.hif8_linear_fwd_wq(a.data_ptr(), w.data_ptr(), None, y.data_ptr(), 64, 60, 64, s) != 0   # N % 8
    assert L.hif8_linear_fwd_wq(a.data_ptr() + 2, w.data_ptr(), None, y.data_ptr(), 64, 64, 64, s) != 0  # align
    assert L.hif8_linear_fwd_wq(None, w.data_ptr(), None, y.data_ptr(), 64, 64, 64, s) != 0
    ns = (ctypes.c_int64 * 2)(100, 64)
    outs = (ctypes.c_void_p * 2)(y.data_ptr(), y.data_ptr())
    assert L.hif8_linear_fwd_wq_grouped(a.data_ptr(), w.data_ptr(), None, outs, ns, 2, 64, 64, s) != 0  # 100 % 256
