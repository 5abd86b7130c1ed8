"""Linears outside the MFMA kernels' tiles, and layers that compute in fp32, on the library's own
GEMMs -- no vendor or torch GEMM on the product path.

* Forward (``F.linear(x_q, w_q, b)``, hif8_linear.py:86) for in_features % 64 != 0 and
  out_features % 8 != 0: the GEMM routes on zero-padded operands (``hif8_pad_2d``), against the
  CPU oracle's linear (``oracle.hif8_ref.linear``, float64 sums of the bit-exact dequantised
  operands).
* Backward (hif8_linear.py:97,104) at such shapes: dgrad and wgrad on padded operands (bf16), and
  for fp32 layers the library's fp32 GEMM (``hif8_gemm_f32``), against float64 products of the
  oracle's dequantised operands.
* ``QLinear`` (QLinear.py:13-70) on the same GEMMs, with and without autocast.

Every product of these calls runs with torch's GEMMs patched to raise.  Tolerances are those of
the other linear tests: max element error relative to max(|ref|, 1e-2 rms) <= 1e-2 and normwise
<= 4e-3 (bf16 outputs; 1e-4 / 1e-5 for fp32 outputs, fp32 sums of exact products).
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_ELEM, TOL_NORM = 1e-2, 4e-3
TOL_ELEM_F32, TOL_NORM_F32 = 1e-4, 1e-5


def rel_errors(y, y_ref):
    y, y_ref = torch.as_tensor(y).double().cpu(), torch.as_tensor(y_ref).double().cpu()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


@contextlib.contextmanager
def no_torch_gemm():
    """torch's GEMM entry points raise while the block runs."""
    def boom(*a, **k):
        raise AssertionError("a torch GEMM was called on the product path")
    saved = (torch.nn.functional.linear, torch.matmul, torch.mm, torch.bmm, torch.addmm, torch.Tensor.__matmul__,
             torch.Tensor.matmul, torch.Tensor.mm)
    torch.nn.functional.linear = torch.matmul = torch.mm = torch.bmm = torch.addmm = boom
    torch.Tensor.__matmul__ = torch.Tensor.matmul = torch.Tensor.mm = boom
    try:
        yield
    finally:
        (torch.nn.functional.linear, torch.matmul, torch.mm, torch.bmm, torch.addmm, torch.Tensor.__matmul__,
         torch.Tensor.matmul, torch.Tensor.mm) = saved


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dev_bf16(bits, shape):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).reshape(shape).to(DEV)


@pytest.mark.parametrize("M,K,N", [(41, 100, 36), (100, 64, 100), (123, 100, 100), (300, 130, 257), (7, 40, 8),
                                   (9000, 100, 100)])
def test_forward_odd_shapes_vs_oracle(pkg, R, M, K, N):
    """F.linear at in/out features outside the tiles, against the oracle's float64 linear; from
    8192 rows the decode-once route."""
    print(f"[any-shape] forward M={M} K={K} N={N}", flush=True)
    x_bits = R.activation_input(seed=M + K, m=M, k=K, n_outlier=2)
    w_bits = R.weight_input(seed=N + 3, n=N, k=K)
    b_bits = R.weight_input(seed=N + 4, n=1, k=N, std=0.1)[0]
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(dev_bf16(w_bits, (N, K)))
        lin.bias.copy_(dev_bf16(b_bits, (N,)))
        x = dev_bf16(x_bits, (M, K))
        with no_torch_gemm():
            y = lin(x)
            lin.prepack()
            y2 = lin(x)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16 and np.array_equal(bits_of(y2), bits_of(y))
    y_ref, xq, wq = R.linear(x_bits, w_bits, b_bits, 15.0, "npu", accumulate="f64")
    elem, norm = rel_errors(y.float(), torch.from_numpy(y_ref))
    assert elem <= TOL_ELEM and norm <= TOL_NORM, (elem, norm)


@pytest.mark.parametrize("M,K,N", [(257, 100, 100), (384, 512, 100), (200, 100, 64), (130, 72, 200)])
def test_backward_odd_shapes_bf16(pkg, R, M, K, N):
    """dgrad (reduction over N, padded to 64) and wgrad (features padded to 8) on the MFMA GEMMs."""
    print(f"[any-shape] backward bf16 M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 7 + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    with no_torch_gemm():
        y = lin(x)
        y.backward(gy)
    xq, _ = pkg._quant(x.detach(), 15.0)
    wq, _ = pkg._quant(lin.weight.detach(), 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    g64, w64, x64 = gq.double().cpu(), wq.double().cpu(), xq.double().cpu()
    for got, want in ((x.grad, g64 @ w64), (lin.weight.grad, g64.t() @ x64), (lin.bias.grad, g64.sum(0))):
        assert got.dtype == torch.bfloat16
        elem, norm = rel_errors(got, want)
        assert elem <= TOL_ELEM and norm <= TOL_NORM, (tuple(got.shape), elem, norm)


@pytest.mark.parametrize("M,K,N,w_dtype", [(300, 256, 192, torch.bfloat16), (257, 100, 100, torch.float32),
                                           (64, 1536, 40, torch.float32)])
def test_backward_fp32_layer(pkg, M, K, N, w_dtype):
    """An fp32 input with an fp32 or bf16 weight.  The forward is F.linear's bf16 autocast (bf16
    output, so the incoming gradient is bf16); the backward's products take the saved tensors'
    dtypes (hif8_linear.py:97,104): with an fp32 weight both run on the fp32 GEMM with fp32
    results; with a bf16 weight dgrad is the bf16 MFMA dgrad and wgrad (x_q fp32) the fp32 GEMM,
    cast to the weight's dtype."""
    print(f"[any-shape] backward fp32 M={M} K={K} N={N} w={w_dtype}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M + 2 * K + 3 * N)
    x = torch.randn(M, K, generator=g).to(DEV).requires_grad_(True)
    lin = pkg.HIF8Linear(K, N, bias=False, device=DEV, dtype=w_dtype)
    with no_torch_gemm():
        y = lin(x)
        gy = torch.randn(y.shape, generator=g).to(y.dtype).to(DEV)
        y.backward(gy)
    assert y.dtype == torch.bfloat16
    assert x.grad.dtype == torch.float32 and lin.weight.grad.dtype == w_dtype
    xq, _ = pkg._quant(x.detach(), 15.0)
    wq, _ = pkg._quant(lin.weight.detach(), 15.0)
    gq, _ = pkg._quant(gy, 224.0)
    g64, w64, x64 = gq.double().cpu(), wq.double().cpu(), xq.double().cpu()
    f32 = w_dtype == torch.float32
    tol = (TOL_ELEM_F32, TOL_NORM_F32) if f32 else (TOL_ELEM, TOL_NORM)
    elem, norm = rel_errors(x.grad, g64 @ w64)
    assert elem <= tol[0] and norm <= tol[1], ("dgrad", elem, norm)
    elem, norm = rel_errors(lin.weight.grad, g64.t() @ x64)
    assert elem <= tol[0] and norm <= tol[1], ("wgrad", elem, norm)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (65, 70, 17), (300, 64, 1000)])
def test_gemm_f32_strides_vs_fp64(pkg, M, N, K):
    """hif8_gemm_f32 on plain, transposed and bf16 operands, against float64 products."""
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(DEV)
    bt = torch.randn(N, K, generator=g).to(DEV)          # b = bt^T as a strided view
    ref = a.double().cpu() @ bt.double().cpu().t()
    c = pkg.gemm_f32(a, bt, M, N, K, (K, 1), (1, K))
    assert rel_errors(c, ref)[1] <= 1e-6
    c16 = pkg.gemm_f32(a.to(torch.bfloat16), bt, M, N, K, (K, 1), (1, K), out_dtype=torch.bfloat16)
    ref16 = a.to(torch.bfloat16).double().cpu() @ bt.double().cpu().t()
    assert c16.dtype == torch.bfloat16 and rel_errors(c16, ref16)[1] <= 4e-3
    at = a.t().contiguous()                               # a given as its transpose's strides
    c2 = pkg.gemm_f32(at, bt, M, N, K, (1, M), (1, K))
    assert torch.equal(c2, c)


@pytest.mark.parametrize("shape", [((5, 7), (9, 12)), ((1, 1), (3, 1)), ((100, 36), (100, 36)), ((33, 16), (16, 8))])
@pytest.mark.parametrize("dtype", [torch.uint8, torch.bfloat16, torch.float32])
def test_pad_2d(pkg, shape, dtype):
    (r, c), (dr, dc) = shape
    src = (torch.arange(r * c, device=DEV) % 251 + 1).to(dtype).view(r, c)
    out = pkg.pad_2d(src, dr, dc)
    want = torch.zeros(dr, dc, dtype=dtype, device=DEV)
    rr, cc = min(r, dr), min(c, dc)
    want[:rr, :cc] = src[:rr, :cc]
    assert torch.equal(out, want)


@pytest.mark.parametrize("autocast", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qlinear_on_library_gemms(pkg, R, autocast, dtype):
    """QLinear's F.linear and backward matmuls (QLinear.py:13-70) on the library's GEMMs at an
    odd shape: bf16 under autocast or for bf16 operands, fp32 otherwise."""
    if dtype == torch.bfloat16 and autocast:
        pytest.skip("autocast of a bf16 layer is the bf16 case")
    print(f"[any-shape] QLinear dtype={dtype} autocast={autocast}", flush=True)
    torch.manual_seed(3)
    lin = pkg.QLinear(100, 36, bias=True).to(DEV).to(dtype)
    lin.assign_qparams("hif8")
    g = torch.Generator(device="cpu").manual_seed(4)
    x = (torch.randn(2, 25, 100, generator=g) * 3).to(dtype).to(DEV).requires_grad_(True)
    gy = torch.randn(2, 25, 36, generator=g).to(DEV)
    with no_torch_gemm(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        y = lin(x)
        y.backward(gy.to(y.dtype))
    low = autocast or dtype == torch.bfloat16
    assert y.dtype == (torch.bfloat16 if low else torch.float32)
    Q = pkg.QType("hif8")
    xq = pkg.quant_dequant_float(x.detach(), Q, force_fp32=True)
    wq = pkg.quant_dequant_float(lin.weight.detach(), Q, force_fp32=True)
    gq = pkg.quant_dequant_float(gy.to(y.dtype), Q, force_fp32=True)
    if low:
        xq, wq = xq.to(torch.bfloat16), wq.to(torch.bfloat16)
    x64, w64, g64 = xq.double().cpu().view(-1, 100), wq.double().cpu(), gq.double().cpu().view(-1, 36)
    bias = lin.bias.detach().to(y.dtype).double().cpu()
    tol = (TOL_ELEM, TOL_NORM) if low else (TOL_ELEM_F32, TOL_NORM_F32)
    for got, want in ((y.view(-1, 36), x64 @ w64.t() + bias), (x.grad.view(-1, 100), g64 @ w64),
                      (lin.weight.grad, g64.t() @ x64)):
        elem, norm = rel_errors(got, want)
        assert elem <= tol[0] and norm <= tol[1], (tuple(got.shape), elem, norm)
