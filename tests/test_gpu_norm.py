"""GPU parity of the modulated LayerNorm producer (osp_next.py:941, :954 with the WanLayerNorm of
want2v.py:96-106, feeding _quant of hif8_linear.py:42-50):

- y (the kernels' optional output) against the oracle's float64 layer norm and bf16
  modulation: equal except on fewer than 1e-3 of the elements (an fp32 layer norm rounds
  differently from the exact one only next to a bf16 rounding boundary), and there within one
  bf16 unit of the product n * (1 + scale) plus one unit of y;
- the state's amax and scale are exactly the reference rule applied to that y;
- x_q is bit-exactly the oracle's _quant of that y, in both qdq semantics, including rows that
  hold NaN or Inf (the degenerate-scale route);
- q, k, v fed by the fused producer equal three HIF8Linear forwards of y, bit for bit;
- at the 14B 720P shape, amax equals torch's and x_q equals the standalone codec's
  fake quant of y (size-independent consistency);
- shapes outside the fused kernels (dim % 8 != 0, dim > 8192) take the GPU op sequence.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def ulp(a, b):
    def key(u):
        u = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


def make(seed, B, N, D, outliers=4, with_mod=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, D, generator=g) * 2 + 0.25
    x[:, :, :min(outliers, D)] *= 25
    x = x.to(torch.bfloat16)
    if not with_mod:
        return x.to(DEV), None, None
    e = (torch.randn(B, 6, D, generator=g) * 0.5).to(torch.bfloat16).chunk(6, dim=1)
    return x.to(DEV), e[0].to(DEV), e[1].to(DEV)


def oracle_y(R, x, shift, scale):
    B, N, D = x.shape
    sh = None if shift is None else bits(shift).reshape(-1, D)
    sc = None if scale is None else bits(scale).reshape(-1, D)
    rpb = N if (shift is not None and shift.reshape(-1, D).shape[0] > 1) else B * N
    return R.modulated_layer_norm_bf16(bits(x).reshape(-1, D), sh, sc, rows_per_batch=rpb, eps=1e-6)


def check_y(R, yb, x, shift, scale, frac=1e-3):
    """y against the oracle: where they differ, by at most one bf16 unit of the product
    u = n * (1 + scale) plus one unit of y (a one-unit difference of the layer norm n passes
    through the product; the sum with shift can cancel, so y's own units are not the measure),
    and on fewer than ``frac`` of the elements."""
    D = x.shape[-1]
    want = oracle_y(R, x, shift, scale)
    u = oracle_y(R, x, None, scale)            # shift = 0: y is the rounded product itself
    a, b = R.bf16_to_f32(yb).astype(np.float64), R.bf16_to_f32(want).astype(np.float64)
    bound = 2.0 ** -7 * (np.abs(R.bf16_to_f32(u)) + np.abs(b))
    fin = np.isfinite(b)
    assert np.array_equal(np.isfinite(a), fin)
    err = np.abs(a - b)[fin]
    assert np.all(err <= bound[fin]), float((err / np.maximum(bound[fin], 1e-30)).max())
    assert (yb != want).mean() < frac, float((yb != want).mean())


@pytest.mark.parametrize("B,N,D", [(1, 300, 1536), (2, 150, 5120), (1, 5, 8), (3, 7, 72), (1, 33, 8192),
                                   (1, 1, 512), (2, 64, 1536)])
@pytest.mark.parametrize("sem", ["npu", "torch"])
def test_modln_matches_oracle(pkg, R, B, N, D, sem):
    x, shift, scale = make(B * 1000 + N + D, B, N, D)
    semc = pkg._lib.SEM_NPU if sem == "npu" else pkg._lib.SEM_TORCH
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, shift, scale, eps=1e-6, scale_max=15.0, semantics=semc,
                                             return_y=True)
    torch.cuda.synchronize()
    yb = bits(y).reshape(-1, D)
    check_y(R, yb, x, shift, scale)
    amax_bits, scale_f = st.read()
    assert amax_bits == R.absmax_bf16(yb)
    sb = R.hif8_scale_bf16(amax_bits, 15.0)
    assert np.float32(scale_f) == R.bf16_to_f32(np.array([sb], np.uint16))[0]
    want, _ = R.quant_bf16(yb, 15.0, sem)
    assert np.array_equal(bits(xq).reshape(-1, D), want)


def test_modln_without_modulation_is_layer_norm(pkg, R):
    x, _, _ = make(11, 1, 200, 1536, with_mod=False)
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, None, None, return_y=True)
    yb = bits(y).reshape(-1, 1536)
    d = ulp(yb, R.layer_norm_bf16(bits(x).reshape(-1, 1536), 1e-6))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3
    want, _ = R.quant_bf16(yb, 15.0, "npu")
    assert np.array_equal(bits(xq).reshape(-1, 1536), want)


def test_modln_constant_rows_and_broadcast_modulation(pkg, R):
    """A constant row normalises to exactly 0, so y = shift there; a [D] / [1, 1, D] modulation
    broadcasts over every row."""
    x, shift, scale = make(12, 1, 64, 512)
    x[0, 3] = 2.5
    x[0, 10] = -7.0
    sh, sc = shift.reshape(512), scale.reshape(1, 1, 512)
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, sh, sc, return_y=True)
    yb = bits(y).reshape(-1, 512)
    assert np.array_equal(yb[3], bits(sh)) and np.array_equal(yb[10], bits(sh))
    check_y(R, yb, x, shift, scale)
    want, _ = R.quant_bf16(yb, 15.0, "npu")
    assert np.array_equal(bits(xq).reshape(-1, 512), want)


@pytest.mark.parametrize("bad", ["nan", "inf"])
def test_modln_non_finite_rows(pkg, R, bad):
    """A NaN or Inf in x makes its row NaN (mean and variance), the amax NaN and the scale NaN:
    x_q is NaN everywhere, as _quant of such a y is in the reference."""
    x, shift, scale = make(13, 1, 16, 256)
    x[0, 5, 17] = float(bad)
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, shift, scale, return_y=True)
    yb = bits(y).reshape(-1, 256)
    assert np.all((yb[5] & 0x7FFF) > 0x7F80)
    assert np.all((np.delete(yb, 5, axis=0) & 0x7FFF) <= 0x7F80)
    amax_bits, _ = st.read()
    assert (amax_bits & 0x7FFF) > 0x7F80
    want, _ = R.quant_bf16(yb, 15.0, "npu")
    assert np.array_equal(bits(xq).reshape(-1, 256), want)


@pytest.mark.parametrize("D", [5120, 1536, 264])
@pytest.mark.parametrize("case", ["mixed", "nan_row", "few_rows", "overflow"])
def test_modln_amax_from_column_extremes(pkg, R, D, case):
    """With one modulation row, pass 1 takes amax|y| from each column's largest and smallest n
    (y is monotone in n per column).  The cases: columns with 1 + scale < 0 (y decreasing in
    n), constant rows (n = 0), a row of huge finite values whose variance overflows (rstd = 0:
    the row goes through the full chain after the loop), a NaN row among finite ones, fewer
    rows than wavefronts, and a modulation whose product overflows to Inf.  The state's amax
    must be the max of |y| over the kernel's own y, bit for bit, and x_q the codec's quant of y."""
    g = torch.Generator().manual_seed(D + len(case))
    N = 3 if case == "few_rows" else 301
    x = torch.randn(1, N, D, generator=g) * 2 + 0.25
    x[:, :, :3] *= 25
    e = (torch.randn(1, 6, D, generator=g) * 0.5).chunk(6, dim=1)
    shift, scale = e[0].clone(), e[1].clone()
    scale[..., 5:9] = -3.0                                   # t = -2: y decreasing in n
    if case in ("mixed", "nan_row"):
        x[0, 7] = 1.5                                        # constant rows
        x[0, 100] = -0.75
        x[0, 200] = torch.randn(D, generator=g) * 1e25       # sum of squares overflows fp32
    if case == "nan_row":
        x[0, 150, D // 3] = float("nan")
    if case == "overflow":
        scale[..., 11] = 1e38                                # n * t overflows for |n| > 3.4
        x[0, 50, 11] = 40.0                                  # n about 17 there
    x, shift, scale = (t.to(torch.bfloat16).to(DEV) for t in (x, shift, scale))
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, shift, scale, return_y=True)
    yb = bits(y).reshape(-1, D)
    amax_bits, _ = st.read()
    assert amax_bits == R.absmax_bf16(yb)
    if case == "nan_row":
        assert (amax_bits & 0x7FFF) > 0x7F80
    if case == "overflow":
        # Inf in column 11; the word-neighbour's y is Inf * 0 + shift = NaN in the dot2 form
        # (only the diagnostic y differs: x_q is NaN everywhere either way, as amax = Inf
        # gives the reference scale 0 and x_q = 0 / 0)
        assert (amax_bits & 0x7FFF) >= 0x7F80
    if case == "mixed":
        assert np.array_equal(yb[7], bits(shift).reshape(D)) and np.array_equal(yb[100], bits(shift).reshape(D))
    want, _ = R.quant_bf16(yb, 15.0, "npu")
    assert np.array_equal(bits(xq).reshape(-1, D), want)


def test_qkv_from_modulated_norm_equals_three_forwards(pkg):
    D = 1536
    x, shift, scale = make(21, 1, 257, D)
    torch.manual_seed(0)
    lins = [pkg.HIF8Linear(D, D, bias=True).to(DEV).to(torch.bfloat16) for _ in range(3)]
    with torch.no_grad():
        for m in lins:
            m.weight.normal_(0, 0.02)
            m.bias.normal_(0, 0.1)
        q, k, v = pkg.qkv_from_modulated_norm(x, shift, scale, *lins)
        _, _, y = pkg.modulated_norm_quant(x, shift, scale, return_y=True)
        for got, m in zip((q, k, v), lins):
            assert torch.equal(got.view(torch.int16), m(y).view(torch.int16))


def test_modln_rejects_autograd(pkg):
    x, shift, scale = make(22, 1, 8, 64)
    x.requires_grad_(True)
    with pytest.raises(RuntimeError):
        pkg.modulated_norm_quant(x, shift, scale)


@pytest.mark.parametrize("D", [100, 8200])
def test_modln_shapes_outside_the_kernels(pkg, R, D):
    x, shift, scale = make(23, 1, 40, D)
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, shift, scale, return_y=True)
    yb = bits(y).reshape(-1, D)
    check_y(R, yb, x, shift, scale, frac=1e-2)
    want, _ = R.quant_bf16(yb, 15.0, "npu")
    assert np.array_equal(bits(xq).reshape(-1, D), want)


def test_modln_full_size_consistency(pkg):
    """14B 720P: x [75600, 5120].  amax equals torch's amax of the kernel's y, and the fused
    x_q equals the standalone codec's fake quant of y with the same state."""
    g = torch.Generator(device=DEV).manual_seed(31)
    x = torch.randn(1, 75600, 5120, generator=g, device=DEV).to(torch.bfloat16)
    e = (torch.randn(1, 6, 5120, generator=g, device=DEV) * 0.5).to(torch.bfloat16).chunk(6, dim=1)
    with torch.no_grad():
        xq, st, y = pkg.modulated_norm_quant(x, e[0], e[1], return_y=True)
    amax_bits, _ = st.read()
    assert amax_bits == int(y.abs().amax().view(torch.int16).item()) & 0x7FFF
    xq2 = pkg.fake_quant(y, st)
    assert torch.equal(xq.view(torch.int16), xq2.view(torch.int16))
    # y against torch's own fp32 layer norm on the GPU, on a row sample
    rows = torch.randint(0, 75600, (512,), generator=g, device=DEV)
    n = torch.nn.functional.layer_norm(x[0, rows].float(), (5120,), eps=1e-6).to(torch.bfloat16)
    u = n * (1 + e[1][0])
    y_t = u + e[0][0]
    err = (y[0, rows].double() - y_t.double()).abs()
    assert bool((err <= 2.0 ** -7 * (u.double().abs() + y_t.double().abs())).all())
    assert float((y[0, rows] != y_t).double().mean()) < 1e-3


# ------------------------------------------------------------------ affine LayerNorm (norm3)

def affine_norm(pkg, D, seed):
    g = torch.Generator().manual_seed(seed)
    norm = pkg.WanLayerNorm(D, eps=1e-6, elementwise_affine=True).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.3 * torch.randn(D, generator=g))
        norm.bias.copy_(0.2 * torch.randn(D, generator=g))
    return norm


def check_affine_y(R, yb, x, norm, frac=1e-3):
    """y against the oracle's float64 affine layer norm: equal except on fewer than ``frac`` of
    the elements, and there within one bf16 unit of y plus fp32-level error of the terms
    n * w and b (their sum can cancel)."""
    D = x.shape[-1]
    w = norm.weight.detach().cpu().numpy()
    b = norm.bias.detach().cpu().numpy()
    want = R.affine_layer_norm_bf16(bits(x).reshape(-1, D), w, b, 1e-6)
    n = R.bf16_to_f32(R.layer_norm_bf16(bits(x).reshape(-1, D), 1e-6)).astype(np.float64)
    terms = np.abs(n * w[None]) + np.abs(b[None])
    a, t = R.bf16_to_f32(yb).astype(np.float64), R.bf16_to_f32(want).astype(np.float64)
    assert np.all(np.abs(a - t) <= 2.0 ** -7 * np.abs(t) + 2.0 ** -16 * terms)
    assert (yb != want).mean() < frac, float((yb != want).mean())


@pytest.mark.parametrize("B,N,D", [(1, 300, 1536), (2, 150, 5120), (1, 5, 8), (3, 7, 72), (1, 1, 512),
                                   (1, 40, 6144)])
@pytest.mark.parametrize("sem", ["npu", "torch"])
def test_affine_norm_quant_matches_oracle(pkg, R, B, N, D, sem):
    x, _, _ = make(B * 1000 + N + D + 7, B, N, D, with_mod=False)
    norm = affine_norm(pkg, D, D + N)
    semc = pkg._lib.SEM_NPU if sem == "npu" else pkg._lib.SEM_TORCH
    print(f"[affine_norm] B={B} N={N} D={D} {sem}", flush=True)
    with torch.no_grad():
        xq, st, y = pkg.affine_norm_quant(x, norm, 15.0, semc, return_y=True)
    torch.cuda.synchronize()
    yb = bits(y).reshape(-1, D)
    check_affine_y(R, yb, x, norm)
    amax_bits, scale_f = st.read()
    assert amax_bits == R.absmax_bf16(yb)
    sb = R.hif8_scale_bf16(amax_bits, 15.0)
    assert np.float32(scale_f) == R.bf16_to_f32(np.array([sb], np.uint16))[0]
    want, _ = R.quant_bf16(yb, 15.0, sem)
    assert np.array_equal(bits(xq).reshape(-1, D), want)


def test_affine_norm_quant_constant_rows_give_the_bias(pkg, R):
    """A constant row normalises to exactly 0, so y there is bf16(bias)."""
    x, _, _ = make(21, 1, 32, 512, with_mod=False)
    x[0, 5] = 3.25
    norm = affine_norm(pkg, 512, 3)
    with torch.no_grad():
        _, _, y = pkg.affine_norm_quant(x, norm, return_y=True)
    want = bits(norm.bias.detach().to(torch.bfloat16))
    assert np.array_equal(bits(y[0, 5]), want)


def test_affine_norm_quant_falls_back_and_rejects(pkg, R):
    """dim > 6144 or a bf16 weight take the module + _quant on the GPU; the C-ABI rejects
    shapes and pointers outside its contract."""
    x, _, _ = make(22, 1, 16, 8192, with_mod=False)
    norm = affine_norm(pkg, 8192, 4)
    with torch.no_grad():
        xq, st, y = pkg.affine_norm_quant(x, norm, return_y=True)
        assert torch.equal(y, norm(x))
        want, _ = pkg._quant(y, 15.0)
    assert torch.equal(xq.view(torch.int16), want.view(torch.int16))
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(torch.device(DEV))
    xs = torch.zeros(8, 1024, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(8192, dtype=torch.float32, device=DEV)
    stats = torch.empty(16, dtype=torch.float32, device=DEV)
    stq = pkg.QuantState(DEV)
    assert L.hif8_ln_affine_amax(xs.data_ptr(), w.data_ptr(), None, 8, 1024, 1e-6, stats.data_ptr(), 15.0, stq.ptr, s) != 0
    assert L.hif8_ln_affine_amax(xs.data_ptr(), w.data_ptr(), w.data_ptr(), 1, 8192, 1e-6, stats.data_ptr(), 15.0,
                                 stq.ptr, s) != 0                       # dim above the LDS limit
    assert L.hif8_ln_affine_amax(xs.data_ptr(), w.data_ptr() + 4, w.data_ptr(), 8, 1024, 1e-6, stats.data_ptr(),
                                 15.0, stq.ptr, s) != 0                 # misaligned weight
    assert L.hif8_ln_affine_amax(xs.data_ptr(), w.data_ptr(), w.data_ptr(), 8, 1020, 1e-6, stats.data_ptr(), 15.0,
                                 stq.ptr, s) != 0                       # dim % 8
