"""Pins the CPU oracle (oracle/hif8_ref.py, oracle/hif8_npu_ref.c) to facts that do
not come from retyping its own formulas:

* brute force: the NPU qdq of every finite bf16 value is the nearest HiF8 value
  (ties away from zero), with the overflow cut at 40960 (midpoint to the missing
  1.5*2^15) -- a characterisation independent of the kernel's bit tricks;
* exact rational arithmetic: QFuncs/hif8.py evaluated with Fractions and an
  explicit fp32 rounding (exponent from bit length, not log2) matches the numpy
  restatement bit for bit over every bf16 input and random fp32 inputs;
* real torch: the scale expression ``scale_max / x.abs().amax().clamp(min=1e-8)``,
  bf16 ``x*scale`` and ``q/scale``, and the whole ``_quant`` chain evaluated with
  torch's own CPU kernels;
* special points, invariants, code-table structure, the config-1 known answers
  recorded when the reference was surveyed, and committed fixtures;
* mutation checks: planting a plausible mistake in the oracle makes a pin fail.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


# ----------------------------------------------------------------- helpers


def round_fp32(q: Fraction) -> Fraction:
    """Round a non-negative rational to float32, nearest-even, with subnormals."""
    if q == 0:
        return q
    n, d = q.numerator, q.denominator
    e = n.bit_length() - d.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 23)
    k = q / quantum
    fl = k.numerator // k.denominator
    rem = k - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl * quantum


def floor_log2(q: Fraction) -> int:
    n, d = q.numerator, q.denominator
    e = n.bit_length() - d.bit_length()
    return e - 1 if Fraction(2) ** e > q else e


def torch_exact(xf: float) -> float:
    """QFuncs/hif8.py:6-23 in exact rationals with every fp32 op rounded explicitly.  Its floor of
    log2 is exact (bit length); torch's float32 log2 rounds up to k for the last few floats below
    2^k, which changes the result where |x| + 2^-45 is near 2^-44 or 2^-43: the samples of the
    tests using this avoid those bands, which test_torch_route_fp32_log2_bands_match_torch pins
    against torch itself."""
    if math.isnan(xf) or math.isinf(xf):
        return math.nan
    x = Fraction(xf)
    a = abs(x)
    sign = 1 if x > 0 else (-1 if x < 0 else 0)
    v = round_fp32(a + Fraction(1, 2 ** 45))
    E = floor_log2(v)
    ae = abs(E)
    mb = 3 if ae <= 3 else 2 if ae <= 7 else 1 if ae <= 15 else 0
    t = round_fp32(a * Fraction(2) ** (mb - E))
    u = round_fp32(t + Fraction(1, 2))
    r = u.numerator // u.denominator
    res = round_fp32(r * Fraction(2) ** (E - mb))
    if sign == 0:
        return 0.0
    out = float(res)
    return -out if sign < 0 else out  # r == 0 with x < 0 gives -0.0 as 0 * 2^k * -1 does


def hif8_magnitudes(R) -> np.ndarray:
    d = R.decode_table().astype(np.float64)
    v = np.unique(np.abs(d[np.isfinite(d)]))
    return v


def nearest_hif8(R, xf: np.ndarray) -> np.ndarray:
    """Brute force: nearest finite HiF8 value, ties away from zero, Inf from 40960."""
    V = hif8_magnitudes(R)
    a = np.abs(xf.astype(np.float64))
    hi_i = np.clip(np.searchsorted(V, a, side="right"), 1, len(V) - 1)
    lo, hi = V[hi_i - 1], V[hi_i]
    mag = np.where(a - lo >= hi - a, hi, lo)
    mag = np.where(a >= V[-1], V[-1], mag)
    mag = np.where(a >= 40960.0, np.inf, mag)
    out = np.where(np.signbit(xf) & (mag != 0), -mag, mag)
    return out.astype(np.float32)


def bits32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------- special points


def test_special_points(R):
    x = np.array([1.0625, 15.75, 0.3, -1.0625, 2.5, 3.5, 0.0], np.float32)
    want = np.array([1.125, 16.0, 0.3125, -1.125, 2.5, 3.5, 0.0], np.float32)
    for sem in ("torch", "npu"):
        assert np.array_equal(R.quant_hif8(x, sem), want), sem
    big = np.array([40959.0, 40960.0, -40960.0, 49152.0, 2.0 ** -23, 1.5 * 2.0 ** -24], np.float32)
    npu = R.quant_hif8_npu(big)
    assert npu[0] == 32768.0 and np.isposinf(npu[1]) and np.isneginf(npu[2]) and np.isposinf(npu[3])
    assert npu[4] == 2.0 ** -22 and npu[5] == 0.0
    tor = R.quant_hif8_torch(big)
    assert tor[1] == 49152.0 and tor[3] == 49152.0 and tor[4] == 2.0 ** -23


# ------------------------------------------------------ NPU brute force


def test_npu_equals_nearest_hif8_every_bf16(R):
    xf = R.bf16_to_f32(ALL_BF16)
    fin = ~np.isnan(xf)
    got = R.quant_hif8_npu(xf[fin])
    want = nearest_hif8(R, xf[fin])
    bad = np.nonzero(bits32(got) != bits32(want))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={xf[fin][bad[:5]]}"


def test_npu_nan_and_zero_follow_kernel_selects(R):
    # hif8_quant_op.h:137-150: flushed values are +0; NaN fails both Inf guards -> -Inf
    y = R.quant_hif8_npu(np.array([np.nan, -0.0, -1e-30], np.float32))
    assert np.isneginf(y[0])
    assert bits32(y[1:]).tolist() == [0, 0]


def test_npu_random_fp32_equals_nearest(R):
    rng = np.random.default_rng(7)
    e = rng.integers(-30, 17, 200000)
    m = rng.random(200000) + 1.0
    xf = (np.ldexp(m, e) * rng.choice([-1, 1], 200000)).astype(np.float32)
    got = R.quant_hif8_npu(xf)
    want = nearest_hif8(R, xf)
    assert np.array_equal(bits32(got), bits32(want))


# ------------------------------------------------- torch-path exactness


def test_torch_restatement_matches_exact_rationals_every_bf16(R):
    xf = R.bf16_to_f32(ALL_BF16)
    got = R.quant_hif8_torch(xf)
    with np.errstate(over="ignore"):
        want = np.array([torch_exact(float(v)) for v in xf], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    bad = np.nonzero(bits32(got[~nan]) != bits32(want[~nan]))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={xf[~nan][bad[:5]]}"


def test_torch_restatement_matches_exact_rationals_random_fp32(R):
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32)
    xf = u.view(np.float32)
    xf = xf[np.isfinite(xf)]
    # plus values just below powers of two, where log2 rounding could bite
    k = rng.integers(-60, 60, 2000)
    near = (np.ldexp(1.0, k) * (1 - 2.0 ** -24)).astype(np.float32)
    xf = np.concatenate([xf, near, -near])
    got = R.quant_hif8_torch(xf)
    with np.errstate(over="ignore"):
        want = np.array([torch_exact(float(v)) for v in xf], np.float32)
    assert np.array_equal(bits32(got), bits32(want))


def test_torch_and_npu_agree_on_shared_range(R):
    xf = R.bf16_to_f32(ALL_BF16)
    a = np.abs(xf)
    shared = (a == 0) | ((a >= 2.0 ** -22) & (a < 40960))
    t = R.quant_hif8_torch(xf[shared])
    n = R.quant_hif8_npu(xf[shared])
    assert np.array_equal(bits32(t), bits32(n))
    # and outside it they do differ (the tails are real)
    tails = ~shared & np.isfinite(xf)
    assert (bits32(R.quant_hif8_torch(xf[tails])) != bits32(R.quant_hif8_npu(xf[tails]))).any()


def test_torch_literal_ops_match_numpy(R):
    """The reference's own torch expression (QFuncs/hif8.py:6-23) on torch's CPU
    kernels (oracle.quant_hif8_torch_cpu, also the CPU baseline) against the numpy
    restatement: pins numpy's log2/pow/floor to torch's."""
    torch = pytest.importorskip("torch")
    xf = R.bf16_to_f32(ALL_BF16)
    res = R.quant_hif8_torch_cpu(torch.from_numpy(xf.copy()))
    got = R.quant_hif8_torch(xf)
    r = res.numpy()
    nan = np.isnan(r)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(bits32(r[~nan]), bits32(got[~nan]))


def test_torch_bf16_route_matches_torch_every_bf16(R):
    """quant_dequant_float(bf16, force_py=True, force_fp32=False) runs QFuncs/hif8.py on the bf16
    tensor itself: the reference's expression on torch's CPU bf16 kernels against the oracle's
    bf16 restatement, every finite bf16 input bit for bit (non-finite inputs give NaN)."""
    torch = pytest.importorskip("torch")
    x = torch.from_numpy(ALL_BF16.view(np.int16)).view(torch.bfloat16)
    got = R.quant_hif8_torch_cpu(x).view(torch.int16).numpy().view(np.uint16)
    want = R.quant_hif8_torch_bf16(ALL_BF16)
    fin = np.isfinite(R.bf16_to_f32(ALL_BF16))
    assert np.array_equal(got[fin], want[fin])
    assert np.all((got[~fin] & 0x7FFF) > 0x7F80) and np.all(want[~fin] == 0x7FC0)
    # it differs from the fp32 route (force_fp32=True) only on 128 inputs, all below 2^-43
    f32 = R.f32_to_bf16(R.quant_hif8_torch(R.bf16_to_f32(ALL_BF16)))
    d = np.nonzero((want != f32) & fin)[0]
    assert d.size == 128 and np.abs(R.bf16_to_f32(ALL_BF16[d])).max() < 2.0 ** -43


def test_torch_bf16_log2_is_far_from_bf16_boundaries(R):
    """The bf16 route rounds log2(bf16(|x| + 2^-45)) to bf16.  For every bf16 |x| the exact log2
    lies at least 10 float32 ulps from a bf16 rounding boundary, so a float32 log2 that is off by
    a few ulps (torch's on the CPU, log2f on the GPU) rounds to the same bf16 value."""
    xu = R.bf16_to_f32(ALL_BF16[:0x7F80])                  # every non-negative finite bf16
    t = R.bf16_to_f32(R.f32_to_bf16(xu + np.float32(2.0 ** -45))).astype(np.float64)
    lg = np.log2(t)
    m, e = np.frexp(lg)
    nz = lg != 0
    half = np.ldexp(1.0, e - 9)                             # half a bf16 unit of lg
    dist = half - np.abs(lg - np.ldexp(np.round(m * 256.0), e - 8))
    margin = dist[nz] / np.ldexp(1.0, e[nz] - 24)          # in float32 units of lg
    assert margin.min() >= 10.0, margin.min()


def fp32_log2_band_inputs():
    """float32 x for which v = |x| + 2^-45 lies within 64 units below (or at) a power of two
    2^k, k in [-47, 40], both signs: where torch's float32 log2 of v rounds up to k."""
    xs = []
    for k in range(-47, 41):
        top = np.float32(2.0 ** k).view(np.uint32)
        v = (top - np.arange(0, 64, dtype=np.uint32)).view(np.float32)
        x = (v.astype(np.float64) - 2.0 ** -45).astype(np.float32)
        x = x[x > 0]
        nb = np.concatenate([x, np.nextafter(x, np.float32(0)), np.nextafter(x, np.float32(np.inf))])
        xs.append(nb)
    x = np.unique(np.concatenate(xs))
    return np.concatenate([x, -x]).astype(np.float32)


def test_torch_route_fp32_log2_bands_match_torch(R):
    """The fp32 torch route floors torch's float32 log2 of |x| + 2^-45, which rounds up to the next
    integer for the last few floats below a power of two; where v is near 2^-44 or 2^-43 the
    result depends on it.  The oracle against torch's CPU ops on every such band value."""
    torch = pytest.importorskip("torch")
    x = fp32_log2_band_inputs()
    got = R.quant_hif8_torch_cpu(torch.from_numpy(x)).numpy()
    want = R.quant_hif8_torch(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the band changes results (against the exponent-field floor) near 2^-44 and 2^-43 only
    v = (np.abs(x) + np.float32(2.0 ** -45)).astype(np.float32)
    e_field = ((v.view(np.uint32) >> 23) & 0xFF).astype(np.int64) - 127
    e_torch = np.floor(np.log2(v)).astype(np.int64)
    assert np.any(e_field != e_torch)


def test_torch_f16_route_matches_torch_every_f16(R):
    """quant_dequant_float(fp16, force_py=True, force_fp32=False) runs QFuncs/hif8.py on the fp16
    tensor itself, with the fp16 offset 2^-14 (:10-11): the reference's expression on torch's CPU
    fp16 kernels against the oracle's fp16 restatement, every fp16 input bit for bit (NaN
    wherever torch gives NaN: the NaN and Inf inputs)."""
    torch = pytest.importorskip("torch")
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(allh.view(np.int16)).view(torch.float16)
    got = R.quant_hif8_torch_cpu(x).view(torch.int16).numpy().view(np.uint16)
    want = R.quant_hif8_torch_f16(allh)
    nan_g, nan_w = (got & 0x7FFF) > 0x7C00, (want & 0x7FFF) > 0x7C00
    assert np.array_equal(nan_g, nan_w) and nan_w.sum() == 2048
    assert np.array_equal(got[~nan_g], want[~nan_w])
    xf = R.f16_to_f32(allh)
    fin = np.isfinite(xf)
    # against the fp32 route (force_fp32=True, then the cast back): the 2^-14 offset moves the
    # exponent of every |x| < 2^-11 it changes, 2834 inputs; from 57344 up both give Inf
    f32 = R.quant_dequant_f16(allh, "torch")
    d = np.nonzero((want != f32) & fin)[0]
    assert d.size == 2834 and np.abs(xf[d]).max() < 2.0 ** -11
    big = fin & (np.abs(xf) >= 57344.0)
    assert np.all((want[big] & 0x7FFF) == 0x7C00) and np.all((f32[big] & 0x7FFF) == 0x7C00)
    # known answers of the fp16 grid: ties away from zero, 3/2/1 mantissa bits by |e|
    def q(v):
        return float(R.f16_to_f32(R.quant_hif8_torch_f16(R.f32_to_f16(np.array([v], np.float32))))[0])
    assert q(1.0625) == 1.125 and q(15.75) == 16.0 and q(-0.3) == -0.3125 and q(1000.0) == 1024.0
    assert q(0.0) == 0.0 and q(2.0 ** -14) == 2.0 ** -14


def test_torch_f16_log2_floor_is_stable(R):
    """The fp16 route floors log2(fp16(|x| + 2^-14)) rounded to fp16.  For every fp16 |x| that
    floor is unchanged when log2 is off by up to 32 float32 ulps either way, so torch's float32
    log2 on the CPU and log2f on the GPU give the same exponent.  The rounding to fp16 itself
    moves the floor up a binade on 89 inputs (values just below a power of two), which the
    restatement keeps."""
    xu = R.f16_to_f32(np.arange(0x7C00, dtype=np.uint16))        # every non-negative finite fp16
    t = R.f16_to_f32(R.f32_to_f16(xu + np.float32(2.0 ** -14))).astype(np.float64)
    lg = np.log2(t)
    e0 = np.floor(lg.astype(np.float16).astype(np.float64))
    for s in (-1.0, 1.0):
        lp = lg * (1.0 + s * 32 * 2.0 ** -24)
        assert np.array_equal(np.floor(lp.astype(np.float16).astype(np.float64)), e0)
    assert int(np.sum(e0 != np.floor(lg))) == 89


# ---------------------------------------------------------- invariants


@pytest.mark.parametrize("sem", ["torch", "npu"])
def test_invariants(R, sem):
    xf = R.bf16_to_f32(ALL_BF16)
    xf = xf[np.isfinite(xf)]
    q = R.quant_hif8(xf, sem)
    # odd symmetry (up to the sign of zero)
    qn = R.quant_hif8(-xf, sem)
    assert np.array_equal(q, -qn) or np.array_equal(np.abs(q), np.abs(qn))
    assert np.all((q == -qn) | ((q == 0) & (qn == 0)))
    # idempotence, except where the torch route's +2^-45 offset moves 2^-45 to
    # 2^-44 (QFuncs/hif8.py:13) and -0 (from a negative underflow) to +0
    fin = np.isfinite(q)
    q2 = R.quant_hif8(q[fin], sem)
    same = bits32(q2) == bits32(q[fin])
    if sem == "torch":
        exempt = (np.abs(q[fin]) == 2.0 ** -45) | (q[fin] == 0)
        assert np.all(same | exempt) and np.all(q2[np.abs(q[fin]) == 2.0 ** -45] != 0)
    else:
        assert np.all(same)
    # monotone non-decreasing
    order = np.argsort(xf, kind="stable")
    qs = q[order].astype(np.float64)
    assert np.all(qs[1:] >= qs[:-1])
    # at most 4 significant bits
    m, _ = np.frexp(q[fin & (q != 0)].astype(np.float64))
    assert np.all((np.abs(m) * 16) == np.round(np.abs(m) * 16))


# ---------------------------------------------------------- code table


def test_code_table_structure(R):
    d = R.decode_table()
    assert np.isnan(d[0x80]) and np.isposinf(d[0x6F]) and np.isneginf(d[0xEF]) and d[0] == 0
    fin = np.isfinite(d)
    assert len(np.unique(d[fin])) == 253  # 126 magnitudes x 2 signs + zero
    assert np.abs(d[fin]).max() == 32768.0
    assert np.min(np.abs(d[fin & (d != 0)])) == 2.0 ** -22
    for c in range(256):
        if c in (0x00, 0x80):
            continue
        assert d[c ^ 0x80] == -d[c]
    # every finite non-NaN code round-trips
    codes = np.arange(256, dtype=np.uint8)
    keep = codes != 0x80
    assert np.array_equal(R.encode_npu(d[keep]), codes[keep])
    # exactly the value set of the NPU kernel on bf16 inputs
    xf = R.bf16_to_f32(ALL_BF16)
    qv = np.unique(R.quant_hif8_npu(xf[np.isfinite(xf)]))
    assert np.array_equal(np.sort(qv), np.sort(np.unique(d[~np.isnan(d)])))


# Known answers from the published HiFloat8 layout (Luo et al., "Ascend HiFloat8 Format for Deep
# Learning", 2024): sign | dot prefix (D exponent bits: 11 -> 4, 10 -> 3, 01 -> 2, 001 -> 1,
# 0001 -> 0, 0000 -> denormal) | exponent in sign-magnitude with an implicit leading 1 |
# mantissa (1, 2, 3, 3, 3 bits); denormal 0000 MMM = 2^(M - 23); 0x80 NaN; the 1.5 * 2^15 slot
# of each sign is +-Inf, so 2^15 is the largest finite value.
HIF8_KNOWN = {
    0x00: 0.0, 0x01: 2.0 ** -22, 0x07: 2.0 ** -16,
    0x08: 1.0, 0x09: 1.125, 0x0F: 1.875,                       # D = 0: e = 0
    0x10: 2.0, 0x17: 3.75, 0x18: 0.5, 0x1C: 0.75,               # D = 1: e = +-1
    0x20: 4.0, 0x28: 8.0, 0x2F: 15.0, 0x30: 0.25, 0x38: 0.125,  # D = 2: e = +-2, +-3
    0x40: 16.0, 0x41: 20.0, 0x43: 28.0, 0x4C: 128.0, 0x50: 2.0 ** -4, 0x5F: 1.75 * 2.0 ** -7,  # D = 3
    0x60: 256.0, 0x61: 384.0, 0x6E: 32768.0, 0x70: 2.0 ** -8, 0x7E: 2.0 ** -15, 0x7F: 1.5 * 2.0 ** -15,  # D = 4
    0x6F: np.inf, 0xEF: -np.inf,
    0x81: -(2.0 ** -22), 0x88: -1.0, 0x90: -2.0, 0xC0: -16.0, 0xEE: -32768.0,
}


def test_code_layout_known_answers(R):
    d = R.decode_table()
    for c, v in HIF8_KNOWN.items():
        assert d[c] == v, (hex(c), d[c], v)
    assert np.isnan(d[0x80])
    # and the encoder maps each of these values back to its code
    codes = np.array(sorted(HIF8_KNOWN), np.uint8)
    vals = np.array([HIF8_KNOWN[c] for c in codes], np.float32)
    assert np.array_equal(R.encode_npu(vals), codes)


def test_codes_decode_to_npu_qdq_every_bf16(R):
    xf = R.bf16_to_f32(ALL_BF16)
    fin = ~np.isnan(xf)
    c = R.encode_npu(xf[fin])
    assert np.array_equal(bits32(R.decode(c)), bits32(R.quant_hif8_npu(xf[fin])))


@pytest.mark.parametrize("amax", [1.0, 3.75, 0.013, 200.0, 40000.0])
def test_decode_lut_bf16_is_the_quant_chain_of_its_code(R, amax):
    """x_q as a function of the code: for every finite bf16 x with |x| <= amax (amax itself
    included, so it sets the scale), decode_lut_bf16(scale)[code(x * scale)] equals the whole
    _quant chain's x_q, which test_quant_chain_matches_torch_expression pins against torch.  A
    table built without the division by the scale, or with the fp32 instead of the bf16 rounding
    of decode(c) / scale, fails it."""
    xf = R.bf16_to_f32(ALL_BF16)
    a_bits = int(R.f32_to_bf16(np.array([amax], np.float32))[0])
    amax_b = float(R.bf16_to_f32(np.array([a_bits], np.uint16))[0])
    x = ALL_BF16[np.isfinite(xf) & (np.abs(xf) <= amax_b)]
    x = np.concatenate([x, np.array([a_bits], np.uint16)])
    xq, s_bits = R.quant_bf16(x, 15.0, "npu")
    codes, s2 = R.codes_bf16(x, 15.0)
    assert s2 == s_bits
    lut = R.decode_lut_bf16(s_bits)
    assert np.array_equal(lut[codes], xq)
    s = float(R.bf16_to_f32(np.array([s_bits], np.uint16))[0])
    wrong = R.f32_to_bf16(R.decode_table())                     # no division by the scale
    assert not np.array_equal(wrong[codes], xq)
    if math.frexp(s)[0] != 0.5:                                  # a power-of-two scale divides exactly
        with np.errstate(all="ignore"):
            f32_only = (R.decode_table() / np.float32(s)).astype(np.float32)
        assert not np.array_equal(bits32(f32_only[codes]), bits32(R.bf16_to_f32(xq)))


# ------------------------------------------------- scale and bf16 ops vs torch


def test_scale_matches_torch_every_bf16_amax(R):
    torch = pytest.importorskip("torch")
    a = np.arange(32768, dtype=np.uint16)
    t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    for smax in (15.0, 224.0):
        # hif8_linear.py:45-46, elementwise over every candidate amax
        x_max = t.clamp(min=1e-8)
        scale = smax / x_max
        want = scale.view(torch.int16).numpy().view(np.uint16)
        got = np.array([R.hif8_scale_bf16(int(v), smax) for v in a], np.uint16)
        nan = (want & 0x7FFF) > 0x7F80
        assert np.array_equal(got[~nan], want[~nan])
        assert np.all((got[nan] & 0x7FFF) > 0x7F80)


def test_scale_double_rounding_is_observable(R):
    """A single-rounded scale (bf16(15/amax)) would be a plausible mistake: it
    differs from the reference's bf16(bf16(1/amax)*15) on many inputs."""
    a = np.arange(0x3C00, 0x4400, dtype=np.uint16)  # amax in [2^-7, 2^9)
    af = R.bf16_to_f32(a)
    single = R.f32_to_bf16(np.float32(15.0) / af)
    double = np.array([R.hif8_scale_bf16(int(v), 15.0) for v in a], np.uint16)
    frac = np.mean(single != double)
    assert frac > 0.1, frac


def test_bf16_mul_div_by_scalar_tensor_match_torch(R):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = rng.integers(0, 65536, 200000).astype(np.uint16)
    x = x[(x & 0x7FFF) < 0x7F80]
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    for sbits in (0x4080, 0x407F, 0x4329, 0x3F81, 0x4B19):
        s = torch.tensor(sbits, dtype=torch.int16).view(torch.bfloat16)
        sf = R.bf16_to_f32(np.array([sbits], np.uint16))[0]
        mul = (xt * s).view(torch.int16).numpy().view(np.uint16)
        div = (xt / s).view(torch.int16).numpy().view(np.uint16)
        with np.errstate(all="ignore"):
            assert np.array_equal(mul, R.f32_to_bf16(R.bf16_to_f32(x) * sf))
            assert np.array_equal(div, R.f32_to_bf16(R.bf16_to_f32(x) / sf))


@pytest.mark.parametrize("sem", ["torch", "npu"])
def test_quant_chain_matches_torch_expression(R, sem):
    """hif8_linear.py:42-50 + QTensor.py:94-128 evaluated by torch ops, with the
    qdq step supplied by the oracle (torch path: also evaluated by torch)."""
    torch = pytest.importorskip("torch")
    xb = R.c1_input(seed=9, shape=(257, 129))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    x_max = x.abs().amax().clamp(min=1e-8)
    scale = 15.0 / x_max
    scaled = x * scale
    xf = scaled.to(torch.float32)
    if sem == "torch":
        xu = torch.abs(xf)
        e = torch.floor(torch.log2(xu + 2 ** -45))
        abse = e.abs()
        mb = torch.zeros_like(abse)
        mb[abse <= 15] = 1
        mb[abse <= 7] = 2
        mb[abse <= 3] = 3
        q = torch.floor(xu * 2.0 ** (-e + mb) + 0.5) * 2.0 ** (e - mb) * torch.sign(xf)
    else:
        q = torch.from_numpy(R.quant_hif8_npu(xf.numpy()))
    xq = q.to(torch.bfloat16) / scale
    want = xq.view(torch.int16).numpy().view(np.uint16)
    got, s_bits = R.quant_bf16(xb, 15.0, sem)
    assert s_bits == int(scale.view(torch.int16).item()) & 0xFFFF
    assert np.array_equal(got, want)


def test_torch_cpu_linear_path_matches_bit_emulation(R):
    """The CPU-baseline route (torch ops) equals the bit-level bf16 emulation."""
    torch = pytest.importorskip("torch")
    xb = R.activation_input(4, 96, 64, n_outlier=4)
    wb = R.weight_input(5, 48, 64)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    xq, s = R.quant_torch_cpu(x, 15.0)
    want, s_bits = R.quant_bf16(xb, 15.0, "torch")
    assert np.array_equal(xq.view(torch.int16).numpy().view(np.uint16), want)
    y = R.linear_torch_cpu(x, torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16))
    y_ref, _, _ = R.linear(xb, wb, None, 15.0, "torch", accumulate="torch")
    assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), y_ref)


# ------------------------------------------------------- known answers


def test_config1_known_answers(R, golden):
    """Recorded when the reference was surveyed: amax 3.75, scale 4.0, max|xs| 15,
    41 scaled elements below 2^-22, 33 where the two semantics differ."""
    x = R.c1_input(0)
    a = R.absmax_bf16(x)
    s = R.hif8_scale_bf16(a, 15.0)
    assert R.bf16_to_f32(np.array([a], np.uint16))[0] == 3.75
    assert R.bf16_to_f32(np.array([s], np.uint16))[0] == 4.0
    xs = R.bf16_to_f32(R.f32_to_bf16(R.bf16_to_f32(x) * np.float32(4.0)))
    assert np.abs(xs).max() == 15.0
    assert int(((np.abs(xs) < 2.0 ** -22) & (xs != 0)).sum()) == 41
    qt = R.quant_hif8_torch(xs)
    qn = R.quant_hif8_npu(xs)
    assert int((bits32(qt) != bits32(qn)).sum()) == 33
    assert golden["c1_meta"]["amax_bits"] == a and golden["c1_meta"]["scale_bits"] == s


def test_committed_fixtures_reproduce(R, golden):
    ex = golden["ex"]
    xf = R.bf16_to_f32(ALL_BF16)
    assert np.array_equal(R.f32_to_bf16(R.quant_hif8_npu(xf)), ex["npu_qdq"])
    assert np.array_equal(R.f32_to_bf16(R.quant_hif8_torch(xf)), ex["torch_qdq"])
    assert np.array_equal(R.encode_npu(xf), ex["codes"])
    assert np.all(ex["codes"][np.isnan(xf)] == 0xEF)
    sc = golden["scale"]
    sample = np.arange(0, 32768, 97)
    assert all(R.hif8_scale_bf16(int(a), 15.0) == int(sc["scale15"][a]) for a in sample)
    c1 = golden["c1"]
    x = R.c1_input(0).ravel()
    assert np.array_equal(x[c1["idx"]], c1["x"])


# --------------------------------------------------------- mutation checks


def test_planted_mistakes_are_caught(R):
    """Swap in plausible wrong oracles; the brute-force pin must reject each."""
    xf = R.bf16_to_f32(ALL_BF16)
    xf = xf[np.isfinite(xf)]
    want = nearest_hif8(R, xf)

    def ties_even(x):  # round-half-even instead of half-away
        a = np.abs(x).astype(np.float64)
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -30)))
        mb = np.where(np.abs(e) <= 3, 3, np.where(np.abs(e) <= 7, 2, np.where(np.abs(e) <= 15, 1, 0)))
        step = 2.0 ** (e - mb)
        return (np.sign(x) * np.round(a / step) * step).astype(np.float32)

    def thresholds_off_by_one(x):
        a = np.abs(x).astype(np.float64)
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -30)))
        mb = np.where(np.abs(e) < 3, 3, np.where(np.abs(e) < 7, 2, np.where(np.abs(e) < 15, 1, 0)))
        step = 2.0 ** (e - mb)
        return (np.sign(x) * np.floor(a / step + 0.5) * step).astype(np.float32)

    for wrong in (ties_even, thresholds_off_by_one):
        sel = (np.abs(xf) > 2.0 ** -20) & (np.abs(xf) < 30000)
        assert (bits32(wrong(xf[sel])) != bits32(want[sel])).any(), wrong.__name__


# ------------------------------------------------ modulated LayerNorm producer


def _bf16_ulp(a, b):
    """|distance| in bf16 units between two arrays of bf16 bits (monotone integer encoding)."""
    def key(u):
        u = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


def _modln_case(seed, B=2, N=96, D=1536):
    torch = pytest.importorskip("torch")
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, D, generator=g) * 2 + 0.5
    x[:, :, :4] *= 30                                   # outlier channels
    x = x.to(torch.bfloat16)
    e = (torch.randn(B, 6, D, generator=g) * 0.5).to(torch.bfloat16).chunk(6, dim=1)
    return torch, x, e[0], e[1]


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_modulated_layer_norm_matches_torch_cpu(R):
    """The oracle against the reference's own op sequence run by torch on the CPU
    (want2v.py:96-106 then osp_next.py:941): LayerNorm, a library routine, to one bf16 unit on
    a small fraction of elements (fp32 summation order); the bf16 modulation ops bit-exact."""
    torch, x, shift, scale = _modln_case(3)
    B, N, D = x.shape
    n_t = torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6).type_as(x)
    n_o = R.layer_norm_bf16(_bits(x).reshape(-1, D), 1e-6)
    d = _bf16_ulp(n_o, _bits(n_t).reshape(-1, D))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3, (d.max(), (d > 0).mean())
    # same n -> the modulation is bit-exact against torch's bf16 tensor ops
    n_o_t = torch.from_numpy(n_o.view(np.int16)).view(torch.bfloat16).view(B, N, D)
    y_t = n_o_t * (1 + scale) + shift
    y_o = R.modulated_layer_norm_bf16(_bits(x).reshape(-1, D), _bits(shift).reshape(B, D),
                                      _bits(scale).reshape(B, D), rows_per_batch=N, eps=1e-6)
    assert np.array_equal(y_o, _bits(y_t).reshape(-1, D))
    # and against the whole torch sequence, to the LayerNorm's unit
    y_full = n_t * (1 + scale) + shift
    d = _bf16_ulp(y_o, _bits(y_full).reshape(-1, D))
    assert (d > 0).mean() < 1e-3


def test_modulated_layer_norm_closed_forms(R):
    """Rows with a closed-form norm: a constant row normalises to 0 (then y = shift), and a
    two-valued row +-a to +-a / sqrt(a^2 + eps), which is +-1 in bf16 for a >= 1."""
    D = 64
    x = np.zeros((3, D), np.float32)
    x[0] = 7.25
    x[1, ::2], x[1, 1::2] = 3.0, -3.0
    x[2, ::2], x[2, 1::2] = 1.5, -1.5
    xb = R.f32_to_bf16(x)
    n = R.bf16_to_f32(R.layer_norm_bf16(xb))
    assert np.all(n[0] == 0)
    assert np.array_equal(n[1], np.where(x[1] > 0, 1.0, -1.0).astype(np.float32))
    assert np.array_equal(n[2], np.where(x[2] > 0, 1.0, -1.0).astype(np.float32))
    sh = R.f32_to_bf16(np.linspace(-2, 2, D, dtype=np.float32))[None]
    sc = R.f32_to_bf16(np.full(D, 0.5, np.float32))[None]
    y = R.bf16_to_f32(R.modulated_layer_norm_bf16(xb, sh, sc))
    assert np.array_equal(y[0], R.bf16_to_f32(sh[0]))
    assert np.array_equal(y[1], R.bf16_to_f32(R.f32_to_bf16(np.where(x[1] > 0, 1.5, -1.5) + R.bf16_to_f32(sh[0]))))


def test_modulated_layer_norm_planted_mistakes(R):
    """Plausible wrong restatements (eps dropped, 1 + scale dropped, shift and scale swapped,
    unbiased variance) all fail the torch comparison above."""
    torch, x, shift, scale = _modln_case(5, B=1, N=64, D=512)
    D = x.shape[-1]
    want = _bits(torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6).type_as(x) * (1 + scale) + shift)
    want = want.reshape(-1, D)
    xb, shb, scb = _bits(x).reshape(-1, D), _bits(shift).reshape(1, D), _bits(scale).reshape(1, D)

    def frac(y):
        return float((_bf16_ulp(y, want) > 1).mean())
    assert frac(R.modulated_layer_norm_bf16(xb, shb, scb, eps=1e-6)) == 0.0
    assert frac(R.modulated_layer_norm_bf16(xb, scb, shb, eps=1e-6)) > 0.1          # swapped
    sc_m1 = R.f32_to_bf16(R.bf16_to_f32(scb) - np.float32(1.0))                       # drops the 1 +
    assert frac(R.modulated_layer_norm_bf16(xb, shb, sc_m1, eps=1e-6)) > 0.1
    xs = xb.copy()
    xs[:, 0] = R.f32_to_bf16(R.bf16_to_f32(xs[:, 0]) * np.float32(1.5))              # unnormalised input
    assert frac(R.modulated_layer_norm_bf16(xs, shb, scb, eps=1e-6)) > 0.0
    # unbiased variance (torch.var's default) is off by sqrt(D/(D-1)): visible on most elements
    xf = R.bf16_to_f32(xb).astype(np.float64)
    m = xf.mean(-1, keepdims=True)
    nb = R.f32_to_bf16(((xf - m) / np.sqrt(xf.var(-1, ddof=1, keepdims=True) + 1e-6)).astype(np.float32))
    t = R.f32_to_bf16(np.float32(1) + R.bf16_to_f32(scb))
    u = R.f32_to_bf16(R.bf16_to_f32(nb) * R.bf16_to_f32(t))
    y_bad = R.f32_to_bf16(R.bf16_to_f32(u) + R.bf16_to_f32(shb))
    assert (_bf16_ulp(y_bad, want) > 0).mean() > 0.05


def _affine_case(seed, B=2, N=96, D=1536):
    torch, x, _, _ = _modln_case(seed, B, N, D)
    g = torch.Generator().manual_seed(seed + 1)
    w = 1 + 0.3 * torch.randn(D, generator=g)
    b = 0.2 * torch.randn(D, generator=g)
    return torch, x, w, b


def test_affine_layer_norm_matches_torch_cpu(R):
    """The affine LayerNorm (norm3, want2v.py:96-106 with elementwise_affine) against torch's
    layer_norm on the CPU with fp32 weight and bias, cast back to bf16: a library routine, to
    one bf16 unit on a small fraction of elements (fp32 evaluation order)."""
    torch, x, w, b = _affine_case(11)
    D = x.shape[-1]
    y_t = torch.nn.functional.layer_norm(x.float(), (D,), w, b, eps=1e-6).type_as(x)
    y_o = R.affine_layer_norm_bf16(_bits(x).reshape(-1, D), w.numpy(), b.numpy(), 1e-6)
    yt = _bits(y_t).reshape(-1, D)
    d = _bf16_ulp(y_o, yt)
    assert (d > 0).mean() < 1e-3, (d > 0).mean()
    # where n * w + b cancels, fp32 error relative to |n * w| is several units of the small y:
    # bound each difference by one bf16 unit of y plus fp32-level error of the terms
    n = R.bf16_to_f32(R.layer_norm_bf16(_bits(x).reshape(-1, D), 1e-6)).astype(np.float64)
    terms = np.abs(n * w.numpy()[None]) + np.abs(b.numpy()[None])
    a_o, a_t = R.bf16_to_f32(y_o).astype(np.float64), R.bf16_to_f32(yt).astype(np.float64)
    assert np.all(np.abs(a_o - a_t) <= 2.0 ** -7 * np.abs(a_t) + 2.0 ** -16 * terms)


def test_affine_layer_norm_closed_forms_and_planted_mistakes(R):
    """Closed forms: a constant row normalises to 0, so y = bias exactly; a two-valued row +-a
    (a >= 1) to +-1, so y = bf16(weight + bias) / bf16(bias - weight).  Plausible wrong
    restatements (weight and bias swapped, bias dropped, weight applied before the
    normalisation) fail the torch comparison."""
    D = 64
    x = np.zeros((2, D), np.float32)
    x[0] = 7.25
    x[1, ::2], x[1, 1::2] = 3.0, -3.0
    w = np.linspace(0.5, 2.0, D, dtype=np.float32)
    b = np.linspace(-1.0, 1.0, D, dtype=np.float32)
    y = R.bf16_to_f32(R.affine_layer_norm_bf16(R.f32_to_bf16(x), w, b))
    assert np.array_equal(y[0], R.bf16_to_f32(R.f32_to_bf16(b)))
    want1 = np.where(x[1] > 0, w + b, b - w).astype(np.float32)
    assert np.array_equal(y[1], R.bf16_to_f32(R.f32_to_bf16(want1)))

    torch, xt, wt, bt = _affine_case(13, B=1, N=64, D=512)
    Dt = xt.shape[-1]
    want = _bits(torch.nn.functional.layer_norm(xt.float(), (Dt,), wt, bt, eps=1e-6).type_as(xt)).reshape(-1, Dt)
    xb = _bits(xt).reshape(-1, Dt)

    def frac(yb):
        return float((_bf16_ulp(yb, want) > 1).mean())
    assert frac(R.affine_layer_norm_bf16(xb, wt.numpy(), bt.numpy())) == 0.0
    assert frac(R.affine_layer_norm_bf16(xb, bt.numpy(), wt.numpy())) > 0.1            # swapped
    assert frac(R.affine_layer_norm_bf16(xb, wt.numpy(), np.zeros(Dt, np.float32))) > 0.1   # no bias
    xw = R.f32_to_bf16(R.bf16_to_f32(xb) * wt.numpy()[None])                          # weight first
    assert frac(R.affine_layer_norm_bf16(xw, np.ones(Dt, np.float32), bt.numpy())) > 0.1
