"""The device scale rule of ``_quant`` (hif8_linear.py:45-46), swept on the GPU.

``x_max = |x|.amax().clamp(min=1e-8)`` and ``scale = scale_max / x_max`` (evaluated by torch as
``x_max.reciprocal() * scale_max``, each op rounded to the tensor dtype), then the decode tables
x_q(code) = rnd(decode(code) / scale).  The device computes them in ``scale_from_amax`` and
``fill_luts`` with IEEE-rounded division: a fast reciprocal or a changed build flag would break
the rule for some amax values.  Here ``hif8_absmax_scale`` runs on a one-element tensor for
EVERY bf16 amax (all 32768 magnitudes, NaN and Inf included) with scale_max 15 and 224, and the
state's amax, scale, flags and both tables are compared bit for bit with the committed fixture
``tests/golden/hif8_scale_bf16.npz`` (written by the oracle, which ``tests/test_oracle.py`` pins
to torch's own scalar ops over the same table) and with the oracle's decode tables.  fp32 states
are checked on a sample that covers every binade, the clamp and the overflow ends.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
# State layout (hif8_internal.h): amax_bits @8, scale (fp32) @12, fast @16, dtype @20, finite @24,
# lut_bf16[256] @32, lut_f32[256] @544
OFF_AMAX, OFF_SCALE, OFF_FAST, OFF_LUT16, OFF_LUT32 = 8, 12, 16, 32, 544


def _run_states(pkg, x_rows: torch.Tensor, dtype_code: int, smaxes):
    """hif8_absmax_scale of row i of x_rows (its first element; n = 1) into state (i, j) for each
    scale_max j; returns the states' leading fields as a host array [rows, len(smaxes), 1568]."""
    L = pkg._lib.load()
    S = pkg._lib.state_size()
    rows = x_rows.shape[0]
    st = torch.zeros(rows * len(smaxes) * S, dtype=torch.uint8, device=DEV)
    s = pkg._lib.stream_ptr(torch.device(DEV))
    base, row_bytes = x_rows.data_ptr(), x_rows.stride(0) * x_rows.element_size()
    assert row_bytes % 16 == 0 and base % 16 == 0
    sb = st.data_ptr()
    for i in range(rows):
        for j, smax in enumerate(smaxes):
            rc = L.hif8_absmax_scale(base + i * row_bytes, dtype_code, 1, float(smax), sb + (i * len(smaxes) + j) * S,
                                     s)
            if rc != 0:
                raise AssertionError(f"hif8_absmax_scale rc {rc} at row {i}")
    torch.cuda.synchronize()
    # the fields compared below end with lut_f32 (byte 1568); the rest of a state is not copied
    return st.view(rows, len(smaxes), S)[:, :, :OFF_LUT32 + 1024].cpu().numpy()


def _fields(h):
    amax = h[..., OFF_AMAX:OFF_AMAX + 4].copy().view(np.uint32)[..., 0]
    scale = h[..., OFF_SCALE:OFF_SCALE + 4].copy().view(np.uint32)[..., 0]
    fast = h[..., OFF_FAST:OFF_FAST + 4].copy().view(np.uint32)[..., 0]
    lut16 = h[..., OFF_LUT16:OFF_LUT16 + 512].copy().view(np.uint16)
    lut32 = h[..., OFF_LUT32:OFF_LUT32 + 1024].copy().view(np.uint32)
    return amax, scale, fast, lut16, lut32


def test_scale_rule_every_bf16_amax(pkg, R, golden):
    sc = golden["scale"]
    amax_bits = sc["amax"].astype(np.uint16)                        # 0 .. 0x7FFF, every magnitude
    rows = np.zeros((amax_bits.size, 8), np.uint16)                # 16-byte rows, the value first
    rows[:, 0] = amax_bits
    x = torch.from_numpy(rows.view(np.int16)).view(torch.bfloat16).to(DEV)
    smaxes = (15.0, 224.0)
    h = _run_states(pkg, x, pkg._lib.DTYPE_BF16, smaxes)
    amax, scale, fast, lut16, lut32 = _fields(h)
    assert np.array_equal(amax[:, 0], amax_bits.astype(np.uint32)) and np.array_equal(amax[:, 1], amax[:, 0])
    table = R.decode_table().astype(np.float32)
    cache = {}
    for j, key in enumerate(("scale15", "scale224")):
        want = sc[key].astype(np.uint32)
        got = scale[:, j]
        nan_w = (want & 0x7FFF) > 0x7F80
        nan_g = (got & 0x7FFFFFFF) > 0x7F800000
        assert np.array_equal(nan_g, nan_w), key
        # the fp32 scale holds the bf16 value exactly
        assert np.array_equal(got[~nan_g], want[~nan_w] << 16), (key, np.nonzero(got[~nan_g] != want[~nan_w] << 16)[0][:8])
        sf = (want << 16).view(np.float32)
        amax_f = R.bf16_to_f32(amax_bits)
        fast_w = np.isfinite(amax_f) & np.isfinite(sf) & (sf > 0)
        assert np.array_equal(fast[:, j].astype(bool), fast_w), key
        # decode tables: bf16 x_q(code) from the oracle, fp32 decode(code) / scale (IEEE division)
        for sb in np.unique(want[~nan_w]):
            if int(sb) not in cache:
                s32 = np.float32((np.uint32(sb) << 16).view(np.float32))
                with np.errstate(all="ignore"):
                    q32 = (table / s32).astype(np.float32).view(np.uint32)
                cache[int(sb)] = (R.decode_lut_bf16(int(sb)), q32)
        for i in np.nonzero(~nan_w)[0]:
            w16, w32 = cache[int(want[i])]
            g16, g32 = lut16[i, j], lut32[i, j]
            ok16 = (g16 == w16) | (((g16 & 0x7FFF) > 0x7F80) & ((w16 & 0x7FFF) > 0x7F80))
            ok32 = (g32 == w32) | (((g32 & 0x7FFFFFFF) > 0x7F800000) & ((w32 & 0x7FFFFFFF) > 0x7F800000))
            assert ok16.all() and ok32.all(), (key, hex(int(amax_bits[i])), np.nonzero(~ok16)[0][:4],
                                               np.nonzero(~ok32)[0][:4])


def _f32_sample():
    rng = np.random.default_rng(2024)
    v = [np.float32(0.0), np.float32(1e-8), np.nextafter(np.float32(1e-8), np.float32(0)),
         np.nextafter(np.float32(1e-8), np.float32(1)), np.float32(np.finfo(np.float32).tiny),
         np.float32(1e-45), np.float32(np.finfo(np.float32).max), np.float32(np.inf), np.float32(np.nan),
         np.float32(15.0), np.float32(224.0), np.float32(1.0), np.float32(3.75)]
    # every binade, random mantissas, plus the largest values (reciprocal near the subnormal range)
    e = np.repeat(np.arange(-149, 128), 24)
    m = rng.random(e.size) + 1.0
    v += list(np.ldexp(m, e).astype(np.float32))
    v += list(np.float32(np.finfo(np.float32).max) * rng.random(200).astype(np.float32))
    v = np.array(v, np.float32)
    return v[np.isnan(v) | (v >= 0)]


def test_scale_rule_f32_sample(pkg, R):
    v = _f32_sample()
    rows = np.zeros((v.size, 4), np.float32)                        # 16-byte rows
    rows[:, 0] = v
    x = torch.from_numpy(rows).to(DEV)
    smaxes = (15.0, 224.0)
    h = _run_states(pkg, x, pkg._lib.DTYPE_F32, smaxes)
    amax, scale, fast, lut16, lut32 = _fields(h)
    assert np.array_equal(amax[:, 0], v.view(np.uint32) & np.uint32(0x7FFFFFFF))
    table = R.decode_table().astype(np.float32)
    for j, smax in enumerate(smaxes):
        want = np.array([R.hif8_scale_f32(a, smax) for a in v], np.float32)
        got = scale[:, j].view(np.float32)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), \
            (smax, v[~nan][got[~nan] != want[~nan]][:6])
        fast_w = np.isfinite(v) & np.isfinite(want) & (want > 0)
        assert np.array_equal(fast[:, j].astype(bool), fast_w)
        for i in np.nonzero(fast_w)[0][::7]:
            with np.errstate(all="ignore"):
                q = (table / want[i]).astype(np.float32)
            assert np.array_equal(lut32[i, j], q.view(np.uint32))
            assert np.array_equal(lut16[i, j], R.f32_to_bf16(q))
