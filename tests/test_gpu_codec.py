"""GPU parity of the HiF8 codec kernels against the CPU oracle and the committed
fixtures: amax/scale, codes, fake-quant (both semantics), decode, and the
unscaled qdq drop-ins.  Integer/byte outputs and every bf16/fp32 value are
compared bit for bit."""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def host_bits(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).cpu().numpy().view(np.uint32)
    return t.cpu().numpy()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_config1_against_fixtures(pkg, golden, R):
    meta = golden["c1_meta"]
    x = dev_bf16(R.c1_input(0))
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    amax, scale = st.read()
    assert amax == meta["amax_bits"]
    assert scale == float(R.bf16_to_f32(np.array([meta["scale_bits"]], np.uint16))[0])
    codes = pkg.encode(x, st)
    assert sha(host_bits(codes)) == meta["sha256_codes"]
    xq_npu = pkg.fake_quant(x, st, pkg._lib.SEM_NPU)
    assert sha(host_bits(xq_npu)) == meta["sha256_xq_npu"]
    xq_torch = pkg.fake_quant(x, st, pkg._lib.SEM_TORCH)
    assert sha(host_bits(xq_torch)) == meta["sha256_xq_torch"]
    assert torch.equal(pkg.decode(codes, st).view(torch.int16), xq_npu.view(torch.int16))
    # the reference module's helper returns the same
    xq2, s2 = pkg._quant(x, 15.0)
    assert torch.equal(xq2.view(torch.int16), xq_npu.view(torch.int16)) and s2.item() == 4.0


def test_raw_qdq_every_bf16(pkg, golden):
    ex = golden["ex"]
    x = dev_bf16(ALL_BF16)
    nan = (ALL_BF16 & 0x7FFF) > 0x7F80
    y = torch.empty_like(x)
    pkg.hif8_quant_bf16(x, y)
    got = host_bits(y)
    assert np.array_equal(got, ex["npu_qdq"])              # NaN included: -Inf, as the Ascend kernel
    assert np.all(got[nan] == 0xFF80)
    yt = pkg.quant_dequant_float(x, pkg.QType("hif8"), force_py=True, force_fp32=True)
    assert np.array_equal(host_bits(yt), ex["torch_qdq"])
    # fp32 drop-in on the same values
    xf = x.float()
    y32 = torch.empty_like(xf)
    pkg.hif8_quant(xf, y32)
    assert np.array_equal(host_bits(y32.to(torch.bfloat16)), ex["npu_qdq"])


def test_torch_bf16_route_every_bf16(pkg, R, golden):
    """quant_dequant_float(bf16, force_py=True) without force_fp32 runs QFuncs/hif8.py in bf16
    arithmetic (HIF8_SEM_TORCH_BF16), every bf16 input against the oracle; with force_fp32 it
    is the fp32 route of the fixture."""
    x = dev_bf16(ALL_BF16)
    want = R.quant_hif8_torch_bf16(ALL_BF16)
    got = host_bits(pkg.quant_dequant_float(x, pkg.QType("hif8"), force_py=True))
    fin = np.isfinite(R.bf16_to_f32(ALL_BF16))
    assert np.array_equal(got[fin], want[fin])
    assert np.all((got[~fin] & 0x7FFF) > 0x7F80)
    y = torch.empty_like(x)
    pkg._lib.check(pkg._lib.load().hif8_quant_bf16(x.data_ptr(), y.data_ptr(), x.numel(), pkg._lib.SEM_TORCH_BF16,
                                                   pkg._lib.stream_ptr(x.device)), "hif8_quant_bf16")
    assert np.array_equal(host_bits(y), got)
    yt = pkg.quant_dequant_float(x, pkg.QType("hif8"), force_py=True, force_fp32=True)
    assert np.array_equal(host_bits(yt), golden["ex"]["torch_qdq"])


def test_fp32_torch_route_log2_bands(pkg, R):
    """The fp32 torch route (HIF8_SEM_TORCH) on every float32 x whose |x| + 2^-45 lies within 64
    units below a power of two 2^k (k in [-47, 40]): the device floors log2 the way torch's
    float32 log2 rounds (up to k for the last few floats below 2^k), bit for bit against the
    oracle, which tests/test_oracle.py pins to torch's CPU ops on the same values."""
    from test_oracle import fp32_log2_band_inputs
    x = fp32_log2_band_inputs()
    xt = torch.from_numpy(x).to(DEV)
    y = torch.empty_like(xt)
    pkg._lib.check(pkg._lib.load().hif8_quant_f32(xt.data_ptr(), y.data_ptr(), xt.numel(), pkg._lib.SEM_TORCH,
                                                  pkg._lib.stream_ptr(xt.device)), "hif8_quant_f32")
    want = R.quant_hif8_torch(x)
    got = host_bits(y)
    bad = np.nonzero(got != want.view(np.uint32))[0]
    assert bad.size == 0, [(float(x[i]), float(y[i]), float(want[i])) for i in bad[:6]]


def test_f16_routes_every_f16(pkg, R):
    """quant_dequant_float of an fp16 tensor (hif8_quant_f16), every fp16 input bit for bit against
    the oracle in its three routes: the NPU kernel on x.float() cast back (force_py=False), the fp32
    torch function cast back (force_py with force_fp32), and the torch function in fp16 arithmetic
    with the 2^-14 offset (force_py alone; the oracle's restatement is pinned to torch's fp16 CPU
    ops).  NaN outputs are compared as NaN."""
    allh = ALL_BF16
    x = torch.from_numpy(allh.view(np.int16)).view(torch.float16).to(DEV)
    Q = pkg.QType("hif8")
    for kw, sem in (({}, "npu"), ({"force_py": True, "force_fp32": True}, "torch"),
                    ({"force_py": True}, "torch_f16")):
        y = pkg.quant_dequant_float(x, Q, **kw)
        assert y.dtype == torch.float16
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        want = R.quant_dequant_f16(allh, sem)
        nan_g, nan_w = (got & 0x7FFF) > 0x7C00, (want & 0x7FFF) > 0x7C00
        assert np.array_equal(nan_g, nan_w), sem
        bad = np.nonzero(got[~nan_g] != want[~nan_w])[0]
        assert bad.size == 0, (sem, [hex(v) for v in allh[~nan_g][bad[:8]]])
    # odd offsets and lengths take the same elementwise route
    xs = x[3:3 + 1001]
    got = pkg.quant_dequant_float(xs, Q, force_py=True).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, R.quant_dequant_f16(allh[3:3 + 1001], "torch_f16"))
    with pytest.raises(ValueError):
        y = torch.empty_like(x)
        pkg.quant._qdq_inplace(x, y, pkg._lib.SEM_TORCH_BF16)


def test_codes_every_bf16_unit_scale(pkg, golden):
    ex = golden["ex"]
    x = dev_bf16(ALL_BF16)
    st = pkg.QuantState(x.device)
    pkg._lib.check(pkg._lib.load().hif8_set_scale(st.ptr, 0, 1.0, pkg._lib.stream_ptr(x.device)), "set_scale")
    got = host_bits(pkg.encode(x, st))
    assert np.array_equal(got, ex["codes"])
    assert np.array_equal(host_bits(pkg.decode(pkg.encode(x, st), st))[(ALL_BF16 & 0x7FFF) <= 0x7F80],
                          ex["npu_qdq"][(ALL_BF16 & 0x7FFF) <= 0x7F80])


def _wide_bf16(rng, n):
    e = rng.integers(-40, 20, n)
    v = np.ldexp(rng.random(n) + 1.0, e) * rng.choice([-1.0, 1.0], n)
    v[rng.random(n) < 0.01] = 0.0
    t = torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("n", [1, 7, 15, 16, 17, 255, 4097, 65539, 1 << 20, (1 << 22) + 4099, 9000011])
def test_bf16_sizes_and_tails(pkg, R, n):
    rng = np.random.default_rng(n)
    xb = _wide_bf16(rng, n)
    x = dev_bf16(xb)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    amax, scale = st.read()
    assert amax == R.absmax_bf16(xb)
    s_bits = R.hif8_scale_bf16(amax, 15.0)
    assert scale == float(R.bf16_to_f32(np.array([s_bits], np.uint16))[0])
    for sem, name in ((pkg._lib.SEM_NPU, "npu"), (pkg._lib.SEM_TORCH, "torch")):
        want, _ = R.quant_bf16(xb, 15.0, name)
        got = host_bits(pkg.fake_quant(x, st, sem))
        assert np.array_equal(got, want), (name, np.nonzero(got != want)[0][:8])
    codes, _ = R.codes_bf16(xb, 15.0)
    c = pkg.encode(x, st)
    assert np.array_equal(host_bits(c), codes)
    want_npu, _ = R.quant_bf16(xb, 15.0, "npu")
    assert np.array_equal(host_bits(pkg.decode(c, st)), want_npu)


@pytest.mark.parametrize("n", [5, 16, 1000, 65536 + 9, (1 << 22) + 771, 6000007])
def test_fp32_path(pkg, R, n):
    rng = np.random.default_rng(100 + n)
    e = rng.integers(-40, 12, n)
    xf = (np.ldexp(rng.random(n) + 1.0, e) * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    x = torch.from_numpy(xf).to(DEV)
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    amax, scale = st.read()
    s_ref = R.hif8_scale_f32(R.absmax_f32(xf), 15.0)
    assert np.float32(scale).view(np.uint32) == np.float32(s_ref).view(np.uint32)
    for sem, name in ((pkg._lib.SEM_NPU, "npu"), (pkg._lib.SEM_TORCH, "torch")):
        want, _ = R.quant_f32(xf, 15.0, name)
        got = host_bits(pkg.fake_quant(x, st, sem))
        assert np.array_equal(got, want.view(np.uint32)), name
    codes = host_bits(pkg.encode(x, st))
    assert np.array_equal(codes, R.encode_npu((xf * np.float32(s_ref)).astype(np.float32)))
    # decode to fp32 and its autocast bf16 rounding
    d32 = pkg.decode(pkg.encode(x, st), st, torch.float32)
    want_npu, _ = R.quant_f32(xf, 15.0, "npu")
    assert np.array_equal(host_bits(d32), want_npu.view(np.uint32))


def test_edge_tensors(pkg, R):
    cases = {
        "zeros": np.zeros(4096, np.uint16),
        "neg_zeros": np.full(4096, 0x8000, np.uint16),
        "one_outlier": np.concatenate([np.full(4095, 0x3C00, np.uint16), [0x4600]]).astype(np.uint16),
        "ties": R.f32_to_bf16(np.array([1.0625, 2.125, 15.75, 0.15625, 7.5, -3.75] * 64, np.float32) / 4),
        "tiny": R.f32_to_bf16(np.ldexp(np.ones(64, np.float32), np.arange(-60, 4)).astype(np.float32)),
    }
    for name, xb in cases.items():
        x = dev_bf16(xb)
        st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
        for sem, sname in ((0, "npu"), (1, "torch")):
            want, _ = R.quant_bf16(xb, 15.0, sname)
            assert np.array_equal(host_bits(pkg.fake_quant(x, st, sem)), want), (name, sname)


def test_nonfinite_tensors_take_the_exact_route(pkg, R):
    """Inf/NaN in the tensor make amax non-finite and the scale 0 or NaN; every
    element then follows the reference's arithmetic one by one, including the NPU
    kernel's -Inf for a NaN scaled value (hif8_quant_op.h:143-150)."""
    for special in (0x7F80, 0xFF80, 0x7FC0):
        xb = np.concatenate([R.f32_to_bf16(np.linspace(-2, 2, 1000).astype(np.float32)), [special]]).astype(np.uint16)
        x = dev_bf16(xb)
        st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
        for sem, sname in ((0, "npu"), (1, "torch")):
            want, _ = R.quant_bf16(xb, 15.0, sname)
            got = host_bits(pkg.fake_quant(x, st, sem))
            wn = (want & 0x7FFF) > 0x7F80
            gn = (got & 0x7FFF) > 0x7F80
            assert np.array_equal(wn, gn), (hex(special), sname)
            assert np.array_equal(got[~wn], want[~wn]), (hex(special), sname)


def test_state_reuse_and_stream_order(pkg, R):
    rng = np.random.default_rng(3)
    st = pkg.QuantState(torch.device(DEV))
    for n in (1 << 18, 1000, 1 << 16):
        xb = _wide_bf16(rng, n)
        x = dev_bf16(xb)
        pkg.absmax_scale(x, 15.0, st)
        want, _ = R.quant_bf16(xb, 15.0, "npu")
        assert np.array_equal(host_bits(pkg.fake_quant(x, st)), want)
        assert st.read()[0] == R.absmax_bf16(xb)


def test_misaligned_views(pkg, R):
    """Offset views are realigned by the Python layer; the C ABI itself refuses them."""
    rng = np.random.default_rng(8)
    xb = _wide_bf16(rng, 4097)
    base = dev_bf16(xb)
    x = base[1:]
    st = pkg.absmax_scale(x, 15.0, pkg.QuantState(x.device))
    want, _ = R.quant_bf16(xb[1:], 15.0, "npu")
    assert np.array_equal(host_bits(pkg.fake_quant(x, st)), want)
    L = pkg._lib.load()
    assert L.hif8_absmax_scale(x.data_ptr(), 0, x.numel(), 15.0, st.ptr, None) == -3
