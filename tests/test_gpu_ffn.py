"""GPU parity of the FFN producer fusion (osp_next.py:873-877): the up-projection's
GELU-statistic epilogue, the down-projection's quantisation of GELU(y) (hif8_gelu_fake_quant,
GELU applied on the way in), and HIF8FFN's fused forward.

- The epilogue's y is the plain linear output bit for bit, and the state it settles from max y is
  exactly what a full pass over GELU(y) gives (hif8_gelu_absmax_scale); the pending path (no
  positive output large enough, or a non-finite one) runs that pass and gives the same x_q.
- x_q = _quant(GELU(y)) against torch's bf16 GELU followed by the library's _quant: GELU is the
  device's tanh, so a GELU value may differ from torch's by one bf16 unit on a few elements (and
  its x_q by one HiF8 step there); everywhere else x_q is identical.
- HIF8FFN's fused forward matches the plain sequence within the linear tolerance."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def rel_errors(y, y_ref):
    y, y_ref = y.double(), y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


def ulp_diff(a, b):
    """|bit distance| between two bf16 tensors of the same sign pattern (monotone encoding)."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return (ai - bi).abs()


def _gelu_quant_vs_torch(pkg, y, xq):
    """x_q of GELU(y) against _quant of torch's bf16 GELU: identical except where the two GELUs
    round one bf16 unit apart (at most 1e-3 of the elements), and there one HiF8 step at most."""
    ref_g = torch.nn.functional.gelu(y, approximate="tanh")
    ref, _ = pkg._quant(ref_g, 15.0)
    d = ulp_diff(xq, ref)
    frac = float((d > 0).float().mean())
    assert frac <= 1e-3, frac
    rel = ((xq.float() - ref.float()).abs() / ref.float().abs().clamp(min=1e-30))[d > 0]
    assert rel.numel() == 0 or float(rel.max()) <= 0.5, float(rel.max())


@pytest.mark.parametrize("M,K,N", [(300, 256, 264), (777, 512, 1024), (2048, 1536, 8960), (1, 64, 8)])
def test_gelu_stat_epilogue(pkg, R, M, K, N):
    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    b = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    y_st = pkg.QuantState(x.device)
    y = pkg.linear_fwd_gelu_stat(a, packed, b, y_st, 15.0)
    lin = pkg.linear_fwd(a, fmt, st, packed, b)
    assert torch.equal(y.view(torch.int16), lin.view(torch.int16))          # the plain output
    # the settled state equals a full amax pass over GELU(y); its scale follows the reference rule
    full = pkg.gelu_absmax_scale(y, 15.0, pkg.QuantState(x.device))
    assert y_st.read() == full.read()
    amax_bits, scale = y_st.read()
    sb = R.hif8_scale_bf16(amax_bits, 15.0)
    assert np.float32(scale) == R.bf16_to_f32(np.array([sb], np.uint16))[0]
    xq = pkg.gelu_fake_quant(y, y_st, 15.0)
    assert torch.equal(xq.view(torch.int16), pkg.gelu_fake_quant(y, full, 15.0).view(torch.int16))
    _gelu_quant_vs_torch(pkg, y, xq)


@pytest.mark.parametrize("case", ["small", "neg", "ninf", "nan"])
def test_gelu_stat_pending_states(pkg, case):
    """max y too small to settle amax|GELU(y)| (every output below ~0.26, or all negative), or a
    non-finite output (a -Inf or NaN bias column; GELU(-Inf) is NaN): the state is pending and
    hif8_gelu_fake_quant runs the amax pass first, giving _quant(GELU(y)) exactly as with a state
    from hif8_gelu_absmax_scale (all NaN for a NaN amax, as _quant gives)."""
    g = torch.Generator(device="cpu").manual_seed(len(case))
    M, K, N = 640, 256, 264
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    if case in ("small", "neg"):
        w = w * 0.001
    b = torch.full((N,), -1.0 if case == "neg" else 0.0, dtype=torch.bfloat16, device=DEV)
    if case == "ninf":
        b[7] = float("-inf")
    elif case == "nan":
        b[7] = float("nan")
    packed = pkg.PackedWeight(w, 15.0)
    a, _, _ = pkg.quantize_activation(x, 15.0, "bf16")
    y_st = pkg.QuantState(DEV)
    y = pkg.linear_fwd_gelu_stat(a, packed, b, y_st, 15.0)
    xq = pkg.gelu_fake_quant(y, y_st, 15.0)                        # runs the pending amax pass
    full = pkg.gelu_absmax_scale(y, 15.0, pkg.QuantState(DEV))
    assert y_st.read()[0] == full.read()[0]
    if case in ("ninf", "nan"):
        assert bool(torch.isnan(xq.float()).all())
        return
    assert float(y.float().max()) < 0.26
    assert y_st.read() == full.read()
    assert torch.equal(xq.view(torch.int16), pkg.gelu_fake_quant(y, full, 15.0).view(torch.int16))
    _gelu_quant_vs_torch(pkg, y, xq)


def test_state_reuse_across_calls(pkg):
    """The epilogue resets its accumulators: a second, smaller call leaves the second statistic."""
    g = torch.Generator(device="cpu").manual_seed(7)
    w = (torch.randn(256, 128, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    y_st = pkg.QuantState(DEV)
    for M, mult in ((1000, 8.0), (300, 1.0)):
        x = (torch.randn(M, 128, generator=g) * mult).to(torch.bfloat16).to(DEV)
        a, _, _ = pkg.quantize_activation(x, 15.0, "bf16")
        y = pkg.linear_fwd_gelu_stat(a, packed, None, y_st, 15.0)
        assert y_st.read() == pkg.gelu_absmax_scale(y, 15.0, pkg.QuantState(DEV)).read()


@pytest.mark.parametrize("dim,ffn,M", [(512, 1536, 600), (1536, 8960, 2048)])
def test_hif8ffn_fused_forward(pkg, dim, ffn, M):
    torch.manual_seed(dim)
    mod = pkg.HIF8FFN(dim, ffn, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in mod.parameters():
            p.normal_(0, 0.02)
    x = torch.randn(2, M // 2, dim, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        assert mod.fused_ok(x)
        y = mod(x)
        y_seq = torch.nn.Sequential.forward(mod, x)
    assert y.shape == (2, M // 2, dim) and y.dtype == torch.bfloat16
    elem, norm = rel_errors(y, y_seq)
    assert elem <= 1e-2 and norm <= 4e-3, (elem, norm)
    # and with autograd the module runs the plain sequence
    x.requires_grad_(True)
    assert not mod.fused_ok(x)
    mod(x).float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()


def _all_bf16():
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to(DEV)


# Finite bf16 inputs whose library GELU may differ from torch's on the GPU by one bf16 unit (the
# device's tanh is 1 - 2 / (1 + e^(2|u|)) from the hardware exp2 and reciprocal, not torch's
# tanhf): none, measured over all 65280 finite inputs.
GELU_TORCH_DIFF_MAX = 0


def test_gelu_bf16_every_input(pkg):
    """GELU of every bf16 value through the window route (the one the quantisation pass applies)
    against torch's tanh GELU on the GPU: the closed forms outside the window hold exactly,
    inside it at most GELU_TORCH_DIFF_MAX of the 65280 finite inputs round one unit apart, and the
    non-finite inputs give GELU(+Inf) = +Inf and NaN for -Inf and NaN."""
    print("[gelu] gelu_bf16 over every bf16 input", flush=True)
    y = _all_bf16()
    g = pkg.gelu_bf16(y)
    ref = torch.nn.functional.gelu(y, approximate="tanh")
    yb = y.view(torch.int16).to(torch.int32) & 0xFFFF
    gb = g.view(torch.int16).to(torch.int32) & 0xFFFF
    rb = ref.view(torch.int16).to(torch.int32) & 0xFFFF
    mag, neg = yb & 0x7FFF, yb >= 0x8000
    finite = mag < 0x7F80
    # closed forms
    tiny = finite & (mag < 0x3B20)
    half = (y.float() * 0.5).to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    assert torch.equal(gb[tiny], half[tiny])
    assert torch.equal(gb[finite & ~neg & (mag >= 0x40C0)], yb[finite & ~neg & (mag >= 0x40C0)])
    assert bool((gb[finite & neg & (mag >= 0x40C0)] == 0x8000).all())
    # torch meets the same closed forms there
    outside = finite & ((mag < 0x3B20) | (mag >= 0x40C0))
    assert torch.equal(gb[outside], rb[outside])
    # inside: equal but for a few one-unit roundings
    diff = finite & (gb != rb)
    n = int(diff.sum())
    print(f"[gelu] {n} finite inputs round one unit apart from torch", flush=True)
    assert n <= GELU_TORCH_DIFF_MAX
    if n:
        assert bool(((gb[diff] - rb[diff]).abs() == 1).all())
    # non-finite
    assert int(gb[yb == 0x7F80]) == 0x7F80
    nan_in = ~finite & ~(yb == 0x7F80)
    assert bool(torch.isnan(g[nan_in].float()).all())


@pytest.mark.parametrize("sem", [0, 1])
def test_gelu_quant_table_route_equals_scalar_route(pkg, sem):
    """The GELU quantisation pass through its table of x_q over y (the route of a state that proved
    its input finite) gives the x_q of the per-element route (GELU evaluated for each element, then
    the reference qdq) for every finite bf16 input, at scales that move the tabled range of |y| over
    the whole bf16 range -- the extreme ones (2^-30, 2^30) need more entries than the table holds,
    so part of the range is evaluated element by element.  The input is long enough for the pass's
    span grid.  A state not proven finite takes the per-element route, with the same x_q."""
    print(f"[gelu] table route vs scalar route, semantics {sem}", flush=True)
    y = _all_bf16()
    y = y[(y.view(torch.int16).to(torch.int32) & 0x7F80) != 0x7F80]
    reps = (256 * 16 * 64 * 300) // y.numel() + 1
    y = y[torch.randperm(y.numel(), generator=torch.Generator().manual_seed(sem)).to(DEV)].repeat(reps).contiguous()
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(y.device)
    for scale in (2.0 ** -30, 2.0 ** -12, 1.0 / 3.0, 1.0, 7.5, 2.0 ** 6, 1000.0, 2.0 ** 18, 2.0 ** 30):
        st = pkg.QuantState(DEV)
        pkg._lib.check(L.hif8_set_scale(st.ptr, 0, float(scale), s), "hif8_set_scale")
        st.buf[24:28].view(torch.int32).fill_(1)   # State.finite = 1 (true of y): the table route
        fast = pkg.gelu_fake_quant(y, st, 15.0, sem)
        slow_st = pkg.QuantState(DEV)
        slow_st.buf.copy_(st.buf)
        slow_st.buf[16:20].zero_()                 # State.fast = 0: the per-element route
        slow = pkg.gelu_fake_quant(y, slow_st, 15.0, sem)
        bad = (fast.view(torch.int16) != slow.view(torch.int16)).nonzero().flatten()
        if bad.numel():
            i = bad[:12].cpu()
            yb = [hex(int(v) & 0xFFFF) for v in y.view(torch.int16)[bad[:12]].cpu()]
            fb = [hex(int(v) & 0xFFFF) for v in fast.view(torch.int16)[bad[:12]].cpu()]
            sb = [hex(int(v) & 0xFFFF) for v in slow.view(torch.int16)[bad[:12]].cpu()]
            print(f"[gelu] scale {scale}: {bad.numel()} differ; y {yb} table {fb} reference {sb}", flush=True)
        assert torch.equal(fast.view(torch.int16), slow.view(torch.int16)), scale
        guard_st = pkg.QuantState(DEV)
        guard_st.buf.copy_(st.buf)
        guard_st.buf[24:28].zero_()                # State.finite = 0: per element too
        guarded = pkg.gelu_fake_quant(y, guard_st, 15.0, sem)
        assert torch.equal(guarded.view(torch.int16), slow.view(torch.int16)), scale
    # a short tensor (the grid-stride route) with a tail
    yt = y[: 5 * 4096 + 7].contiguous()
    st = pkg.QuantState(DEV)
    pkg._lib.check(L.hif8_set_scale(st.ptr, 0, 2.5, s), "hif8_set_scale")
    st.buf[24:28].view(torch.int32).fill_(1)
    slow_st = pkg.QuantState(DEV)
    slow_st.buf.copy_(st.buf)
    slow_st.buf[16:20].zero_()
    assert torch.equal(pkg.gelu_fake_quant(yt, st, 15.0, sem).view(torch.int16),
                       pkg.gelu_fake_quant(yt, slow_st, 15.0, sem).view(torch.int16))
