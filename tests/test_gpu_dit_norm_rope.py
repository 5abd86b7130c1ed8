"""GPU parity of hif8_rms_norm_rope (the DiT block's q/k RMSNorm + 3-D RoPE + bf16 cast in one
pass) against the harness's torch op sequence: OSPNextRMSNorm (fp32 weight, bf16 output), then
SkiparseRopeWrapper.apply_rope (fp32), then the attention's cast to bf16.

The kernel keeps every rounding point of that sequence; only the sum of squares is taken in a
different order, so rsqrt can differ by an ulp and y = rnd_bf16(x * rsqrt) by one bf16 step where
x * rsqrt lies next to a rounding boundary.  The check: fewer than 1 % of outputs differ at all,
and each output is within 2^-7 of the norm of its rotated pair (one bf16 step of the pair, which
the rotation preserves).  A wrong pair, angle, head or weight index breaks both."""
from __future__ import annotations

import ctypes

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def torch_path(D, x, norm, rope, grid, rearrange, H):
    B, N, dim = x.shape
    y = norm(x)
    if rope is None:
        return y
    y = rope.apply_rope(y.view(B, N, H, dim // H), grid, rearrange)
    return y.to(torch.bfloat16).reshape(B, N, dim)


def check(got, want, pairs=True):
    g, w = got.float(), want.float()
    diff = (g - w).abs()
    if pairs:
        mag = w.view(*w.shape[:-1], -1, 2).norm(dim=-1, keepdim=True).expand(*w.shape[:-1], w.shape[-1] // 2, 2)
        mag = mag.reshape(w.shape)
    else:
        mag = w.abs()
    assert bool((diff <= mag * 2.0 ** -7 + 1e-30).all()), float((diff / (mag + 1e-30)).max())
    frac = float((got.view(torch.int16) != want.view(torch.int16)).float().mean())
    assert frac < 0.01, frac


@pytest.mark.parametrize("B,grid,P,kind", [(1, (3, 8, 10), 1, "identity"), (4, (3, 8, 10), 2, "token"),
                                            (8, (2, 6, 8), 2, "group")])
def test_norm_rope_matches_torch(pkg, B, grid, P, kind):
    D = pkg.dit
    H, hd = 40, 128
    dim = H * hd
    rt = {"identity": D.RearrangeType.Identity, "token": D.RearrangeType.Skiparse2DToken,
          "group": D.RearrangeType.Skiparse2DGroup}[kind]
    rearr = D.SkiparseRearrange(P, rt)
    rope = D.SkiparseRopeWrapper(D.rope_freqs(hd).to(DEV))
    N = rope.prepare_freqs(grid, hd // 2, rearr)[0].shape[1]   # tokens per sequence, padding included
    g = torch.Generator().manual_seed(B * 100 + N)
    x = (torch.randn(B, N, dim, generator=g) * 3).to(torch.bfloat16).to(DEV)
    norm = D.OSPNextRMSNorm(dim, eps=1e-6, device=DEV)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.3 * torch.randn(dim, generator=g)).to(DEV))
    print(f"[norm_rope] B={B} N={N} grid={grid} {kind}", flush=True)
    with torch.no_grad():
        want = torch_path(D, x, norm, rope, grid, rearr, H)
        cos_f, sin_f = rope.prepare_freqs(grid, hd // 2, rearr)
        got = D.rms_norm_rope(x, norm, cos_f, sin_f, hd)
    torch.cuda.synchronize()
    check(got, want)


def test_norm_only_matches_torch(pkg):
    D = pkg.dit
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(2, 333, 5120, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    norm = D.OSPNextRMSNorm(5120, eps=1e-6, device=DEV)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.3 * torch.randn(5120, generator=g)).to(DEV))
        want = norm(x)
        got = D.rms_norm_rope(x, norm)
    check(got, want, pairs=False)


def test_rejects_bad_shapes(pkg):
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(torch.device(DEV))
    x = torch.zeros(8, 1024, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(1024, dtype=torch.float32, device=DEV)
    c = torch.ones(8, 64, dtype=torch.float32, device=DEV)
    o = torch.empty_like(x)
    assert L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), None, None, o.data_ptr(), 8, 1000, 128, 1, 1, 1e-6, s) != 0
    assert L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), c.data_ptr(), None, o.data_ptr(), 8, 1024, 128, 8, 1, 1e-6, s) != 0
    assert L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), c.data_ptr(), c.data_ptr(), o.data_ptr(), 8, 1024, 96, 8, 1,
                                1e-6, s) != 0   # 512 % head_dim
    assert L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), c.data_ptr(), c.data_ptr(), o.data_ptr(), 8, 1024, 128, 3, 1,
                                1e-6, s) != 0   # rows % seq
    assert L.hif8_rms_norm_rope(x.data_ptr() + 2, w.data_ptr(), None, None, o.data_ptr(), 4, 1024, 128, 1, 1, 1e-6, s) != 0
    assert L.hif8_rms_norm_rope(None, w.data_ptr(), None, None, o.data_ptr(), 8, 1024, 128, 1, 1, 1e-6, s) != 0


@pytest.mark.parametrize("B,N,D,gate", [(2, 300, 5120, "batch"), (1, 777, 1536, "one"), (3, 65, 512, "none"),
                                        (1, 5, 8, "batch")])
def test_gated_residual_equals_torch_ops(pkg, B, N, D, gate):
    """hif8_gated_residual against the block's own torch ops (osp_next.py:947, :949, :955):
    x + y * gate with bf16 tensors, bit for bit (the same fp32 op and RNE at each step)."""
    D_ = pkg.dit
    g = torch.Generator().manual_seed(B * 7 + N + D)
    x = (torch.randn(B, N, D, generator=g) * 4).to(torch.bfloat16).to(DEV)
    y = (torch.randn(B, N, D, generator=g) * 3).to(torch.bfloat16).to(DEV)
    y[0, 0, :4] = torch.tensor([float("inf"), -0.0, 1e-38, 3e38])
    x[0, 0, 4:6] = torch.tensor([float("nan"), float("-inf")])          # NaN in, and inf - inf
    y[0, 0, 5] = float("inf")
    gt = None
    if gate == "batch":
        gt = torch.randn(B, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    elif gate == "one":
        gt = torch.randn(1, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    print(f"[gated_residual] B={B} N={N} D={D} {gate}", flush=True)
    got = D_.gated_residual(x, y, gt)
    want = x + y if gt is None else x + y * gt
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_gated_residual_fallback_and_rejects(pkg):
    D_ = pkg.dit
    x = torch.randn(2, 10, 12, device=DEV).to(torch.bfloat16)       # D % 8 != 0: torch ops
    y = torch.randn(2, 10, 12, device=DEV).to(torch.bfloat16)
    gt = torch.randn(2, 1, 12, device=DEV).to(torch.bfloat16)
    assert torch.equal(D_.gated_residual(x, y, gt), x + y * gt)
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(torch.device(DEV))
    a = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    assert L.hif8_gated_residual(a.data_ptr(), a.data_ptr(), a.data_ptr(), a.data_ptr(), 4, 64, 3, s) != 0  # rows % rpb
    assert L.hif8_gated_residual(a.data_ptr(), a.data_ptr(), None, a.data_ptr(), 4, 60, 1, s) != 0          # dim % 8
    assert L.hif8_gated_residual(a.data_ptr() + 2, a.data_ptr(), None, a.data_ptr(), 2, 64, 1, s) != 0      # alignment
    assert L.hif8_gated_residual(None, a.data_ptr(), None, a.data_ptr(), 4, 64, 1, s) != 0


@pytest.mark.parametrize("kind,grid,B", [("token", (3, 10, 14), 1), ("token", (2, 8, 12), 2), ("group", (3, 10, 14), 1),
                                         ("token_rev", (3, 10, 14), 1), ("group_rev", (2, 8, 12), 2),
                                         ("t2g", (3, 10, 14), 1), ("g2t", (2, 8, 12), 1)])
def test_layout_gather_equals_torch(pkg, kind, grid, B):
    """SkiparseRearrange with ``gather`` (hif8_gather_rows over a map of source rows) against its
    torch path (skiparse_func.py:18-52 with the padding and cropping of osp_next.py:239-283): every
    layout change, with and without padding rows (H, W not multiples of P * P), bit for bit, and
    again with other values through the kept map."""
    D = pkg.dit
    RT = D.RearrangeType
    P, C = 2, 136
    T, H, W = grid
    g = torch.Generator().manual_seed(len(kind) * 10 + T)
    full = torch.randn(B, T * H * W, C, generator=g).to(torch.bfloat16).to(DEV)
    src_rt, rt = {"token": (None, RT.Skiparse2DToken), "group": (None, RT.Skiparse2DGroup),
                  "token_rev": (RT.Skiparse2DToken, RT.Skiparse2DTokenReverse),
                  "group_rev": (RT.Skiparse2DGroup, RT.Skiparse2DGroupReverse),
                  "t2g": (RT.Skiparse2DToken, RT.Skiparse2DToken2Group),
                  "g2t": (RT.Skiparse2DGroup, RT.Skiparse2DGroup2Token)}[kind]
    prep = (lambda t: t) if src_rt is None else (lambda t: D.SkiparseRearrange(P, src_rt)(t, grid))
    r = D.SkiparseRearrange(P, rt)
    print(f"[gather] {kind} grid={grid} B={B}", flush=True)
    for rep in range(2):
        x = prep(full if rep == 0 else torch.randn(full.shape, generator=g).to(torch.bfloat16).to(DEV))
        want = r(x, grid)
        got = r(x, grid, gather=True)
        torch.cuda.synchronize()
        assert got.shape == want.shape
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert len(r._maps) == 1


def test_layout_gather_rejects_bad_arguments(pkg):
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(torch.device(DEV))
    x = torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV)
    o = torch.empty_like(x)
    src = torch.arange(8, dtype=torch.int32, device=DEV)
    assert L.hif8_gather_rows(x.data_ptr(), 8, src.data_ptr(), 8, 60, o.data_ptr(), s) != 0       # cols % 8
    assert L.hif8_gather_rows(x.data_ptr() + 2, 8, src.data_ptr(), 4, 64, o.data_ptr(), s) != 0   # alignment
    assert L.hif8_gather_rows(x.data_ptr(), 8, None, 8, 64, o.data_ptr(), s) != 0
    assert L.hif8_gather_rows(x.data_ptr(), 0, src.data_ptr(), 8, 64, o.data_ptr(), s) != 0
    # a source row out of range gives a zero row
    x.fill_(1.0)
    src[3] = 9
    src[5] = -1
    assert L.hif8_gather_rows(x.data_ptr(), 8, src.data_ptr(), 8, 64, o.data_ptr(), s) == 0
    torch.cuda.synchronize()
    assert float(o[3].abs().sum()) == 0.0 and float(o[5].abs().sum()) == 0.0 and bool((o[4] == 1).all())


@pytest.mark.parametrize("rope_on", [True, False])
def test_quantising_producer_equals_codec(pkg, rope_on):
    """quant_attn's q/k producer (hif8_rms_norm_rope_amax + _fake_quant): the output it quantises
    is the one hif8_rms_norm_rope writes (fp32 with rope; its bf16 cast equal bit for bit), the
    state it leaves equals hif8_absmax_scale of that output (fp32 rule with rope, bf16 without),
    and x_q equals the codec's fake quant of it with that state (the bf16 cast of the fp32 x_q
    with rope), bit for bit: _quant of the q the reference hands the attention, then its cast."""
    D = pkg.dit
    H, hd = 40, 128
    dim = H * hd
    B, grid, P = 4, (3, 8, 10), 2
    rearr = D.SkiparseRearrange(P, D.RearrangeType.Skiparse2DToken)
    rope = D.SkiparseRopeWrapper(D.rope_freqs(hd).to(DEV))
    N = rope.prepare_freqs(grid, hd // 2, rearr)[0].shape[1]
    g = torch.Generator().manual_seed(31 + int(rope_on))
    x = (torch.randn(B, N, dim, generator=g) * 3).to(torch.bfloat16).to(DEV)
    norm = D.OSPNextRMSNorm(dim, eps=1e-6, device=DEV)
    print(f"[norm_rope] quantising producer rope={rope_on}", flush=True)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.3 * torch.randn(dim, generator=g)).to(DEV))
        if rope_on:
            cos_f, sin_f = rope.prepare_freqs(grid, hd // 2, rearr)
            xq, st, y = D.rms_norm_rope_quant(x, norm, 15.0, cos_f, sin_f, hd, return_y=True)
            plain = D.rms_norm_rope(x, norm, cos_f, sin_f, hd)
            assert y.dtype == torch.float32
        else:
            xq, st, y = D.rms_norm_rope_quant(x, norm, 15.0, return_y=True)
            plain = D.rms_norm_rope(x, norm)
            assert y.dtype == torch.bfloat16
        assert torch.equal(y.to(torch.bfloat16).view(torch.int16), plain.view(torch.int16))
        y2 = y.reshape(-1, dim)
        full = pkg.absmax_scale(y2, 15.0, pkg.QuantState(DEV))
        want = pkg.fake_quant_to_bf16(y2, full) if rope_on else pkg.fake_quant(y2, full)
    torch.cuda.synchronize()
    assert st.read() == full.read()
    assert torch.equal(xq.reshape(-1, dim).view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("rope_on", [True, False])
@pytest.mark.parametrize("sem", ["npu", "torch"])
def test_quantising_producer_scales_and_semantics(pkg, rope_on, sem):
    """The fake-quant pass (hif8_rms_norm_rope_fake_quant) under states set to explicit scales and
    both semantics: a regular scale, scales that put most values past 40960 (Inf codes; the torch
    route's own rounding there) and below 2^-22 (flushed; torch keeps them), and non-finite and zero
    scales (the scalar route), with a NaN row (the state did not prove the tensor finite).  x_q must
    equal the codec's fake quant of the output the pass wrote (y_out) with the same state and
    semantics, bit for bit: fake_quant_to_bf16 of the fp32 rope output, fake_quant of the bf16 norm
    output."""
    D = pkg.dit
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(torch.device(DEV))
    H, hd = 8, 128
    dim = H * hd
    B, grid, P = 4, (2, 4, 6), 2    # B: the P * P sub-grids of one video
    rearr = D.SkiparseRearrange(P, D.RearrangeType.Skiparse2DToken)
    rope = D.SkiparseRopeWrapper(D.rope_freqs(hd).to(DEV))
    cos_f, sin_f = rope.prepare_freqs(grid, hd // 2, rearr)
    N = cos_f.shape[1]
    g = torch.Generator().manual_seed(77 + int(rope_on))
    x = (torch.randn(B, N, dim, generator=g) * 3).to(torch.bfloat16)
    x[0, 1, 5] = float("nan")                                   # a NaN row
    x = x.to(DEV)
    norm = D.OSPNextRMSNorm(dim, eps=1e-6, device=DEV)
    semantics = pkg._lib.SEM_NPU if sem == "npu" else pkg._lib.SEM_TORCH
    dtype = torch.float32 if rope_on else torch.bfloat16
    with torch.no_grad():
        norm.weight.copy_((1 + 0.3 * torch.randn(dim, generator=g)).to(DEV))
    w = norm.weight.detach().contiguous()
    c, sn = cos_f.to(torch.float32).contiguous(), sin_f.to(torch.float32).contiguous()
    cp, sp = (c.data_ptr(), sn.data_ptr()) if rope_on else (None, None)
    seq, rep = (N, B // cos_f.shape[0] if cos_f.shape[0] > 1 else B) if rope_on else (1, 1)
    for scale in (15.0 / 4.0, 20000.0, 3e-7, float("inf"), 0.0):
        print(f"[norm_rope] fake-quant pass rope={rope_on} sem={sem} scale={scale}", flush=True)
        st = pkg.QuantState(DEV)
        assert L.hif8_set_scale(st.ptr, pkg._lib.dtype_code(dtype), scale, stream) == 0
        xq = torch.empty_like(x)
        y = torch.empty(x.shape, dtype=dtype, device=DEV)
        assert L.hif8_rms_norm_rope_fake_quant(x.data_ptr(), w.data_ptr(), cp, sp, B * N, dim, hd, seq, rep,
                                               float(norm.eps), st.ptr, semantics, xq.data_ptr(), y.data_ptr(),
                                               stream) == 0
        y2 = y.reshape(-1, dim)
        want = (pkg.fake_quant_to_bf16(y2, st, semantics) if rope_on else pkg.fake_quant(y2, st, semantics))
        torch.cuda.synchronize()
        assert torch.isnan(y2[1]).all()
        got = xq.reshape(-1, dim).view(torch.int16)
        assert torch.equal(got, want.view(torch.int16)), \
            f"scale {scale}: {(got != want.view(torch.int16)).sum().item()} of {got.numel()} differ"


def test_quantising_producer_rejects_bad_arguments(pkg):
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(torch.device(DEV))
    x = torch.zeros(8, 1024, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(1024, dtype=torch.float32, device=DEV)
    o = torch.empty_like(x)
    st = pkg.QuantState(DEV)
    assert L.hif8_rms_norm_rope_amax(x.data_ptr(), w.data_ptr(), None, None, 8, 1024, 128, 1, 1, 1e-6, 15.0, None, s) != 0
    assert L.hif8_rms_norm_rope_amax(x.data_ptr(), w.data_ptr(), None, None, 8, 1024, 128, 1, 1, 1e-6, 0.0, st.ptr, s) != 0
    assert L.hif8_rms_norm_rope_amax(x.data_ptr(), w.data_ptr(), None, None, 8, 1000, 128, 1, 1, 1e-6, 15.0, st.ptr, s) != 0
    assert L.hif8_rms_norm_rope_fake_quant(x.data_ptr(), w.data_ptr(), None, None, 8, 1024, 128, 1, 1, 1e-6, st.ptr, 7,
                                           o.data_ptr(), None, s) != 0
    assert L.hif8_rms_norm_rope_fake_quant(x.data_ptr(), w.data_ptr(), None, None, 8, 1024, 128, 1, 1, 1e-6, st.ptr, 0,
                                           None, None, s) != 0
    assert L.hif8_rms_norm_rope_fake_quant(x.data_ptr(), w.data_ptr(), None, None, 8, 1024, 128, 1, 1, 1e-6, st.ptr, 0,
                                           o.data_ptr(), o.data_ptr() + 4, s) != 0
