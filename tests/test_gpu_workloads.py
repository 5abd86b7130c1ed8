"""GPU correctness at the full BASELINE workloads.

- Config 3 (Wan-14B 720P linears, x [75600, K]): FFN-down [13824 -> 5120] and the
  q/k/v/o shape [5120 -> 5120] on HIF8Linear's default route for that M (the weight decoded
  once, then the decode-free GEMM) and on the fused dequant-GEMM: the two routes equal bit for
  bit on the whole output, sampled rows of the output against fp32 torch on the same
  operands, and sampled x_q and w_q rows bit-exact against the oracle under the full tensors'
  scales (FFN-up at this size is in test_gpu_linear.py).
- Config 4 (one 14B block at 720P: dim 5120, 40 heads, grid 21x45x80 padded to 48, text 512,
  osp_next.py:926-957): every linear of both routes is intercepted where it runs; each x_q is
  checked against the oracle on sampled rows with the full tensor's scale and, for the fused
  producers, against the standalone _quant of the producer's own output on the whole tensor;
  each GEMM's output rows against fp32 torch; on the fused route, sampled queries of each
  attention kernel call against float32 softmax over the kept keys, and the o input quantised
  with the state the kernel's epilogue left is the standalone _quant of the attention output;
  the two routes' block outputs agree within the block tolerance of tests/test_dit_cpu.py and
  are finite.
- Config 5 (the 40-block 14B step at 768P, osp_next.py:1287-1331): the fused step's output
  is finite; the per-linear probe of config 4 runs on the stack's full block 0, its full ->
  Skiparse token block 4 and the group block 5 that follows (fed block 4's output), both
  routes each, and the routes agree within the block tolerance.
"""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import numpy as np  # noqa: E402

import workload_checks as W  # noqa: E402
from test_dit_cpu import TOL_HIF8, block_errors  # noqa: E402

DEV = "cuda:0"


def _route(pkg, name):
    class _Ctx:
        def __enter__(self):
            self.old = pkg.hif8_linear.GEMM_ROUTE
            pkg.hif8_linear.GEMM_ROUTE = name

        def __exit__(self, *exc):
            pkg.hif8_linear.GEMM_ROUTE = self.old
    return _Ctx()


def _config3_operands(M, K, N, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=DEV)
    ch = torch.randperm(K, generator=g, device=DEV)[:16]
    x[:, ch] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    return x, w, b


@pytest.mark.parametrize("name,N,K", [("ffn_down", 5120, 13824), ("qkvo", 5120, 5120)])
def test_config3_full_size_both_routes(pkg, R, name, N, K):
    M = 75600
    print(f"[config3] {name} M={M} K={K} N={N}", flush=True)
    x, w, b = _config3_operands(M, K, N, seed=31 + N + K)
    packed = pkg.PackedWeight(w, 15.0)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    assert pkg.hif8_linear.decode_once(M, K)       # the default route at this M
    y_auto = pkg.linear_fwd(a, fmt, st, packed, b)
    with _route(pkg, "fused"):
        y_fused = pkg.linear_fwd(a, fmt, st, packed, b)
    torch.cuda.synchronize()
    # the same MFMA products in the same order: identical bits on the whole output
    assert torch.equal(y_auto.view(torch.int16), y_fused.view(torch.int16))
    assert bool(torch.isfinite(y_auto).all())
    rows = W.sample_rows(M, seed=N + K)
    w_q = packed.dequantize()
    W.check_linear_rows(a, w_q, b, y_auto, rows)
    # operands: x_q and w_q rows bit-exact against the oracle under the full tensors' scales
    W.check_xq_rows(R, x, a, st, 15.0, rows)
    W.check_xq_rows(R, w, w_q, packed.state, 15.0, W.sample_rows(N, seed=K, n=64, tail=16))
    # the layer itself (autograd off) takes the same route and gives the same bits
    lin = pkg.HIF8Linear(K, N, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
        y_mod = lin(x)
    assert torch.equal(y_mod.view(torch.int16), y_auto.view(torch.int16))


# ----------------------------------------------------------------------- config 4


class BlockProbe:
    """Intercepts the functions through which a DiT block's linears and their producers run
    and checks each call (see the module docstring).  ``calls`` counts the sites visited."""

    def __init__(self, pkg, R, monkeypatch, seed, label="config4"):
        self.pkg, self.R, self.seed, self.label = pkg, R, seed, label
        self.calls = {}
        self.errors = []
        from ospnext_amd import dit, ffn, hif8_linear, norm
        self.mods = dict(dit=dit, ffn=ffn, hif8_linear=hif8_linear, norm=norm)
        hl = hif8_linear
        wrap_mn = self._modln(norm.modulated_norm_quant)
        monkeypatch.setattr(norm, "modulated_norm_quant", wrap_mn)
        monkeypatch.setattr(dit, "modulated_norm_quant", wrap_mn)
        monkeypatch.setattr(dit, "affine_norm_quant", self._affine(dit.affine_norm_quant))
        wrap_g = self._grouped(hl.linear_fwd_grouped)
        monkeypatch.setattr(norm, "linear_fwd_grouped", wrap_g)
        monkeypatch.setattr(dit, "linear_fwd_grouped", wrap_g)
        wrap_any = self._linear_any(hl.linear_any)
        monkeypatch.setattr(hl, "linear_any", wrap_any)
        monkeypatch.setattr(ffn, "linear_any", wrap_any)
        monkeypatch.setattr(ffn, "linear_fwd_gelu_stat", self._gelu(hl.linear_fwd_gelu_stat))
        monkeypatch.setattr(ffn, "gelu_fake_quant", self._down_quant(hl.gelu_fake_quant))
        monkeypatch.setattr(dit, "fake_quant", self._text_quant(dit.fake_quant))
        wrap_q = self._qact(hl.quantize_activation)
        monkeypatch.setattr(hl, "quantize_activation", wrap_q)
        monkeypatch.setattr(ffn, "quantize_activation", wrap_q)
        monkeypatch.setattr(dit, "attention_fwd", self._attention(dit.attention_fwd))
        monkeypatch.setattr(hl.HIF8Linear, "forward_settled", self._settled(hl.HIF8Linear.forward_settled))

    def _hit(self, site):
        self.calls[site] = self.calls.get(site, 0) + 1
        print(f"[{self.label}]   {site}", flush=True)

    def _rows(self, M):
        return W.sample_rows(M, seed=self.seed + sum(self.calls.values()))

    def _modln(self, orig):
        def wrapped(x, shift=None, scale=None, eps=1e-6, scale_max=15.0, semantics=0, return_y=False):
            xq, st, y = orig(x, shift, scale, eps, scale_max, semantics, return_y=True)
            self._hit("modulated_norm_quant")
            ref_y = self.pkg.modulate(self.pkg.WanLayerNorm(x.shape[-1], eps).to(x.device)(x), shift, scale)
            self._check_y(y, ref_y, shift)
            self._check_producer(xq, st, y, scale_max)
            return (xq, st, y) if return_y else (xq, st)
        return wrapped

    def _affine(self, orig):
        def wrapped(x, norm, scale_max=15.0, semantics=0, return_y=False):
            xq, st, y = orig(x, norm, scale_max, semantics, return_y=True)
            self._hit("affine_norm_quant")
            self._check_y(y, norm(x), norm.bias.detach())
            self._check_producer(xq, st, y, scale_max)
            return (xq, st, y) if return_y else (xq, st)
        return wrapped

    def _check_y(self, y, ref_y, shift=None):
        """The producer's y against torch's fp32 layer norm (+ bf16 modulation): equal except next
        to a bf16 rounding boundary (fewer than 1e-3 of the elements), and there within one bf16
        unit of the product n * (1 + scale) (or w * n) plus one of y, together below 2^-6 of
        |y| + |shift| (``shift``: the modulation shift, or the affine norm's bias, which y can
        cancel down to a small value) plus 2^-16 of rms(y): where x is within a few float32 units
        of its row mean, x - mean cancels and the last bit of the mean (summation order) is the
        whole of a tiny normalised value (torch gives ~1e-8 where the producer gives 0)."""
        ref_y = ref_y.reshape(y.shape)
        d = (y.float() - ref_y.float()).abs()
        frac = float((d != 0).float().mean())
        mag = ref_y.float().abs() + 2.0 ** -16 * float(ref_y.float().square().mean().sqrt())
        if shift is not None:
            mag = mag + shift.float().abs().reshape(1, 1, -1)
        assert frac < 1e-3, frac
        assert bool((d <= mag * 2.0 ** -6).all()), float((d / mag.clamp(min=1e-30)).max())

    def _check_producer(self, xq, st, y, scale_max):
        xq_std, st_std = W.standalone_quant(self.pkg, y, scale_max)
        assert torch.equal(xq.reshape(-1).view(torch.int16), xq_std.reshape(-1).view(torch.int16))
        assert st.read()[1] == st_std.read()[1]
        W.check_xq_rows(self.R, y, xq, st, scale_max, self._rows(y.numel() // y.shape[-1]))

    def _grouped(self, orig):
        def wrapped(a, gw):
            ys = orig(a, gw)
            self._hit(f"linear_fwd_grouped[{len(ys)}]")
            rows = self._rows(a.shape[0])
            for p, y, i in zip(gw.packs, ys, range(len(ys))):
                b = None
                if gw.bias is not None:
                    off = sum(gw.ns[:i])
                    b = gw.bias[off:off + gw.ns[i]]
                W.check_linear_rows(a, p.dequantize(torch.bfloat16), b, y, rows)
            return ys
        return wrapped

    def _linear_any(self, orig):
        def wrapped(a, a_fmt, a_state, w, bias):
            y = orig(a, a_fmt, a_state, w, bias)
            self._hit("linear_any")
            assert a_fmt == self.pkg._lib.A_BF16
            W.check_linear_rows(a, w.dequantize(torch.bfloat16), bias, y, self._rows(a.shape[0]))
            return y
        return wrapped

    def _gelu(self, orig):
        def wrapped(a, w, bias, y_state, scale_max):
            y = orig(a, w, bias, y_state, scale_max)
            self._hit("linear_fwd_gelu_stat")
            W.check_linear_rows(a, w.dequantize(torch.bfloat16), bias, y, self._rows(a.shape[0]))
            # the statistic settled the amax a full pass over GELU(y) finds
            st_full = self.pkg.gelu_absmax_scale(y, scale_max, self.pkg.QuantState(y.device))
            assert y_state.read() == st_full.read()
            return y
        return wrapped

    def _down_quant(self, orig):
        def wrapped(y, state, scale_max=15.0, semantics=0):
            yq = orig(y, state, scale_max, semantics)
            self._hit("ffn_down_quant")
            # x_q of GELU(y) against the library's GELU written out and the standalone _quant of it
            g = self.pkg.gelu_fake_quant(y, self.pkg.gelu_absmax_scale(y, scale_max, self.pkg.QuantState(y.device)),
                                         scale_max)
            assert torch.equal(yq.reshape(-1).view(torch.int16), g.reshape(-1).view(torch.int16))
            ref_g = torch.nn.functional.gelu(y, approximate="tanh")
            ref, _ = W.standalone_quant(self.pkg, ref_g, scale_max)
            diff = float((yq.reshape(-1).view(torch.int16) != ref.reshape(-1).view(torch.int16)).float().mean())
            assert diff <= 1e-3, diff
            return yq
        return wrapped

    def _text_quant(self, orig):
        def wrapped(t2, state, semantics=0):
            tq = orig(t2, state, semantics)
            self._hit("text_quant")
            W.check_xq_rows(self.R, t2, tq, state, 15.0, self._rows(t2.shape[0]))
            return tq
        return wrapped

    def _attention(self, orig):
        def wrapped(q, k, v, key_idx=None, key_count=None, softmax_scale=None, o_state=None, o_as_f32=False,
                    scale_max=15.0):
            out = orig(q, k, v, key_idx, key_count, softmax_scale, o_state, o_as_f32, scale_max)
            self._hit("attention_fwd" + ("[f32]" if o_as_f32 else ""))
            W.check_attention_rows(q, k, v, key_idx, key_count, out, seed=self.seed + sum(self.calls.values()))
            # the epilogue's state is the one an amax pass over the output leaves
            st_full = self.pkg.absmax_scale(out.reshape(-1, out.shape[2] * out.shape[3]), scale_max,
                                            self.pkg.QuantState(out.device), as_f32=o_as_f32)
            assert o_state.read() == st_full.read()
            return out
        return wrapped

    def _settled(self, orig):
        def wrapped(lin, x, x_state, as_f32=False):
            self._hit("forward_settled" + ("[f32]" if as_f32 else ""))
            # the o input quantised with the settled state is the standalone _quant of x (of its
            # fp32 copy, then the autocast, for the self-attention)
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            if as_f32:
                a = self.pkg.fake_quant_to_bf16(x2, x_state, as_f32=True)
                want = W.standalone_quant(self.pkg, x2.float(), lin.scale_max_forward)[0].to(torch.bfloat16)
            else:
                a = self.pkg.fake_quant(x2, x_state)
                want = W.standalone_quant(self.pkg, x2, lin.scale_max_forward)[0]
            assert torch.equal(a.view(torch.int16), want.view(torch.int16))
            W.check_xq_rows(self.R, x2, a, x_state, lin.scale_max_forward, self._rows(x2.shape[0]), as_f32=as_f32)
            return orig(lin, x, x_state, as_f32)
        return wrapped

    def _qact(self, orig):
        def wrapped(x2, scale_max, a_format, as_f32=False):
            a, fmt, st = orig(x2, scale_max, a_format, as_f32)
            self._hit("quantize_activation" + ("[f32]" if (as_f32 or x2.dtype == torch.float32) else ""))
            W.check_xq_rows(self.R, x2, a, st, scale_max, self._rows(x2.shape[0]), as_f32=as_f32)
            if as_f32:
                # the bf16 attention output quantised as its fp32 copy: the fp32 _quant, then the cast
                xq32, _ = W.standalone_quant(self.pkg, x2.float(), scale_max)
                assert torch.equal(a.view(torch.int16), xq32.to(torch.bfloat16).view(torch.int16))
            return a, fmt, st
        return wrapped


def _block_720p(pkg):
    D = pkg.dit
    dim, ffn, heads, grid, L = 5120, 13824, 40, (21, 45, 80), 512
    torch.manual_seed(4)
    blk = D.OSPNextAttentionBlock(dim, ffn, heads, cross_attn_norm=True, sparse_ratio=2,
                                  skiparse_block_type="token", is_full2skiparse_block=True, quant="hif8",
                                  device=DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    D.init_block_weights(blk, 0.02, g)
    with torch.no_grad():
        for n, p in blk.named_parameters():
            if n.endswith("bias"):
                p.normal_(0.0, 0.02, generator=g)
            elif "norm" in n:
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g, device=DEV))
    for m in blk.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack()
    T, H, W_ = grid
    x = torch.randn(1, T * H * W_, dim, generator=g, device=DEV).to(torch.bfloat16)
    e = torch.randn(1, 6, dim, generator=g, device=DEV).to(torch.bfloat16)
    text = torch.randn(1, L, dim, generator=g, device=DEV).to(torch.bfloat16)
    return blk, x, e, text, grid


FUSED_SITES = {"modulated_norm_quant": 2, "linear_fwd_grouped[3]": 1, "attention_fwd[f32]": 1,
               "forward_settled[f32]": 1, "linear_any": 4, "linear_fwd_grouped[2]": 1, "text_quant": 1,
               "affine_norm_quant": 1, "attention_fwd": 1, "forward_settled": 1, "linear_fwd_gelu_stat": 1,
               "ffn_down_quant": 1}


def probe_both_routes(probe, blk, x, mask, e, grid, rope, text, x_ref, label):
    """Run the block on both routes under the probe: every linear, producer and attention call
    checked where it runs; the sites of each route counted; the two outputs within the block
    tolerance of each other.  Returns the fused route's output."""
    outs = {}
    for fused in (True, False):
        probe.calls = {}
        print(f"[{label}] route fused={fused}", flush=True)
        with torch.no_grad():
            y = blk(x, mask, mask, e, grid, grid, rope, text, fused=fused)
        torch.cuda.synchronize()
        assert y.shape == x_ref.shape and y.dtype == torch.bfloat16
        assert bool(torch.isfinite(y).all())
        outs[fused] = y
        print(f"[{label}] fused={fused} sites {probe.calls}", flush=True)
        if fused:
            assert probe.calls == FUSED_SITES, probe.calls
        else:
            # q, k, v, o (fp32 input), cross q, k, v, o, FFN up: each quantises its own input
            assert probe.calls.get("quantize_activation", 0) + probe.calls.get("quantize_activation[f32]", 0) == 9
            assert probe.calls["quantize_activation[f32]"] == 1
            assert probe.calls["linear_fwd_gelu_stat"] == 1 and probe.calls["ffn_down_quant"] == 1
    nw, mx = block_errors(outs[True], outs[False], x_ref)
    frac = float((outs[True].view(torch.int16) != outs[False].view(torch.int16)).float().mean())
    print(f"[{label}] routes: normwise {nw:.3e} max {mx:.3e}, {frac:.4%} of outputs differ", flush=True)
    assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (nw, mx)
    return outs[True]


def test_config4_block_720p_every_linear(pkg, R, monkeypatch):
    D = pkg.dit
    print("[config4] building the 14B block at 720P", flush=True)
    blk, x, e, text, grid = _block_720p(pkg)
    rope = D.SkiparseRopeWrapper(D.rope_freqs(128).to(DEV))
    tm, _ = D.skiparse_masks(1, grid, 2, DEV)
    assert tm is not None and tm.shape == (4, 20160)       # H 45 padded to 48
    probe = BlockProbe(pkg, R, monkeypatch, seed=44)
    x_ref = D.SkiparseRearrange(2, D.RearrangeType.Skiparse2DToken)(x, grid)
    y = probe_both_routes(probe, blk, x, tm, e, grid, rope, text, x_ref, "config4")
    assert y.shape == (4, 20160, 5120)


# ----------------------------------------------------------------------- config 5


@pytest.fixture(scope="module")
def stack_768p(pkg):
    """The 40-block 14B stack (8 full blocks, dual-end schedule, osp_hif8_14b.yaml:35-37) with
    prepacked random-init weights, and the 768P step inputs: x [1, 84672, 5120], e, and the text
    context (512 x 4096 through the text embedding)."""
    D = pkg.dit
    dim, ffn, heads, grid, L, text_dim = 5120, 13824, 40, (21, 48, 84), 512, 4096
    print("[config5] building the 40-block 14B stack", flush=True)
    torch.manual_seed(5)
    stack = D.OSPNextBlocks(dim, ffn, heads, num_layers=40, num_full_blocks=8, quant="hif8", device=DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    D.init_block_weights(stack, 0.02, g)
    for m in stack.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack(drop_weight=True)
    torch.cuda.empty_cache()
    emb = torch.nn.Sequential(torch.nn.Linear(text_dim, dim), torch.nn.GELU(approximate="tanh"),
                              torch.nn.Linear(dim, dim)).to(DEV, torch.bfloat16)
    D.init_block_weights(emb, 0.02, g)
    T, H, W_ = grid
    x = torch.randn(1, T * H * W_, dim, generator=g, device=DEV).to(torch.bfloat16)
    e = torch.randn(1, 6, dim, generator=g, device=DEV).to(torch.bfloat16)
    text_in = torch.randn(1, L, text_dim, generator=g, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        text = emb(text_in)
    yield stack, x, e, text, grid
    del stack
    torch.cuda.empty_cache()


def test_config5_step_768p(pkg, stack_768p):
    D = pkg.dit
    stack, x, e, text, grid = stack_768p
    with torch.no_grad():
        print("[config5] the fused 40-block step", flush=True)
        y = stack(x, e, text, grid)
        torch.cuda.synchronize()
        assert y.shape == x.shape and bool(torch.isfinite(y).all())
        assert float((y.float() - x.float()).norm()) > 0
        tm, gm = D.skiparse_masks(1, grid, 2, DEV)
        assert tm is None and gm is None                 # 48 and 84 are multiples of 4: no padding


def test_config5_blocks_768p_every_linear(pkg, R, monkeypatch, stack_768p):
    """The per-linear probe of config 4 on the 768P stack's three block kinds at full size: the
    first full block (0), the full -> Skiparse token block (4) and the group block after it (5),
    which reads the token block's output in the token layout and changes it to the group layout
    (osp_next.py:1287-1331, the group layout of skiparse_func.py:26-31).  Each runs on both
    routes; block 5's input is block 4's fused output, as in the step."""
    D = pkg.dit
    stack, x, e, text, grid = stack_768p
    rope = stack.rope
    kinds = [stack.blocks[i].skiparse_block_type for i in (0, 4, 5)]
    assert kinds == ["full", "token", "group"], kinds
    probe = BlockProbe(pkg, R, monkeypatch, seed=55, label="config5")
    y0 = probe_both_routes(probe, stack.blocks[0], x, None, e, grid, rope, text, x, "config5 block 0 full")
    assert y0.shape == x.shape
    x_tok = D.SkiparseRearrange(2, D.RearrangeType.Skiparse2DToken)(x, grid)
    y4 = probe_both_routes(probe, stack.blocks[4], x, None, e, grid, rope, text, x_tok, "config5 block 4 token")
    assert y4.shape == (4, 21168, 5120)
    x_grp = D.SkiparseRearrange(2, D.RearrangeType.Skiparse2DToken2Group)(y4, grid)
    y5 = probe_both_routes(probe, stack.blocks[5], y4, None, e, grid, rope, text, x_grp, "config5 block 5 group")
    assert y5.shape == (4, 21168, 5120)
