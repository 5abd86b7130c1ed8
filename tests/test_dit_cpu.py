"""The DiT block harness on CPU: rearranges, masks, RoPE and the block schedule against the
oracle's restatement of the reference (einops patterns, exact angles), and the block's glue
(norms, modulation, attention, rearranges) with the oracle's HiF8 linears plugged in.

The linears here are the oracle's (CPU); the HIP linears are exercised in test_gpu_dit.py."""
from __future__ import annotations

import math

import pytest

torch = pytest.importorskip("torch")
import torch.nn as nn  # noqa: E402

from oracle import dit_ref  # noqa: E402

GRIDS = [(2, 6, 8), (1, 8, 12), (3, 5, 7), (2, 4, 4)]


@pytest.fixture(scope="module")
def dit(pkg):
    from ospnext_amd import dit as D  # loaded by the pkg fixture
    return D


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("B", [1, 2])
def test_rearranges_match_reference_patterns(dit, grid, B):
    T, H, W = grid
    P = 2
    g = torch.Generator().manual_seed(T * 100 + H * 10 + W + B)
    x = torch.randn(B, T * H * W, 3, generator=g)
    R = dit.RearrangeType
    for kind in (R.Skiparse2DToken, R.Skiparse2DGroup):
        got = dit.SkiparseRearrange(P, kind)(x, grid)
        want = dit_ref.skiparse_rearrange(x, kind, grid, P)
        assert torch.equal(got, want), kind
    tok = dit.SkiparseRearrange(P, R.Skiparse2DToken)(x, grid)
    grp = dit.SkiparseRearrange(P, R.Skiparse2DToken2Group)(tok, grid)
    assert torch.equal(grp, dit_ref.skiparse_rearrange(tok, R.Skiparse2DToken2Group, grid, P))
    assert torch.equal(grp, dit.SkiparseRearrange(P, R.Skiparse2DGroup)(x, grid))
    back = dit.SkiparseRearrange(P, R.Skiparse2DGroup2Token)(grp, grid)
    assert torch.equal(back, tok)
    for kind, fwd in ((R.Skiparse2DTokenReverse, tok), (R.Skiparse2DGroupReverse, grp)):
        got = dit.SkiparseRearrange(P, kind)(fwd, grid)
        assert torch.equal(got, dit_ref.skiparse_rearrange(fwd, kind, grid, P))
        assert torch.equal(got, x), kind        # crop of the padding restores the input


def test_token_layout_is_strided_subgrid(dit):
    """Sub-sequence p*P+q of the token layout holds the tokens at rows p, p+P, ... and columns
    q, q+P, ... of every frame, in (t, h, w) order."""
    T, H, W, P = 2, 4, 6, 2
    pos = torch.arange(T * H * W, dtype=torch.float32).reshape(1, -1, 1)
    tok = dit.skiparse_2d_token(pos, (T, H, W), P)
    for p in range(P):
        for q in range(P):
            want = [t * H * W + h * W + w for t in range(T) for h in range(p, H, P) for w in range(q, W, P)]
            assert tok[p * P + q, :, 0].long().tolist() == want


@pytest.mark.parametrize("grid", GRIDS)
def test_masks(dit, grid):
    tm, gm = dit.skiparse_masks(1, grid, 2, "cpu")
    rtm, rgm = dit_ref.masks(1, grid, 2)
    for a, b in ((tm, rtm), (gm, rgm)):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)
            T, H, W = grid
            assert int(a.sum()) == T * H * W     # exactly the real tokens


def test_rope_table_and_rotation(dit):
    f = dit.rope_freqs(128)
    assert f.shape == (1024, 64) and f.dtype == torch.float32
    # t, h and w parts: 22 + 21 + 21 angles, each pos / 10000^(2i/dim) for its own dim
    assert float(f[5, 3]) == pytest.approx(5 / 10000 ** (6 / 44), rel=1e-6)
    assert float(f[7, 22 + 4]) == pytest.approx(7 / 10000 ** (8 / 42), rel=1e-6)
    assert float(f[9, 43 + 20]) == pytest.approx(9 / 10000 ** (40 / 42), rel=1e-6)
    rope = dit.SkiparseRopeWrapper(f)
    grid = (3, 6, 8)
    g = torch.Generator().manual_seed(3)
    for kind in ("identity", "skiparse_2d_token", "skiparse_2d_group"):
        P = 1 if kind == "identity" else 2
        ra = dit.SkiparseRearrange(P, kind)
        ang = dit_ref.rope_angles(grid, 128, kind, P)
        x = torch.randn(ang.shape[0], ang.shape[1], 2, 128, generator=g).to(torch.bfloat16)
        got = rope.apply_rope(x, grid, ra)
        want = dit_ref.apply_rope(x, ang)
        assert got.dtype == torch.float32
        assert torch.allclose(got, want, rtol=0, atol=2e-6 * float(x.float().abs().max()))
        # a rotation: pair norms unchanged; the token at (0, 0, 0) is not rotated
        n_in = x.float().reshape(*x.shape[:3], 64, 2).square().sum(-1)
        n_out = got.reshape(*x.shape[:3], 64, 2).square().sum(-1)
        assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)
        assert torch.equal(got[0, 0], x[0, 0].float())


def test_block_schedule(dit):
    s = dit.block_schedule(40, "dual_end", 8)
    kinds = [k for k, _, _ in s]
    assert kinds[:4] == ["full"] * 4 and kinds[36:] == ["full"] * 4
    assert kinds[4:36] == ["token", "group"] * 16
    assert [i for i, (_, f2s, _) in enumerate(s) if f2s] == [4]
    assert [i for i, (_, _, s2f) in enumerate(s) if s2f] == [35]
    assert all(k == "full" for k, _, _ in dit.block_schedule(6, "full"))
    s0 = dit.block_schedule(4, "dual_end", 0)    # no full blocks: the virtual ones at -1 and 4
    assert s0 == [("token", True, False), ("group", False, False), ("token", False, False), ("group", False, True)]
    with pytest.raises(ValueError):
        dit.block_schedule(40, "dual_end", 6)


class OracleLinear(nn.Module):
    """An nn.Linear whose forward is the oracle's linear (HiF8 fake quant, or exact)."""

    def __init__(self, lin: nn.Linear, kind: str):
        super().__init__()
        self.weight = lin.weight
        self.bias = lin.bias
        self.kind = kind

    def forward(self, x):
        b = None if self.bias is None else self.bias.detach()
        if self.kind == "exact":
            return dit_ref.exact_linear(x, self.weight.detach(), b)
        return dit_ref.hif8_linear(x, self.weight.detach(), b)


def _swap_linears(mod, kind="hif8"):
    for name, child in list(mod.named_children()):
        if isinstance(child, nn.Linear):
            setattr(mod, name, OracleLinear(child, kind))
        else:
            _swap_linears(child, kind)


def make_block(dit, kind, f2s, s2f, dim=256, heads=2, ffn=512, seed=0, quant=None, device="cpu", quant_attn=None):
    torch.manual_seed(seed)
    blk = dit.OSPNextAttentionBlock(dim, ffn, heads, cross_attn_norm=True, sparse_ratio=2 if kind != "full" else 1,
                                    skiparse_block_type=kind, is_full2skiparse_block=f2s, is_skiparse2full_block=s2f,
                                    quant=quant, quant_attn=quant_attn, device=device, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for n, p in blk.named_parameters():
            if n.endswith("norm_q.weight") or n.endswith("norm_k.weight") or n.startswith("norm3"):
                p.copy_((1 + 0.1 * torch.randn(p.shape, generator=g)).to(p.dtype))
            elif n == "modulation":
                p.copy_((torch.randn(p.shape, generator=g) / dim ** 0.5).to(p.dtype))
            elif n.endswith("bias"):
                p.copy_((0.02 * torch.randn(p.shape, generator=g)).to(p.dtype))
            else:
                p.copy_((0.02 * torch.randn(p.shape, generator=g)).to(p.dtype))
    return blk


def block_inputs(grid, dim=256, L=16, seed=5, B=1):
    T, H, W = grid
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T * H * W, dim, generator=g).to(torch.bfloat16)
    e = torch.randn(B, 6, dim, generator=g).to(torch.bfloat16)
    text = torch.randn(B, L, dim, generator=g).to(torch.bfloat16)
    return x, e, text


def out_layout(kind, f2s, s2f, x_in, grid):
    """The block input in the block's output layout (padding tokens zero)."""
    if kind == "token" and f2s:
        return dit_ref.skiparse_rearrange(x_in, "skiparse_2d_token", grid, 2)
    if kind == "group" and s2f:
        return dit_ref.skiparse_rearrange(x_in, "skiparse_2d_token_reverse", grid, 2)
    return x_in


def block_errors(got, want, x_ref=None):
    """(normwise, max) errors of the block's update (output minus ``x_ref``, the input in the
    output layout), relative to the update's norm and max magnitude."""
    got, want = got.double(), want.double()
    if x_ref is not None:
        got, want = got - x_ref.double(), want - x_ref.double()
    d = got - want
    return float(d.norm() / want.norm()), float(d.abs().max() / want.abs().max())


# Tolerances on the block update.  With exact linears the two evaluations differ by the
# rounding of bf16 intermediates (attention output, norms, GELU: one bf16 unit, 2^-8, on part
# of the elements), and the residual stream x + update is rounded to bf16 at the scale of x,
# which is a few times the update here: one unit of x is up to ~1e-2 of the update.  With HiF8
# linears every quantisation can also turn a one-unit bf16 difference at a HiF8 rounding
# boundary into a one-step HiF8 difference (1/8 to 1/2 of that element), on the few per cent of
# elements whose bf16 value moved; the block quantises eight times.  A structural mistake (a
# wrong permutation, modulation chunk, gate or mask) moves the update by O(1).
TOL_EXACT = (1.5e-2, 5e-2)
TOL_HIF8 = (6e-2, 1.5e-1)


CASES = [("token", True, False, (2, 6, 8)), ("group", False, True, (2, 6, 8)), ("full", False, False, (2, 4, 8)),
         ("token", False, False, (1, 8, 8)), ("group", False, False, (1, 8, 12))]


def _layout_in(dit, kind, f2s, x, grid):
    """The input layout a non-first skiparse block receives (token or group with padding)."""
    R = dit.RearrangeType
    if kind == "token" and not f2s:
        return dit.SkiparseRearrange(2, R.Skiparse2DGroup)(x, grid)
    if kind == "group":
        return dit.SkiparseRearrange(2, R.Skiparse2DToken)(x, grid)
    return x


@pytest.mark.parametrize("linear", ["exact", "hif8"])
@pytest.mark.parametrize("kind,f2s,s2f,grid", CASES)
def test_block_glue_matches_oracle(dit, kind, f2s, s2f, grid, linear):
    blk = make_block(dit, kind, f2s, s2f)
    _swap_linears(blk, linear)
    x, e, text = block_inputs(grid)
    xin = _layout_in(dit, kind, f2s, x, grid)
    rope = dit.SkiparseRopeWrapper(dit.rope_freqs(128))
    tm, gm = dit.skiparse_masks(1, grid, 2, "cpu")
    am = {"token": tm, "group": gm, "full": None}[kind]
    with torch.no_grad():
        got = blk(xin, am, am, e, grid, grid, rope, text, fused=False)
    sd = {k: v.detach() for k, v in blk.state_dict().items()}
    want = dit_ref.block(sd, xin, e, text, grid, kind, f2s, s2f, num_heads=2, linear=linear)
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    nw, mx = block_errors(got, want, out_layout(kind, f2s, s2f, xin, grid))
    tol = TOL_EXACT if linear == "exact" else TOL_HIF8
    assert nw < tol[0] and mx < tol[1], (nw, mx)


def test_state_dict_keys_follow_reference(dit):
    blk = make_block(dit, "token", True, False)
    keys = set(blk.state_dict().keys())
    for k in ("modulation", "norm3.weight", "norm3.bias", "self_attn.q.weight", "self_attn.o.bias",
              "self_attn.norm_q.weight", "cross_attn.k.weight", "cross_attn.norm_k.weight", "ffn.0.weight",
              "ffn.2.bias"):
        assert k in keys, k
    assert blk.self_attn.norm_q.weight.dtype == torch.float32 and blk.norm3.weight.dtype == torch.float32
    assert blk.self_attn.q.weight.dtype == torch.bfloat16 and blk.modulation.dtype == torch.bfloat16


# Mistakes planted in a copy of the oracle's block: each must move the exact-linear comparison
# outside its tolerance (the check has the power to see them).
MUTATIONS = {
    "shift and scale swapped": ('* (1 + ee[1]) + ee[0]', '* (1 + ee[0]) + ee[1]'),
    "wrong FFN gate": ('lin("ffn.2", h) * ee[5]', 'lin("ffn.2", h) * ee[2]'),
    "k not rotated": ('q, k = apply_rope(q, ang), apply_rope(k, ang)', 'q, k = apply_rope(q, ang), k.float()'),
    "group angles in a token block": ('rope_kind, Pk = "identity", "skiparse_2d_token", P',
                                      'rope_kind, Pk = "identity", "skiparse_2d_group", P'),
    "padding keys attended": ('key_mask = tm if kind == "token" else gm', 'key_mask = None'),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_block_check_rejects_planted_mistakes(dit, name):
    import types
    src_path = dit_ref.__file__
    with open(src_path) as f:
        src = f.read()
    a, b = MUTATIONS[name]
    assert a in src
    mod = types.ModuleType("oracle.dit_ref_mutant")
    mod.__package__ = "oracle"
    exec(compile(src.replace(a, b, 1), src_path, "exec"), mod.__dict__)
    kind, f2s, s2f, grid = CASES[0]
    blk = make_block(dit, kind, f2s, s2f)
    _swap_linears(blk, "exact")
    x, e, text = block_inputs(grid)
    rope = dit.SkiparseRopeWrapper(dit.rope_freqs(128))
    tm, _ = dit.skiparse_masks(1, grid, 2, "cpu")
    with torch.no_grad():
        got = blk(x, tm, tm, e, grid, grid, rope, text, fused=False)
    sd = {k: v.detach() for k, v in blk.state_dict().items()}
    want = mod.block(sd, x, e, text, grid, kind, f2s, s2f, num_heads=2, linear="exact")
    nw, mx = block_errors(got, want, out_layout(kind, f2s, s2f, x, grid))
    assert not (nw < TOL_EXACT[0] and mx < TOL_EXACT[1]), (name, nw, mx)


def test_key_list_cache_is_per_mask(dit):
    """The attention's key lists are kept per mask tensor and version: masks used in turn (the
    token and group masks of alternating Skiparse blocks) keep their own lists, the lists of a mask
    stay while it lives (a captured graph reads their addresses), a mask modified in place gets new
    lists without dropping the old ones, and a mask's entry goes when the mask does."""
    import gc
    a = torch.tensor([[True, False, True, True], [True, True, False, False]])
    b = torch.tensor([[False, True, True, True], [True, False, True, False]])
    la = dit._cached_key_list(a)
    lb = dit._cached_key_list(b)
    assert dit._cached_key_list(a)[0] is la[0] and dit._cached_key_list(b)[1] is lb[1]
    assert la[1].tolist() == [3, 2] and la[0][0, :3].tolist() == [0, 2, 3] and la[0][1, :2].tolist() == [0, 1]
    a_copy = a.clone()
    assert dit._cached_key_list(a_copy)[0] is not la[0]
    assert dit._cached_key_list(a)[0] is la[0]                 # the copy did not evict a's lists
    a[0, 1] = True                                             # in place: a new version
    la2 = dit._cached_key_list(a)
    assert la2[0] is not la[0] and la2[1].tolist() == [4, 2]
    ent = dit._KEY_LISTS[id(a)][1]
    assert len(ent) == 2 and any(v[0] is la[0] for v in ent.values())
    n = len(dit._KEY_LISTS)
    del a, a_copy
    gc.collect()
    assert len(dit._KEY_LISTS) == n - 2
    assert dit._cached_key_list(None) == (None, None)
