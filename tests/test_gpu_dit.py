"""GPU parity of the DiT block harness (osp_next.py:819-1022, the HiF8 linears at their call
sites): every linear, the modulated-norm producers, the grouped q/k/v and k/v launches and the
FFN's GELU + amax epilogue on the HIP kernels, against the oracle's CPU block
(oracle/dit_ref.py) on the same parameters and inputs.

Tolerances are those of the CPU glue check with HiF8 linears (test_dit_cpu.TOL_HIF8, reasoned
there): the GPU block differs from the exactly evaluated one by fp32 accumulation order in the
GEMMs and attention, which moves some bf16 intermediates by one unit and, through the next
quantisation, a few HiF8 codes by one step."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from oracle import dit_ref  # noqa: E402
from test_dit_cpu import (CASES, TOL_HIF8, _layout_in, block_errors, block_inputs, make_block,  # noqa: E402
                          out_layout)

DEV = "cuda:0"


@pytest.fixture(scope="module")
def dit(pkg):
    from ospnext_amd import dit as D
    return D


def run_block(dit, blk, xin, e, text, grid, kind, fused):
    rope = dit.SkiparseRopeWrapper(dit.rope_freqs(128).to(DEV))
    tm, gm = dit.skiparse_masks(1, grid, 2, DEV)
    am = {"token": tm, "group": gm, "full": None}[kind]
    with torch.no_grad():
        y = blk(xin.to(DEV), am, am, e.to(DEV), grid, grid, rope, text.to(DEV), fused=fused)
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("kind,f2s,s2f,grid", CASES)
def test_block_matches_oracle(dit, kind, f2s, s2f, grid):
    print(f"[dit] block {kind} f2s={f2s} s2f={s2f} grid={grid}", flush=True)
    blk = make_block(dit, kind, f2s, s2f, quant="hif8", device=DEV)
    x, e, text = block_inputs(grid)
    xin = _layout_in(dit, kind, f2s, x, grid)
    sd = {k: v.detach().cpu() for k, v in blk.state_dict().items()}
    want = dit_ref.block(sd, xin, e, text, grid, kind, f2s, s2f, num_heads=2)
    ref_layout = out_layout(kind, f2s, s2f, xin, grid)
    outs = {}
    for fused in (False, True):
        got = run_block(dit, blk, xin, e, text, grid, kind, fused)
        assert got.shape == want.shape and got.dtype == torch.bfloat16
        assert torch.isfinite(got.float()).all()
        nw, mx = block_errors(got, want, ref_layout)
        assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (fused, nw, mx)
        outs[fused] = got
    # the two routes quantise the same tensors; they differ only where the producer's layer norm
    # or the epilogue's GELU rounds a value one unit differently
    nw, mx = block_errors(outs[True], outs[False], ref_layout)
    assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (nw, mx)


@pytest.mark.parametrize("kind,f2s,s2f,grid", [CASES[0], CASES[2], CASES[4]])
def test_block_fused_norm_rope_matches_oracle(dit, kind, f2s, s2f, grid, monkeypatch):
    """dim 512 (4 heads of 128): the fused route runs the q/k norms and the rope through
    hif8_rms_norm_rope (self-attention q/k with rope, cross-attention q/k without) and norm3
    with the cross-attention q's quantisation through hif8_ln_affine_*."""
    calls = []
    orig = dit.rms_norm_rope

    def spy(*a, **k):
        calls.append(a[3] is not None if len(a) > 3 else k.get("cos_f") is not None)
        return orig(*a, **k)

    monkeypatch.setattr(dit, "rms_norm_rope", spy)
    aff = []
    orig_aff = dit.affine_norm_quant

    def spy_aff(*a, **k):
        aff.append(1)
        return orig_aff(*a, **k)

    monkeypatch.setattr(dit, "affine_norm_quant", spy_aff)
    blk = make_block(dit, kind, f2s, s2f, dim=512, heads=4, ffn=1024, quant="hif8", device=DEV, seed=4)
    x, e, text = block_inputs(grid, dim=512, seed=5)
    xin = _layout_in(dit, kind, f2s, x, grid)
    sd = {k: v.detach().cpu() for k, v in blk.state_dict().items()}
    want = dit_ref.block(sd, xin, e, text, grid, kind, f2s, s2f, num_heads=4)
    got = run_block(dit, blk, xin, e, text, grid, kind, True)
    assert sorted(calls) == [False, False, True, True], calls
    assert aff == [1], aff          # norm3 + the cross-attention q's quantisation in one producer
    nw, mx = block_errors(got, want, out_layout(kind, f2s, s2f, xin, grid))
    assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (nw, mx)


def test_block_with_hif8_attention(dit):
    """quant_attn="hif8" (configs/infer/npu/osp_hif8_14b.yaml:42): Q/K/V quantised before SDPA."""
    kind, f2s, s2f, grid = CASES[0]
    blk = make_block(dit, kind, f2s, s2f, quant="hif8", device=DEV, quant_attn="hif8")
    x, e, text = block_inputs(grid, seed=9)
    sd = {k: v.detach().cpu() for k, v in blk.state_dict().items()}
    want = dit_ref.block(sd, x, e, text, grid, kind, f2s, s2f, num_heads=2, quant_attn="hif8")
    got = run_block(dit, blk, x, e, text, grid, kind, None)
    nw, mx = block_errors(got, want, out_layout(kind, f2s, s2f, x, grid))
    assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (nw, mx)


def test_block_with_hif8_attention_producers(dit, monkeypatch):
    """quant_attn="hif8" at dim 512 (head dim 128), where the fused route's q and k come out of the
    quantising norm + rope producer (self-attention with rope, cross-attention without) and the
    attention kernel runs on the quantised operands: against the oracle's CPU block."""
    kind, f2s, s2f, grid = CASES[0]
    blk = make_block(dit, kind, f2s, s2f, dim=512, heads=4, ffn=1024, quant="hif8", device=DEV, quant_attn="hif8")
    x, e, text = block_inputs(grid, dim=512, seed=11)
    sd = {k: v.detach().cpu() for k, v in blk.state_dict().items()}
    want = dit_ref.block(sd, x, e, text, grid, kind, f2s, s2f, num_heads=4, quant_attn="hif8")
    calls = []
    orig = dit.rms_norm_rope_quant

    def spy(x_, norm, scale_max, cos_f=None, sin_f=None, head_dim=128, return_y=False):
        calls.append(cos_f is not None)
        return orig(x_, norm, scale_max, cos_f, sin_f, head_dim, return_y)
    monkeypatch.setattr(dit, "rms_norm_rope_quant", spy)
    got = run_block(dit, blk, x, e, text, grid, kind, None)
    assert sorted(calls) == [False, False, True, True], calls
    nw, mx = block_errors(got, want, out_layout(kind, f2s, s2f, x, grid))
    assert nw < TOL_HIF8[0] and mx < TOL_HIF8[1], (nw, mx)


def test_block_stack_dual_end(dit):
    """The block loop with the dual-end schedule (8 layers, 4 full): full, full, token (from full),
    group, token, group (to full), full, full; the output is in (t, h, w) order again."""
    dim, heads, ffn, grid = 256, 2, 512, (2, 6, 8)
    torch.manual_seed(0)
    stack = dit.OSPNextBlocks(dim, ffn, heads, num_layers=8, num_full_blocks=4, quant="hif8", device=DEV)
    g = torch.Generator().manual_seed(21)
    with torch.no_grad():
        for n, p in stack.named_parameters():
            if "norm" in n:
                p.copy_((1 + 0.1 * torch.randn(p.shape, generator=g)).to(p.dtype))
            elif n.endswith("modulation"):
                p.copy_((torch.randn(p.shape, generator=g) / dim ** 0.5).to(p.dtype))
            else:
                p.copy_((0.02 * torch.randn(p.shape, generator=g)).to(p.dtype))
    x, e, text = block_inputs(grid, dim=dim, seed=22)
    with torch.no_grad():
        got = stack(x.to(DEV), e.to(DEV), text.to(DEV), grid).cpu()
    sched = dit.block_schedule(8, "dual_end", 4)
    sds = [{k: v.detach().cpu() for k, v in b.state_dict().items()} for b in stack.blocks]
    want = dit_ref.blocks(sds, sched, x, e, text, grid, num_heads=heads)
    assert got.shape == x.shape == want.shape
    # eight blocks: each one's tolerance on its own update, which the stack sums
    nw, mx = block_errors(got, want, x)
    assert nw < TOL_HIF8[0] and mx < 2 * TOL_HIF8[1], (nw, mx)
