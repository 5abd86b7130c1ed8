"""The inference paths under HIP graph capture (torch.cuda.CUDAGraph): HIF8Linear on both GEMM
routes, the fused FFN (GELU-statistic GEMM, settle kernel, GELU fake quant) and the modulated
LayerNorm producer launch only kernels -- no host synchronisation, allocation outside torch's
graph pool, or memset nodes -- so a captured step replays them.  Each graph is replayed several
times with eager work on the same modules and states in between, and every replay is compared
bit for bit with the eager result."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def capture(fn):
    """Warm fn up on a side stream, then capture one call; returns (graph, output)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def bits(t):
    return t.view(torch.int16)


def replay_and_check(graph, out, ref, eager):
    for rep in range(3):
        eager()                       # eager work on the same modules and states
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), f"replay {rep}"


@pytest.mark.parametrize("M", [1000, 9000])   # the fused route, and the decode-once route from 8192 rows
def test_hif8linear_forward_replays(pkg, M):
    print(f"[graph] HIF8Linear M={M}", flush=True)
    torch.manual_seed(M)
    lin = pkg.HIF8Linear(1024, 768, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.bias.normal_(0, 0.02)
        lin.prepack()
        x = torch.randn(M, 1024, device=DEV).to(torch.bfloat16)
        x2 = (x * 3).contiguous()
        ref = lin(x).clone()
        graph, out = capture(lambda: lin(x))
        replay_and_check(graph, out, ref, lambda: lin(x2))


def test_fused_ffn_replays(pkg):
    """The GELU route: the up-projection's statistic settles the down-projection's scale inside
    the graph, and an eager call on other data between replays leaves nothing behind."""
    print("[graph] HIF8FFN", flush=True)
    torch.manual_seed(5)
    ffn = pkg.HIF8FFN(512, 1536, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in ffn.parameters():
            p.normal_(0, 0.05)
        ffn[0].prepack()
        ffn[2].prepack()
        x = torch.randn(2048, 512, device=DEV).to(torch.bfloat16)
        x2 = (-2 * x).contiguous()   # mostly negative pre-activations: the pending path
        ref = ffn(x).clone()
        graph, out = capture(lambda: ffn(x))
        replay_and_check(graph, out, ref, lambda: ffn(x2))


def test_modulated_norm_quant_replays(pkg):
    print("[graph] modulated_norm_quant", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(4096, 1024, generator=g, device=DEV).to(torch.bfloat16)
    shift = torch.randn(1, 1024, generator=g, device=DEV).to(torch.bfloat16)
    scale = (torch.randn(1, 1024, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    with torch.no_grad():
        ref, _ = pkg.modulated_norm_quant(x, shift, scale, 1e-6, 15.0)
        ref = ref.clone()
        graph, out = capture(lambda: pkg.modulated_norm_quant(x, shift, scale, 1e-6, 15.0)[0])
        replay_and_check(graph, out, ref, lambda: pkg.modulated_norm_quant(x * 2, shift, scale, 1e-6, 15.0))


def test_static_producer_replays(pkg):
    """The allocation-free producer (static device workspace) is what graph-captured callers that
    cannot allocate use: its workspace clear is a kernel, not a memset node."""
    print("[graph] modulated_norm_quant_static", flush=True)
    g = torch.Generator(device=DEV).manual_seed(8)
    x = torch.randn(3000, 1024, generator=g, device=DEV).to(torch.bfloat16)
    shift = torch.randn(1, 1024, generator=g, device=DEV).to(torch.bfloat16)
    scale = (torch.randn(1, 1024, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    with torch.no_grad():
        ref, _ = pkg.modulated_norm_quant(x, shift, scale, 1e-6, 15.0)
        ref = ref.clone()
        graph, out = capture(lambda: pkg.modulated_norm_quant_static(x, shift, scale, 1e-6, 15.0))
        replay_and_check(graph, out, ref, lambda: pkg.modulated_norm_quant_static(x[:1000] * 2, shift, scale, 1e-6, 15.0))


def test_dit_block_fused_route_replays(pkg):
    """A whole DiT block on its inference route -- producers, grouped GEMMs, q/k norm + rope, the
    attention kernel with a key padding mask and the o amax in its epilogue, the FFN's GELU route,
    residual updates -- captured once and replayed bit-identically, with eager calls on other
    data in between (grid 2x5x8: H padded to 6 for the 2x2 sub-grids, so the mask has padding)."""
    print("[graph] DiT block, fused route", flush=True)
    from ospnext_amd import dit as D
    from test_dit_cpu import block_inputs, make_block
    blk = make_block(D, "token", True, False, quant="hif8", device=DEV)
    for m in blk.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack()
    grid = (2, 5, 8)
    x, e, text = (t.to(DEV) for t in block_inputs(grid))
    x2 = (x * -1.5).contiguous()
    rope = D.SkiparseRopeWrapper(D.rope_freqs(128).to(DEV))
    tm, _ = D.skiparse_masks(1, grid, 2, DEV)
    assert tm is not None and not bool(tm.all())
    with torch.no_grad():
        ref = blk(x, tm, tm, e, grid, grid, rope, text, fused=True).clone()
        graph, out = capture(lambda: blk(x, tm, tm, e, grid, grid, rope, text, fused=True))
        replay_and_check(graph, out, ref, lambda: blk(x2, tm, tm, e, grid, grid, rope, text, fused=True))


def test_dit_block_replays_with_other_masks_between(pkg):
    """The block's captured graph holds the device addresses of its mask's key lists.  Eager calls
    on other mask objects between the replays -- a copy of the mask, and a mask with more padding --
    must not free or replace those lists: each replay still equals the eager result (the key lists
    are kept per mask tensor, for as long as the mask lives)."""
    print("[graph] DiT block, other masks between replays", flush=True)
    from ospnext_amd import dit as D
    from test_dit_cpu import block_inputs, make_block
    blk = make_block(D, "token", True, False, quant="hif8", device=DEV)
    for m in blk.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack()
    grid = (2, 5, 8)
    x, e, text = (t.to(DEV) for t in block_inputs(grid))
    rope = D.SkiparseRopeWrapper(D.rope_freqs(128).to(DEV))
    tm, _ = D.skiparse_masks(1, grid, 2, DEV)
    other = tm.clone()
    other[:, -7:] = False
    with torch.no_grad():
        ref = blk(x, tm, tm, e, grid, grid, rope, text, fused=True).clone()
        ref_other = blk(x, other, other, e, grid, grid, rope, text, fused=True).clone()
        assert not torch.equal(bits(ref), bits(ref_other))
        graph, out = capture(lambda: blk(x, tm, tm, e, grid, grid, rope, text, fused=True))
        for rep in range(3):
            copy = tm.clone()                      # a new mask object, new lists
            y1 = blk(x, copy, copy, e, grid, grid, rope, text, fused=True)
            y2 = blk(x, other, other, e, grid, grid, rope, text, fused=True)
            del copy
            torch.cuda.synchronize()
            assert torch.equal(bits(y1), bits(ref)) and torch.equal(bits(y2), bits(ref_other))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(bits(out), bits(ref)), f"replay {rep}"
