"""GPU parity of the attention kernel (hif8_attention_fwd) and of the amax its epilogue leaves for
the o projection.

The attention (attention_with_mask, ospnext/modules/attention.py:460-518, SDPA branch) is floating
point: the kernel is compared with softmax(scale q k^T) v computed in float64 on the CPU (float32 on
the GPU for the larger shapes) on the same bf16 inputs, over exactly the keys each batch keeps.
Tolerance: the kernel rounds the probabilities to bf16 for the P.V products and the output to
bf16, each a relative error of at most 2^-9, so the output's normwise error stays near 2^-9 of its
norm; the tests require normwise <= 1e-2 and elementwise <= 2e-2 of the output's largest magnitude.
The epilogue's state must equal, bit for bit, the state an amax pass over the kernel's own output
gives (hif8_absmax_scale with the same dtype rule), and the quantised o input must then be the same."""
from __future__ import annotations

import math

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = 128


def make(B, Nq, Nkv, H, seed, kb=None, qscale=1.0, kscale=1.0):
    g = torch.Generator().manual_seed(seed)
    kb = B if kb is None else kb
    q = (torch.randn(B, Nq, H, D, generator=g) * qscale).to(torch.bfloat16)
    k = (torch.randn(kb, Nkv, H, D, generator=g) * kscale).to(torch.bfloat16)
    v = torch.randn(kb, Nkv, H, D, generator=g).to(torch.bfloat16)
    return q, k, v


def reference(q, k, v, rows=None, scale=None, dtype=torch.float64, device="cpu"):
    """softmax(scale q k^T) v per batch over the key rows given (all keys when None)."""
    B, Nq, H, _ = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = torch.zeros(B, Nq, H, D, dtype=dtype, device=device)
    for b in range(B):
        kb = k[b if k.shape[0] == B else 0].to(device, dtype)
        vb = v[b if v.shape[0] == B else 0].to(device, dtype)
        if rows is not None:
            r = rows[b]
            if len(r) == 0:
                continue
            idx = torch.as_tensor(r, dtype=torch.long, device=device)
            kb, vb = kb[idx], vb[idx]
        qh = q[b].to(device, dtype).permute(1, 0, 2).contiguous()     # [H, Nq, D]
        kt = kb.permute(1, 2, 0).contiguous()                         # [H, D, Nk]
        vh = vb.permute(1, 0, 2).contiguous()                         # [H, Nk, D]
        p = torch.softmax(torch.matmul(qh, kt) * scale, dim=-1)
        out[b] = torch.matmul(p, vh).permute(1, 0, 2)
    return out


def check(got, want, tag):
    got = got.double().cpu()
    want = want.double().cpu()
    assert torch.isfinite(got).all(), tag
    err = (got - want).norm() / want.norm().clamp_min(1e-30)
    mx = (got - want).abs().max() / want.abs().max().clamp_min(1e-30)
    assert err <= 1e-2 and mx <= 2e-2, f"{tag}: normwise {float(err):.3e}, max {float(mx):.3e}"


def run(pkg, q, k, v, **kw):
    return pkg.attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), **kw)


def test_all_keys_ragged_sizes(pkg):
    print("[attn] all keys", flush=True)
    for (B, Nq, Nkv, H, seed) in ((2, 300, 200, 3, 0), (1, 5, 1, 1, 1), (1, 257, 64, 2, 2), (3, 16, 65, 1, 3)):
        q, k, v = make(B, Nq, Nkv, H, seed)
        check(run(pkg, q, k, v), reference(q, k, v), f"B{B} Nq{Nq} Nkv{Nkv} H{H}")


def test_key_list_and_counts(pkg):
    """Per-batch lists of kept key rows in any order, ragged counts (one of them a single key)."""
    print("[attn] key list", flush=True)
    B, Nq, Nkv, H = 3, 200, 300, 2
    q, k, v = make(B, Nq, Nkv, H, 4)
    g = torch.Generator().manual_seed(5)
    counts = [137, 1, 300]
    idx = torch.zeros(B, Nkv, dtype=torch.int32)
    rows = []
    for b, c in enumerate(counts):
        r = torch.randperm(Nkv, generator=g)[:c]
        idx[b, :c] = r.to(torch.int32)
        rows.append(r.tolist())
    cnt = torch.tensor(counts, dtype=torch.int32)
    out = run(pkg, q, k, v, key_idx=idx.to(DEV), key_count=cnt.to(DEV))
    check(out, reference(q, k, v, rows), "key list")
    # counts alone: the first count keys
    out = run(pkg, q, k, v, key_count=cnt.to(DEV))
    check(out, reference(q, k, v, [list(range(c)) for c in counts]), "key counts")


def test_key_list_from_mask(pkg):
    """key_list turns a [B, Nkv] mask into the kernel's rows and counts on the device; the result
    is the masked attention."""
    print("[attn] key mask", flush=True)
    B, Nq, Nkv, H = 2, 130, 190, 2
    q, k, v = make(B, Nq, Nkv, H, 6)
    g = torch.Generator().manual_seed(7)
    mask = torch.rand(B, Nkv, generator=g) < 0.7
    idx, cnt = pkg.key_list(mask.to(DEV))
    assert cnt.cpu().tolist() == mask.sum(1).tolist()
    for b in range(B):
        assert idx[b, :int(cnt[b])].cpu().tolist() == mask[b].nonzero().squeeze(-1).tolist()
    out = run(pkg, q, k, v, key_idx=idx, key_count=cnt)
    check(out, reference(q, k, v, [mask[b].nonzero().squeeze(-1).tolist() for b in range(B)]), "mask")


def test_shared_keys_and_strided_rows(pkg):
    """Keys of batch 1 serving every batch (the cross-attention's text), and q a view of a wider
    row (token stride larger than heads * 128)."""
    print("[attn] shared keys, strided q", flush=True)
    B, Nq, Nkv, H = 3, 100, 96, 2
    q, k, v = make(B, Nq, Nkv, H, 8, kb=1)
    wide = torch.zeros(B, Nq, 2 * H * D, dtype=torch.bfloat16)
    wide[:, :, H * D:] = q.reshape(B, Nq, H * D)
    qs = wide.to(DEV)[:, :, H * D:].view(B, Nq, H, D)
    assert qs.stride(1) == 2 * H * D
    out = pkg.attention_fwd(qs, k.to(DEV), v.to(DEV))
    check(out, reference(q, k, v), "shared keys")


def test_empty_key_set_gives_zeros(pkg):
    print("[attn] empty key set", flush=True)
    B, Nq, Nkv, H = 2, 40, 70, 1
    q, k, v = make(B, Nq, Nkv, H, 9)
    cnt = torch.tensor([0, 70], dtype=torch.int32, device=DEV)
    out = run(pkg, q, k, v, key_count=cnt)
    assert torch.count_nonzero(out[0]) == 0
    check(out[1:], reference(q[1:], k[1:], v[1:]), "batch 1")


def test_lazy_rescale_with_growing_scores(pkg):
    """Scores that grow along the keys by far more than the kernel's headroom (the reference max
    moves many times) and large in magnitude (up to ~300 in the exponent)."""
    print("[attn] growing scores", flush=True)
    B, Nq, Nkv, H = 1, 64, 1024, 2
    q, k, v = make(B, Nq, Nkv, H, 10, qscale=2.0)
    ramp = torch.linspace(0.1, 12.0, Nkv).view(1, Nkv, 1, 1)
    k = (k.float() * ramp).to(torch.bfloat16)
    out = run(pkg, q, k, v)
    check(out, reference(q, k, v), "growing")
    # decreasing: the first tile holds the max, later tiles underflow
    kr = torch.flip(k, dims=[1])
    vr = torch.flip(v, dims=[1])
    check(run(pkg, q, kr, vr), reference(q, kr, vr), "decreasing")


def test_one_dominant_key_in_each_lane_group(pkg):
    """One key per batch scores ~230 above the others for every query (exp2 of that difference
    overflows fp32): the output must be that key's value row.  The key sits in each of the four
    4-key groups of a 16-key block (one per batch), which four different lanes of the score
    accumulators hold, in different tiles: a tile max that missed any lane group would overflow."""
    print("[attn] dominant key", flush=True)
    B, Nq, Nkv, H = 4, 48, 600, 1
    g = torch.Generator().manual_seed(15)
    u = torch.randn(D, generator=g)
    u = u / u.norm() * math.sqrt(D)
    q = (u.view(1, 1, 1, D) + 0.05 * torch.randn(B, Nq, H, D, generator=g)).to(torch.bfloat16)
    k = (0.1 * torch.randn(B, Nkv, H, D, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, Nkv, H, D, generator=g).to(torch.bfloat16)
    spikes = [64 * 3 + 2, 64 * 5 + 16 + 6, 32 + 9, 64 * 7 + 48 + 15]   # lane groups 0, 1, 2, 3
    for b, j in enumerate(spikes):
        k[b, j, 0] = (20.0 * u).to(torch.bfloat16)
    out = run(pkg, q, k, v)
    assert torch.isfinite(out.float()).all()
    for b, j in enumerate(spikes):
        want = v[b, j, 0].float().expand(Nq, D)
        assert torch.allclose(out[b, :, 0].float().cpu(), want, atol=2e-2 * float(want.abs().max()), rtol=0)
    check(out, reference(q, k, v), "dominant key")


def test_dit_shape_against_float32(pkg):
    """40 heads (the 14B model's), a padded-grid key mask, a few query tiles; compared with float32
    on the GPU and with torch's SDPA on the kept keys."""
    print("[attn] 40 heads", flush=True)
    B, N, H = 1, 1100, 40
    q, k, v = make(B, N, N, H, 11)
    keep = torch.ones(B, N, dtype=torch.bool)
    keep[:, 1000:] = False
    idx, cnt = pkg.key_list(keep.to(DEV))
    out = run(pkg, q, k, v, key_idx=idx, key_count=cnt)
    ref = reference(q.to(DEV), k.to(DEV), v.to(DEV), [list(range(1000))], dtype=torch.float32, device=DEV)
    check(out, ref, "40 heads vs fp32")
    qt, kt, vt = (t.to(DEV).transpose(1, 2) for t in (q, k[:, :1000], v[:, :1000]))
    sd = torch.nn.functional.scaled_dot_product_attention(qt, kt.contiguous(), vt.contiguous()).transpose(1, 2)
    check(out, sd.float(), "40 heads vs SDPA")


@pytest.mark.parametrize("as_f32", [True, False])
def test_epilogue_state_equals_amax_pass(pkg, as_f32):
    """The state the kernel leaves equals hif8_absmax_scale over its output (amax, scale, flags,
    tables), for the fp32 rule (self-attention o input) and the bf16 rule (cross-attention); a
    second call on other data leaves no trace of the first."""
    print(f"[attn] epilogue state as_f32={as_f32}", flush=True)
    for seed, scale in ((12, 1.0), (13, 40.0)):
        B, Nq, Nkv, H = 2, 520, 300, 4
        q, k, v = make(B, Nq, Nkv, H, seed)
        v = (v.float() * scale).to(torch.bfloat16)
        st = pkg.QuantState(DEV)
        out = run(pkg, q, k, v, o_state=st, o_as_f32=as_f32, scale_max=15.0)
        want = pkg.absmax_scale(out.reshape(-1, H * D), 15.0, pkg.QuantState(DEV), as_f32=as_f32)
        torch.cuda.synchronize()
        assert st.read() == want.read()
        # every field of the state: counters, amax, scale, flags, both tables (the buffer's tail
        # past them is padding)
        n = 32 + 2 * 256 + 4 * 256
        assert torch.equal(st.buf[:n], want.buf[:n]), "state fields (tables, flags) differ"
        x2 = out.reshape(-1, H * D)
        if as_f32:
            a = pkg.fake_quant_to_bf16(x2, st, as_f32=True)
            b = pkg.fake_quant_to_bf16(x2, want, as_f32=True)
        else:
            a, b = pkg.fake_quant(x2, st), pkg.fake_quant(x2, want)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_o_projection_settled_equals_forward(pkg):
    """HIF8Linear.forward_settled on the attention output with the epilogue's state is exactly
    forward(out.float()) (self-attention) and forward(out) (cross-attention)."""
    print("[attn] forward_settled", flush=True)
    B, Nq, Nkv, H = 1, 600, 256, 4
    q, k, v = make(B, Nq, Nkv, H, 14)
    lin = pkg.HIF8Linear(H * D, H * D, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.bias.normal_(0, 0.02)
        lin.prepack()
        for as_f32 in (True, False):
            st = pkg.QuantState(DEV)
            out = run(pkg, q, k, v, o_state=st, o_as_f32=as_f32, scale_max=lin.scale_max_forward).reshape(B, Nq, H * D)
            got = lin.forward_settled(out, st, as_f32=as_f32)
            want = lin(out.float()) if as_f32 else lin(out)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"as_f32={as_f32}"


@pytest.mark.parametrize("o_as_f32", [True, False])
def test_quant_attn_route_equals_hif8_qkv_quant(pkg, o_as_f32):
    """quant_attn="hif8" on the attention kernel (the block's inference route): its inputs are the
    bf16 casts of _HIF8QKVQuantFunction's outputs (hif8_attention.py:60-74, the per-tensor _quant
    of q and k in fp32 for the self-attention, of v in bf16), so its output equals the kernel run
    on those tensors bit for bit, and the o state equals an amax pass over the output."""
    print(f"[attn] quant_attn route o_as_f32={o_as_f32}", flush=True)
    B, N, H = 2, 300, 2
    att = pkg.dit.OSPNextSelfAttention(H * D, H, quant="hif8", quant_attn="hif8", device=DEV, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(16)
    dt = torch.float32 if o_as_f32 else torch.bfloat16
    q = (torch.randn(B, N, H, D, generator=g) * 2).to(dt).to(DEV)
    k = torch.randn(B, N, H, D, generator=g).to(dt).to(DEV)
    v = torch.randn(B, N, H, D, generator=g).to(torch.bfloat16).to(DEV)
    mask = (torch.rand(B, N, generator=g) < 0.8).to(DEV)
    with torch.no_grad():
        out, st = att._quantised_attention(q, k, v, mask, o_as_f32=o_as_f32)
        qq, kq, vq = pkg._HIF8QKVQuantFunction.apply(q, k, v, 15.0, 224.0)
        idx, cnt = pkg.key_list(mask)
        want = pkg.attention_fwd(qq.to(torch.bfloat16), kq.to(torch.bfloat16), vq, idx, cnt)
        full = pkg.absmax_scale(out.reshape(-1, H * D), 15.0, pkg.QuantState(DEV), as_f32=o_as_f32)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert st.read() == full.read()
