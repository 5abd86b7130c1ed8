"""GPU parity of the grouped fused linear (several HIF8Linear layers on one input, e.g. the
self-attention q/k/v of osp_next.py:742-744, in one launch): every group's output equals the
single-weight fused linear of that weight bit for bit, with and without biases, for group sets
whose tiles end inside the last group; and the q/k/v helper follows weight updates."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def weights(seed, ns, K, bias_mask):
    g = torch.Generator().manual_seed(seed)
    out = []
    for n, has_b in zip(ns, bias_mask):
        w = (torch.randn(n, K, generator=g) * 0.02 * (1 + len(out))).to(torch.bfloat16).to(DEV)
        b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(DEV) if has_b else None
        out.append((w, b))
    return out


@pytest.mark.parametrize("M,K,ns,bias_mask", [
    (300, 512, (256, 512, 264), (True, True, True)),
    (300, 512, (256, 512, 264), (True, False, True)),
    (1000, 5120, (5120, 5120, 5120), (True, True, True)),
    (77, 1536, (1536,), (False,)),
    (513, 256, (256,) * 7 + (8,), (True,) * 8),
    (64, 64, (256, 256), (False, False)),
])
def test_grouped_equals_separate(pkg, M, K, ns, bias_mask):
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    ws = weights(K, ns, K, bias_mask)
    packs = [pkg.PackedWeight(w, 15.0) for w, _ in ws]
    assert pkg.grouped_ok(packs)
    gw = pkg.GroupedWeight(packs, [b for _, b in ws])
    ys = pkg.linear_fwd_grouped(a, gw)
    for y, p, (_, b) in zip(ys, packs, ws):
        want = pkg.linear_fwd(a, fmt, st, p, b)
        assert y.shape == want.shape
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_grouped_rejects_what_it_cannot_take(pkg):
    K = 256
    ws = weights(1, (264, 256), K, (False, False))
    packs = [pkg.PackedWeight(w, 15.0) for w, _ in ws]
    assert not pkg.grouped_ok(packs)                      # a group other than the last not a multiple of 256
    with pytest.raises(ValueError):
        pkg.GroupedWeight(packs, [None, None])
    mixed = [pkg.PackedWeight(weights(2, (256,), 256, (False,))[0][0], 15.0),
             pkg.PackedWeight(weights(3, (256,), 512, (False,))[0][0], 15.0)]
    assert not pkg.grouped_ok(mixed)                      # different in_features


def test_qkv_helper_follows_weight_updates(pkg):
    D = 512
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 70, D, generator=g).to(torch.bfloat16).to(DEV)
    e = (torch.randn(1, 6, D, generator=g) * 0.5).to(torch.bfloat16).to(DEV).chunk(6, dim=1)
    torch.manual_seed(1)
    lins = [pkg.HIF8Linear(D, D).to(DEV).to(torch.bfloat16) for _ in range(3)]
    with torch.no_grad():
        for m in lins:
            m.weight.normal_(0, 0.02)
            m.bias.normal_(0, 0.1)
        _, _, y = pkg.modulated_norm_quant(x, e[0], e[1], return_y=True)
        first = pkg.qkv_from_modulated_norm(x, e[0], e[1], *lins)
        for got, m in zip(first, lins):
            assert torch.equal(got.view(torch.int16), m(y).view(torch.int16))
        lins[1].weight.mul_(3.0)                          # in place: the packed weight is rebuilt
        lins[2].bias.add_(1.0)
        second = pkg.qkv_from_modulated_norm(x, e[0], e[1], *lins)
        for got, m in zip(second, lins):
            assert torch.equal(got.view(torch.int16), m(y).view(torch.int16))
        assert not torch.equal(first[1], second[1]) and not torch.equal(first[2], second[2])
