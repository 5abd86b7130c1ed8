"""GPU parity of the HiF8 Q/K/V quantisation around attention (ospnext/modules/hif8_attention.py).

Q/K (fp32) and V (bf16) forward quantisation and the backward gradient quantisation
(scale_max_backward = 224) are bit-exact against the CPU restatement of _quant.  The
attention itself is torch SDPA (the reference's non-flash branch); it is run here in
float32 and compared with a float32 softmax(QK^T/sqrt(D))V on the quantised inputs."""
from __future__ import annotations

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def bits16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_qkv_quant_forward_bit_exact(pkg, R):
    g = torch.Generator(device="cpu").manual_seed(0)
    B, N, H, D = 1, 96, 4, 64
    q = torch.randn(B, N, H, D, generator=g)
    k = torch.randn(B, N, H, D, generator=g) * 3
    v = torch.randn(B, N, H, D, generator=g).to(torch.bfloat16)
    qq, kq, vq = pkg._HIF8QKVQuantFunction.apply(q.to(DEV), k.to(DEV), v.to(DEV), 15.0, 224.0)
    for got, src in ((qq, q), (kq, k)):
        want, _ = R.quant_f32(src.numpy(), 15.0, "npu")
        assert got.dtype == torch.float32
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    want_v, _ = R.quant_bf16(bits16(v), 15.0, "npu")
    assert vq.dtype == torch.bfloat16 and np.array_equal(bits16(vq), want_v.reshape(v.shape))


def test_qkv_quant_backward_quantises_grads(pkg, R):
    g = torch.Generator(device="cpu").manual_seed(1)
    shape = (1, 64, 2, 64)
    q = torch.randn(shape, generator=g).to(DEV).requires_grad_(True)
    k = torch.randn(shape, generator=g).to(DEV).requires_grad_(True)
    v = torch.randn(shape, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    outs = pkg._HIF8QKVQuantFunction.apply(q, k, v, 15.0, 224.0)
    grads = [torch.randn(shape, generator=g) * 1e-2 for _ in range(2)] + [
        (torch.randn(shape, generator=g) * 1e-2).to(torch.bfloat16)]
    torch.autograd.backward(outs, [t.to(DEV) for t in grads])
    for leaf, gin in ((q, grads[0]), (k, grads[1])):
        want, _ = R.quant_f32(gin.numpy(), 224.0, "npu")
        assert np.array_equal(leaf.grad.cpu().numpy().view(np.uint32), want.view(np.uint32))
    want_v, _ = R.quant_bf16(bits16(grads[2]), 224.0, "npu")
    assert np.array_equal(bits16(v.grad), want_v.reshape(shape))
    # one grad missing (None): that input gets no gradient, the others still quantised
    q2 = q.detach().clone().requires_grad_(True)
    outs2 = pkg._HIF8QKVQuantFunction.apply(q2, k.detach(), v.detach(), 15.0, 224.0)
    outs2[0].backward(grads[0].to(DEV))
    want, _ = R.quant_f32(grads[0].numpy(), 224.0, "npu")
    assert np.array_equal(q2.grad.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("masked", [False, True])
def test_hif8_attention_with_mask(pkg, R, masked):
    g = torch.Generator(device="cpu").manual_seed(2)
    B, N, H, D = 2, 80, 3, 64
    q, k, v = (torch.randn(B, N, H, D, generator=g) for _ in range(3))
    mask = None
    if masked:
        mask = torch.ones(B, N, dtype=torch.bool)
        mask[1, 60:] = False
    out = pkg.hif8_attention_with_mask(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask_kv=None if mask is None else mask.to(DEV),
                                       dtype=torch.float32)
    assert out.shape == (B, N, H, D) and out.dtype == torch.float32
    qq, kq, vq = (torch.from_numpy(R.quant_f32(t.numpy(), 15.0, "npu")[0]).double() for t in (q, k, v))
    s = torch.einsum("bnhd,bmhd->bhnm", qq, kq) / math.sqrt(D)
    if mask is not None:
        s = s.masked_fill(~mask[:, None, None, :], float("-inf"))
    ref = torch.einsum("bhnm,bmhd->bnhd", torch.softmax(s, -1), vq)
    err = float((out.cpu().double() - ref).abs().max() / ref.abs().max())
    assert err < 1e-4, err
