"""HiF8 fake quant of Q/K/V around attention, mirroring ``ospnext/modules/hif8_attention.py``.

Forward (hif8_attention.py:60-74)::

    Q_q = qdq(Q * s_q) / s_q,  s_q = scale_max_forward / max|Q|     (same for K, V)
    out = attention_with_mask(Q_q, K_q, V_q, ...)

Backward (hif8_attention.py:76-87) quantises each incoming gradient dQ_q, dK_q,
dV_q with ``scale_max_backward`` the same way.  The per-tensor quantisation is
``_quant`` of ``hif8_linear`` (one amax pass and one quantise pass on the GPU).

The attention kernel itself is outside the HiF8 path: ``attention_with_mask`` is
the reference's SDPA route (``ospnext/modules/attention.py:433-518``, the branch
taken when no flash-attention package is present), on torch's
``scaled_dot_product_attention``.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .hif8_linear import _quant


class _HIF8QKVQuantFunction(torch.autograd.Function):
    """hif8_attention.py:40-87: quantised (Q_q, K_q, V_q) forward, quantised grads backward."""

    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor, v: Tensor, scale_max_forward: float, scale_max_backward: float):
        q_q, _ = _quant(q, scale_max_forward)
        k_q, _ = _quant(k, scale_max_forward)
        v_q, _ = _quant(v, scale_max_forward)
        # the reference keeps the backward scale as a tensor of q's dtype and reads it
        # back with .item(): the value is scale_max_backward rounded to that dtype
        ctx.smb = float(torch.tensor(scale_max_backward, dtype=q.dtype).item())
        return q_q, k_q, v_q

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        def qg(g):
            return None if g is None else _quant(g, ctx.smb)[0]
        return qg(grad_q), qg(grad_k), qg(grad_v), None, None


def scaled_dot_product_attention_with_mask(q: Tensor, k: Tensor, v: Tensor, attn_mask: Optional[Tensor] = None,
                                           causal: bool = False, dropout_p: float = 0.0) -> Tensor:
    """attention.py:433-458: [B, N, H, D] in and out; a [B, Nkv] mask is a key-side mask."""
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if attn_mask is not None:
        if attn_mask.dtype != torch.bool:
            attn_mask = attn_mask.to(q.dtype)
        attn_mask = attn_mask[:, None, None, :]
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=causal,
                                                           dropout_p=dropout_p)
    return out.transpose(1, 2)


def attention_with_mask(q: Tensor, k: Tensor, v: Tensor, attn_mask: Optional[Tensor] = None,
                        attn_mask_kv: Optional[Tensor] = None, is_cross_attn: bool = False, causal: bool = False,
                        softmax_scale: Optional[float] = None, deterministic: bool = False, dropout_p: float = 0.0,
                        dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """attention.py:460-518, SDPA branch: computes in ``dtype``, returns q's dtype.  As in
    that branch, ``attn_mask`` (query-side), ``is_cross_attn``, ``softmax_scale`` and
    ``deterministic`` do not change the result (SDPA uses 1/sqrt(D))."""
    out_dtype = q.dtype
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    out = scaled_dot_product_attention_with_mask(q, k, v, attn_mask=attn_mask_kv, causal=causal, dropout_p=dropout_p)
    return out.to(out_dtype)


def hif8_attention_with_mask(q: Tensor, k: Tensor, v: Tensor, attn_mask: Optional[Tensor] = None,
                             attn_mask_kv: Optional[Tensor] = None, is_cross_attn: bool = False,
                             causal: bool = False, softmax_scale: Optional[float] = None,
                             deterministic: bool = False, dropout_p: float = 0.0,
                             dtype: torch.dtype = torch.bfloat16, scale_max_forward: float = 15.0,
                             scale_max_backward: float = 224.0) -> Tensor:
    """hif8_attention.py:93-126: HiF8 qdq of Q, K, V, then attention_with_mask."""
    q_q, k_q, v_q = _HIF8QKVQuantFunction.apply(q, k, v, scale_max_forward, scale_max_backward)
    return attention_with_mask(q_q, k_q, v_q, attn_mask=attn_mask, attn_mask_kv=attn_mask_kv,
                               is_cross_attn=is_cross_attn, causal=causal, softmax_scale=softmax_scale,
                               deterministic=deterministic, dropout_p=dropout_p, dtype=dtype)
