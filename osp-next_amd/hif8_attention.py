"""HiF8 fake quant of Q/K/V around attention, mirroring ``ospnext/modules/hif8_attention.py``.

Forward (hif8_attention.py:60-74)::

    Q_q = qdq(Q * s_q) / s_q,  s_q = scale_max_forward / max|Q|     (same for K, V)
    out = attention_with_mask(Q_q, K_q, V_q, ...)

Backward (hif8_attention.py:76-87) quantises each incoming gradient dQ_q, dK_q,
dV_q with ``scale_max_backward`` the same way.  The per-tensor quantisation is
``_quant`` of ``hif8_linear`` (one amax pass and one quantise pass on the GPU).

``attention_with_mask`` is the reference's SDPA route
(``ospnext/modules/attention.py:433-518``, the branch taken when no flash-attention package is
present), on torch's ``scaled_dot_product_attention``.  ``attention_fwd`` is the library's own
attention kernel (``hif8_attention_fwd``): the same attention on a list of kept keys, whose
epilogue also leaves the o projection's amax and scale in a quantisation state, so that
``_quant`` of the attention output (``osp_next.py:777``) needs no amax pass.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib
from .hif8_linear import QuantState, _quant


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


def key_list(key_mask: Tensor) -> Tuple[Tensor, Tensor]:
    """A [B, Nkv] key mask as ``attention_fwd`` takes it: the rows of the kept keys, in order and
    first in each row of an int32 [B, Nkv] tensor, and their number per batch (int32 [B]).
    Computed on the device, with no host synchronisation."""
    if key_mask.dim() != 2 or key_mask.dtype != torch.bool:
        raise ValueError("key_mask must be a [batch, keys] bool tensor")
    counts = key_mask.sum(1, dtype=torch.int32)
    order = torch.argsort((~key_mask).to(torch.uint8), dim=1, stable=True).to(torch.int32)
    return order.contiguous(), counts.contiguous()


def attention_fwd_ok(q: Tensor, k: Tensor, v: Tensor) -> bool:
    """True when ``attention_fwd`` takes these operands (bf16 on the GPU, head dim 128, heads
    contiguous in each token row)."""
    if not (q.is_cuda and q.dtype == k.dtype == v.dtype == torch.bfloat16):
        return False
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or q.shape[-1] != 128:
        return False
    if k.shape != v.shape or k.shape[2:] != q.shape[2:] or k.shape[0] not in (1, q.shape[0]):
        return False
    return all(t.stride(3) == 1 and t.stride(2) == 128 and t.data_ptr() % 16 == 0 for t in (q, k, v))


def attention_fwd(q: Tensor, k: Tensor, v: Tensor, key_idx: Optional[Tensor] = None,
                  key_count: Optional[Tensor] = None, softmax_scale: Optional[float] = None,
                  o_state: Optional[QuantState] = None, o_as_f32: bool = False,
                  scale_max: float = 15.0) -> Tensor:
    """``attention_with_mask(q, k, v, attn_mask_kv=...)`` (attention.py:460-518, SDPA branch) on
    the library's kernel: q [B, Nq, H, 128], k and v [B or 1, Nkv, H, 128] bf16 (k, v with batch 1
    serve every batch); returns out [B, Nq, H, 128] bf16.  Keys: every key, or ``key_count`` [B]
    int32 (the first key_count[b]), or ``key_idx`` [B, Nkv] int32 with ``key_count`` (the rows
    key_idx[b, :key_count[b]], as ``key_list`` gives them).  ``softmax_scale`` defaults to
    1/sqrt(128), SDPA's.  With ``o_state``, the amax of out is left in it with the scale rule
    for ``scale_max`` (as fp32 values with ``o_as_f32``, the self-attention's o input), as
    ``absmax_scale(out, scale_max, o_state, o_as_f32)`` would leave it.  Inference only (no
    backward)."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise RuntimeError("attention_fwd has no backward; use attention_with_mask under autograd")
    if not attention_fwd_ok(q, k, v):
        raise ValueError("attention_fwd takes bf16 GPU tensors [B, N, H, 128] with heads contiguous per token")
    if key_idx is not None and key_count is None:
        raise ValueError("key_idx needs key_count")
    B, Nq, H, D = q.shape
    Nkv = k.shape[1]
    out = torch.empty(B, Nq, H, D, dtype=torch.bfloat16, device=q.device)
    rs = (ctypes.c_int64 * 4)(q.stride(1), k.stride(1), v.stride(1), out.stride(1))
    bs = (ctypes.c_int64 * 4)(q.stride(0), k.stride(0) if k.shape[0] == B else 0,
                              v.stride(0) if v.shape[0] == B else 0, out.stride(0))
    idx_ptr, idx_bs, cnt_ptr = 0, 0, 0
    if key_count is not None:
        if key_count.dtype != torch.int32 or key_count.shape != (B,) or not key_count.is_contiguous():
            raise ValueError("key_count must be a contiguous int32 [batch] tensor")
        cnt_ptr = key_count.data_ptr()
    if key_idx is not None:
        if key_idx.dtype != torch.int32 or key_idx.dim() != 2 or key_idx.shape[0] != B or key_idx.stride(1) != 1:
            raise ValueError("key_idx must be an int32 [batch, keys] tensor with contiguous rows")
        # the kernel reads key_count[b] entries of row b, clamped only to the row stride: a row
        # shorter than the keys (a narrow or sliced list) would let a larger count run past it
        if key_idx.shape[1] != Nkv:
            raise ValueError(f"key_idx rows must hold one entry per key ({Nkv}), got {key_idx.shape[1]}")
        idx_ptr, idx_bs = key_idx.data_ptr(), key_idx.stride(0)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    st_ptr = o_state.ptr if o_state is not None else 0
    st_dtype = _lib.DTYPE_BF16_AS_F32 if o_as_f32 else _lib.DTYPE_BF16
    _lib.check(_lib.load().hif8_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Nq, Nkv,
                                              H, D, rs, bs, idx_ptr, idx_bs, cnt_ptr, scale, st_ptr, st_dtype,
                                              float(scale_max), _lib.stream_ptr(q.device)),
               "hif8_attention_fwd")
    return out
