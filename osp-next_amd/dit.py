"""OSP-Next DiT attention blocks with every linear on the HiF8 path.

This is the caller of the HiF8 linear in the reference: ``OSPNextAttentionBlock``
(``ospnext/modules/osp_next.py:819-1022``) with its self-attention (``:646-779``),
cross-attention (``:782-816``) and FFN (``:873-877``), the Skiparse-2D rearranges
(``ospnext/modules/skiparse_func.py:7-52``, ``osp_next.py:146-283``), the rearranged 3-D RoPE
(``osp_next.py:64-70,550-644``), the padding masks (``osp_next.py:467-548``) and the block
schedule of ``OSPNextModel`` (``osp_next.py:1105-1158``).  Module and argument names follow
the reference so that its state dict loads unchanged.

Two routes through a block, chosen per call:

* **reference order** (autograd, or ``fused=False``): each ``HIF8Linear`` quantises its own
  input, as ``block_forward`` (``osp_next.py:926-957``) does -- q, k and v each quantise the
  same modulated norm.
* **fused** (inference): ``modulated_norm_quant`` produces the quantised q/k/v input once and
  the three projections run as one grouped GEMM; cross-attention's k and v quantise the text
  once and run grouped; cross-attention's q takes the quantised affine norm of ``norm3`` from
  ``affine_norm_quant``; the FFN takes the quantised modulated norm of ``norm2`` and runs its
  up-projection with the GELU + amax epilogue; the self- and cross-attention run on the
  library's attention kernel (``attention_fwd``), whose epilogue leaves the ``o`` projection's
  amax and scale, so ``o`` quantises its input without an amax pass.  Every quantised operand
  is the one the reference would build from the attention output (the producers are bit-exact
  after the layer norm; the attention itself agrees with SDPA within floating-point tolerance).

dtypes follow the reference's inference setting (FSDP2 mixed precision with bf16 block
parameters, fp32 norm parameters with bf16 outputs, ``osp_next.py:1390-1395``,
``fsdp2_wrapper.py:23-77``): the residual stream, modulation and linears are bf16; RMSNorm and
the affine LayerNorm compute in fp32 and hand bf16 on; RoPE runs in fp32, so the
self-attention output and the ``o`` projection's input are fp32 (``osp_next.py:644``,
``attention.py:473,518``).  Attention is the reference's SDPA branch
(``attention.py:433-458``); a key-side padding mask is applied by attending each sequence to
its unmasked keys only, which is the masked softmax without an [N, N] mask tensor (on the
fused route, the kernel reads the list of unmasked key rows).
"""
from __future__ import annotations

import math
import weakref
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import _lib
from .ffn import HIF8FFN
from .hif8_attention import _HIF8QKVQuantFunction, attention_fwd, attention_fwd_ok, key_list
from .hif8_linear import (HIF8Linear, QuantState, absmax_scale, fake_quant, fake_quant_to_bf16, grouped_ok,
                          linear_fwd_grouped, make_linear)
from .norm import (WanLayerNorm, affine_fused_ok, affine_norm_quant, grouped_weight, modulated_norm_quant,
                   qkv_from_modulated_norm)


# ----------------------------------------------------------------- block kinds


class SkiparseBlockType:
    Full = "full"
    Token = "token"
    Group = "group"


class SkiparseModelType:
    DualEnd = "dual_end"
    Full = "full"


class RearrangeType:
    """Rearrange kinds (``osp_next.py:88-144``)."""
    Identity = "identity"
    Skiparse2DToken = "skiparse_2d_token"
    Skiparse2DTokenReverse = "skiparse_2d_token_reverse"
    Skiparse2DGroup = "skiparse_2d_group"
    Skiparse2DGroupReverse = "skiparse_2d_group_reverse"
    Skiparse2DToken2Group = "skiparse_2d_token_to_group"
    Skiparse2DGroup2Token = "skiparse_2d_group_to_token"

    FROM_FULL = (Skiparse2DToken, Skiparse2DGroup)
    TO_FULL = (Skiparse2DTokenReverse, Skiparse2DGroupReverse)
    SWAP = (Skiparse2DToken2Group, Skiparse2DGroup2Token)


# ------------------------------------------------------- Skiparse-2D rearranges
#
# Sequences hold tokens in (t, h, w) order.  With stride P, the token layout gathers every
# P-th row and column into one of P*P sub-sequences (skiparse_func.py:18-20); the group layout
# gathers P x P blocks of P-strided tokens (skiparse_func.py:26-31); token <-> group is one
# permutation and its own inverse (skiparse_func.py:40-52).  Each is a view + permute + copy.


def skiparse_2d_token(x: Tensor, grid, P: int) -> Tensor:
    """[b, T*H*W, c] -> [P*P*b, T*(H/P)*(W/P), c]; batch index (p*P + q)*b + i."""
    T, H, W = grid
    b, _, c = x.shape
    h, w = H // P, W // P
    return x.reshape(b, T, h, P, w, P, c).permute(3, 5, 0, 1, 2, 4, 6).reshape(P * P * b, T * h * w, c)


def skiparse_2d_token_reverse(x: Tensor, grid, P: int) -> Tensor:
    T, H, W = grid
    pb, _, c = x.shape
    b = pb // (P * P)
    h, w = H // P, W // P
    return x.reshape(P, P, b, T, h, w, c).permute(2, 3, 4, 0, 5, 1, 6).reshape(b, T * H * W, c)


def skiparse_2d_group(x: Tensor, grid, P: int) -> Tensor:
    """[b, (T*H/P^2) P P (W/P^2) P P, c] -> [P*P*b, (T*H/P^2) P (W/P^2) P, c]."""
    T, H, W = grid
    b, n, c = x.shape
    w = W // (P * P)
    th = n // (P * P * w * P * P)
    return x.reshape(b, th, P, P, w, P, P, c).permute(2, 5, 0, 1, 3, 4, 6, 7).reshape(P * P * b, th * P * w * P, c)


def skiparse_2d_group_reverse(x: Tensor, grid, P: int) -> Tensor:
    T, H, W = grid
    pb, n, c = x.shape
    b = pb // (P * P)
    w = W // (P * P)
    th = n // (P * w * P)
    return x.reshape(P, P, b, th, P, w, P, c).permute(2, 3, 0, 4, 5, 1, 6, 7).reshape(b, th * P * P * w * P * P, c)


def skiparse_2d_token_to_group(x: Tensor, grid, P: int) -> Tensor:
    """token layout <-> group layout (one permutation, its own inverse)."""
    T, H, W = grid
    pb, n, c = x.shape
    b = pb // (P * P)
    w = W // (P * P)
    th = n // (P * w * P)
    return x.reshape(P, P, b, th, P, w, P, c).permute(4, 6, 2, 3, 0, 5, 1, 7).reshape(pb, n, c)


_DISPATCH = {
    RearrangeType.Skiparse2DToken: skiparse_2d_token,
    RearrangeType.Skiparse2DTokenReverse: skiparse_2d_token_reverse,
    RearrangeType.Skiparse2DGroup: skiparse_2d_group,
    RearrangeType.Skiparse2DGroupReverse: skiparse_2d_group_reverse,
    RearrangeType.Skiparse2DToken2Group: skiparse_2d_token_to_group,
    RearrangeType.Skiparse2DGroup2Token: skiparse_2d_token_to_group,
}


class SkiparseRearrange:
    """``SkiparseRearrange.forward`` (osp_next.py:239-283) on one GPU: H and W are padded with
    zero tokens to multiples of P*P before a full -> skiparse rearrange, and the padding is
    cropped after a skiparse -> full one.  With ``gather`` (the block's fused route) a bf16 CUDA
    tensor is moved in one pass (``hif8_gather_rows``) by a map of source rows that the torch
    path itself makes of a row-index tensor (padding rows -1), built on the first call for a
    shape and kept; the same bits as the torch path."""

    def __init__(self, sparse_ratio: int = 1, rearrange_type: str = RearrangeType.Identity):
        if rearrange_type != RearrangeType.Identity and rearrange_type not in _DISPATCH:
            raise ValueError(f"unsupported rearrange {rearrange_type}")
        self.sparse_ratio = sparse_ratio
        self.rearrange_type = rearrange_type
        self._maps = {}

    def paddings(self, grid) -> Tuple[int, int]:
        """osp_next.py:222-237."""
        if self.rearrange_type == RearrangeType.Identity:
            return 0, 0
        bs = self.sparse_ratio ** 2
        return (bs - grid[1] % bs) % bs, (bs - grid[2] % bs) % bs

    def __call__(self, x: Optional[Tensor], grid=None, gather: bool = False) -> Optional[Tensor]:
        rt = self.rearrange_type
        if x is None or rt == RearrangeType.Identity:
            return x
        if (gather and x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.numel() > 0
                and x.shape[-1] % 8 == 0):
            out = self._gather(x, grid)
            if out is not None:
                return out
        return self._torch(x, grid)

    def _gather(self, x: Tensor, grid) -> Optional[Tensor]:
        B, N, C = x.shape
        key = (B, N, tuple(grid), x.device)
        hit = self._maps.get(key)
        if hit is None:
            ids = torch.arange(B * N, dtype=torch.int32, device=x.device).view(B, N, 1)
            m = self._torch(ids, grid, pad_value=-1)
            if len(self._maps) >= 8:
                self._maps.clear()
            hit = self._maps[key] = (m.reshape(-1).contiguous(), tuple(m.shape[:2]))
        src, (Bo, No) = hit
        x = x.contiguous()
        if x.data_ptr() % 16 != 0 or src.numel() * (C // 8) >= 2 ** 31:
            return None
        out = torch.empty((Bo, No, C), dtype=x.dtype, device=x.device)
        _lib.check(_lib.load().hif8_gather_rows(x.data_ptr(), B * N, src.data_ptr(), src.numel(), C,
                                                out.data_ptr(), _lib.stream_ptr(x.device)), "hif8_gather_rows")
        return out

    def _torch(self, x: Tensor, grid, pad_value: int = 0) -> Tensor:
        rt = self.rearrange_type
        P = self.sparse_ratio
        T, H, W = grid
        ph, pw = self.paddings(grid)
        Hp, Wp = H + ph, W + pw
        fn = _DISPATCH[rt]
        B, N, C = x.shape
        if rt in RearrangeType.FROM_FULL:
            x = x.contiguous()
            if ph or pw:
                x = F.pad(x.view(B, T, H, W, C), (0, 0, 0, pw, 0, ph), value=pad_value).view(B, -1, C)
            return fn(x, (T, Hp, Wp), P)
        if rt in RearrangeType.TO_FULL:
            x = fn(x.contiguous(), (T, Hp, Wp), P)
            if ph or pw:
                b = x.shape[0]
                x = x.view(b, T, Hp, Wp, C)[:, :, :H, :W].contiguous().view(b, -1, C)
            return x
        return fn(x.contiguous(), (T, Hp, Wp), P)


def skiparse_masks(batch: int, grid, sparse_ratio: int, device) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """(token mask, group mask): [P*P*batch, N'] bool, False at padding tokens, or None when no
    token is padding (``SkiparseMaskPreprocessor.preprocess``, osp_next.py:498-548, one GPU)."""
    T, H, W = grid
    ones = torch.ones((batch, T * H * W, 1), dtype=torch.bool, device=device)
    out = []
    for rt in (RearrangeType.Skiparse2DToken, RearrangeType.Skiparse2DGroup):
        m = SkiparseRearrange(sparse_ratio, rt)(ones, grid).squeeze(-1).bool()
        out.append(None if bool(m.all()) else m.contiguous())
    return out[0], out[1]


# ------------------------------------------------------------------------ RoPE


def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> Tensor:
    """osp_next.py:64-70: angles pos / theta^(2i/dim) in float64, returned as fp32."""
    assert dim % 2 == 0
    freqs = torch.outer(torch.arange(max_seq_len),
                        1.0 / torch.pow(theta, torch.arange(0, dim, 2).to(torch.float64).div(dim)))
    return freqs.float()


def rope_freqs(head_dim: int, max_seq_len: int = 1024) -> Tensor:
    """The model's angle table (osp_next.py:1236-1243): t, h and w parts side by side,
    [max_seq_len, head_dim / 2]."""
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)), rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


class SkiparseRopeWrapper:
    """osp_next.py:550-644 on one GPU: per-token angles from the (t, h, w) position, laid out
    like the attention's tokens (the block's rearrange, padding at angle 0)."""

    def __init__(self, freqs: Tensor):
        self.freqs = freqs
        self.cache = {}

    def prepare_freqs(self, grid, head_dim: int, rearrange: Optional[SkiparseRearrange] = None):
        T, H, W = grid
        rt = rearrange.rearrange_type if rearrange is not None else RearrangeType.Identity
        key = (T, H, W, rt, self.freqs.device)
        hit = self.cache.get(key)
        if hit is not None:
            return hit
        f = self.freqs.split([head_dim - 2 * (head_dim // 3), head_dim // 3, head_dim // 3], dim=1)
        fi = torch.cat([f[0][:T].view(T, 1, 1, -1).expand(T, H, W, -1),
                        f[1][:H].view(1, H, 1, -1).expand(T, H, W, -1),
                        f[2][:W].view(1, 1, W, -1).expand(T, H, W, -1)], dim=-1).reshape(1, T * H * W, -1)
        if rearrange is not None:
            fi = rearrange(fi, grid)
        fi = fi.to(torch.float32)
        res = (fi.cos().unsqueeze(2), fi.sin().unsqueeze(2))
        self.cache[key] = res
        return res

    def apply_rope(self, x: Tensor, grid, rearrange: Optional[SkiparseRearrange] = None) -> Tensor:
        """x [B, S, heads, 2d] -> fp32, pairs (x[2i], x[2i+1]) rotated by the token's angle i."""
        B, S, Hh, D = x.shape
        d = D // 2
        x = x.to(torch.float32).reshape(B, S, Hh, d, 2)
        x1, x2 = x[..., 0], x[..., 1]
        cos_f, sin_f = self.prepare_freqs(grid, d, rearrange)
        fb = cos_f.shape[0]
        if fb > 1 and B != fb:
            cos_f = cos_f.repeat_interleave(B // fb, dim=0)
            sin_f = sin_f.repeat_interleave(B // fb, dim=0)
        o1 = x1 * cos_f - x2 * sin_f
        o2 = x1 * sin_f + x2 * cos_f
        return torch.stack([o1, o2], dim=-1).flatten(3).float()


# ----------------------------------------------------------------------- norms


def fused_norm_ok(x: Tensor, norm: nn.Module) -> bool:
    """Whether ``norm(x)`` (and the rope after it) can take hif8_rms_norm_rope: inference on a bf16
    CUDA tensor, an OSPNextRMSNorm with its fp32 weight and bf16 output, a row of 512k <= 8192."""
    return (isinstance(norm, OSPNextRMSNorm) and norm.output_dtype == torch.bfloat16 and x.is_cuda
            and x.dtype == torch.bfloat16 and norm.weight.dtype == torch.float32 and x.shape[-1] % 512 == 0
            and x.shape[-1] <= 8192 and not (torch.is_grad_enabled() and (x.requires_grad or norm.weight.requires_grad)))


def gated_residual(x: Tensor, y: Tensor, gate: Optional[Tensor] = None) -> Tensor:
    """``x + y * gate`` (``osp_next.py:947, :955``; ``x + y`` without gate, ``:949``) as torch's
    bf16 ops compute it, in one pass (``hif8_gated_residual``): the same bits as the two torch
    ops.  ``gate`` is [B, 1, D] / [1, 1, D] for x of [B, N, D].  Other dtypes, layouts or
    shapes run the torch ops."""
    ok = (x.is_cuda and x.dtype == y.dtype == torch.bfloat16 and x.shape == y.shape and x.dim() == 3
          and x.is_contiguous() and y.is_contiguous() and x.shape[-1] % 8 == 0 and x.numel() > 0
          and x.data_ptr() % 16 == 0 and y.data_ptr() % 16 == 0)
    if ok and gate is not None:
        B, N, D = x.shape
        ok = (gate.dtype == torch.bfloat16 and gate.dim() == 3 and gate.shape[1] == 1 and gate.shape[2] == D
              and gate.shape[0] in (1, B) and gate.device == x.device)
    if not ok:
        return x + y if gate is None else x + y * gate
    B, N, D = x.shape
    out = torch.empty_like(x)
    g = None
    rpb = B * N
    if gate is not None:
        g = gate.reshape(-1, D).contiguous()
        rpb = N if g.shape[0] == B else B * N
    _lib.check(_lib.load().hif8_gated_residual(x.data_ptr(), y.data_ptr(), g.data_ptr() if g is not None else None,
                                               out.data_ptr(), B * N, D, rpb, _lib.stream_ptr(x.device)),
               "hif8_gated_residual")
    return out


def rms_norm_rope(x: Tensor, norm: "OSPNextRMSNorm", cos_f: Optional[Tensor] = None,
                  sin_f: Optional[Tensor] = None, head_dim: int = 128) -> Tensor:
    """``norm(x)``, and with the angle tables of SkiparseRopeWrapper.prepare_freqs the rotation of
    apply_rope and the attention's bf16 cast of its fp32 result, in one pass over x
    (hif8_rms_norm_rope).  x bf16 [B, N, dim] -> bf16 [B, N, dim] (heads of ``head_dim``)."""
    B, N, dim = x.shape
    x = x.contiguous()
    out = torch.empty_like(x)
    w = norm.weight.detach().contiguous()
    L = _lib.load()
    s = _lib.stream_ptr(x.device)
    if cos_f is None:
        _lib.check(L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), None, None, out.data_ptr(), B * N, dim, head_dim,
                                        1, 1, float(norm.eps), s), "hif8_rms_norm_rope")
        return out
    fb = cos_f.shape[0]
    if cos_f.shape[1] != N or (fb > 1 and B % fb != 0):
        raise ValueError(f"angle tables {tuple(cos_f.shape)} do not match x {tuple(x.shape)}")
    c = cos_f.to(torch.float32).contiguous()
    sn = sin_f.to(torch.float32).contiguous()
    _lib.check(L.hif8_rms_norm_rope(x.data_ptr(), w.data_ptr(), c.data_ptr(), sn.data_ptr(), out.data_ptr(), B * N,
                                    dim, head_dim, N, B if fb == 1 else B // fb, float(norm.eps), s),
               "hif8_rms_norm_rope")
    return out


def rms_norm_rope_quant(x: Tensor, norm: "OSPNextRMSNorm", scale_max: float, cos_f: Optional[Tensor] = None,
                        sin_f: Optional[Tensor] = None, head_dim: int = 128,
                        return_y: bool = False):
    """quant_attn="hif8" on q or k as a producer: the attention's bf16 cast of
    ``_quant(apply_rope(norm(x)))`` (the rope output in fp32, hif8_attention.py:60-74), or without
    the angle tables of ``_quant(norm(x))`` (the bf16 norm output), in two passes over x
    (hif8_rms_norm_rope_amax, hif8_rms_norm_rope_fake_quant), never writing the fp32 rope output.
    Returns (x_q bf16 [B, N, dim], state), and with ``return_y`` the output that was quantised
    (fp32 with rope, bf16 without) as a third element."""
    B, N, dim = x.shape
    x = x.contiguous()
    w = norm.weight.detach().contiguous()
    L = _lib.load()
    s = _lib.stream_ptr(x.device)
    st = QuantState(x.device)
    xq = torch.empty_like(x)
    y = None
    if return_y:
        y = torch.empty(x.shape, dtype=torch.float32 if cos_f is not None else torch.bfloat16, device=x.device)
    yp = y.data_ptr() if y is not None else None
    if cos_f is None:
        c = sn = None
        cp = sp = None
        seq, rep = 1, 1
    else:
        fb = cos_f.shape[0]
        if cos_f.shape[1] != N or (fb > 1 and B % fb != 0):
            raise ValueError(f"angle tables {tuple(cos_f.shape)} do not match x {tuple(x.shape)}")
        c = cos_f.to(torch.float32).contiguous()
        sn = sin_f.to(torch.float32).contiguous()
        cp, sp = c.data_ptr(), sn.data_ptr()
        seq, rep = N, (B if fb == 1 else B // fb)
    _lib.check(L.hif8_rms_norm_rope_amax(x.data_ptr(), w.data_ptr(), cp, sp, B * N, dim, head_dim, seq, rep,
                                         float(norm.eps), float(scale_max), st.ptr, s), "hif8_rms_norm_rope_amax")
    _lib.check(L.hif8_rms_norm_rope_fake_quant(x.data_ptr(), w.data_ptr(), cp, sp, B * N, dim, head_dim, seq, rep,
                                               float(norm.eps), st.ptr, _lib.SEM_NPU, xq.data_ptr(), yp, s),
               "hif8_rms_norm_rope_fake_quant")
    return (xq, st, y) if return_y else (xq, st)


class OSPNextRMSNorm(nn.Module):
    """WanRMSNorm (want2v.py:77-93) with an fp32 weight and a bf16 output, as the model runs it
    under FSDP2's high-precision policy for norms (``output_dtype`` bf16)."""

    def __init__(self, dim: int, eps: float = 1e-5, device=None, output_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.output_dtype = output_dtype
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=torch.float32))

    def forward(self, x: Tensor) -> Tensor:
        y = self._norm(x.float()).type_as(x) * self.weight
        return y.to(self.output_dtype) if self.output_dtype is not None else y

    def _norm(self, x: Tensor) -> Tensor:
        return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + self.eps)


class OSPNextLayerNorm(WanLayerNorm):
    """WanLayerNorm (want2v.py:96-106); an affine one keeps fp32 parameters (norm3)."""

    def __init__(self, dim: int, eps: float = 1e-6, elementwise_affine: bool = False, device=None):
        super().__init__(dim, eps=eps, elementwise_affine=elementwise_affine)
        if device is not None:
            self.to(device)


# ------------------------------------------------------------------- attention


def _sdpa(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """SDPA on [B, N, H, D] bf16 tensors (attention.py:433-458 without a mask).  On the GPU only
    the fused attention kernels are allowed (flash, memory-efficient): a shape they do not take
    raises instead of running the [N, N] math path."""
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = F.scaled_dot_product_attention(qt, kt, vt)
    else:
        out = F.scaled_dot_product_attention(qt, kt, vt)
    return out.transpose(1, 2)


def attention_key_masked(q: Tensor, k: Tensor, v: Tensor, key_mask: Optional[Tensor] = None,
                         dtype: torch.dtype = torch.bfloat16, out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """``attention_with_mask(q, k, v, attn_mask_kv=key_mask)`` of the SDPA branch
    (attention.py:460-518): computed in ``dtype``, returned in q's dtype (or ``out_dtype``).
    Keys where ``key_mask`` is False take no weight; each sequence attends to its unmasked keys
    directly, which is that masked softmax without materialising an [N, N] mask (every query
    row, padding queries included, gets its output)."""
    out_dtype = out_dtype or q.dtype
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    if key_mask is None:
        return _sdpa(q, k, v).to(out_dtype)
    if key_mask.shape != k.shape[:2]:
        raise ValueError(f"key mask {tuple(key_mask.shape)} does not match keys {tuple(k.shape[:2])}")
    outs = []
    for b in range(q.shape[0]):
        keep = key_mask[b].nonzero().squeeze(-1)
        if keep.numel() == k.shape[1]:
            outs.append(_sdpa(q[b:b + 1], k[b:b + 1], v[b:b + 1]))
        elif keep.numel() == 0:
            raise ValueError("a sequence with every key masked has no attention output")
        else:
            outs.append(_sdpa(q[b:b + 1], k[b:b + 1, keep], v[b:b + 1, keep]))
    return torch.cat(outs, 0).to(out_dtype)


# Key lists of the attention masks, per mask tensor and per version of its contents: mask id ->
# (weak reference to the mask, {version: (key rows, counts)}).  An entry lives exactly as long as
# its mask (a finaliser drops it), so a HIP graph that captured an attention over a mask keeps
# valid key-list memory for as long as the caller keeps that mask, like any other static input of
# the graph; lists of earlier versions of a mask modified in place stay too.
_KEY_LISTS: dict = {}


def _drop_key_lists(key: int, ref) -> None:
    ent = _KEY_LISTS.get(key)
    if ent is not None and ent[0] is ref:
        del _KEY_LISTS[key]


def _cached_key_list(key_mask: Optional[Tensor]) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """``key_list(key_mask)``, built once per mask tensor (and version): the blocks of a step
    alternate between a few masks (token and group masks of the Skiparse blocks), and each keeps
    its own lists."""
    if key_mask is None:
        return None, None
    key = id(key_mask)
    ent = _KEY_LISTS.get(key)
    if ent is None or ent[0]() is not key_mask:
        ref = weakref.ref(key_mask)
        ent = (ref, {})
        _KEY_LISTS[key] = ent
        weakref.finalize(key_mask, _drop_key_lists, key, ref)
    lists = ent[1]
    hit = lists.get(key_mask._version)
    if hit is None:
        hit = key_list(key_mask.bool())
        lists[key_mask._version] = hit
    return hit


def _grouped_kv(k: HIF8Linear, v: HIF8Linear, text: Tensor) -> Optional[Tuple[Tensor, Tensor]]:
    """k(text), v(text) with the text quantised once and one grouped GEMM (inference), or None."""
    if not (isinstance(k, HIF8Linear) and isinstance(v, HIF8Linear) and text.is_cuda
            and text.dtype == torch.bfloat16 and k.scale_max_forward == v.scale_max_forward
            and k.a_format == v.a_format == "bf16"):
        return None
    gw = grouped_weight((k, v))
    if gw is None:
        return None
    t2 = text.reshape(-1, text.shape[-1]).contiguous()
    st = absmax_scale(t2, k.scale_max_forward, QuantState(t2.device))
    tq = fake_quant(t2, st)
    ys = linear_fwd_grouped(tq, gw)
    return tuple(y.view(*text.shape[:-1], y.shape[-1]) for y in ys)


class OSPNextSelfAttention(nn.Module):
    """osp_next.py:646-779 on one GPU (no all-to-all)."""

    def __init__(self, dim: int, num_heads: int, window_size=(-1, -1), qk_norm: bool = True, eps: float = 1e-6,
                 sparse_ratio: int = 2, skiparse_block_type: str = SkiparseBlockType.Full, quant: Optional[str] = None,
                 quant_attn: Optional[str] = None, scale_max_forward: float = 15.0,
                 scale_max_backward: float = 224.0, device=None, dtype=None):
        assert dim % num_heads == 0
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.window_size = window_size
        self.qk_norm = qk_norm
        self.eps = eps
        self.quant_attn = quant_attn
        self.scale_max_forward = scale_max_forward
        self.scale_max_backward = scale_max_backward
        kw = dict(device=device, dtype=dtype)
        self.q = make_linear(quant, dim, dim, scale_max_forward, scale_max_backward, **kw)
        self.k = make_linear(quant, dim, dim, scale_max_forward, scale_max_backward, **kw)
        self.v = make_linear(quant, dim, dim, scale_max_forward, scale_max_backward, **kw)
        self.o = make_linear(quant, dim, dim, scale_max_forward, scale_max_backward, **kw)
        self.norm_q = OSPNextRMSNorm(dim, eps=eps, device=device) if qk_norm else nn.Identity()
        self.norm_k = OSPNextRMSNorm(dim, eps=eps, device=device) if qk_norm else nn.Identity()
        self.skiparse_block_type = skiparse_block_type
        if skiparse_block_type == SkiparseBlockType.Token:
            self.rearrange_rope = SkiparseRearrange(sparse_ratio, RearrangeType.Skiparse2DToken)
        elif skiparse_block_type == SkiparseBlockType.Group:
            self.rearrange_rope = SkiparseRearrange(sparse_ratio, RearrangeType.Skiparse2DGroup)
        else:
            self.rearrange_rope = SkiparseRearrange(1, RearrangeType.Identity)

    def _attend(self, q: Tensor, k: Tensor, v: Tensor, key_mask: Optional[Tensor],
                out_dtype: Optional[torch.dtype] = None) -> Tensor:
        if self.quant_attn == "hif8":   # hif8_attention.py:93-126
            q, k, v = _HIF8QKVQuantFunction.apply(q, k, v, self.scale_max_forward, self.scale_max_backward)
        return attention_key_masked(q, k, v, key_mask, out_dtype=out_dtype)

    def _kernel_ok(self, q: Tensor) -> bool:
        """The attention can run on the attention kernel: inference on the GPU, head dim 128, an
        HIF8Linear o (which takes the state the kernel's epilogue leaves)."""
        return (q.is_cuda and not torch.is_grad_enabled() and q.shape[-1] == 128
                and isinstance(self.o, HIF8Linear))

    def _kernel_quant_attn_ok(self, q: Tensor) -> bool:
        """quant_attn="hif8" on the attention kernel."""
        return self.quant_attn == "hif8" and self._kernel_ok(q)

    def _quantise_v(self, v: Tensor) -> Tensor:
        """_quant(v) of the bf16 v (hif8_attention.py:60-74), in its shape."""
        v2 = v.reshape(-1, v.shape[-1]).contiguous()
        return fake_quant(v2, absmax_scale(v2, self.scale_max_forward, QuantState(v.device))).view(v.shape)

    def _quantised_attention(self, q: Tensor, k: Tensor, v: Tensor, key_mask: Optional[Tensor],
                             o_as_f32: bool) -> Tuple[Tensor, QuantState]:
        """quant_attn="hif8" on the attention kernel: the kernel's inputs are bf16(_quant(q)),
        bf16(_quant(k)) and _quant(v) -- the HiF8 qdq of each with its own per-tensor scale
        (hif8_attention.py:60-74), then the attention's bf16 cast (attention.py:460-518) -- and
        the o projection's state comes from its epilogue.  Returns (out bf16, o state)."""
        def quantised(t: Tensor) -> Tensor:
            t2 = t.reshape(-1, t.shape[-1]).contiguous()
            st = absmax_scale(t2, self.scale_max_forward, QuantState(t.device))
            tq = fake_quant_to_bf16(t2, st) if t.dtype == torch.float32 else fake_quant(t2, st)
            return tq.view(t.shape)
        qq, kq, vq = quantised(q), quantised(k), quantised(v)
        st = QuantState(q.device)
        out = attention_fwd(qq, kq, vq, *_cached_key_list(key_mask), o_state=st, o_as_f32=o_as_f32,
                            scale_max=self.o.scale_max_forward)
        return out, st

    def forward(self, x: Optional[Tensor], attn_mask: Optional[Tensor], grid_sizes_for_rope,
                rope_wrapper: SkiparseRopeWrapper, qkv: Optional[Sequence[Tensor]] = None) -> Tensor:
        """``qkv`` = the three projections of x computed by the caller (the fused route, which
        also hands the bf16 attention output to ``o`` without its fp32 copy)."""
        qkv_given = qkv is not None
        if qkv is None:
            qkv = (self.q(x), self.k(x), self.v(x))
        ql, kl, vl = qkv
        B, N = ql.shape[:2]
        H, D = self.num_heads, self.head_dim
        if (qkv_given and self._kernel_quant_attn_ok(ql.view(B, N, H, D)) and fused_norm_ok(ql, self.norm_q)
                and fused_norm_ok(kl, self.norm_k) and vl.dtype == torch.bfloat16):
            # quant_attn="hif8": q and k quantised by the norm + rope producer (two passes each,
            # the fp32 rope output never written), v by the codec, then the attention kernel
            cos_f, sin_f = rope_wrapper.prepare_freqs(grid_sizes_for_rope, D // 2, self.rearrange_rope)
            qq, _ = rms_norm_rope_quant(ql, self.norm_q, self.scale_max_forward, cos_f, sin_f, D)
            kq, _ = rms_norm_rope_quant(kl, self.norm_k, self.scale_max_forward, cos_f, sin_f, D)
            vq = self._quantise_v(vl.view(B, N, H, D))
            st = QuantState(ql.device)
            x = attention_fwd(qq.view(B, N, H, D), kq.view(B, N, H, D), vq, *_cached_key_list(attn_mask), o_state=st,
                              o_as_f32=True, scale_max=self.o.scale_max_forward)
            return self.o.forward_settled(x.flatten(2), st, as_f32=True)
        if (qkv_given and self.quant_attn is None and isinstance(self.o, HIF8Linear) and fused_norm_ok(ql, self.norm_q)
                and fused_norm_ok(kl, self.norm_k)):
            # norms, rope and the attention's bf16 cast in one pass each; the attention output
            # is the bf16 value of what the reference returns as fp32 (q's dtype)
            cos_f, sin_f = rope_wrapper.prepare_freqs(grid_sizes_for_rope, D // 2, self.rearrange_rope)
            q = rms_norm_rope(ql, self.norm_q, cos_f, sin_f, D).view(B, N, H, D)
            k = rms_norm_rope(kl, self.norm_k, cos_f, sin_f, D).view(B, N, H, D)
            v = vl.view(B, N, H, D)
            if attention_fwd_ok(q, k, v):
                # the attention kernel leaves the o input's amax and scale in st: no amax pass
                st = QuantState(q.device)
                x = attention_fwd(q, k, v, *_cached_key_list(attn_mask), o_state=st, o_as_f32=True,
                                  scale_max=self.o.scale_max_forward)
                return self.o.forward_settled(x.flatten(2), st, as_f32=True)
            x = self._attend(q, k, v, attn_mask, out_dtype=torch.bfloat16)
            return self.o.forward_f32_of_bf16(x.flatten(2))
        q = self.norm_q(ql).view(B, N, H, D)
        k = self.norm_k(kl).view(B, N, H, D)
        v = vl.view(B, N, H, D)
        q = rope_wrapper.apply_rope(q, grid_sizes_for_rope, self.rearrange_rope)
        k = rope_wrapper.apply_rope(k, grid_sizes_for_rope, self.rearrange_rope)
        if qkv_given and isinstance(self.o, HIF8Linear) and q.dtype == torch.float32:
            # the attention output is bf16 values returned as fp32: quantise them as such
            if self._kernel_quant_attn_ok(q) and k.dtype == torch.float32 and v.dtype == torch.bfloat16:
                x, st = self._quantised_attention(q, k, v, attn_mask, o_as_f32=True)
                return self.o.forward_settled(x.flatten(2), st, as_f32=True)
            if self.quant_attn is None and self._kernel_ok(q) and v.dtype == torch.bfloat16:
                # the attention's bf16 cast of q and k (attention.py:460-518), then the kernel
                q16, k16 = q.to(torch.bfloat16), k.to(torch.bfloat16)
                if attention_fwd_ok(q16, k16, v):
                    st = QuantState(q.device)
                    x = attention_fwd(q16, k16, v, *_cached_key_list(attn_mask), o_state=st, o_as_f32=True,
                                      scale_max=self.o.scale_max_forward)
                    return self.o.forward_settled(x.flatten(2), st, as_f32=True)
            x = self._attend(q, k, v, attn_mask, out_dtype=torch.bfloat16)
            return self.o.forward_f32_of_bf16(x.flatten(2))
        x = self._attend(q, k, v, attn_mask)
        return self.o(x.flatten(2))


class OSPNextCrossAttention(OSPNextSelfAttention):
    """osp_next.py:782-816.  ``text`` may have batch 1 where x has P*P (the reference repeats
    the text per sub-sequence, ``osp_next.py:973``): every query then attends to the same keys,
    so the sub-sequences are attended as one."""

    def forward(self, x: Optional[Tensor], attn_mask: Optional[Tensor], text: Tensor, fused: bool = False,
                x_q: Optional[Tensor] = None) -> Tensor:
        """``x_q``: the q input already quantised with q's ``scale_max_forward`` (``_quant(x)[0]``,
        e.g. from ``affine_norm_quant``) in place of x; q then runs the GEMM alone."""
        B = (x if x_q is None else x_q).shape[0]
        H, D = self.num_heads, self.head_dim
        kv = _grouped_kv(self.k, self.v, text) if fused else None
        if kv is None:
            kv = (self.k(text), self.v(text))
        ql = self.q(x) if x_q is None else self.q.forward_quantized(x_q)
        # quant_attn="hif8" through the norm producers: q and k come out quantised
        qa = (fused and self.quant_attn == "hif8" and D == 128 and ql.is_cuda and not torch.is_grad_enabled()
              and isinstance(self.o, HIF8Linear) and fused_norm_ok(ql, self.norm_q)
              and fused_norm_ok(kv[0], self.norm_k) and kv[1].dtype == torch.bfloat16)
        if qa:
            q, _ = rms_norm_rope_quant(ql, self.norm_q, self.scale_max_forward, head_dim=D)
            k, _ = rms_norm_rope_quant(kv[0], self.norm_k, self.scale_max_forward, head_dim=D)
        elif fused and self.quant_attn is None and fused_norm_ok(ql, self.norm_q) and fused_norm_ok(kv[0], self.norm_k):
            q = rms_norm_rope(ql, self.norm_q, head_dim=D)
            k = rms_norm_rope(kv[0], self.norm_k, head_dim=D)
        else:
            q = self.norm_q(ql)
            k = self.norm_k(kv[0])
        v = self._quantise_v(kv[1]) if qa else kv[1]
        tb = text.shape[0]
        if tb != B:
            if tb != 1:
                raise ValueError(f"text batch {tb} does not match x batch {B}")
            q = q.reshape(1, -1, H, D)          # the P*P sub-sequences against one text
        else:
            q = q.view(B, -1, H, D)
        k = k.view(tb, -1, H, D)
        v = v.view(tb, -1, H, D)
        if (fused and self.quant_attn is None and isinstance(self.o, HIF8Linear) and q.dtype == torch.bfloat16
                and attention_fwd_ok(q, k, v)):
            # attn_mask is query-side: no effect (as in SDPA); the o input's amax comes from the
            # attention kernel's epilogue
            st = QuantState(q.device)
            out = attention_fwd(q, k, v, o_state=st, scale_max=self.o.scale_max_forward)
            return self.o.forward_settled(out.reshape(B, -1, H * D), st)
        if qa and attention_fwd_ok(q, k, v):
            st = QuantState(q.device)
            out = attention_fwd(q, k, v, o_state=st, scale_max=self.o.scale_max_forward)
            return self.o.forward_settled(out.reshape(B, -1, H * D), st)
        if fused and not qa and self._kernel_quant_attn_ok(q) and q.dtype == k.dtype == v.dtype == torch.bfloat16:
            out, st = self._quantised_attention(q, k, v, None, o_as_f32=False)
            return self.o.forward_settled(out.reshape(B, -1, H * D), st)
        if qa:   # the quantised operands on SDPA (the kernel does not take these strides)
            out = attention_key_masked(q, k, v, None)
            return self.o(out.reshape(B, -1, H * D))
        out = self._attend(q, k, v, None)       # attn_mask is query-side: no effect in SDPA
        return self.o(out.reshape(B, -1, H * D))


class OSPNextAttentionBlock(nn.Module):
    """osp_next.py:819-1022 on one GPU."""

    def __init__(self, dim: int, ffn_dim: int, num_heads: int, window_size=(-1, -1), qk_norm: bool = True,
                 cross_attn_norm: bool = False, eps: float = 1e-6, sparse_ratio: int = 2,
                 skiparse_block_type: str = SkiparseBlockType.Full, is_full2skiparse_block: bool = False,
                 is_skiparse2full_block: bool = False, quant: Optional[str] = None, quant_attn: Optional[str] = None,
                 scale_max_forward: float = 15.0, scale_max_backward: float = 224.0, device=None,
                 dtype=torch.bfloat16):
        super().__init__()
        self.dim = dim
        self.ffn_dim = ffn_dim
        self.num_heads = num_heads
        self.eps = eps
        self.quant = quant
        self.scale_max_forward = scale_max_forward
        kw = dict(device=device, dtype=dtype)
        self.norm1 = OSPNextLayerNorm(dim, eps, device=device)
        self.self_attn = OSPNextSelfAttention(dim, num_heads, window_size, qk_norm, eps, sparse_ratio=sparse_ratio,
                                              skiparse_block_type=skiparse_block_type, quant=quant,
                                              quant_attn=quant_attn, scale_max_forward=scale_max_forward,
                                              scale_max_backward=scale_max_backward, **kw)
        self.norm3 = (OSPNextLayerNorm(dim, eps, elementwise_affine=True, device=device) if cross_attn_norm
                      else nn.Identity())
        self.cross_attn = OSPNextCrossAttention(dim, num_heads, window_size, qk_norm, eps, quant=quant,
                                                quant_attn=quant_attn, scale_max_forward=scale_max_forward,
                                                scale_max_backward=scale_max_backward, **kw)
        self.norm2 = OSPNextLayerNorm(dim, eps, device=device)
        if quant == "hif8":
            self.ffn = HIF8FFN(dim, ffn_dim, scale_max_forward, scale_max_backward, **kw)
        else:
            self.ffn = nn.Sequential(nn.Linear(dim, ffn_dim, **kw), nn.GELU(approximate="tanh"),
                                     nn.Linear(ffn_dim, dim, **kw))
        self.modulation = nn.Parameter(torch.randn(1, 6, dim, device=device) / dim ** 0.5)
        if dtype is not None:
            self.modulation.data = self.modulation.data.to(dtype)

        self.sparse_ratio = sparse_ratio
        self.skiparse_block_type = skiparse_block_type
        self.is_full2skiparse_block = is_full2skiparse_block
        self.is_skiparse2full_block = is_skiparse2full_block
        ident = SkiparseRearrange(1, RearrangeType.Identity)
        self.rearrange_input = self.rearrange_output = ident
        self.repeats = 1 if skiparse_block_type == SkiparseBlockType.Full else sparse_ratio ** 2
        if skiparse_block_type == SkiparseBlockType.Token:
            self.rearrange_input = SkiparseRearrange(
                sparse_ratio, RearrangeType.Skiparse2DToken if is_full2skiparse_block
                else RearrangeType.Skiparse2DGroup2Token)
        elif skiparse_block_type == SkiparseBlockType.Group:
            self.rearrange_input = SkiparseRearrange(sparse_ratio, RearrangeType.Skiparse2DToken2Group)
            if is_skiparse2full_block:
                self.rearrange_output = SkiparseRearrange(sparse_ratio, RearrangeType.Skiparse2DGroupReverse)

    # ------------------------------------------------------------------ routes

    def fused_ok(self, x: Tensor) -> bool:
        grad = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        sa = self.self_attn
        return (not grad and self.quant == "hif8" and x.is_cuda and x.dtype == torch.bfloat16
                and all(m.a_format == "bf16" for m in (sa.q, sa.k, sa.v))
                and sa.q.scale_max_forward == sa.k.scale_max_forward == sa.v.scale_max_forward)

    def block_forward(self, x: Tensor, attn_mask: Optional[Tensor], cross_attn_mask: Optional[Tensor], e: Tensor,
                      grid_sizes_for_rope, rope_wrapper: SkiparseRopeWrapper, text: Tensor,
                      fused: Optional[bool] = None) -> Tensor:
        """osp_next.py:926-957.  ``fused=None`` takes the fused route whenever it applies."""
        if fused is None:
            fused = self.fused_ok(x)
        elif fused and not self.fused_ok(x):
            raise ValueError("the fused route needs bf16 CUDA input, HiF8 linears and no autograd")
        e = (self.modulation + e).chunk(6, dim=1)
        sa = self.self_attn
        if fused:
            qkv = qkv_from_modulated_norm(x, e[0], e[1], sa.q, sa.k, sa.v, self.eps)
            y = sa(None, attn_mask, grid_sizes_for_rope, rope_wrapper, qkv=qkv)
        else:
            y = sa(self.norm1(x) * (1 + e[1]) + e[0], attn_mask, grid_sizes_for_rope, rope_wrapper)
        x = gated_residual(x, y, e[2]) if fused else x + y * e[2]
        ca = self.cross_attn
        if (fused and isinstance(ca.q, HIF8Linear) and ca.q.a_format == "bf16"
                and affine_fused_ok(x, self.norm3)):
            xq3, _ = affine_norm_quant(x, self.norm3, ca.q.scale_max_forward)
            x = gated_residual(x, ca(None, cross_attn_mask, text, fused=True, x_q=xq3))
        else:
            x = x + ca(self.norm3(x), cross_attn_mask, text, fused=fused)
        if fused and isinstance(self.ffn, HIF8FFN) and self.ffn.fused_ok(x):
            xq, _ = modulated_norm_quant(x, e[3], e[4], self.eps, self.ffn[0].scale_max_forward)
            y = self.ffn.forward_quantized(xq)
        else:
            y = self.ffn(self.norm2(x) * (1 + e[4]) + e[3])
        return gated_residual(x, y, e[5]) if fused else x + y * e[5]

    def forward(self, x: Tensor, attn_mask: Optional[Tensor], cross_attn_mask: Optional[Tensor], e: Tensor,
                sub_grid_sizes, grid_sizes_for_rope, rope_wrapper: SkiparseRopeWrapper, text: Tensor,
                fused: Optional[bool] = None) -> Tensor:
        """osp_next.py:960-1022 (no checkpointing).  With batch 1 the repeated text and
        modulation of a skiparse block (``context_rearrange_input``) are kept as one copy:
        broadcasting one row gives the same values as its P*P copies."""
        # the fused route moves bf16 rows with one gather per layout change
        g = self.fused_ok(x) if fused is None else bool(fused)
        x = self.rearrange_input(x, sub_grid_sizes, gather=g)
        if self.repeats > 1 and text.shape[0] > 1:
            text = text.repeat(self.repeats, 1, 1)
            e = e.repeat(self.repeats, 1, 1)
        x = self.block_forward(x, attn_mask, cross_attn_mask, e, grid_sizes_for_rope, rope_wrapper, text, fused)
        return self.rearrange_output(x, sub_grid_sizes, gather=g)


# -------------------------------------------------------------- block schedule


def block_schedule(num_layers: int, skiparse_model_type: str = SkiparseModelType.DualEnd,
                   num_full_blocks: int = 0) -> List[Tuple[str, bool, bool]]:
    """(block type, is_full2skiparse, is_skiparse2full) per layer, osp_next.py:1105-1146."""
    if skiparse_model_type == SkiparseModelType.Full:
        full = list(range(num_layers))
    else:
        if not (num_layers % 2 == 0 and num_full_blocks % 2 == 0 and num_full_blocks <= num_layers // 2):
            raise ValueError("num_full_blocks must be even and at most num_layers // 2")
        if num_full_blocks == 0:
            full = []
        elif skiparse_model_type == SkiparseModelType.DualEnd:
            if num_full_blocks % 4:
                raise ValueError("num_full_blocks should be divisible by 4")
            start = num_full_blocks // 2
            end = num_layers - num_full_blocks // 2 - 1
            full = list(range(0, start)) + list(range(end + 1, num_layers))
        else:
            raise ValueError(f"unsupported skiparse model type {skiparse_model_type}")
    full = [-1] + full + [num_layers]
    out = []
    for i in range(num_layers):
        if i in full:
            kind = SkiparseBlockType.Full
        elif i % 2 == 0:
            kind = SkiparseBlockType.Token
        else:
            kind = SkiparseBlockType.Group
        out.append((kind, (i - 1) in full and i not in full, (i + 1) in full and i not in full))
    return out


class OSPNextBlocks(nn.Module):
    """The block loop of ``OSPNextModel.forward`` (osp_next.py:1287-1331) on one GPU: blocks
    built by the model's schedule, the padding masks and the rope table.  Input and output are
    the patchified tokens [B, T*H*W, dim] in (t, h, w) order."""

    def __init__(self, dim: int = 5120, ffn_dim: int = 13824, num_heads: int = 40, num_layers: int = 40,
                 skiparse_model_type: str = SkiparseModelType.DualEnd, sparse_ratio: int = 2,
                 num_full_blocks: int = 8, qk_norm: bool = True, cross_attn_norm: bool = True, eps: float = 1e-6,
                 quant: Optional[str] = "hif8", quant_attn: Optional[str] = None, scale_max_forward: float = 15.0,
                 scale_max_backward: float = 224.0, device=None, dtype=torch.bfloat16):
        super().__init__()
        if skiparse_model_type == SkiparseModelType.Full:
            sparse_ratio = 1
        self.sparse_ratio = sparse_ratio
        self.head_dim = dim // num_heads
        self.blocks = nn.ModuleList()
        for kind, f2s, s2f in block_schedule(num_layers, skiparse_model_type, num_full_blocks):
            self.blocks.append(OSPNextAttentionBlock(
                dim, ffn_dim, num_heads, (-1, -1), qk_norm, cross_attn_norm, eps,
                sparse_ratio=sparse_ratio if kind != SkiparseBlockType.Full else 1, skiparse_block_type=kind,
                is_full2skiparse_block=f2s, is_skiparse2full_block=s2f, quant=quant, quant_attn=quant_attn,
                scale_max_forward=scale_max_forward, scale_max_backward=scale_max_backward, device=device,
                dtype=dtype))
        self.rope = SkiparseRopeWrapper(rope_freqs(self.head_dim).to(device))

    def forward(self, x: Tensor, e0: Tensor, text: Tensor, grid, fused: Optional[bool] = None) -> Tensor:
        """x [B, T*H*W, dim] bf16, e0 [B, 6, dim] (the time projection), text [B, L, dim] (embedded)."""
        B = x.shape[0]
        token_mask, group_mask = (skiparse_masks(B, grid, self.sparse_ratio, x.device)
                                  if self.sparse_ratio > 1 else (None, None))
        for blk in self.blocks:
            if blk.skiparse_block_type == SkiparseBlockType.Token:
                am = cm = token_mask
            elif blk.skiparse_block_type == SkiparseBlockType.Group:
                am = cm = group_mask
            else:
                am = cm = None
            x = blk(x, am, cm, e0, grid, grid, self.rope, text, fused)
        return x

    @torch.no_grad()
    def prepack(self) -> "OSPNextBlocks":
        for m in self.modules():
            if isinstance(m, HIF8Linear):
                m.prepack()
        return self


def init_block_weights(module: nn.Module, std: float = 0.02, generator: Optional[torch.Generator] = None):
    """N(0, std) linear weights, zero biases (BASELINE configs 4-5 random init)."""
    with torch.no_grad():
        for m in module.modules():
            if isinstance(m, nn.Linear):
                m.weight.normal_(0.0, std, generator=generator)
                if m.bias is not None:
                    m.bias.zero_()
