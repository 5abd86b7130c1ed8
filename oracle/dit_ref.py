"""CPU restatement of OSP-Next's DiT attention block around the HiF8 linears.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as the checker of the
GPU block; the product path never does.

It evaluates ``OSPNextAttentionBlock.forward`` (``ospnext/modules/osp_next.py:926-1022``) on
CPU torch tensors from a state dict with the reference's parameter names, in the reference's
inference dtypes (bf16 block parameters and residual stream, fp32 norm parameters with bf16
outputs, fp32 RoPE and ``o`` input), with every non-elementwise step evaluated exactly:

* Skiparse-2D rearranges: the einops patterns of ``skiparse_func.py:18-52`` as written there,
  with the padding and cropping of ``SkiparseRearrange.forward`` (``osp_next.py:239-283``);
* padding masks: ``SkiparseMaskPreprocessor.preprocess`` (``osp_next.py:498-548``);
* RoPE: ``rope_params`` (``osp_next.py:64-70``), the model's angle table (``:1236-1243``) and
  ``SkiparseRopeWrapper`` (``:558-644``), the rotation in float64 rounded to fp32;
* WanRMSNorm / WanLayerNorm (``want2v.py:77-106``): float64, rounded as the fp32 result is;
* attention: the SDPA branch (``attention.py:433-518``), float64 softmax on the bf16 q, k, v,
  output rounded to bf16;
* HIF8Linear (``hif8_linear.py:68-86``): ``hif8_ref.quant_bf16`` / ``quant_f32`` for x and W,
  float64 product plus bias, rounded to bf16 (F.linear's autocast output);
* GELU(tanh) in float64 on the bf16 up-projection output.
Elementwise bf16 steps (modulation sums, ``(1 + e)``, gates, residual adds) are torch's own
bf16 CPU ops, which round the fp32 result as the GPU's do.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch
from einops import rearrange

from . import hif8_ref as R

BF16 = torch.bfloat16
F32 = torch.float32
F64 = torch.float64


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(BF16)


# ------------------------------------------------------------------ rearranges


def _token(x, grid, P):
    T, H, W = grid
    return rearrange(x, 'b (t h p w q) c -> (p q b) (t h w) c', p=P, q=P, h=H // P, w=W // P)


def _token_reverse(x, grid, P):
    T, H, W = grid
    return rearrange(x, '(p q b) (t h w) c -> b (t h p w q) c', p=P, q=P, h=H // P, w=W // P)


def _group(x, grid, P):
    T, H, W = grid
    return rearrange(x, 'b (txh p1 p2 w q1 q2) c -> (p1 q1 b) (txh p2 w q2) c',
                     p1=P, q1=P, p2=P, q2=P, w=W // (P ** 2))


def _group_reverse(x, grid, P):
    T, H, W = grid
    return rearrange(x, '(p1 q1 b) (txh p2 w q2) c -> b (txh p1 p2 w q1 q2) c',
                     p1=P, q1=P, p2=P, q2=P, w=W // (P ** 2))


def _token_to_group(x, grid, P):
    T, H, W = grid
    return rearrange(x, '(p2 q2 b) (txh_p1 p1 w_q1 q1) c -> (p1 q1 b) (txh_p1 p2 w_q1 q2) c',
                     p1=P, q1=P, p2=P, q2=P, w_q1=W // (P ** 2))


_FNS = {"skiparse_2d_token": _token, "skiparse_2d_token_reverse": _token_reverse,
        "skiparse_2d_group": _group, "skiparse_2d_group_reverse": _group_reverse,
        "skiparse_2d_token_to_group": _token_to_group, "skiparse_2d_group_to_token": _token_to_group}


def skiparse_rearrange(x, kind: str, grid, P: int):
    """SkiparseRearrange.forward (osp_next.py:239-283) without sequence parallelism."""
    if kind == "identity" or x is None:
        return x
    T, H, W = grid
    bs = P ** 2
    ph, pw = (bs - H % bs) % bs, (bs - W % bs) % bs
    B, N, C = x.shape
    if kind in ("skiparse_2d_token", "skiparse_2d_group"):
        if ph or pw:
            x = torch.nn.functional.pad(x.reshape(B, T, H, W, C), (0, 0, 0, pw, 0, ph)).reshape(B, -1, C)
        return _FNS[kind](x, (T, H + ph, W + pw), P)
    if kind in ("skiparse_2d_token_reverse", "skiparse_2d_group_reverse"):
        x = _FNS[kind](x, (T, H + ph, W + pw), P)
        if ph or pw:
            b = x.shape[0]
            x = x.reshape(b, T, H + ph, W + pw, C)[:, :, :H, :W].reshape(b, -1, C)
        return x
    return _FNS[kind](x, (T, H + ph, W + pw), P)


def masks(batch: int, grid, P: int):
    """(token mask, group mask) as SkiparseMaskPreprocessor.preprocess returns them."""
    T, H, W = grid
    ones = torch.ones((batch, T * H * W, 1), dtype=torch.bool)
    out = []
    for kind in ("skiparse_2d_token", "skiparse_2d_group"):
        m = skiparse_rearrange(ones, kind, grid, P).squeeze(-1).bool()
        out.append(None if bool(m.all()) else m)
    return tuple(out)


# ------------------------------------------------------------------------ RoPE


def rope_angles(grid, head_dim: int, kind: str, P: int) -> torch.Tensor:
    """Per-token angles [P*P or 1, seq, head_dim/2] (fp32), osp_next.py:64-70,558-607."""
    d = head_dim

    def params(n, dim):
        i = torch.arange(0, dim, 2, dtype=F64)
        return torch.outer(torch.arange(n, dtype=F64), 1.0 / torch.pow(10000.0, i / dim)).to(F32)

    freqs = torch.cat([params(1024, d - 4 * (d // 6)), params(1024, 2 * (d // 6)), params(1024, 2 * (d // 6))], 1)
    h = d // 2
    f0, f1, f2 = freqs.split([h - 2 * (h // 3), h // 3, h // 3], dim=1)
    T, H, W = grid
    fi = torch.cat([f0[:T].reshape(T, 1, 1, -1).expand(T, H, W, -1), f1[:H].reshape(1, H, 1, -1).expand(T, H, W, -1),
                    f2[:W].reshape(1, 1, W, -1).expand(T, H, W, -1)], dim=-1).reshape(1, T * H * W, -1)
    return skiparse_rearrange(fi, kind, grid, P)


def apply_rope(x: torch.Tensor, ang: torch.Tensor) -> torch.Tensor:
    """x [B, S, heads, D] -> fp32: (x[2i], x[2i+1]) rotated by angle i (osp_next.py:609-644)."""
    B, S, Hh, D = x.shape
    xx = x.to(F64).reshape(B, S, Hh, D // 2, 2)
    a = ang.to(F64)
    if a.shape[0] > 1 and a.shape[0] != B:
        a = a.repeat_interleave(B // a.shape[0], dim=0)
    c = torch.cos(a).to(F32).to(F64).unsqueeze(2)
    s = torch.sin(a).to(F32).to(F64).unsqueeze(2)
    o1 = xx[..., 0] * c - xx[..., 1] * s
    o2 = xx[..., 0] * s + xx[..., 1] * c
    return torch.stack([o1, o2], -1).flatten(3).to(F32)


# ----------------------------------------------------------------------- norms


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """WanRMSNorm: normalise in fp32 (here float64), type_as(x), * fp32 weight, output bf16."""
    xf = x.to(F64)
    n = (xf / torch.sqrt(xf.square().mean(-1, keepdim=True) + eps)).to(F32).to(x.dtype)
    return (n.to(F32) * w.to(F32)).to(BF16)


def layer_norm(x: torch.Tensor, eps: float, w: Optional[torch.Tensor] = None,
               b: Optional[torch.Tensor] = None) -> torch.Tensor:
    """WanLayerNorm of a bf16 tensor (affine with fp32 parameters), output bf16."""
    xf = x.to(F64)
    mean = xf.mean(-1, keepdim=True)
    var = (xf - mean).square().mean(-1, keepdim=True)
    n = (xf - mean) / torch.sqrt(var + float(np.float32(eps)))
    if w is not None:
        n = n * w.to(F64) + b.to(F64)
    return n.to(F32).to(BF16)


# -------------------------------------------------------------------- linears


def hif8_linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], smax: float = 15.0) -> torch.Tensor:
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    if x.dtype == BF16:
        xq = R.bf16_to_f32(R.quant_bf16(_bits(x2), smax)[0])
    else:
        xq32, _ = R.quant_f32(x2.numpy(), smax)
        xq = R.bf16_to_f32(R.f32_to_bf16(xq32))       # autocast: F.linear on bf16(x_q)
    wq = R.bf16_to_f32(R.quant_bf16(_bits(w.contiguous()), smax)[0])
    y = xq.astype(np.float64) @ wq.astype(np.float64).T
    if b is not None:
        y = y + R.bf16_to_f32(_bits(b)).astype(np.float64)
    return torch.from_numpy(y.astype(np.float32)).to(BF16).reshape(*x.shape[:-1], -1)


def exact_linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    """F.linear under bf16 autocast, summed exactly: bf16(x) @ W^T + b, rounded to bf16."""
    y = x.to(BF16).to(F64) @ w.to(F64).T
    if b is not None:
        y = y + b.to(F64)
    return y.to(F32).to(BF16)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    xf = x.to(F64)
    return (0.5 * xf * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (xf + 0.044715 * xf ** 3)))).to(F32).to(x.dtype)


def attention(q, k, v, key_mask=None) -> torch.Tensor:
    """SDPA on bf16 [B, N, H, D] q, k, v (attention.py:433-518), exact softmax, bf16 output."""
    qf, kf, vf = (t.to(BF16).to(F64).transpose(1, 2) for t in (q, k, v))
    s = qf @ kf.transpose(-1, -2) / math.sqrt(q.shape[-1])
    if key_mask is not None:
        s = s.masked_fill(~key_mask[:, None, None, :], float("-inf"))
    out = torch.softmax(s, -1) @ vf
    return out.transpose(1, 2).to(F32).to(BF16)


def hif8_qdq(t: torch.Tensor, smax: float = 15.0) -> torch.Tensor:
    """_quant(t)[0] (hif8_attention.py:60-74)."""
    if t.dtype == BF16:
        return _from_bits(R.quant_bf16(_bits(t.reshape(-1)), smax)[0]).reshape(t.shape)
    q, _ = R.quant_f32(t.reshape(-1).numpy(), smax)
    return torch.from_numpy(q).reshape(t.shape)


# ---------------------------------------------------------------------- block


def block(sd: Dict[str, torch.Tensor], x: torch.Tensor, e: torch.Tensor, text: torch.Tensor, grid,
          kind: str, full2skiparse: bool, skiparse2full: bool, num_heads: int, P: int = 2, eps: float = 1e-6,
          quant_attn: Optional[str] = None, smax: float = 15.0, cross_attn_norm: bool = True,
          linear: str = "hif8") -> torch.Tensor:
    """OSPNextAttentionBlock.forward (osp_next.py:960-1022) of one block: x [B, T*H*W or skiparse
    layout, dim] bf16, e [B, 6, dim] bf16, text [B, L, dim] bf16.  ``linear="exact"`` replaces
    the HiF8 linears by exact ones on the bf16 input (a check of the glue alone)."""
    if kind == "full":
        r_in, r_out, rope_kind, Pk = "identity", "identity", "identity", 1
    elif kind == "token":
        r_in = "skiparse_2d_token" if full2skiparse else "skiparse_2d_group_to_token"
        r_out, rope_kind, Pk = "identity", "skiparse_2d_token", P
    else:
        r_in = "skiparse_2d_token_to_group"
        r_out = "skiparse_2d_group_reverse" if skiparse2full else "identity"
        rope_kind, Pk = "skiparse_2d_group", P
    full_in = kind == "full" or (kind == "token" and full2skiparse)
    B = x.shape[0] if full_in else x.shape[0] // (P * P)     # the batch before any rearrange
    tm, gm = masks(B, grid, P) if kind != "full" else (None, None)
    key_mask = tm if kind == "token" else gm
    x = skiparse_rearrange(x, r_in, grid, Pk)
    if kind != "full":
        text = text.repeat(P * P, 1, 1)      # 'b n c -> (p b) n c'
        e = e.repeat(P * P, 1, 1)
    dim = x.shape[-1]
    Hh = num_heads
    D = dim // Hh
    ang = rope_angles(grid, D, rope_kind, Pk)

    def lin(name, t):
        if linear == "exact":
            return exact_linear(t, sd[name + ".weight"], sd.get(name + ".bias"))
        return hif8_linear(t, sd[name + ".weight"], sd.get(name + ".bias"), smax)

    def attend(q, k, v, km):
        if quant_attn == "hif8":
            q, k, v = hif8_qdq(q, smax), hif8_qdq(k, smax), hif8_qdq(v, smax)
        return attention(q, k, v, km).to(q.dtype)

    ee = (sd["modulation"] + e).chunk(6, dim=1)
    # self-attention (osp_next.py:732-779) on norm1(x) * (1 + e1) + e0
    y = layer_norm(x, eps) * (1 + ee[1]) + ee[0]
    Bx, N = x.shape[:2]
    q = rms_norm(lin("self_attn.q", y), sd["self_attn.norm_q.weight"], eps).reshape(Bx, N, Hh, D)
    k = rms_norm(lin("self_attn.k", y), sd["self_attn.norm_k.weight"], eps).reshape(Bx, N, Hh, D)
    v = lin("self_attn.v", y).reshape(Bx, N, Hh, D)
    q, k = apply_rope(q, ang), apply_rope(k, ang)
    a = attend(q, k, v, key_mask)
    x = x + lin("self_attn.o", a.flatten(2)) * ee[2]
    # cross-attention (osp_next.py:784-816)
    xn = layer_norm(x, eps, sd["norm3.weight"], sd["norm3.bias"]) if cross_attn_norm else x
    q = rms_norm(lin("cross_attn.q", xn), sd["cross_attn.norm_q.weight"], eps).reshape(Bx, -1, Hh, D)
    k = rms_norm(lin("cross_attn.k", text), sd["cross_attn.norm_k.weight"], eps).reshape(Bx, -1, Hh, D)
    v = lin("cross_attn.v", text).reshape(Bx, -1, Hh, D)
    x = x + lin("cross_attn.o", attend(q, k, v, None).flatten(2))
    # FFN (osp_next.py:873-877, :954)
    y = layer_norm(x, eps) * (1 + ee[4]) + ee[3]
    h = gelu_tanh(lin("ffn.0", y))
    x = x + lin("ffn.2", h) * ee[5]
    return skiparse_rearrange(x, r_out, grid, Pk)


def blocks(sds, schedule, x, e, text, grid, num_heads, P=2, **kw):
    """The block loop (osp_next.py:1287-1331) over ``schedule`` = [(kind, f2s, s2f)]."""
    for sd, (kind, f2s, s2f) in zip(sds, schedule):
        x = block(sd, x, e, text, grid, kind, f2s, s2f, num_heads, P, **kw)
    return x
