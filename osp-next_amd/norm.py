"""Producer fusion for the modulated LayerNorm in front of q/k/v and the FFN.

``block_forward`` (``ospnext/modules/osp_next.py:937-957``) feeds its self-attention and FFN
with ``norm(x) * (1 + e[1]) + e[0]`` and ``norm(x) * (1 + e[4]) + e[3]``, ``norm`` the
WanLayerNorm (``ospnext/modules/want2v.py:96-106``); every consuming HIF8Linear then runs
``_quant`` on that tensor (``hif8_linear.py:42-50``), so q, k and v quantise the same input
three times.  ``modulated_norm_quant`` produces the quantised input directly, in two passes
over x (``hif8_modln_amax`` and ``hif8_modln_fake_quant``), and ``qkv_from_modulated_norm``
feeds it to the three projections with one quantisation.  ``affine_norm_quant`` does the same
for the affine LayerNorm (norm3) in front of the cross-attention's q projection.

The fused route is inference-only (no autograd through the producer) and takes bf16 x with
``dim % 8 == 0`` and ``dim <= 8192``; anything else runs the reference's op sequence with the
library's ``_quant`` on the GPU.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from . import _lib
from .hif8_linear import (GroupedWeight, HIF8Linear, QuantState, absmax_scale, fake_quant, grouped_ok,
                          linear_fwd_grouped)

MAX_DIM = 8192


class WanLayerNorm(nn.LayerNorm):
    """want2v.py:96-106: fp32 layer norm over the last dim, cast back to the input dtype."""

    def __init__(self, dim: int, eps: float = 1e-6, elementwise_affine: bool = False):
        super().__init__(dim, elementwise_affine=elementwise_affine, eps=eps)

    def forward(self, x: Tensor) -> Tensor:
        return super().forward(x.float()).type_as(x)


def modulate(n: Tensor, shift: Optional[Tensor], scale: Optional[Tensor]) -> Tensor:
    """``n * (1 + scale) + shift`` as block_forward writes it (osp_next.py:941, :954)."""
    y = n if scale is None else n * (1 + scale)
    return y if shift is None else y + shift


def _modulation_rows(t: Optional[Tensor], x: Tensor, name: str) -> Tuple[Optional[Tensor], int]:
    """[B, 1, D] / [B, D] / [1, D] / [D] modulation -> contiguous [batches, D] and rows per batch."""
    if t is None:
        return None, 0
    D = x.shape[-1]
    if t.shape[-1] != D:
        raise ValueError(f"{name} has last dim {t.shape[-1]}, x has {D}")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 like x, got {t.dtype}")
    t2 = t.reshape(-1, D)
    batches = t2.shape[0]
    rows = x.numel() // D
    if batches == 1:
        rpb = rows
    else:
        if x.dim() < 3 or x.shape[0] != batches or any(s != 1 for s in t.shape[1:-1]):
            raise ValueError(f"{name} of shape {tuple(t.shape)} does not broadcast per batch over x {tuple(x.shape)}")
        rpb = rows // batches
    return t2.contiguous(), rpb


def fused_ok(x: Tensor) -> bool:
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() >= 1 and x.numel() > 0
            and x.shape[-1] % 8 == 0 and x.shape[-1] <= MAX_DIM)


def modulated_norm_quant(x: Tensor, shift: Optional[Tensor] = None, scale: Optional[Tensor] = None,
                         eps: float = 1e-6, scale_max: float = 15.0, semantics: int = _lib.SEM_NPU,
                         return_y: bool = False):
    """x_q = _quant(WanLayerNorm(x) * (1 + scale) + shift)[0] in bf16, the input every HIF8Linear
    fed by this modulated norm quantises to.  Returns ``(x_q, state)`` (``state`` holds amax,
    scale and decode tables of y), plus y itself with ``return_y``."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, shift, scale)):
        raise RuntimeError("modulated_norm_quant has no autograd; use WanLayerNorm, modulate and "
                           "HIF8Linear.forward when gradients are needed")
    if not fused_ok(x):
        y = modulate(WanLayerNorm(x.shape[-1], eps).to(x.device)(x), shift, scale).contiguous()
        st = absmax_scale(y, scale_max, QuantState(y.device))
        xq = fake_quant(y, st, semantics)
        return (xq, st, y) if return_y else (xq, st)
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    D = x.shape[-1]
    rows = x.numel() // D
    sh, rpb_s = _modulation_rows(shift, x, "shift")
    sc, rpb_c = _modulation_rows(scale, x, "scale")
    if sh is not None and sc is not None and rpb_s != rpb_c:
        raise ValueError("shift and scale have different batch counts")
    rpb = rpb_s or rpb_c or rows
    stats = torch.empty(rows * 2, dtype=torch.float32, device=x.device)
    st = QuantState(x.device)
    L = _lib.load()
    s = _lib.stream_ptr(x.device)
    sh_p = sh.data_ptr() if sh is not None else None
    sc_p = sc.data_ptr() if sc is not None else None
    _lib.check(L.hif8_modln_amax(x.data_ptr(), sh_p, sc_p, rows, D, rpb, float(eps), stats.data_ptr(),
                                 float(scale_max), st.ptr, s), "hif8_modln_amax")
    xq = torch.empty_like(x)
    y = torch.empty_like(x) if return_y else None
    _lib.check(L.hif8_modln_fake_quant(x.data_ptr(), sh_p, sc_p, rows, D, rpb, stats.data_ptr(), st.ptr,
                                       int(semantics), xq.data_ptr(), y.data_ptr() if y is not None else None, s),
               "hif8_modln_fake_quant")
    return (xq, st, y) if return_y else (xq, st)


STATIC_MAX_ROWS = 131072


def modulated_norm_quant_static(x: Tensor, shift: Optional[Tensor] = None, scale: Optional[Tensor] = None,
                                eps: float = 1e-6, scale_max: float = 15.0, semantics: int = _lib.SEM_NPU) -> Tensor:
    """``modulated_norm_quant(x, shift, scale, eps, scale_max)[0]`` through the allocation-free entry
    point ``hif8_modln_quant_static``: the row statistics and the state live in the library's static
    device workspace (at most STATIC_MAX_ROWS rows), so the library allocates nothing; only x_q is
    returned (it has no state object).  Calls overlapping on one GPU race on that workspace."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, shift, scale)):
        raise RuntimeError("modulated_norm_quant_static has no autograd")
    if not fused_ok(x):
        raise ValueError("modulated_norm_quant_static takes bf16 CUDA x with dim % 8 == 0 and dim <= 8192")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    D = x.shape[-1]
    rows = x.numel() // D
    sh, rpb_s = _modulation_rows(shift, x, "shift")
    sc, rpb_c = _modulation_rows(scale, x, "scale")
    if sh is not None and sc is not None and rpb_s != rpb_c:
        raise ValueError("shift and scale have different batch counts")
    rpb = rpb_s or rpb_c or rows
    xq = torch.empty_like(x)
    _lib.check(_lib.load().hif8_modln_quant_static(x.data_ptr(), sh.data_ptr() if sh is not None else None,
                                                   sc.data_ptr() if sc is not None else None, rows, D, rpb, float(eps),
                                                   float(scale_max), int(semantics), xq.data_ptr(),
                                                   _lib.stream_ptr(x.device)), "hif8_modln_quant_static")
    return xq


AFFINE_MAX_DIM = 6144


def affine_fused_ok(x: Tensor, norm: nn.Module) -> bool:
    """The fused affine producer takes bf16 CUDA x with dim % 8 == 0, dim <= 6144, and a
    WanLayerNorm with fp32 weight and bias."""
    w, b = getattr(norm, "weight", None), getattr(norm, "bias", None)
    return (fused_ok(x) and x.shape[-1] <= AFFINE_MAX_DIM and isinstance(norm, nn.LayerNorm)
            and w is not None and b is not None and w.dtype == torch.float32 and b.dtype == torch.float32
            and tuple(norm.normalized_shape) == (x.shape[-1],) and w.device == x.device)


def affine_norm_quant(x: Tensor, norm: nn.Module, scale_max: float = 15.0, semantics: int = _lib.SEM_NPU,
                      return_y: bool = False):
    """x_q = _quant(norm(x))[0] in bf16 for the affine WanLayerNorm ``norm`` (norm3,
    osp_next.py:860-864, 949-951): the input the cross-attention's q projection quantises.
    Returns ``(x_q, state)``, plus y = norm(x) with ``return_y``.  Two passes over x
    (``hif8_ln_affine_amax`` and ``hif8_ln_affine_fake_quant``); other shapes and dtypes run
    the module and the library's ``_quant`` on the GPU."""
    if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in norm.parameters())):
        raise RuntimeError("affine_norm_quant has no autograd; use the norm module and HIF8Linear.forward "
                           "when gradients are needed")
    if not affine_fused_ok(x, norm):
        y = norm(x).contiguous()
        st = absmax_scale(y, scale_max, QuantState(y.device))
        xq = fake_quant(y, st, semantics)
        return (xq, st, y) if return_y else (xq, st)
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    w = norm.weight.detach().contiguous()
    b = norm.bias.detach().contiguous()
    D = x.shape[-1]
    rows = x.numel() // D
    stats = torch.empty(rows * 2, dtype=torch.float32, device=x.device)
    st = QuantState(x.device)
    L = _lib.load()
    s = _lib.stream_ptr(x.device)
    _lib.check(L.hif8_ln_affine_amax(x.data_ptr(), w.data_ptr(), b.data_ptr(), rows, D, float(norm.eps),
                                     stats.data_ptr(), float(scale_max), st.ptr, s), "hif8_ln_affine_amax")
    xq = torch.empty_like(x)
    y = torch.empty_like(x) if return_y else None
    _lib.check(L.hif8_ln_affine_fake_quant(x.data_ptr(), w.data_ptr(), b.data_ptr(), rows, D, stats.data_ptr(),
                                           st.ptr, int(semantics), xq.data_ptr(),
                                           y.data_ptr() if y is not None else None, s),
               "hif8_ln_affine_fake_quant")
    return (xq, st, y) if return_y else (xq, st)


def qkv_from_modulated_norm(x: Tensor, shift: Optional[Tensor], scale: Optional[Tensor], q: HIF8Linear,
                            k: HIF8Linear, v: HIF8Linear, eps: float = 1e-6) -> Tuple[Tensor, Tensor, Tensor]:
    """``q(y), k(y), v(y)`` for ``y = norm(x) * (1 + scale) + shift`` (osp_next.py:742-744 fed by :941)
    with y quantised once and the three products in one grouped launch when the shapes allow
    (each output bit-identical to the layer's own forward).  Inference only; the three layers
    must share ``scale_max_forward``."""
    smf = q.scale_max_forward
    if k.scale_max_forward != smf or v.scale_max_forward != smf:
        raise ValueError("q, k and v quantise their input with different scale_max_forward")
    xq, _ = modulated_norm_quant(x, shift, scale, eps, smf)
    gw = grouped_weight((q, k, v))
    if gw is None:
        return q.forward_quantized(xq), k.forward_quantized(xq), v.forward_quantized(xq)
    K = xq.shape[-1]
    ys = linear_fwd_grouped(xq.reshape(-1, K).contiguous(), gw)
    return tuple(y.view(*xq.shape[:-1], y.shape[-1]) for y in ys)


def grouped_weight(layers) -> Optional[GroupedWeight]:
    """The layers' weights concatenated for one grouped launch (cached on the first layer and
    rebuilt when any packed weight or bias changes), or None when they do not fit one."""
    packs = [m._packed_weight() for m in layers]
    if not grouped_ok(packs):
        return None
    key = tuple((id(p), None if m.bias is None else (m.bias.data_ptr(), m.bias._version))
                for p, m in zip(packs, layers))
    cached = getattr(layers[0], "_grouped_cache", None)
    if cached is not None and cached.key == key:
        return cached
    gw = GroupedWeight(packs, [m.bias for m in layers], key)
    layers[0]._grouped_cache = gw
    return gw
