"""Quantised-layer API and packed-weight files.

``QLinear`` / ``replace_linear`` mirror ``ospnext/quant_cy_npu/layers/QLinear.py:13-156``
and ``quant_cy_npu/utils/utils.py:16-37``: a plain ``nn.Linear`` whose input, weight
and (optionally) output gradient go through ``quant_dequant_float`` with an assigned
``QType`` -- the raw HiF8 qdq, without the per-tensor scale of ``HIF8Linear``.

``save_packed`` / ``load_packed`` / ``pack_state_dict`` keep ``HIF8Linear`` weights on
disk as 8-bit HiF8 codes plus the per-tensor scale (safetensors), so that an inference
model is built without ever materialising its bf16 weights.  The reference has no packed
format: it re-quantises the bf16 checkpoint weights at every call (hif8_linear.py:73).

File layout (one entry per HIF8Linear, ``<name>`` its module path)::

    <name>.codes   uint8   [out, in]   HiF8 codes of W * s (NPU semantics)
    <name>.scale   float32 [1]         s = rnd(rnd(1/amax) * scale_max) in W's dtype
    <name>.bias    bias dtype [out]    only if the layer has a bias
    metadata: "format" = "hif8-packed-1", "<name>.dtype" = W's dtype, "<name>.scale_max"
"""
from __future__ import annotations

from typing import Dict, List, Optional, Union

import torch
import torch.nn as nn
from torch import Tensor
from torch.autograd import Function

from . import _lib
from .hif8_linear import HIF8Linear, PackedWeight, QuantState, dense_linear, dense_mm
from .quant import QType, quant_dequant_float

FORMAT = "hif8-packed-1"
_DTYPES = {"torch.bfloat16": torch.bfloat16, "torch.float32": torch.float32}


# ------------------------------------------------------------------ QLinear


def _linear(x_q: Tensor, w_q: Tensor, b: Optional[Tensor]) -> Tensor:
    """F.linear on the library's GEMMs (dense_linear), any leading dims."""
    y = dense_linear(x_q.reshape(-1, x_q.shape[-1]), w_q, b)
    return y.view(*x_q.shape[:-1], y.shape[-1])


def _mm(a: Tensor, b: Tensor) -> Tensor:
    """a @ b for a [..., R] (flattened to 2-D) and b [R, N] on the library's GEMMs (dense_mm)."""
    y = dense_mm(a.reshape(-1, a.shape[-1]), b)
    return y.view(*a.shape[:-1], y.shape[-1])


class LinearForward(Function):
    """QLinear.py:13-43: saves x and w, re-quantises both in backward.  The products run on the
    library's GEMMs (dense_linear, dense_mm) in the dtype autocast gives them."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, w, b, qp, qp_in, quant_grad):
        x_q = quant_dequant_float(x, qp_in, force_fp32=True)
        w_q = quant_dequant_float(w, qp, force_fp32=True)
        ctx.save_for_backward(x, w)
        ctx.qp, ctx.qp_in, ctx.quant_grad = qp, qp_in, quant_grad
        ctx.has_bias = b is not None
        return _linear(x_q, w_q, b)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_out):
        x, w = ctx.saved_tensors
        x_q = quant_dequant_float(x, ctx.qp_in, force_fp32=True)
        w_q = quant_dequant_float(w, ctx.qp, force_fp32=True)
        if ctx.quant_grad:
            g_q = quant_dequant_float(grad_out, ctx.qp_in, force_fp32=True)
            g_t = quant_dequant_float(grad_out.flatten(0, -2).transpose(-1, -2).contiguous(), ctx.qp_in, force_fp32=True)
        else:
            g_q, g_t = grad_out, grad_out.flatten(0, -2).transpose(-1, -2)
        grad_in = _mm(g_q, w_q)
        grad_w = _mm(g_t, x_q.flatten(0, -2))
        grad_b = grad_out.flatten(0, -2).sum(0) if ctx.has_bias else None
        return grad_in, grad_w, grad_b, None, None, None


class LinearForwardFast(Function):
    """QLinear.py:46-70: saves the quantised x_q and w_q instead (products as LinearForward)."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, w, b, qp, qp_in, quant_grad):
        x_q = quant_dequant_float(x, qp_in, force_fp32=True)
        w_q = quant_dequant_float(w, qp, force_fp32=True)
        ctx.save_for_backward(x_q, w_q)
        ctx.qp_in, ctx.quant_grad = qp_in, quant_grad
        ctx.has_bias = b is not None
        return _linear(x_q, w_q, b)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_out):
        x_q, w_q = ctx.saved_tensors
        g_q = quant_dequant_float(grad_out, ctx.qp_in, force_fp32=True) if ctx.quant_grad else grad_out
        grad_in = _mm(g_q, w_q)
        grad_w = _mm(g_q.flatten(0, -2).transpose(-1, -2), x_q.flatten(0, -2))
        grad_b = grad_out.flatten(0, -2).sum(0) if ctx.has_bias else None
        return grad_in, grad_w, grad_b, None, None, None


class QLinear(nn.Linear):
    """QLinear.py:73-156 (``compute_err``, a debugging printout, is not carried over)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.qparams: Optional[QType] = None
        self.in_qparams: Optional[QType] = None
        self._quant_grad = True
        self._fast_forward = False

    def set_quant_grad(self, value: bool):
        self._quant_grad = value

    def forward(self, x: Tensor) -> Tensor:
        assert self.qparams is not None, "QLinear has no weight QType: call assign_qparams() before forward"
        qp = self.qparams.dim(-1)
        qp_in = self.qparams.dim(-1) if self.in_qparams is None else self.in_qparams.dim(-1)
        if not x.is_contiguous():
            x = x.contiguous()
        fn = LinearForwardFast if self._fast_forward else LinearForward
        return fn.apply(x, self.weight, self.bias, qp, qp_in, self._quant_grad)

    def transfer(self, layer: Union["QLinear", nn.Linear]):
        self.to(layer.weight.device)
        self.to(layer.weight.dtype)
        with torch.no_grad():
            self.weight.copy_(layer.weight.reshape(self.weight.shape))
            if self.bias is not None:
                self.bias.copy_(layer.bias)

    def assign_qparams(self, Q: Union[QType, str]):
        self.qparams = QType(Q) if isinstance(Q, str) else Q.copy()

    def assign_input_qparams(self, Q: Union[QType, str]):
        self.in_qparams = QType(Q) if isinstance(Q, str) else Q.copy()

    def __deepcopy__(self, memo):
        layer = QLinear(self.weight.shape[1], self.weight.shape[0], self.bias is not None)
        layer.transfer(self)
        assert self.qparams is not None, "a QLinear is copied only once its weight QType is assigned"
        layer.assign_qparams(self.qparams)
        if self.in_qparams is not None:
            layer.assign_input_qparams(self.in_qparams)
        layer.set_quant_grad(self._quant_grad)
        return layer


def replace_linear(module: nn.Module, w_Q: Union[QType, str], in_Q: Union[QType, str, None] = None,
                   quant_grad: bool = True, exclude_layers: Optional[List[str]] = None) -> None:
    """utils.py:16-37: swap every nn.Linear below ``module`` (not ``exclude_layers``) for a QLinear.
    As in the reference, subclasses of nn.Linear (QLinear, HIF8Linear) are replaced too."""
    exclude_layers = [] if exclude_layers is None else exclude_layers
    assert isinstance(exclude_layers, list), "exclude_layers takes a list of module names"
    mods = dict(module.named_modules())
    for name, m in list(module.named_modules()):
        if name in exclude_layers or not isinstance(m, nn.Linear):
            continue
        new = QLinear(m.in_features, m.out_features, m.bias is not None)
        new.transfer(m)
        new.assign_qparams(w_Q)
        new.set_quant_grad(quant_grad)
        if in_Q is not None:
            new.assign_input_qparams(in_Q)
        parent = mods[".".join(name.split(".")[:-1])]
        setattr(parent, name.split(".")[-1], new)


# ------------------------------------------------------------ packed files


def packed_from_codes(codes: Tensor, scale: float, dtype: torch.dtype, scale_max: float) -> PackedWeight:
    """A PackedWeight from stored codes and scale (no bf16 weight needed): the state is
    set to the scale (hif8_set_scale builds the decode tables)."""
    _lib.require_gpu_tensor(codes, "codes")
    pw = PackedWeight.__new__(PackedWeight)
    pw.shape = tuple(codes.shape)
    pw.src_dtype = dtype
    pw.state = QuantState(codes.device)
    _lib.check(_lib.load().hif8_set_scale(pw.state.ptr, _lib.dtype_code(dtype), float(scale),
                                          _lib.stream_ptr(codes.device)), "hif8_set_scale")
    pw.codes = codes.contiguous()
    pw.scale_max = float(scale_max)
    pw.key = None
    pw._codes_t = None
    return pw


def _layer_entries(name: str, packed: PackedWeight, bias: Optional[Tensor], tensors: Dict[str, Tensor],
                   meta: Dict[str, str]) -> None:
    _, scale = packed.state.read()
    tensors[f"{name}.codes"] = packed.codes.detach().contiguous().cpu()
    tensors[f"{name}.scale"] = torch.tensor([scale], dtype=torch.float32)
    if bias is not None:
        tensors[f"{name}.bias"] = bias.detach().contiguous().cpu()
    meta[f"{name}.dtype"] = str(packed.src_dtype)
    meta[f"{name}.scale_max"] = repr(packed.scale_max)


def save_packed(module: nn.Module, path: str) -> List[str]:
    """Write every HIF8Linear of ``module`` as codes + scale (+ bias); returns the names."""
    from safetensors.torch import save_file
    tensors: Dict[str, Tensor] = {}
    meta = {"format": FORMAT}
    names = []
    for name, m in module.named_modules():
        if isinstance(m, HIF8Linear):
            _layer_entries(name, m._packed_weight(), m.bias, tensors, meta)
            names.append(name)
    save_file(tensors, path, metadata=meta)
    return names


def pack_state_dict(state_dict: Dict[str, Tensor], names: List[str], path: str, scale_max: float = 15.0,
                    device: Union[str, torch.device] = "cuda") -> None:
    """Convert ``<name>.weight`` (and ``<name>.bias``) entries of a checkpoint state dict into a
    packed file, quantising each weight on ``device`` once."""
    from safetensors.torch import save_file
    tensors: Dict[str, Tensor] = {}
    meta = {"format": FORMAT}
    for name in names:
        w = state_dict[f"{name}.weight"].to(device)
        packed = PackedWeight(w, scale_max)
        _layer_entries(name, packed, state_dict.get(f"{name}.bias"), tensors, meta)
        del w, packed
    save_file(tensors, path, metadata=meta)


def load_packed(module: nn.Module, path: str, drop_weight: bool = True) -> List[str]:
    """Install packed weights from ``path`` into the HIF8Linear layers of ``module`` (which must
    already sit on the GPU); with ``drop_weight`` the bf16 weight parameters are released."""
    from safetensors import safe_open
    loaded = []
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (format={meta.get('format')!r})")
        keys = set(f.keys())
        for name, m in module.named_modules():
            if not isinstance(m, HIF8Linear) or f"{name}.codes" not in keys:
                continue
            dev = m.bias.device if m.bias is not None else m.weight.device
            codes = f.get_tensor(f"{name}.codes").to(dev)
            if tuple(codes.shape) != (m.out_features, m.in_features):
                raise ValueError(f"{name}: packed shape {tuple(codes.shape)} != {(m.out_features, m.in_features)}")
            scale = float(f.get_tensor(f"{name}.scale")[0])
            dtype = _DTYPES[meta[f"{name}.dtype"]]
            smax = float(meta[f"{name}.scale_max"])
            m._packed = packed_from_codes(codes, scale, dtype, smax)
            m._prepacked = True
            m.scale_max_forward = smax
            if f"{name}.bias" in keys and m.bias is not None:
                with torch.no_grad():
                    m.bias.copy_(f.get_tensor(f"{name}.bias").to(m.bias.device, m.bias.dtype))
            if drop_weight:
                m.weight = nn.Parameter(torch.empty(0, device=dev, dtype=dtype), requires_grad=False)
            loaded.append(name)
    return loaded
