"""HiF8 quantise-dequantise API, mirroring OSP-Next's ``quant_cy_npu`` surface.

* ``QType``               -- ``ospnext/quant_cy_npu/base/QType.py:5-43`` (only the
  fields the ``'hif8'`` path reads).
* ``quant_dequant_float`` -- ``ospnext/quant_cy_npu/base/QTensor.py:94-128``.
* ``quant_func``          -- ``QTensor.py:131-144`` (straight-through estimator).
* ``quant_slide_window``  -- ``QTensor.py:147-174`` (qdq outside a trailing window, in place).
* ``hif8_quant`` / ``hif8_quant_bf16`` -- the pybind entry points
  ``npu_quant.hif8_quant(x, y)`` / ``npu_quant.hif8_quant_bf16(x, y)``
  (``cusrc/npu_quant.cpp:19-39``): in-place into a caller-allocated ``y``.

All arithmetic runs in the HIP library; tensors must live on the GPU.
"""
from __future__ import annotations

from copy import deepcopy

import torch
from torch import Tensor
from torch.autograd import Function

from . import _lib


class QType:
    """Format descriptor (QType.py:5-43).  For ``'hif8'`` only ``desc`` and
    ``q_dim`` matter: ``blk_size = blk_outer_size = 1`` means no padding."""

    desc: str
    exp_bits: int = -1
    man_bits: int = -1
    k_bits: int = -1
    k_outer_bits: int = 0
    blk_size: int = 1
    blk_outer_size: int = 1
    exp_max: int = -1
    exp_min: int = -1
    k_max: int = -1
    fp_val_max: float = -1
    q_dim: int = -1
    man_shift_bit: int = -1
    exp_offset: int = 0
    do_carry: bool = True

    def __init__(self, desc: str):
        self.desc = desc

    def dim_(self, dim: int) -> "QType":
        self.q_dim = dim
        return self

    def dim(self, dim: int) -> "QType":
        out = deepcopy(self)
        out.q_dim = dim
        return out

    def copy(self) -> "QType":
        return deepcopy(self)

    def __repr__(self) -> str:
        return f"QType: {self.desc}   Dim: {self.q_dim}  ExpOffset: {self.exp_offset}"


def _qdq_inplace(x: Tensor, y: Tensor, semantics: int) -> None:
    _lib.require_gpu_tensor(x, "x")
    _lib.require_gpu_tensor(y, "y")
    if x.dtype != y.dtype or x.numel() != y.numel():
        raise ValueError("x and y must have the same dtype and number of elements")
    n = x.numel()
    if n == 0:
        return
    if x.data_ptr() % 16:
        x = x.clone()
    if y.data_ptr() % 16:
        tmp = torch.empty_like(y)
        _qdq_inplace(x, tmp, semantics)
        y.copy_(tmp)
        return
    L = _lib.load()
    s = _lib.stream_ptr(x.device)
    if x.dtype == torch.float16:
        if semantics == _lib.SEM_TORCH_BF16:
            raise ValueError("the bf16-arithmetic torch route takes a bfloat16 tensor")
        _lib.check(L.hif8_quant_f16(x.data_ptr(), y.data_ptr(), n, semantics, s), "hif8_quant_f16")
    elif semantics == _lib.SEM_TORCH_F16:
        raise ValueError("the fp16-arithmetic torch route takes a float16 tensor")
    elif x.dtype == torch.bfloat16:
        _lib.check(L.hif8_quant_bf16(x.data_ptr(), y.data_ptr(), n, semantics, s), "hif8_quant_bf16")
    elif semantics == _lib.SEM_TORCH_BF16:
        raise ValueError("the bf16-arithmetic torch route takes a bfloat16 tensor")
    elif x.dtype == torch.float32:
        _lib.check(L.hif8_quant_f32(x.data_ptr(), y.data_ptr(), n, semantics, s), "hif8_quant_f32")
    else:
        raise TypeError(f"unsupported dtype {x.dtype}")


def hif8_quant(x: Tensor, y: Tensor) -> None:
    """``npu_quant.hif8_quant`` (fp32, npu_quant.cpp:19-25): y <- qdq(x)."""
    if x.dtype != torch.float32:
        raise TypeError("hif8_quant takes float32 tensors")
    _qdq_inplace(x, y, _lib.SEM_NPU)


def hif8_quant_bf16(x: Tensor, y: Tensor) -> None:
    """``npu_quant.hif8_quant_bf16`` (bf16, npu_quant.cpp:27-33): y <- qdq(x)."""
    if x.dtype != torch.bfloat16:
        raise TypeError("hif8_quant_bf16 takes bfloat16 tensors")
    _qdq_inplace(x, y, _lib.SEM_NPU)


@torch.no_grad()
def quant_dequant_float(x: Tensor, Q: QType, force_py: bool = False, force_fp32: bool = False,
                        **kwargs) -> Tensor:
    """QTensor.py:94-128 for ``Q.desc == 'hif8'``.

    ``force_py=False`` follows the NPU kernel (``hif8_quant_op.h``), ``True`` the
    torch function ``quant_hif8`` (``QFuncs/hif8.py:6-23``).  The output has the
    input's dtype (QTensor.py:126-127).  The torch function runs in the tensor's
    own precision unless ``force_fp32`` (QTensor.py:101-102): on a bf16 tensor every
    op then rounds to bf16 (HIF8_SEM_TORCH_BF16), on an fp16 tensor to fp16 with the
    fp16 offset 2^-14 of QFuncs/hif8.py:10-11 (HIF8_SEM_TORCH_F16).  The NPU kernel
    computes in fp32 for bf16 and fp32 alike; an fp16 tensor takes the fp32 kernel on
    its fp32 values and is cast back (QTensor.py:72-79), in one pass of
    ``hif8_quant_f16``; other dtypes go through fp32.
    """
    if Q.desc in ("fp16", "bf16", "fp32"):
        return x
    if Q.desc != "hif8":
        raise NotImplementedError(f"only the 'hif8' format is implemented, got {Q.desc!r}")
    semantics = _lib.SEM_TORCH if force_py else _lib.SEM_NPU
    if force_py and not force_fp32:
        if x.dtype == torch.bfloat16:
            semantics = _lib.SEM_TORCH_BF16
        elif x.dtype == torch.float16:
            semantics = _lib.SEM_TORCH_F16
    dtype_ori = x.dtype
    xc = x.contiguous()
    if xc.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        xc = xc.to(torch.float32)
    out = torch.empty_like(xc)
    _qdq_inplace(xc, out, semantics)
    if out.dtype != dtype_ori:
        out = out.to(dtype_ori)
    return out


class QuantFunc(Function):
    """Straight-through qdq (QTensor.py:131-140)."""

    @staticmethod
    def forward(ctx, x, Q, force_py, force_fp32):
        return quant_dequant_float(x, Q, force_py, force_fp32)

    @staticmethod
    def backward(ctx, grad):
        return grad, None, None, None


def quant_func(x: Tensor, Q: QType, force_py: bool = False, force_fp32: bool = False) -> Tensor:
    return QuantFunc.apply(x, Q, force_py, force_fp32)


class QuantSlideWindow(Function):
    """qdq of everything but a trailing window, in place, with a straight-through gradient
    (QTensor.py:147-167).  ``dim`` -1: the last ``win_size`` columns keep their values; -2: the
    last ``win_size`` rows of the last two dims; a pair ``(rows, cols)``: the region outside the
    top-left ``[:-rows, :-cols]`` block keeps its values.  A tensor no larger than the window
    along a windowed dim is returned unchanged.  ``x`` itself is modified and returned."""

    @staticmethod
    def forward(ctx, x, Q, force_py, force_fp32, dim, win_size):
        if isinstance(win_size, (list, tuple)):
            wr, wc = int(win_size[0]), int(win_size[1])
            if x.shape[-2] > wr and x.shape[-1] > wc:
                x[..., :-wr, :-wc] = quant_dequant_float(x[..., :-wr, :-wc], Q, force_py, force_fp32)
        elif dim == -1:
            if x.shape[-1] > win_size:
                x[..., :-win_size] = quant_dequant_float(x[..., :-win_size], Q, force_py, force_fp32)
        elif dim == -2:
            if x.shape[-2] > win_size:
                x[..., :-win_size, :] = quant_dequant_float(x[..., :-win_size, :], Q, force_py, force_fp32)
        else:
            raise NotImplementedError(f"quant_slide_window takes qdim -1 or -2, got {dim}")
        return x

    @staticmethod
    def backward(ctx, grad):
        return grad, None, None, None, None, None


def quant_slide_window(x: Tensor, Q: QType, force_py: bool = False, force_fp32: bool = False, qdim: int = -2,
                       win_size=128) -> Tensor:
    """QTensor.py:170-174: a non-negative ``qdim`` counts from the front (converted to the
    negative index); the window is kept at full precision, the rest quantised."""
    if qdim > 0:
        qdim = qdim - x.dim()
    return QuantSlideWindow.apply(x, Q, force_py, force_fp32, qdim, win_size)
