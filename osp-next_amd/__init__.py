"""MI355X-native HiF8 fake-quant linear path for OSP-Next.

Imported under the module name ``ospnext_amd`` (the directory name is not a
Python identifier; see ``__graft_entry__.load_package``).

Public surface, mirroring the reference:
  QType, quant_dequant_float, quant_func            (ospnext/quant_cy_npu/base/QTensor.py)
  hif8_quant, hif8_quant_bf16                       (cusrc/npu_quant.cpp pybind entry points)
  HIF8Linear, _quant, make_linear                   (ospnext/modules/hif8_linear.py, osp_next.py)
plus the tensor-level HIP ops (absmax_scale, encode, fake_quant, decode,
linear_fwd), QuantState and PackedWeight.
"""
from . import _lib  # noqa: F401
from .quant import QType, quant_dequant_float, quant_func, hif8_quant, hif8_quant_bf16  # noqa: F401
from .hif8_linear import (  # noqa: F401
    HIF8Linear,
    PackedWeight,
    QuantState,
    _HIF8LinearFunction,
    _quant,
    absmax_scale,
    decode,
    encode,
    fake_quant,
    fake_quant_tiled,
    linear_fwd,
    linear_fwd_tiled,
    make_linear,
    quantize_activation,
    tile_weight_codes,
    tiled_rows,
)

__all__ = [
    "QType", "quant_dequant_float", "quant_func", "hif8_quant", "hif8_quant_bf16",
    "HIF8Linear", "PackedWeight", "QuantState", "_quant", "absmax_scale", "decode", "encode",
    "fake_quant", "linear_fwd", "make_linear", "quantize_activation", "fake_quant_tiled",
    "tile_weight_codes", "tiled_rows", "linear_fwd_tiled",
]
