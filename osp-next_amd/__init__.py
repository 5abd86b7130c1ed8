"""MI355X-native HiF8 fake-quant linear path for OSP-Next.

Imported under the module name ``ospnext_amd`` (the directory name is not a
Python identifier; see ``__graft_entry__.load_package``).

Public surface, mirroring the reference:
  QType, quant_dequant_float, quant_func,
  quant_slide_window                                (ospnext/quant_cy_npu/base/QTensor.py)
  hif8_quant, hif8_quant_bf16                       (cusrc/npu_quant.cpp pybind entry points)
  HIF8Linear, _quant, make_linear                   (ospnext/modules/hif8_linear.py, osp_next.py)
  hif8_attention_with_mask, _HIF8QKVQuantFunction   (ospnext/modules/hif8_attention.py)
  QLinear, replace_linear                           (quant_cy_npu/layers/QLinear.py, utils/utils.py)
  WanLayerNorm                                      (ospnext/modules/want2v.py)
  OSPNextAttentionBlock, OSPNextBlocks (dit)        (ospnext/modules/osp_next.py, the call sites)
plus the tensor-level HIP ops (absmax_scale, encode, fake_quant, decode,
linear_fwd), QuantState and PackedWeight.
"""
from . import _lib  # noqa: F401
from .quant import (QType, QuantSlideWindow, quant_dequant_float, quant_func, quant_slide_window,  # noqa: F401
                    hif8_quant, hif8_quant_bf16)
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
    fake_quant_to_bf16,
    linear_fwd,
    make_linear,
    quantize_activation,
    transpose_codes,
    linear_dgrad,
    dgrad_fused_ok,
    fused_shape_ok,
    linear_any,
    linear_fwd_gelu_stat,
    gelu_absmax_scale,
    gelu_fake_quant,
    gelu_bf16,
    GroupedWeight,
    grouped_ok,
    linear_fwd_grouped,
    linear_fwd_wq,
    linear_wgrad,
    linear_fwd_wq_split,
    transpose_bf16,
    wgrad_ok,
    pad_2d,
    gemm_f32,
    dense_linear,
    dense_mm,
)
from .ffn import HIF8FFN  # noqa: F401
from . import dit  # noqa: F401
from .dit import OSPNextAttentionBlock, OSPNextBlocks  # noqa: F401
from .norm import (WanLayerNorm, affine_norm_quant, grouped_weight, modulate, modulated_norm_quant,  # noqa: F401
                   modulated_norm_quant_static, qkv_from_modulated_norm)
from .hif8_attention import (  # noqa: F401
    _HIF8QKVQuantFunction,
    attention_fwd,
    attention_fwd_ok,
    attention_with_mask,
    hif8_attention_with_mask,
    key_list,
    scaled_dot_product_attention_with_mask,
)
from .qlinear import (  # noqa: F401
    LinearForward,
    LinearForwardFast,
    QLinear,
    load_packed,
    pack_state_dict,
    packed_from_codes,
    replace_linear,
    save_packed,
)

__all__ = [
    "QType", "quant_dequant_float", "quant_func", "quant_slide_window", "QuantSlideWindow", "hif8_quant",
    "hif8_quant_bf16",
    "HIF8Linear", "PackedWeight", "QuantState", "_quant", "absmax_scale", "decode", "encode",
    "fake_quant", "fake_quant_to_bf16", "linear_fwd", "make_linear", "quantize_activation", "transpose_codes",
    "linear_dgrad", "dgrad_fused_ok",
    "_HIF8QKVQuantFunction", "attention_with_mask", "hif8_attention_with_mask",
    "scaled_dot_product_attention_with_mask", "LinearForward", "LinearForwardFast", "QLinear", "replace_linear",
    "save_packed", "load_packed", "pack_state_dict", "packed_from_codes", "fused_shape_ok", "linear_any",
    "linear_fwd_gelu_stat", "gelu_absmax_scale", "gelu_fake_quant", "gelu_bf16", "HIF8FFN", "WanLayerNorm", "modulate", "modulated_norm_quant", "affine_norm_quant",
    "qkv_from_modulated_norm", "modulated_norm_quant_static", "GroupedWeight", "grouped_ok", "linear_fwd_grouped", "grouped_weight",
    "attention_fwd", "attention_fwd_ok", "key_list",
    "dit", "OSPNextAttentionBlock", "OSPNextBlocks", "linear_fwd_wq", "linear_fwd_wq_split", "linear_wgrad", "transpose_bf16", "wgrad_ok",
    "pad_2d", "gemm_f32", "dense_linear", "dense_mm",
]
