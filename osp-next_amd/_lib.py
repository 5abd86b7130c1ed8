"""ctypes binding of libhif8_mi355x.so (the C ABI in include/hif8_mi355x.h).

The library is the only compute path: if it is missing or fails to load, every
entry point raises.  There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhif8_mi355x.so")

HIF8_OK = 0
ERR_SHAPE = -2    # HIF8_ERR_SHAPE: a shape the entry point does not take
DTYPE_BF16, DTYPE_F32, DTYPE_BF16_AS_F32 = 0, 1, 2
SEM_NPU, SEM_TORCH, SEM_TORCH_BF16, SEM_TORCH_F16 = 0, 1, 2, 3
# formats of a quantised activation held by the Python layer: bf16 x_q, or its 8-bit codes
A_BF16, A_CODES = 0, 1

# Every symbol the header declares, with (restype, argtypes).
_p, _i, _i64, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "hif8_strerror": (ctypes.c_char_p, [_i]),
    "hif8_state_size": (_sz, []),
    "hif8_state_init": (_i, [_p, _p]),
    "hif8_state_read": (_i, [_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_float), _p]),
    "hif8_absmax_scale": (_i, [_p, _i, _i64, _f, _p, _p]),
    "hif8_set_scale": (_i, [_p, _i, _f, _p]),
    "hif8_encode": (_i, [_p, _i, _i64, _p, _p, _p]),
    "hif8_fake_quant": (_i, [_p, _i, _i64, _p, _p, _i, _p]),
    "hif8_fake_quant_to_bf16": (_i, [_p, _i, _i64, _p, _p, _i, _p]),
    "hif8_decode": (_i, [_p, _i64, _p, _i, _p, _p]),
    "hif8_quant_f32": (_i, [_p, _p, _i64, _i, _p]),
    "hif8_quant_bf16": (_i, [_p, _p, _i64, _i, _p]),
    "hif8_quant_f16": (_i, [_p, _p, _i64, _i, _p]),
    "hif8_linear_fwd": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "hif8_transpose_codes": (_i, [_p, _i64, _i64, _p, _p]),
    "hif8_transpose_bf16": (_i, [_p, _i64, _i64, _i64, _p, _p]),
    "hif8_linear_split_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "hif8_linear_fwd_wq_split": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "hif8_linear_wgrad": (_i, [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "hif8_gemm_f32": (_i, [_p, _i, _p, _i, _p, _i, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "hif8_pad_2d": (_i, [_p, _i64, _i64, _p, _i64, _i64, _i, _p]),
    "hif8_linear_fwd_gelu_stat": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p, _p]),
    "hif8_gelu_absmax_scale": (_i, [_p, _i64, _f, _p, _p]),
    "hif8_gelu_fake_quant": (_i, [_p, _i64, _p, _f, _p, _i, _p]),
    "hif8_gelu_bf16": (_i, [_p, _p, _i64, _p]),
    "hif8_modln_amax": (_i, [_p, _p, _p, _i64, _i64, _i64, _f, _p, _f, _p, _p]),
    "hif8_linear_fwd_grouped": (_i, [_p, _p, ctypes.POINTER(_p), _p, ctypes.POINTER(_p), ctypes.POINTER(_i64), _i,
                                     _i64, _i64, _p]),
    "hif8_modln_fake_quant": (_i, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _i, _p, _p, _p]),
    "hif8_modln_quant_static": (_i, [_p, _p, _p, _i64, _i64, _i64, _f, _f, _i, _p, _p]),
    "hif8_ln_affine_amax": (_i, [_p, _p, _p, _i64, _i64, _f, _p, _f, _p, _p]),
    "hif8_gated_residual": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "hif8_gather_rows": (_i, [_p, _i64, _p, _i64, _i64, _p, _p]),
    "hif8_ln_affine_fake_quant": (_i, [_p, _p, _p, _i64, _i64, _p, _p, _i, _p, _p, _p]),
    "hif8_linear_fwd_wq": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "hif8_linear_fwd_wq_gelu_stat": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p, _p]),
    "hif8_linear_fwd_wq_grouped": (_i, [_p, _p, _p, ctypes.POINTER(_p), ctypes.POINTER(_i64), _i, _i64, _i64, _p]),
    "hif8_rms_norm_rope": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _p]),
    "hif8_rms_norm_rope_amax": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _f, _p, _p]),
    "hif8_rms_norm_rope_fake_quant": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _p, _i, _p, _p, _p]),
    "hif8_attention_fwd": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64), _p, _i64, _p, _f, _p, _i, _f, _p]),
}

_lib = None
_lock = threading.Lock()


class HIF8Error(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it is absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() "
                    "(make -C osp-next_amd/csrc).  There is no fallback path.")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != HIF8_OK:
        msg = load().hif8_strerror(status).decode()
        raise HIF8Error(f"{what} failed: {msg} (status {status})")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise TypeError(f"HiF8 kernels take bfloat16 or float32 tensors, got {dt}")


def state_size() -> int:
    return int(load().hif8_state_size())


def new_state(device: torch.device) -> torch.Tensor:
    """Allocate and initialise one per-tensor quantisation state on ``device``."""
    st = torch.empty(state_size(), dtype=torch.uint8, device=device)
    check(load().hif8_state_init(ptr(st), stream_ptr(device)), "hif8_state_init")
    return st


def require_gpu_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the HiF8 path has no CPU route)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
