"""HiF8 fake-quant linear layer, mirroring ``ospnext/modules/hif8_linear.py``.

Forward (hif8_linear.py:68-86)::

    x_q = qdq(x * s_x) / s_x,  s_x = scale_max_forward / max|x|
    w_q = qdq(W * s_w) / s_w,  s_w = scale_max_forward / max|W|
    y   = x_q @ w_q.T + bias

Here ``x_q`` comes from one amax pass and one quantise pass (HIP kernels), ``W``
is held as packed 8-bit HiF8 codes plus a per-tensor state, and the product is
the fused dequant-GEMM ``hif8_linear_fwd``.  The dequantised operands are
bit-identical to the reference's; only the fp32 accumulation order differs.

Backward (hif8_linear.py:88-111) quantises the incoming gradient with
``scale_max_backward`` through the same HIP kernels.  dgrad ``grad_q @ w_q``
runs on the forward's GEMM against the transposed weight codes, and wgrad
``grad_q^T @ x_q`` on the decode-free GEMM reading both operands token-major,
when the operands are bf16 (the reference's autocast case); an fp32 operand takes
the library's fp32 GEMM (``hif8_gemm_f32``) on the same dequantised operands.
Shapes outside the MFMA tiles (in_features % 64, out_features % 8, or the dgrad's
reduction % 64) run those GEMMs on zero-padded operands (``hif8_pad_2d``).  No
product runs on a vendor or torch GEMM.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from . import _lib


# --------------------------------------------------------------------- state


class QuantState:
    """Device-side per-tensor quantisation state (amax, scale, decode tables)."""

    def __init__(self, device: torch.device):
        self.device = torch.device(device)
        self.buf = _lib.new_state(self.device)

    @property
    def ptr(self) -> int:
        return self.buf.data_ptr()

    def scale(self) -> Tensor:
        """The scale as a 0-dim fp32 device tensor (a copy; no host sync)."""
        return self.buf[12:16].view(torch.float32).reshape(()).clone()

    def read(self) -> Tuple[int, float]:
        """(amax bits, scale) on the host (synchronises the stream)."""
        import ctypes
        a = ctypes.c_uint32()
        s = ctypes.c_float()
        _lib.check(_lib.load().hif8_state_read(self.ptr, ctypes.byref(a), ctypes.byref(s),
                                               _lib.stream_ptr(self.device)), "hif8_state_read")
        return int(a.value), float(s.value)

    def lut_bf16(self) -> Tensor:
        """The 256-entry bf16 decode table x_q(code) (a device view)."""
        return self.buf[32:544].view(torch.bfloat16)


def _aligned(t: Tensor) -> Tensor:
    """The kernels use 128-bit accesses: realign offset views with one copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def pad_2d(t: Tensor, rows: int, cols: int) -> Tensor:
    """t [R, C] into a new [rows, cols] tensor with zeros outside t, or cropped where smaller
    (hif8_pad_2d)."""
    _lib.require_gpu_tensor(t, "t")
    if t.dim() != 2:
        raise ValueError("pad_2d takes a 2-D tensor")
    R_, C_ = t.shape
    out = torch.empty((rows, cols), dtype=t.dtype, device=t.device)
    if R_ == 0 or C_ == 0:
        return out.zero_()
    _lib.check(_lib.load().hif8_pad_2d(t.data_ptr(), R_, C_, out.data_ptr(), rows, cols, t.element_size(),
                                       _lib.stream_ptr(t.device)), "hif8_pad_2d")
    return out


def gemm_f32(a: Tensor, b: Tensor, M: int, N: int, K: int, a_strides, b_strides,
             out_dtype: torch.dtype = torch.float32) -> Tensor:
    """c[M, N] = sum_k a[m, k] b[k, n] with fp32 accumulation on bf16 or fp32 operands given by
    their element strides (m, k) and (k, n) (hif8_gemm_f32): the backward's products of a layer
    computing in fp32."""
    if not (a.is_cuda and b.is_cuda):
        raise ValueError("gemm_f32 takes GPU tensors (the HiF8 path has no CPU route)")
    c = torch.empty((M, N), dtype=out_dtype, device=a.device)
    _lib.check(_lib.load().hif8_gemm_f32(a.data_ptr(), _lib.dtype_code(a.dtype), b.data_ptr(),
                                         _lib.dtype_code(b.dtype), c.data_ptr(), _lib.dtype_code(out_dtype), M, N, K,
                                         int(a_strides[0]), int(a_strides[1]), int(b_strides[0]), int(b_strides[1]),
                                         _lib.stream_ptr(a.device)), "hif8_gemm_f32")
    return c


def _dtype_arg(x: Tensor, as_f32: bool) -> int:
    """The library's dtype code for x; ``as_f32`` quantises a bf16 x as x.float() would be."""
    if as_f32:
        if x.dtype != torch.bfloat16:
            raise TypeError("as_f32 applies to a bfloat16 tensor")
        return _lib.DTYPE_BF16_AS_F32
    return _lib.dtype_code(x.dtype)


def absmax_scale(x: Tensor, scale_max: float, state: QuantState, as_f32: bool = False) -> QuantState:
    """hif8_linear.py:45-46 into ``state`` (amax, scale and decode tables).  ``as_f32``: the
    fp32 rule for a bf16 x, as ``_quant(x.float())`` computes it."""
    _lib.require_gpu_tensor(x, "x")
    x = _aligned(x)
    if x.numel() == 0:
        raise ValueError("amax of an empty tensor")
    _lib.check(_lib.load().hif8_absmax_scale(x.data_ptr(), _dtype_arg(x, as_f32), x.numel(),
                                             float(scale_max), state.ptr, _lib.stream_ptr(x.device)),
               "hif8_absmax_scale")
    return state


def encode(x: Tensor, state: QuantState, as_f32: bool = False) -> Tensor:
    """HiF8 codes of qdq(x * scale) (NPU semantics), one byte per element."""
    _lib.require_gpu_tensor(x, "x")
    x = _aligned(x)
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    if x.numel():
        _lib.check(_lib.load().hif8_encode(x.data_ptr(), _dtype_arg(x, as_f32), x.numel(), state.ptr,
                                           codes.data_ptr(), _lib.stream_ptr(x.device)), "hif8_encode")
    return codes


def fake_quant_to_bf16(x: Tensor, state: QuantState, semantics: int = _lib.SEM_NPU, as_f32: bool = False) -> Tensor:
    """bf16(x_q): the GEMM operand F.linear's bf16 autocast makes of ``_quant(x)[0]``
    (hif8_linear.py:86); for an fp32 x (or ``as_f32``) the fp32 x_q is never stored."""
    _lib.require_gpu_tensor(x, "x")
    x = _aligned(x)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    if x.numel():
        _lib.check(_lib.load().hif8_fake_quant_to_bf16(x.data_ptr(), _dtype_arg(x, as_f32), x.numel(), state.ptr,
                                                       y.data_ptr(), semantics, _lib.stream_ptr(x.device)),
                   "hif8_fake_quant_to_bf16")
    return y


def fake_quant(x: Tensor, state: QuantState, semantics: int = _lib.SEM_NPU) -> Tensor:
    """qdq(x * scale) / scale in x's dtype (hif8_linear.py:47-48)."""
    _lib.require_gpu_tensor(x, "x")
    x = _aligned(x)
    y = torch.empty_like(x)
    if x.numel():
        _lib.check(_lib.load().hif8_fake_quant(x.data_ptr(), _lib.dtype_code(x.dtype), x.numel(), state.ptr,
                                               y.data_ptr(), semantics, _lib.stream_ptr(x.device)),
                   "hif8_fake_quant")
    return y


def decode(codes: Tensor, state: QuantState, dtype: torch.dtype = torch.bfloat16, out: Optional[Tensor] = None) -> Tensor:
    """x_q = decode(code) / scale in ``dtype`` (into ``out`` when given: contiguous, 16-byte aligned)."""
    _lib.require_gpu_tensor(codes, "codes")
    codes = _aligned(codes)
    if out is None:
        y = torch.empty(codes.shape, dtype=dtype, device=codes.device)
    else:
        if out.dtype != dtype or out.numel() != codes.numel() or not out.is_contiguous() or out.data_ptr() % 16:
            raise ValueError("decode: out must be a contiguous, 16-byte aligned tensor of the codes' size and dtype")
        y = out
    if codes.numel():
        _lib.check(_lib.load().hif8_decode(codes.data_ptr(), codes.numel(), state.ptr, _lib.dtype_code(dtype),
                                           y.data_ptr(), _lib.stream_ptr(codes.device)), "hif8_decode")
    return y


def _quant(x: Tensor, scale_max: float, semantics: int = _lib.SEM_NPU) -> Tuple[Tensor, Tensor]:
    """hif8_linear.py:42-50: returns ``(x_q, scale)``, scale a 0-dim tensor of x's dtype."""
    xc = x.contiguous()
    st = absmax_scale(xc, scale_max, QuantState(xc.device))
    xq = fake_quant(xc, st, semantics)
    return xq.view(x.shape), st.scale().to(x.dtype)


# ------------------------------------------------------------ packed weight


class PackedWeight:
    """8-bit HiF8 weight storage: codes [N, K] (uint8) + the weight's state.

    Halves the bytes of a bf16 weight; ``dequantize()`` gives the reference's
    ``w_q`` exactly.
    """

    def __init__(self, weight: Tensor, scale_max: float):
        w = weight.detach().contiguous()
        self.shape = tuple(w.shape)
        self.src_dtype = w.dtype
        self.state = absmax_scale(w, scale_max, QuantState(w.device))
        self.codes = encode(w, self.state)
        self.scale_max = float(scale_max)
        self.key = (w.data_ptr(), weight._version, w.device)
        self._codes_t: Optional[Tensor] = None
        self._padded: dict = {}

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> Tensor:
        return decode(self.codes, self.state, dtype or self.src_dtype)

    def codes_t(self) -> Tensor:
        """The codes transposed, [K, N] (built once): the dgrad weight operand."""
        if self._codes_t is None:
            self._codes_t = transpose_codes(self.codes)
        return self._codes_t

    def codes_t_padded(self, k_rows: int, n_cols: int) -> Tensor:
        """The transposed codes zero-padded to [k_rows, n_cols] (built once per shape)."""
        key = ("t", k_rows, n_cols)
        if key not in self._padded:
            self._padded[key] = pad_2d(self.codes_t(), k_rows, n_cols)
        return self._padded[key]

    def padded(self, n_rows: int, k_cols: int) -> "PackedWeight":
        """The same weight with its codes zero-padded to [n_rows, k_cols] (zero codes decode to
        0), sharing the state: the operand of a GEMM over zero-padded shapes (built once)."""
        key = (n_rows, k_cols)
        p = self._padded.get(key)
        if p is None:
            p = object.__new__(PackedWeight)
            p.shape = (n_rows, k_cols)
            p.src_dtype, p.state, p.scale_max, p.key = self.src_dtype, self.state, self.scale_max, self.key
            p.codes = pad_2d(self.codes, n_rows, k_cols)
            p._codes_t, p._padded = None, {}
            self._padded[key] = p
        return p


def transpose_codes(codes: Tensor) -> Tensor:
    """[R, C] uint8 -> [C, R] (hif8_transpose_codes)."""
    _lib.require_gpu_tensor(codes, "codes")
    R, C = codes.shape
    out = torch.empty((C, R), dtype=torch.uint8, device=codes.device)
    _lib.check(_lib.load().hif8_transpose_codes(codes.data_ptr(), R, C, out.data_ptr(), _lib.stream_ptr(codes.device)),
               "hif8_transpose_codes")
    return out


def dgrad_fused_ok(grad_q: Tensor, w: "PackedWeight") -> bool:
    """Dtypes the MFMA dgrad takes: bf16 gradient and weight (other shapes than the tiles'
    are zero-padded by ``linear_dgrad``)."""
    N, K = w.shape
    return grad_q.dtype == torch.bfloat16 and w.src_dtype == torch.bfloat16 and _round_up(N, 64) < (1 << 22)


def linear_dgrad(grad_q2: Tensor, w: "PackedWeight") -> Tensor:
    """grad_q [M, N] @ w_q [N, K] -> [M, K] bf16 (hif8_linear.py:97): the forward GEMM with the
    transposed weight codes [K, N] as its weight, on the route the forward takes at this M (the
    fused GEMM, or the transposed codes decoded once and the decode-free GEMM with its last
    partial wave of tiles split over k ranges).  The reduction (N) is padded to a multiple of 64
    and the output features (K) to a multiple of 8 with zeros where they are not."""
    M, N = grad_q2.shape
    K = w.shape[1]
    Np, Kp = _round_up(N, 64), _round_up(K, 8)
    g = _aligned(grad_q2.contiguous())
    if Np != N:
        g = pad_2d(g, M, Np)
    codes_t = w.codes_t() if (Np, Kp) == (N, K) else w.codes_t_padded(Kp, Np)
    if decode_once(M, Np):
        y = linear_fwd_wq_split(g, decode(codes_t, w.state, torch.bfloat16))
    else:
        y = torch.empty((M, Kp), dtype=torch.bfloat16, device=g.device)
        _lib.check(_lib.load().hif8_linear_fwd(g.data_ptr(), codes_t.data_ptr(), w.state.ptr, None, y.data_ptr(),
                                               M, Kp, Np, _lib.stream_ptr(g.device)), "hif8_linear_fwd (dgrad)")
    return y if Kp == K else pad_2d(y, M, K)


def transpose_bf16(x2: Tensor, rows_pad: Optional[int] = None) -> Tensor:
    """[R, C] bf16 -> [C, rows_pad] bf16 with zeros past R (hif8_transpose_bf16)."""
    _lib.require_gpu_tensor(x2, "x")
    if x2.dtype != torch.bfloat16 or x2.dim() != 2:
        raise ValueError("transpose_bf16 takes a 2-D bfloat16 tensor")
    R, C = x2.shape
    rp = R if rows_pad is None else int(rows_pad)
    out = torch.empty((C, rp), dtype=torch.bfloat16, device=x2.device)
    _lib.check(_lib.load().hif8_transpose_bf16(x2.data_ptr(), R, C, rp, out.data_ptr(), _lib.stream_ptr(x2.device)),
               "hif8_transpose_bf16")
    return out


def wgrad_ok(grad_q2: Tensor, x_q2: Tensor) -> bool:
    """Operands linear_wgrad takes: bf16, the same tokens (features that are not multiples of 8
    are zero-padded by linear_wgrad)."""
    return (grad_q2.dtype == torch.bfloat16 and x_q2.dtype == torch.bfloat16
            and grad_q2.shape[0] == x_q2.shape[0] and grad_q2.shape[0] > 0)


def linear_wgrad(grad_q2: Tensor, x_q2: Tensor, split_tail: bool = True, transposed: bool = False) -> Tensor:
    """grad_weight = grad_q^T [N, M] @ x_q [M, K] -> [N, K] bf16 (hif8_linear.py:100-105, fp32
    accumulation): hif8_linear_wgrad, the decode-free GEMM reading both operands token-major as
    they are, with the last partial wave of tiles split over token ranges unless ``split_tail`` is
    False.  Operands too large for its 32-bit offsets (or ``transposed=True``) take the transposed
    route: both operands transposed with the tokens zero-padded to a multiple of 64, then the
    row-major GEMM over the padded tokens (the zeros add nothing)."""
    M, N = grad_q2.shape
    K = x_q2.shape[1]
    Np, Kp = _round_up(N, 8), _round_up(K, 8)
    if (Np, Kp) != (N, K):
        g = pad_2d(grad_q2.contiguous(), M, Np) if Np != N else grad_q2
        x = pad_2d(x_q2.contiguous(), M, Kp) if Kp != K else x_q2
        return pad_2d(linear_wgrad(g, x, split_tail, transposed), N, K)
    g = _aligned(grad_q2.contiguous())
    x = _aligned(x_q2.contiguous())
    L = _lib.load()
    if not transposed:
        dw = torch.empty((N, K), dtype=torch.bfloat16, device=g.device)
        nbytes = int(L.hif8_linear_split_workspace_bytes(N, K, M)) if split_tail else 0
        ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=g.device) if nbytes > 0 else None
        rc = L.hif8_linear_wgrad(g.data_ptr(), x.data_ptr(), dw.data_ptr(), M, N, K,
                                 ws.data_ptr() if ws is not None else None, nbytes, _lib.stream_ptr(g.device))
        if rc != _lib.ERR_SHAPE:
            _lib.check(rc, "hif8_linear_wgrad")
            return dw
    Mp = (M + 63) // 64 * 64
    g_t = transpose_bf16(g, Mp)
    x_t = transpose_bf16(x, Mp)
    return linear_fwd_wq_split(g_t, x_t, split_tail=split_tail)


def linear_fwd_wq_split(a: Tensor, w_q: Tensor, bias: Optional[Tensor] = None, split_tail: bool = True) -> Tensor:
    """hif8_linear_fwd_wq_split: y = a @ w_q^T (+ bias), bf16, with the tail of the tile grid split
    over k ranges into a transient fp32 workspace (hif8_linear_split_workspace_bytes) unless
    ``split_tail`` is False."""
    M, K = a.shape
    N = w_q.shape[0]
    if w_q.shape[1] != K or w_q.dtype != torch.bfloat16 or a.dtype != torch.bfloat16:
        raise ValueError("linear_fwd_wq_split takes bf16 a [M, K] and bf16 w_q [N, K]")
    L = _lib.load()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    b_ptr = None
    if bias is not None:
        bias = bias.detach().to(torch.bfloat16).contiguous()
        b_ptr = bias.data_ptr()
    nbytes = int(L.hif8_linear_split_workspace_bytes(M, N, K)) if split_tail else 0
    ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=a.device) if nbytes > 0 else None
    _lib.check(L.hif8_linear_fwd_wq_split(a.data_ptr(), w_q.data_ptr(), b_ptr, y.data_ptr(), M, N, K,
                                          ws.data_ptr() if ws is not None else None, nbytes,
                                          _lib.stream_ptr(a.device)), "hif8_linear_fwd_wq_split")
    return y


# GEMM route for bf16 activations: "fused" decodes the packed weight inside the GEMM (each
# element once per 256-row tile of x), "decode_once" decodes it into a bf16 buffer per call and
# runs the decode-free twin (hif8_linear_fwd_wq), "auto" takes decode_once from
# DECODE_ONCE_MIN_ROWS rows up, or from DECODE_ONCE_MIN_ROWS_SHORT_K rows up when the reduction
# depth K is at most SHORT_K.  Both issue the same MFMA products in the same order: the same bits.
# Measured fused / decode-once times (decode included; alternating A/B on one box): K = 1536 (the
# 1.3B q/k/v/o and FFN-up) 0.82-0.98 at 4096-16384 rows, 0.99-1.01 at 32760 (config 2), 1.02-1.03
# from 49152; K = 5120 or more 0.96-1.01 at 4096-8192 rows, 1.01-1.05 from 16384.
GEMM_ROUTE = "auto"
DECODE_ONCE_MIN_ROWS = 8192
DECODE_ONCE_MIN_ROWS_SHORT_K = 24576
SHORT_K = 2048


def decode_once(M: int, K: int) -> bool:
    """Whether a GEMM of M rows and reduction depth K takes the decode-once route."""
    if GEMM_ROUTE not in ("auto", "fused", "decode_once"):
        raise ValueError(f"GEMM_ROUTE must be auto, fused or decode_once, not {GEMM_ROUTE!r}")
    if GEMM_ROUTE != "auto":
        return GEMM_ROUTE == "decode_once"
    return M >= (DECODE_ONCE_MIN_ROWS_SHORT_K if K <= SHORT_K else DECODE_ONCE_MIN_ROWS)


def linear_fwd_wq(a: Tensor, w_q: Tensor, bias: Optional[Tensor], y_state: Optional[QuantState] = None,
                  scale_max: float = 15.0) -> Tensor:
    """hif8_linear_fwd_wq[_gelu_stat]: y = x_q @ w_q^T + bias with w_q the dequantised bf16 weight
    [N, K] (``PackedWeight.dequantize()``); with ``y_state`` the GELU-statistic epilogue."""
    M, K = a.shape
    N = w_q.shape[0]
    if w_q.shape[1] != K or w_q.dtype != torch.bfloat16 or a.dtype != torch.bfloat16:
        raise ValueError("linear_fwd_wq takes bf16 x_q [M, K] and bf16 w_q [N, K]")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    b_ptr = None
    if bias is not None:
        bias = bias.detach().to(torch.bfloat16).contiguous()
        b_ptr = bias.data_ptr()
    L = _lib.load()
    s = _lib.stream_ptr(a.device)
    if y_state is None:
        _lib.check(L.hif8_linear_fwd_wq(a.data_ptr(), w_q.data_ptr(), b_ptr, y.data_ptr(), M, N, K, s),
                   "hif8_linear_fwd_wq")
    else:
        _lib.check(L.hif8_linear_fwd_wq_gelu_stat(a.data_ptr(), w_q.data_ptr(), b_ptr, y.data_ptr(), M, N, K,
                                                  float(scale_max), y_state.ptr, s), "hif8_linear_fwd_wq_gelu_stat")
    return y


def _autocast_bf16() -> bool:
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def dense_linear(x2: Tensor, w: Tensor, bias: Optional[Tensor]) -> Tensor:
    """``F.linear(x2, w, bias)`` for already dequantised operands x2 [M, K], w [N, K] on the
    library's GEMMs: in bf16 (the autocast case, or bf16 operands) the decode-free MFMA GEMM on
    zero-padded shapes where needed, output bf16; otherwise the fp32 GEMM in the operands' result
    dtype."""
    M, K = x2.shape
    N = w.shape[0]
    if _autocast_bf16() or (x2.dtype == torch.bfloat16 and w.dtype == torch.bfloat16):
        a = _aligned(x2.to(torch.bfloat16).contiguous())
        wq = _aligned(w.to(torch.bfloat16).contiguous())
        Np, Kp = _round_up(N, 8), _round_up(K, 64)
        b = None
        if bias is not None:
            b = bias.detach().to(torch.bfloat16).reshape(1, N).contiguous()
            b = pad_2d(b, 1, Np).view(Np) if Np != N else b.view(N)
        if Kp != K:
            a = pad_2d(a, M, Kp)
        if (Np, Kp) != (N, K):
            wq = pad_2d(wq, Np, Kp)
        y = linear_fwd_wq(a, wq, b)
        return y if Np == N else pad_2d(y, M, N)
    ct = torch.promote_types(x2.dtype, w.dtype)
    y = gemm_f32(x2.contiguous(), w.contiguous(), M, N, K, (K, 1), (1, K), out_dtype=ct)
    return y if bias is None else y + bias.to(ct)


def dense_mm(a: Tensor, b: Tensor) -> Tensor:
    """``a @ b`` for 2-D a [M, R], b [R, N] on the library's GEMMs: in bf16 (autocast or bf16
    operands) the token-major MFMA GEMM on a^T (one transpose) and b, output bf16; otherwise the
    fp32 GEMM on the strided operands."""
    M, R = a.shape
    N = b.shape[1]
    if _autocast_bf16() or (a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16):
        a_t = transpose_bf16(_aligned(a.to(torch.bfloat16).contiguous()))        # [R, M]
        return linear_wgrad(a_t, _aligned(b.to(torch.bfloat16).contiguous()))   # a_t^T @ b
    ct = torch.promote_types(a.dtype, b.dtype)
    return gemm_f32(a, b, M, N, R, (a.stride(0), a.stride(1)), (b.stride(0), b.stride(1)), out_dtype=ct)


def fused_shape_ok(N: int, K: int) -> bool:
    """Shapes hif8_linear_fwd takes: in_features K % 64 == 0, out_features N % 8 == 0."""
    return K % 64 == 0 and N % 8 == 0 and K < (1 << 22)


def linear_any(a: Tensor, a_fmt: int, a_state: Optional[QuantState], w: PackedWeight,
               bias: Optional[Tensor]) -> Tensor:
    """y = x_q @ w_q^T + bias in bf16 for any shape: the GEMM routes of linear_fwd, on operands
    zero-padded to in_features % 64 == 0 and out_features % 8 == 0 where the layer's are not (the
    zeros add nothing to the sums; the output is cropped back)."""
    N, K = w.shape
    if fused_shape_ok(N, K):
        return linear_fwd(a, a_fmt, a_state, w, bias)
    M = a.shape[0]
    Np, Kp = _round_up(N, 8), _round_up(K, 64)
    if not fused_shape_ok(Np, Kp):
        raise ValueError(f"in_features {K} is beyond the GEMMs' k range")
    xq = a if a_fmt == _lib.A_BF16 else decode(a, a_state, torch.bfloat16)
    xq = pad_2d(_aligned(xq.contiguous()), M, Kp) if Kp != K else xq
    bp = None
    if bias is not None:
        bp = bias.detach().to(torch.bfloat16).reshape(1, N).contiguous()
        bp = pad_2d(bp, 1, Np).view(Np) if Np != N else bp.view(N)
    y = linear_fwd(xq, _lib.A_BF16, None, w.padded(Np, Kp), bp)
    return y if Np == N else pad_2d(y, M, N)


def linear_fwd(a: Tensor, a_fmt: int, a_state: Optional[QuantState], w: PackedWeight,
               bias: Optional[Tensor]) -> Tensor:
    """y[M,N] = x_q[M,K] @ w_q[N,K]^T + bias, bf16 out: hif8_linear_fwd (the fused dequant-GEMM),
    or where decode_once(M, K) the weight decoded once and hif8_linear_fwd_wq.  An
    activation given as codes (``a_fmt`` A_CODES, with its ``a_state``) is decoded to its bf16
    x_q first (bit-exact: decode(encode(x)) is the fake quant of x)."""
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"in_features mismatch: x has {K}, weight has {w.shape[1]}")
    if a_fmt == _lib.A_CODES:
        if a_state is None:
            raise ValueError("codes activations need their quantisation state")
        a = decode(a, a_state, torch.bfloat16)
    elif a_fmt != _lib.A_BF16:
        raise ValueError(f"unknown activation format {a_fmt}")
    if decode_once(M, K):
        return linear_fwd_wq(a, w.dequantize(torch.bfloat16), bias)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    b_ptr = None
    if bias is not None:
        bias = bias.detach().to(torch.bfloat16).contiguous()
        b_ptr = bias.data_ptr()
    _lib.check(_lib.load().hif8_linear_fwd(a.data_ptr(), w.codes.data_ptr(), w.state.ptr, b_ptr, y.data_ptr(),
                                           M, N, K, _lib.stream_ptr(a.device)), "hif8_linear_fwd")
    return y


MAX_GROUPS = 8


def grouped_ok(packs: "List[PackedWeight]") -> bool:
    """Weights hif8_linear_fwd_grouped takes together: same in_features (K % 64 == 0), every
    out_features a multiple of 256 except the last (a multiple of 8), at most 8 of them."""
    if not 1 <= len(packs) <= MAX_GROUPS:
        return False
    K = packs[0].shape[1]
    if any(p.shape[1] != K for p in packs) or not fused_shape_ok(packs[-1].shape[0], K):
        return False
    return all(p.shape[0] % 256 == 0 for p in packs[:-1])


class GroupedWeight:
    """The weights of several HIF8Linear layers that read the same input, concatenated along the
    output features (codes, and biases with zeros for a layer without one) for one launch of
    hif8_linear_fwd_grouped.  Built from the layers' packed weights; ``key`` identifies them."""

    def __init__(self, packs: "List[PackedWeight]", biases: "List[Optional[Tensor]]", key=None):
        if not grouped_ok(packs):
            raise ValueError("weights do not fit one grouped launch (see grouped_ok)")
        self.packs = list(packs)
        self.ns = [p.shape[0] for p in packs]
        self.K = packs[0].shape[1]
        self.codes = torch.cat([p.codes for p in packs], 0).contiguous()
        if any(b is not None for b in biases):
            dev = self.codes.device
            self.bias = torch.cat([b.detach().to(torch.bfloat16).reshape(-1) if b is not None
                                   else torch.zeros(n, dtype=torch.bfloat16, device=dev)
                                   for b, n in zip(biases, self.ns)]).contiguous()
        else:
            self.bias = None
        self.key = key


def linear_fwd_grouped(a: Tensor, gw: GroupedWeight) -> "List[Tensor]":
    """hif8_linear_fwd_grouped: ``[a @ w_q_i^T + b_i for each group]`` in one launch, each equal
    bit for bit to linear_fwd of that weight alone.  ``a`` is the bf16 x_q [M, K]."""
    M, K = a.shape
    if K != gw.K:
        raise ValueError(f"in_features mismatch: x has {K}, weights have {gw.K}")
    if a.dtype != torch.bfloat16:
        raise TypeError("the grouped GEMM takes the bf16 x_q")
    ys = [torch.empty((M, n), dtype=torch.bfloat16, device=a.device) for n in gw.ns]
    g = len(ys)
    outs = (ctypes.c_void_p * g)(*[y.data_ptr() for y in ys])
    ns = (ctypes.c_int64 * g)(*gw.ns)
    b_ptr = gw.bias.data_ptr() if gw.bias is not None else None
    if decode_once(M, K):
        w_q = torch.empty((sum(gw.ns), K), dtype=torch.bfloat16, device=a.device)
        row = 0
        for p, n in zip(gw.packs, gw.ns):
            decode(p.codes, p.state, torch.bfloat16, out=w_q[row:row + n])
            row += n
        _lib.check(_lib.load().hif8_linear_fwd_wq_grouped(a.data_ptr(), w_q.data_ptr(), b_ptr, outs, ns, g, M, K,
                                                          _lib.stream_ptr(a.device)), "hif8_linear_fwd_wq_grouped")
        return ys
    states = (ctypes.c_void_p * g)(*[p.state.ptr for p in gw.packs])
    _lib.check(_lib.load().hif8_linear_fwd_grouped(a.data_ptr(), gw.codes.data_ptr(), states, b_ptr, outs, ns,
                                                   g, M, K, _lib.stream_ptr(a.device)), "hif8_linear_fwd_grouped")
    return ys


def linear_fwd_gelu_stat(a: Tensor, w: PackedWeight, bias: Optional[Tensor], y_state: QuantState,
                         scale_max: float) -> Tensor:
    """hif8_linear_fwd[_wq]_gelu_stat: y = x_q @ w_q^T + bias in bf16 (bf16 x_q), with the GELU
    statistic of y in ``y_state``: amax|GELU(y)| and its scale for ``scale_max`` when max y settles
    it, else the state is pending.  ``gelu_fake_quant(y, y_state, scale_max)`` then gives the next
    linear's x_q of GELU(y)."""
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"in_features mismatch: x has {K}, weight has {w.shape[1]}")
    if a.dtype != torch.bfloat16:
        raise TypeError("the GELU-statistic epilogue takes bf16 activations")
    if decode_once(M, K):
        return linear_fwd_wq(a, w.dequantize(torch.bfloat16), bias, y_state, scale_max)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    b_ptr = None
    if bias is not None:
        bias = bias.detach().to(torch.bfloat16).contiguous()
        b_ptr = bias.data_ptr()
    _lib.check(_lib.load().hif8_linear_fwd_gelu_stat(a.data_ptr(), w.codes.data_ptr(), w.state.ptr, b_ptr,
                                                     y.data_ptr(), M, N, K, float(scale_max), y_state.ptr,
                                                     _lib.stream_ptr(a.device)), "hif8_linear_fwd_gelu_stat")
    return y


def gelu_absmax_scale(y: Tensor, scale_max: float, state: QuantState) -> QuantState:
    """amax|GELU(y)| and its scale into ``state`` (hif8_gelu_absmax_scale) for a bf16 y."""
    _lib.require_gpu_tensor(y, "y")
    if y.dtype != torch.bfloat16:
        raise TypeError("gelu_absmax_scale takes a bfloat16 tensor")
    y = _aligned(y)
    _lib.check(_lib.load().hif8_gelu_absmax_scale(y.data_ptr(), y.numel(), float(scale_max), state.ptr,
                                                  _lib.stream_ptr(y.device)), "hif8_gelu_absmax_scale")
    return state


def gelu_bf16(y: Tensor) -> Tensor:
    """GELU(y) of a bf16 tensor as the library's GELU quantisation applies it (hif8_gelu_bf16):
    nn.GELU(approximate="tanh") on bf16, ``osp_next.py:875``."""
    _lib.require_gpu_tensor(y, "y")
    if y.dtype != torch.bfloat16:
        raise TypeError("gelu_bf16 takes a bfloat16 tensor")
    y = _aligned(y)
    out = torch.empty_like(y)
    if y.numel():
        _lib.check(_lib.load().hif8_gelu_bf16(y.data_ptr(), out.data_ptr(), y.numel(), _lib.stream_ptr(y.device)),
                   "hif8_gelu_bf16")
    return out


def gelu_fake_quant(y: Tensor, state: QuantState, scale_max: float = 15.0, semantics: int = _lib.SEM_NPU) -> Tensor:
    """``_quant(GELU(y))[0]`` in bf16 without writing GELU(y) (hif8_gelu_fake_quant), with the state
    from ``linear_fwd_gelu_stat`` or ``gelu_absmax_scale`` (a pending state is completed first)."""
    _lib.require_gpu_tensor(y, "y")
    if y.dtype != torch.bfloat16:
        raise TypeError("gelu_fake_quant takes a bfloat16 tensor")
    y = _aligned(y)
    out = torch.empty_like(y)
    if y.numel():
        _lib.check(_lib.load().hif8_gelu_fake_quant(y.data_ptr(), y.numel(), state.ptr, float(scale_max),
                                                    out.data_ptr(), semantics, _lib.stream_ptr(y.device)),
                   "hif8_gelu_fake_quant")
    return out


def quantize_activation(x2: Tensor, scale_max: float, a_format: str, as_f32: bool = False):
    """Quantise a [M,K] activation for the fused GEMM: returns (a, a_fmt, state).  An fp32
    activation (or a bf16 one with ``as_f32``) is quantised in fp32 and handed over as its
    bf16 autocast rounding; ``a_format="codes"`` gives the 8-bit codes instead."""
    st = absmax_scale(x2, scale_max, QuantState(x2.device), as_f32)
    if a_format == "codes":
        return encode(x2, st, as_f32), _lib.A_CODES, st
    if x2.dtype == torch.bfloat16 and not as_f32:
        return fake_quant(x2, st), _lib.A_BF16, st
    return fake_quant_to_bf16(x2, st, as_f32=as_f32), _lib.A_BF16, st


# --------------------------------------------------------------- autograd


def _forward_no_grad(x: Tensor, packed: PackedWeight, bias: Optional[Tensor], scale_max_forward: float,
                     a_format: str = "bf16") -> Tensor:
    """_HIF8LinearFunction.forward without autograd bookkeeping (nothing kept for a backward)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"HIF8Linear takes bfloat16 or float32 input, got {x.dtype}")
    K = x.shape[-1]
    a, a_fmt, a_st = quantize_activation(x.reshape(-1, K).contiguous(), scale_max_forward,
                                         "codes" if a_format == "codes" else "bf16")
    y = linear_any(a, a_fmt, a_st, packed, bias)
    return y.view(*x.shape[:-1], y.shape[-1])


class _HIF8LinearFunction(torch.autograd.Function):
    """hif8_linear.py:56-111 with the fused HIP forward."""

    @staticmethod
    def forward(ctx, x, weight, bias, scale_max_forward: float, scale_max_backward: float,
                packed: Optional[PackedWeight] = None, a_format: str = "bf16"):
        if x.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"HIF8Linear takes bfloat16 or float32 input, got {x.dtype}")
        K = x.shape[-1]
        x2 = x.reshape(-1, K).contiguous()
        if packed is None:
            packed = PackedWeight(weight, scale_max_forward)
        needs_grad = any(ctx.needs_input_grad[:3])
        a, a_fmt, a_st = quantize_activation(x2, scale_max_forward, "codes" if a_format == "codes" else "bf16")
        y = linear_any(a, a_fmt, a_st, packed, bias)
        if needs_grad:
            if x.dtype != torch.bfloat16 and a_fmt == _lib.A_BF16:
                # the backward's x_q is the fp32 one (hif8_linear.py:78-82): keep its codes
                a, a_fmt = encode(x2, a_st), _lib.A_CODES
            ctx.a, ctx.a_fmt, ctx.a_st, ctx.packed = a, a_fmt, a_st, packed
            ctx.x_dtype, ctx.w_dtype = x.dtype, weight.dtype
            ctx.x_shape = x.shape
            ctx.has_bias = bias is not None
            ctx.b_dtype = bias.dtype if bias is not None else None
            ctx.smb = float(scale_max_backward)
        return y.view(*x.shape[:-1], y.shape[-1])

    @staticmethod
    def backward(ctx, grad_output):
        # x_q and w_q as the reference saves them (hif8_linear.py:78-82)
        if ctx.a_fmt == _lib.A_CODES:
            x_q = decode(ctx.a, ctx.a_st, torch.bfloat16 if ctx.x_dtype == torch.bfloat16 else torch.float32)
        else:
            x_q = ctx.a
        grad_q, _ = _quant(grad_output.contiguous(), ctx.smb)            # :93
        g_2d = grad_q.reshape(-1, grad_q.shape[-1]).contiguous()
        M, N = g_2d.shape
        K = ctx.packed.shape[1]
        if dgrad_fused_ok(g_2d, ctx.packed):                              # :97, grad_q @ w_q
            grad_input = linear_dgrad(g_2d, ctx.packed)
        else:                                                             # fp32: the fp32 GEMM
            w_q = ctx.packed.dequantize(ctx.w_dtype)                      # [N, K]
            grad_input = gemm_f32(g_2d, w_q, M, K, N, (N, 1), (K, 1))
        grad_input = grad_input.to(ctx.x_dtype).view(ctx.x_shape)
        x_2d = x_q.reshape(-1, x_q.shape[-1]).contiguous()
        if wgrad_ok(g_2d, x_2d):                                            # :104, g^T @ x_q
            grad_weight = linear_wgrad(g_2d, x_2d).to(ctx.w_dtype)
        else:                                                               # g[M, N]^T x[M, K]
            grad_weight = gemm_f32(g_2d, x_2d, N, K, M, (1, N), (K, 1)).to(ctx.w_dtype)
        grad_bias = g_2d.sum(0).to(ctx.b_dtype) if ctx.has_bias else None                   # :107
        return grad_input, grad_weight, grad_bias, None, None, None, None


# ------------------------------------------------------------------ module


class HIF8Linear(nn.Linear):
    """Drop-in ``nn.Linear`` with HiF8 qdq of input and weight
    (hif8_linear.py:117-170; same constructor and forward).

    Extras beyond the reference interface:
      * ``prepack(drop_weight=False)`` stores the weight as 8-bit HiF8 codes once
        (inference); without it the packed weight is rebuilt whenever the weight
        tensor changes (version counter or storage), which matches the
        reference's per-call re-quantisation.
      * ``a_format`` = ``"bf16"`` (default: the bf16 x_q is the GEMM operand and, with
        autograd, what the backward keeps) or ``"codes"`` (x_q is held as its 8-bit
        codes -- half the bytes a training step keeps for the backward -- and decoded
        to bf16 for the GEMM).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 scale_max_forward: float = 15.0, scale_max_backward: float = 224.0,
                 device=None, dtype=None):
        super().__init__(in_features, out_features, bias, device=device, dtype=dtype)
        self.scale_max_forward = scale_max_forward
        self.scale_max_backward = scale_max_backward
        self.a_format = "bf16"
        self._packed: Optional[PackedWeight] = None
        self._prepacked = False

    def _packed_weight(self) -> PackedWeight:
        w = self.weight
        key = (w.data_ptr(), w._version, w.device)
        p = self._packed
        if self._prepacked and p is not None:
            return p
        if p is None or p.key != key or p.scale_max != float(self.scale_max_forward):
            p = PackedWeight(w, self.scale_max_forward)
            self._packed = p
        return p

    @torch.no_grad()
    def prepack(self, drop_weight: bool = False) -> "HIF8Linear":
        self._packed = PackedWeight(self.weight, self.scale_max_forward)
        self._prepacked = True
        if drop_weight:
            self.weight = nn.Parameter(torch.empty(0, device=self.weight.device, dtype=self.weight.dtype),
                                       requires_grad=False)
        return self

    def forward(self, x: Tensor) -> Tensor:
        packed = self._packed_weight()
        grad = torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad
                                            or (self.bias is not None and self.bias.requires_grad))
        if not grad:
            return _forward_no_grad(x, packed, self.bias, self.scale_max_forward, self.a_format)
        return _HIF8LinearFunction.apply(x, self.weight, self.bias, self.scale_max_forward,
                                         self.scale_max_backward, packed, self.a_format)

    def forward_quantized(self, x_q: Tensor) -> Tensor:
        """The forward of an input already quantised with this layer's ``scale_max_forward``
        (``x_q = _quant(x)[0]``, e.g. from ``modulated_norm_quant``): the GEMM alone.  Equals
        ``forward(x)`` exactly, since ``_quant`` is deterministic.  Inference only."""
        if torch.is_grad_enabled() and (x_q.requires_grad or self.weight.requires_grad
                                        or (self.bias is not None and self.bias.requires_grad)):
            raise RuntimeError("forward_quantized has no autograd; call forward(x) when gradients are needed")
        if x_q.dtype != torch.bfloat16:
            raise TypeError(f"forward_quantized takes the bf16 x_q, got {x_q.dtype}")
        K = x_q.shape[-1]
        x2 = x_q.reshape(-1, K).contiguous()
        y = linear_any(x2, _lib.A_BF16, None, self._packed_weight(), self.bias)
        return y.view(*x_q.shape[:-1], y.shape[-1])

    def forward_f32_of_bf16(self, x: Tensor) -> Tensor:
        """``forward(x.float())`` for a bf16 x without the fp32 copy: x quantised with fp32
        arithmetic as ``_quant`` does for the fp32 tensor, the GEMM on its bf16 autocast
        rounding.  The self-attention ``o`` input is such a tensor (the bf16 attention output
        returned as fp32, attention.py:473,518).  Inference only."""
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad
                                        or (self.bias is not None and self.bias.requires_grad)):
            raise RuntimeError("forward_f32_of_bf16 has no autograd; call forward(x.float())")
        if x.dtype != torch.bfloat16:
            raise TypeError(f"forward_f32_of_bf16 takes a bfloat16 tensor, got {x.dtype}")
        K = x.shape[-1]
        x2 = x.reshape(-1, K).contiguous()
        a, a_fmt, a_st = quantize_activation(x2, self.scale_max_forward, "bf16", as_f32=True)
        y = linear_any(a, a_fmt, a_st, self._packed_weight(), self.bias)
        return y.view(*x.shape[:-1], y.shape[-1])

    def forward_settled(self, x: Tensor, x_state: QuantState, as_f32: bool = False) -> Tensor:
        """``forward(x)`` (``as_f32``: ``forward(x.float())``) for a bf16 x whose amax, scale and
        tables ``x_state`` already holds for this layer's ``scale_max_forward``, left there by the
        kernel that wrote x (the attention's epilogue): the quantisation pass and the GEMM, no
        amax pass.  Inference only."""
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad
                                        or (self.bias is not None and self.bias.requires_grad)):
            raise RuntimeError("forward_settled has no autograd; call forward(x)")
        if x.dtype != torch.bfloat16:
            raise TypeError(f"forward_settled takes a bfloat16 tensor, got {x.dtype}")
        K = x.shape[-1]
        x2 = x.reshape(-1, K).contiguous()
        a = fake_quant_to_bf16(x2, x_state, as_f32=True) if as_f32 else fake_quant(x2, x_state)
        y = linear_any(a, _lib.A_BF16, x_state, self._packed_weight(), self.bias)
        return y.view(*x.shape[:-1], y.shape[-1])

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, "
                f"scale_max_fwd={self.scale_max_forward}, "
                f"scale_max_bwd={self.scale_max_backward}")


def make_linear(quant: str, in_features: int, out_features: int, scale_max_forward: float = 15.0,
                scale_max_backward: float = 224.0, bias: bool = True, **kw) -> nn.Module:
    """``_make_linear`` (ospnext/modules/osp_next.py:42-58)."""
    if quant == "hif8":
        return HIF8Linear(in_features, out_features, bias=bias, scale_max_forward=scale_max_forward,
                          scale_max_backward=scale_max_backward, **kw)
    return nn.Linear(in_features, out_features, bias=bias, **kw)
