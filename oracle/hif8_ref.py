"""CPU restatement of OSP-Next's per-tensor HiF8 fake-quant linear path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker; the product path (the HIP library and its Python mirror) never does.

What it restates (citations are into the reference tree):

* ``quant_hif8_torch``  -- ``ospnext/quant_cy_npu/base/QFuncs/hif8.py:6-23``, the
  torch ("CPU") HiF8 qdq, op by op in explicit float32 numpy.
* ``quant_hif8_npu``    -- ``ospnext/quant_cy_npu/base/cusrc/hif8_quant_op.h:88-151``,
  the Ascend kernel, through the C restatement in ``hif8_npu_ref.c``.
* ``hif8_scale``        -- ``ospnext/modules/hif8_linear.py:45-46``:
  ``x_max = |x|.amax().clamp(min=1e-8)`` and ``scale = scale_max / x_max``, which
  torch evaluates as ``x_max.reciprocal() * scale_max`` (``torch/_tensor.py``
  ``__rdiv__``), each op rounded to the tensor dtype.
* ``quant``             -- ``hif8_linear.py:42-50`` with ``quant_dequant_float``
  (``QTensor.py:94-128``, ``force_fp32=True``): ``xs = x*scale``; fp32 qdq; cast
  back to the input dtype; ``/ scale``.
* ``linear``            -- ``hif8_linear.py:68-86``: ``F.linear(_quant(x), _quant(W), b)``.
* ``modulated_layer_norm_bf16`` -- the producer of the q/k/v and FFN-up inputs,
  ``norm(x) * (1 + scale) + shift`` (``osp_next.py:941``, ``:954``) with the WanLayerNorm
  (``want2v.py:96-106``); its ``_quant`` is ``quant_bf16`` above.

bf16 arithmetic is emulated bit-exactly: every bf16 op of the reference is an
fp32 op followed by round-to-nearest-even (torch CPU's ``c10::BFloat16``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

F32 = np.float32
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libhif8_oracle.so")
BF16_1E_8 = 0x322C  # bf16(1e-8): clamp(min=1e-8) on a bf16 tensor converts the bound first

# --------------------------------------------------------------------------- bf16


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns (uint16) -> exact float32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7FC0 (c10::BFloat16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    r[np.isnan(x)] = 0x7FC0
    return r


def f32_to_bf16_trunc(x) -> np.ndarray:
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ------------------------------------------------------------- torch-path qdq


def quant_hif8_torch(x) -> np.ndarray:
    """QFuncs/hif8.py:6-23 for float32 input (the ``force_fp32=True`` route).

    ``sign`` is torch.sign, which is +0 for +-0 and 0 for NaN
    ((0 < a) - (a < 0)); everything else is a float32 op in the same order.
    """
    x = np.asarray(x, dtype=F32)
    x_unsigned = np.abs(x)                                              # :7
    sign = (x > 0).astype(F32) - (x < 0).astype(F32)                    # :8
    with np.errstate(all="ignore"):
        e = np.floor(np.log2(x_unsigned + F32(2.0 ** -45)))             # :13
        abse = np.abs(e)                                                # :15
        mant_bits = np.zeros_like(abse)                                 # :16
        mant_bits[abse <= 15] = 1                                       # :17
        mant_bits[abse <= 7] = 2                                        # :18
        mant_bits[abse <= 3] = 3                                        # :19
        res = (np.floor(x_unsigned * np.power(F32(2.0), -e + mant_bits) + F32(0.5))
               * np.power(F32(2.0), e - mant_bits) * sign)               # :21
    return res.astype(F32)


def quant_hif8_torch_bf16(x_bits) -> np.ndarray:
    """QFuncs/hif8.py:6-23 on a bf16 tensor without ``force_fp32`` (QTensor.py:101-102 not
    taken): every op computes in float32 and rounds its result to bf16, as torch's bf16 tensor
    ops do.  bf16 bits in, bf16 bits out.  log2 is evaluated in float64 and rounded straight to
    bf16 (torch rounds its float32 log2 to bf16; the tests pin that the two agree on every input)."""
    x = bf16_to_f32(x_bits)
    rb = lambda v: bf16_to_f32(f32_to_bf16(v))                            # noqa: E731
    with np.errstate(all="ignore"):
        xu = np.abs(x)                                                      # :7
        sign = (x > 0).astype(F32) - (x < 0).astype(F32)                    # :8
        t = rb(xu + F32(2.0 ** -45))                                        # :13, the sum in bf16
        lg = np.log2(t.astype(np.float64))
        e = np.floor(bf16_to_f32(_f64_to_bf16(lg)))                         # :13, log2 then floor
        abse = np.abs(e)
        mant_bits = np.zeros_like(abse)
        mant_bits[abse <= 15] = 1
        mant_bits[abse <= 7] = 2
        mant_bits[abse <= 3] = 3
        m = rb(xu * np.power(F32(2.0), -e + mant_bits))                     # :21
        f = np.floor(rb(m + F32(0.5)))
        r = rb(f * np.power(F32(2.0), e - mant_bits))
        res = rb(r * sign)
    out = f32_to_bf16(res)
    out[~np.isfinite(x)] = 0x7FC0
    return out


def f16_to_f32(bits) -> np.ndarray:
    """fp16 bit patterns (uint16) -> exact float32 values."""
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(F32)


def f32_to_f16(x) -> np.ndarray:
    """float32 -> fp16 bits, round-to-nearest-even with subnormals, overflow to Inf
    (c10::Half's conversion; numpy's float32 -> float16 cast is the same IEEE rounding)."""
    with np.errstate(all="ignore"):
        return np.ascontiguousarray(np.asarray(x, dtype=F32).astype(np.float16)).view(np.uint16)


def quant_hif8_torch_f16(x_bits) -> np.ndarray:
    """QFuncs/hif8.py:6-23 on an fp16 tensor without ``force_fp32`` (QTensor.py:101-102 not
    taken): the fp16 branch of :10-11, offset 2^-14, and every op computing in float32 and
    rounding its result to fp16, as torch's fp16 CPU ops do.  fp16 bits in, fp16 bits out.
    log2 is evaluated in float64 and rounded straight to fp16 (torch rounds its float32 log2 to
    fp16; the tests pin that the two agree on every input).  In fp16 the rounded log2 of a value
    just below a power of two can be that power's exponent, so ``floor`` moves up a binade there
    (the tests count those inputs); 2^(e - mb) overflows to Inf for e = 16."""
    x = f16_to_f32(x_bits)
    rh = lambda v: f16_to_f32(f32_to_f16(v))                            # noqa: E731
    with np.errstate(all="ignore"):
        xu = np.abs(x)                                                      # :7
        sign = (x > 0).astype(F32) - (x < 0).astype(F32)                    # :8
        t = rh(xu + F32(2.0 ** -14))                                        # :11, the sum in fp16
        lg = np.log2(t.astype(np.float64)).astype(np.float16).astype(F32)   # log2, one rounding
        e = np.floor(lg)                                                    # :11
        abse = np.abs(e)                                                    # :15
        mant_bits = np.zeros_like(abse)                                     # :16-19
        mant_bits[abse <= 15] = 1
        mant_bits[abse <= 7] = 2
        mant_bits[abse <= 3] = 3
        p1 = rh(np.power(np.float64(2.0), (-e + mant_bits).astype(np.float64)).astype(F32))  # 2.0**(-e+mb)
        m = rh(xu * p1)                                                     # :21
        f = np.floor(rh(m + F32(0.5)))
        p2 = rh(np.power(np.float64(2.0), (e - mant_bits).astype(np.float64)).astype(F32))   # 2.0**(e-mb)
        r = rh(f * p2)
        res = rh(r * sign)
    return f32_to_f16(res)


def quant_dequant_f16(x_bits, semantics: str) -> np.ndarray:
    """``quant_dequant_float`` on an fp16 tensor (QTensor.py:94-128), fp16 bits in and out:
    ``"npu"`` -- the NPU table has no fp16 kernel, so the fp32 kernel on x.float() and the result
    cast back (QTensor.py:66-79, 126-127); ``"torch"`` -- ``force_py=True, force_fp32=True``: the
    float32 torch function, then the cast back; ``"torch_f16"`` -- ``force_py=True`` alone: the
    torch function in fp16 arithmetic (``quant_hif8_torch_f16``)."""
    if semantics == "torch_f16":
        return quant_hif8_torch_f16(x_bits)
    return f32_to_f16(quant_hif8(f16_to_f32(x_bits), semantics))


def _f64_to_bf16(v) -> np.ndarray:
    """float64 -> bf16 bits, one round-to-nearest-even from the exact value (finite inputs)."""
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)                                  # v = m 2^e, 0.5 <= |m| < 1
    r = np.ldexp(np.round(m * 256.0), e - 8)            # 8 significant bits, ties to even
    return f32_to_bf16(r.astype(F32))


# --------------------------------------------------------------- NPU-path qdq

_lib = None


def build_lib(force: bool = False) -> str:
    """Compile hif8_npu_ref.c with gcc (oracle/Makefile)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "build/libhif8_oracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build_lib()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        L.hif8_npu_qdq_f32_n.argtypes = [p, p, ctypes.c_int64]
        L.hif8_npu_qdq_bf16_n.argtypes = [p, p, ctypes.c_int64]
        L.hif8_npu_encode_f32_n.argtypes = [p, p, ctypes.c_int64]
        L.hif8_npu_encode_f32_n.restype = ctypes.c_int64
        L.hif8_decode_n.argtypes = [p, p, ctypes.c_int64]
        _lib = L
    return _lib


def quant_hif8_npu(x) -> np.ndarray:
    """hif8_quant_op.h:88-151 on float32 input (``npu_quant.hif8_quant``)."""
    x = np.ascontiguousarray(x, dtype=F32)
    y = np.empty_like(x)
    lib().hif8_npu_qdq_f32_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def encode_npu(x) -> np.ndarray:
    """HiF8 codes of the NPU-semantics qdq of float32 ``x``."""
    x = np.ascontiguousarray(x, dtype=F32)
    c = np.empty(x.shape, dtype=np.uint8)
    bad = lib().hif8_npu_encode_f32_n(x.ctypes.data, c.ctypes.data, x.size)
    if bad:
        raise AssertionError(f"{bad} NPU qdq outputs outside the HiF8 value set")
    return c


def decode(codes) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    y = np.empty(c.shape, dtype=F32)
    lib().hif8_decode_n(c.ctypes.data, y.ctypes.data, c.size)
    return y


def decode_table() -> np.ndarray:
    return decode(np.arange(256, dtype=np.uint8))


def quant_hif8(x, semantics: str) -> np.ndarray:
    if semantics == "torch":
        return quant_hif8_torch(x)
    if semantics == "npu":
        return quant_hif8_npu(x)
    raise ValueError(semantics)


# ------------------------------------------------------------------ _quant


def absmax_bf16(x_bits) -> int:
    """``x.abs().amax()`` on bf16: max of the magnitude bits; NaN propagates."""
    m = np.asarray(x_bits, dtype=np.uint16) & np.uint16(0x7FFF)
    if m.size == 0:
        raise ValueError("amax of an empty tensor")
    return int(m.max())


def hif8_scale_bf16(amax_bits: int, scale_max: float) -> int:
    """hif8_linear.py:45-46 for a bf16 tensor: bf16 bits of the scale."""
    a = amax_bits & 0x7FFF
    if a <= 0x7F80:                     # clamp(min=1e-8); NaN passes through
        a = max(a, BF16_1E_8)
    af = bf16_to_f32(np.array([a], np.uint16))
    with np.errstate(all="ignore"):
        r = f32_to_bf16(F32(1.0) / af)                          # reciprocal()
        s = f32_to_bf16(bf16_to_f32(r) * F32(scale_max))        # * scale_max
    return int(s[0])


def absmax_f32(x) -> float:
    x = np.asarray(x, dtype=F32)
    m = np.abs(x)
    return F32(np.nan) if np.isnan(m).any() else F32(m.max())


def hif8_scale_f32(amax: float, scale_max: float) -> float:
    a = F32(amax)
    if not np.isnan(a):
        a = max(a, F32(1e-8))
    with np.errstate(all="ignore"):
        return F32(F32(F32(1.0) / a) * F32(scale_max))


def quant_bf16(x_bits, scale_max: float = 15.0, semantics: str = "npu"):
    """``_quant`` (hif8_linear.py:42-50) on a bf16 tensor.

    Returns ``(x_q_bits, scale_bits)``; every intermediate is rounded to bf16
    exactly where the reference's bf16 tensor ops round.
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    s_bits = hif8_scale_bf16(absmax_bf16(x_bits), scale_max)
    s = bf16_to_f32(np.array([s_bits], np.uint16))[0]
    with np.errstate(all="ignore"):
        xs = f32_to_bf16(bf16_to_f32(x_bits) * s)                   # x * scale (bf16)
        q = quant_hif8(bf16_to_f32(xs), semantics)                  # fp32 qdq
        q = f32_to_bf16(q)                                          # out.to(bf16)
        xq = f32_to_bf16(bf16_to_f32(q) / s)                        # / scale (bf16)
    return xq, s_bits


def quant_f32(x, scale_max: float = 15.0, semantics: str = "npu"):
    """``_quant`` on a float32 tensor (the self-attention ``o`` input)."""
    x = np.asarray(x, dtype=F32)
    s = hif8_scale_f32(absmax_f32(x), scale_max)
    with np.errstate(all="ignore"):
        xq = (quant_hif8(x * s, semantics) / s).astype(F32)
    return xq, s


def codes_bf16(x_bits, scale_max: float = 15.0):
    """HiF8 codes of ``x*scale`` for a bf16 tensor plus the scale bits."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    s_bits = hif8_scale_bf16(absmax_bf16(x_bits), scale_max)
    s = bf16_to_f32(np.array([s_bits], np.uint16))[0]
    xs = f32_to_bf16(bf16_to_f32(x_bits) * s)
    return encode_npu(bf16_to_f32(xs)), s_bits


def decode_lut_bf16(s_bits: int) -> np.ndarray:
    """bf16 bits of ``decode(c) / scale`` for the 256 codes (x_q as a function of the code)."""
    s = bf16_to_f32(np.array([s_bits], np.uint16))[0]
    v = f32_to_bf16(decode_table())             # exact: <= 4 significant bits
    with np.errstate(all="ignore"):
        return f32_to_bf16(bf16_to_f32(v) / s)


# ------------------------------------------------------------------ linear


def linear(x_bits, w_bits, b_bits=None, scale_max: float = 15.0, semantics: str = "npu",
           accumulate: str = "f64"):
    """``_HIF8LinearFunction.forward`` (hif8_linear.py:68-86) for bf16 x [M,K], W [N,K].

    Returns ``(y, x_q_bits, w_q_bits)``.  ``accumulate="f64"`` gives an exactly
    summed reference of the (bit-exact) dequantized operands, returned as float64
    (the output rounding is left to the comparison); ``"torch"`` runs the
    reference's own ``F.linear`` on CPU in bf16 and returns bf16 bits.
    """
    xq, _ = quant_bf16(x_bits, scale_max, semantics)
    wq, _ = quant_bf16(w_bits, scale_max, semantics)
    if accumulate == "f64":
        y = bf16_to_f32(xq).astype(np.float64) @ bf16_to_f32(wq).astype(np.float64).T
        if b_bits is not None:
            y = y + bf16_to_f32(b_bits).astype(np.float64)
        return y, xq, wq
    if accumulate == "torch":
        import torch
        import torch.nn.functional as F
        xt = torch.from_numpy(xq.view(np.int16)).view(torch.bfloat16)
        wt = torch.from_numpy(wq.view(np.int16)).view(torch.bfloat16)
        bt = None if b_bits is None else torch.from_numpy(
            np.asarray(b_bits, np.uint16).view(np.int16)).view(torch.bfloat16)
        y = F.linear(xt, wt, bt)
        return y.view(torch.int16).numpy().view(np.uint16), xq, wq
    raise ValueError(accumulate)


# ------------------------------------------- modulated LayerNorm (producer)


def layer_norm_bf16(x_bits, eps: float = 1e-6):
    """WanLayerNorm (``ospnext/modules/want2v.py:96-106``) of a bf16 [rows, dim] tensor:
    ``layer_norm(x.float(), eps)`` without affine, ``.type_as(x)``.  The normalisation is
    evaluated in float64 (mean, biased variance, ``(x - mean) / sqrt(var + eps)``) and rounded
    to fp32 and then to bf16: the exact result to well below one bf16 unit, where an fp32
    implementation can differ only at a rounding boundary."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = np.square(x - mean).mean(axis=-1, keepdims=True)
    with np.errstate(all="ignore"):
        n = (x - mean) / np.sqrt(var + np.float64(F32(eps)))
    return f32_to_bf16(n.astype(F32))


def affine_layer_norm_bf16(x_bits, weight, bias, eps: float = 1e-6):
    """The affine WanLayerNorm (norm3: ``osp_next.py:860-864``, applied at ``:949-951``;
    ``want2v.py:96-106``) of a bf16 [rows, dim] tensor: ``layer_norm(x.float(), (dim,), weight,
    bias, eps).type_as(x)`` with fp32 weight and bias.  Evaluated in float64 (mean, biased
    variance, ``(x - mean) / sqrt(var + eps) * weight + bias``) and rounded to fp32 and then to
    bf16, as ``layer_norm_bf16``."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = np.asarray(weight, F32).astype(np.float64)
    b = np.asarray(bias, F32).astype(np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = np.square(x - mean).mean(axis=-1, keepdims=True)
    with np.errstate(all="ignore"):
        n = (x - mean) / np.sqrt(var + np.float64(F32(eps)))
        y = n * w + b
    return f32_to_bf16(y.astype(F32))


def modulated_layer_norm_bf16(x_bits, shift_bits=None, scale_bits=None, rows_per_batch=None, eps: float = 1e-6):
    """``norm(x) * (1 + scale) + shift`` of ``block_forward`` (``osp_next.py:941``, ``:954``) with
    bf16 tensors: ``n = layer_norm_bf16(x)``, ``t = bf16(1 + scale)``, ``u = bf16(n * t)``,
    ``y = bf16(u + shift)`` (each bf16 tensor op an fp32 op rounded to bf16).  ``shift`` and
    ``scale`` are [batches, dim]; row r uses modulation row ``r // rows_per_batch``; None is 0."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    rows, dim = x_bits.shape
    rpb = rows if rows_per_batch is None else rows_per_batch
    n = layer_norm_bf16(x_bits, eps)
    bidx = np.arange(rows) // rpb
    zero = np.zeros((int(bidx.max()) + 1, dim), np.uint16)
    sh = zero if shift_bits is None else np.asarray(shift_bits, np.uint16).reshape(-1, dim)
    sc = zero if scale_bits is None else np.asarray(scale_bits, np.uint16).reshape(-1, dim)
    with np.errstate(all="ignore"):
        t = f32_to_bf16(F32(1.0) + bf16_to_f32(sc))
        u = f32_to_bf16(bf16_to_f32(n) * bf16_to_f32(t)[bidx])
        y = f32_to_bf16(bf16_to_f32(u) + bf16_to_f32(sh)[bidx])
    return y


# ------------------------------------------------------------- input recipes


def c1_input(seed: int = 0, shape=(4096, 5120)):
    """Config 1: N(0,0.02) with 0.1% of entries x50, bf16 bits (CPU torch generator)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 0.02
    n = x.numel()
    idx = torch.randperm(n, generator=g)[: n // 1000]
    x.view(-1)[idx] *= 50
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def activation_input(seed: int, m: int, k: int, n_outlier: int, mult: float = 20.0):
    """N(0,1) activations with ``n_outlier`` channels scaled by ``mult`` (configs 2/3)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g)
    ch = torch.randperm(k, generator=g)[:n_outlier]
    x[:, ch] *= mult
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def weight_input(seed: int, n: int, k: int, std: float = 0.02):
    import torch
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((n, k), generator=g) * std
    return w.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------ reference CPU path, torch ops


def quant_hif8_torch_cpu(x):
    """QFuncs/hif8.py:6-23 on a torch CPU tensor (the reference's own op sequence, with its
    fp16 branch, multi-threaded by torch); pinned to ``quant_hif8_torch`` (float32),
    ``quant_hif8_torch_bf16`` and ``quant_hif8_torch_f16`` in the tests."""
    import torch
    x_unsigned = torch.abs(x)
    sign = torch.sign(x)
    if x.dtype == torch.float16:
        e = torch.floor(torch.log2(x_unsigned + 2 ** -14))
    else:
        e = torch.floor(torch.log2(x_unsigned + 2 ** -45))
    abse = e.abs()
    mant_bits = torch.zeros_like(abse)
    mant_bits[abse <= 15] = 1
    mant_bits[abse <= 7] = 2
    mant_bits[abse <= 3] = 3
    return torch.floor(x_unsigned * 2.0 ** (-e + mant_bits) + 0.5) * 2.0 ** (e - mant_bits) * sign


def quant_torch_cpu(x, scale_max: float = 15.0):
    """``_quant`` (hif8_linear.py:42-50) on a torch CPU tensor, torch-path qdq
    (``quant_dequant_float(..., force_fp32=True)`` with the CPU function)."""
    import torch
    x_max = x.abs().amax().clamp(min=1e-8)
    scale = scale_max / x_max
    scaled = x * scale
    q = quant_hif8_torch_cpu(scaled.to(torch.float32)).to(x.dtype)
    return q / scale, scale


def linear_torch_cpu(x, w, b=None, scale_max: float = 15.0):
    """``_HIF8LinearFunction.forward`` (hif8_linear.py:68-86) on CPU torch tensors."""
    import torch.nn.functional as F
    xq, _ = quant_torch_cpu(x, scale_max)
    wq, _ = quant_torch_cpu(w, scale_max)
    return F.linear(xq, wq, b)
