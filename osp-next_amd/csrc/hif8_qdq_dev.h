// Device-side HiF8 quantisation helpers shared by the codec and the fused producers (the
// LayerNorm kernels): the scalar reference route of one element, the LDS layout of the
// encode/decode tables and the sign fix-up of packed magnitude codes.  Every fp32 operation
// here is IEEE-rounded in source order; translation units including this header are built
// with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_common.h"
#include "hif8_internal.h"
#include "hif8_state_dev.h"

namespace hif8 {

// Encode table (magnitude code of each clamped bf16 magnitude), one copy per translation unit.
static __constant__ EncTable kEncTable = make_enc_table();

// ---------------------------------------------------------------- helpers

// Packed RNE convert of two finite floats (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f2bf_pk(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    bf16x2 r = __builtin_convertvector(v, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

// floor of the float32 log2 of a normal float v, as torch takes it (torch.floor(torch.log2(v))):
// the exponent field E, except that log2(v) of the last few v below 2^(E+1) rounds up to the
// integer k = E + 1.  v = 2^k (1 - j 2^-24) has log2 k - delta, delta = -log2(1 - j 2^-24), and
// rounds to k when delta is below half the float32 spacing there, 2^(b-24) with 2^b the binade of
// |k - delta|: for j < 2^b ln 2, i.e. j <= c(b) = ceil(2^b ln 2) - 1 = 0, 1, 2, 5, 11, 22, 44, 88
// for b = 0 .. 7.  (numpy's and torch's float32 log2 round the same way on the 256 floats below
// every power of two in [2^-50, 2^19].)  It matters when v = |x| + 2^-45 lies a few units below
// 2^-44 or 2^-43: there x is half of v or less, and the two floors round x differently.
__device__ __forceinline__ int floor_log2_f32(float v)
{
    const uint32_t vb = f2u(v);
    const int E = int((vb >> 23) & 0xFF) - 127;
    const int k = E + 1;
    const uint32_t ak = uint32_t(k < 0 ? -k : k);
    // b = floor(log2 |k - delta|): for k > 0 that of k - 1 (k - delta lies below k), for k < 0 that
    // of |k| (|k - delta| lies above |k|); no round-up for |k - delta| < 2 (c = 0)
    const uint32_t m = k > 0 ? ak - 1u : ak;
    if (m < 2u) return E;
    const int b = 31 - __builtin_clz(m);
    constexpr uint8_t kC[8] = {0, 1, 2, 5, 11, 22, 44, 88};
    const uint32_t below = 0x7FFFFFu - (vb & 0x7FFFFFu);      // j - 1 for v = 2^k (1 - j 2^-24)
    return below < kC[b] ? k : E;
}

// QFuncs/hif8.py:6-23 on one fp32 value, with the same fp32 operations; floor(log2(v)) of the
// normal value v = |x| + 2^-45 as torch's float32 log2 gives it (floor_log2_f32).
static __device__ float qdq_torch(float x)
{
    float xu = fabsf(x);
    float sign = float(x > 0.0f) - float(x < 0.0f);
    if (!(xu <= 3.402823466e38f)) return __builtin_nanf("");   // NaN, Inf -> NaN
    float v = xu + 0x1p-45f;
    int e = floor_log2_f32(v);
    int ae = e < 0 ? -e : e;
    int mb = ae <= 3 ? 3 : ae <= 7 ? 2 : ae <= 15 ? 1 : 0;
    float t = xu * __builtin_ldexpf(1.0f, mb - e);
    float r = __builtin_floorf(t + 0.5f);
    return r * __builtin_ldexpf(1.0f, e - mb) * sign;
}

__device__ __forceinline__ float qdq_npu(float x) { return u2f(decode_bits(encode_npu_bits(f2u(x)))); }


// Scalar reference route for one element: returns the qdq output in the
// tensor's dtype (bf16 bits in the low half, or fp32 bits) and the code.
template <int DT>
__device__ __forceinline__ void slow_elem(uint32_t xbits, float s, int sem, uint32_t &ybits, uint32_t &code)
{
    if (DT == kBF16) {
        uint32_t xs = f2bf(bf2f(xbits) * s);                  // x * scale   (bf16)
        code = encode_npu_bits(xs << 16);
        float q = sem == kSemTorch ? qdq_torch(bf2f(xs)) : qdq_npu(bf2f(xs));
        uint32_t qb = f2bf(q);                                // out.to(bf16)
        ybits = f2bf(bf2f(qb) / s);                           // / scale     (bf16)
    } else {
        float xs = u2f(xbits) * s;
        code = encode_npu_bits(f2u(xs));
        float q = sem == kSemTorch ? qdq_torch(xs) : qdq_npu(xs);
        ybits = f2u(q / s);
    }
}

// LDS map of the quantise kernels: [0,512) bf16 decode table, [1024,2048) fp32
// decode table, [kTabLo, kTabHi] the encode table (so the clamped magnitude
// bits are the LDS address).
constexpr uint32_t kLdsLutBf16 = 0;
constexpr uint32_t kLdsLutF32 = 1024;
constexpr uint32_t kLdsBytes = (kTabLo + sizeof(EncTable) + 15) & ~15u;
static_assert(kLdsLutF32 + 1024 <= kTabLo, "LDS map overlap");

__device__ __forceinline__ uint32_t clampu(uint32_t u)
{
    return u < kTabLo ? kTabLo : (u > kTabHi ? kTabHi : u);
}

// Table route of one element whose fake quant is wanted as bf16 bits (an attention or GEMM
// operand), for a fast state (finite scale s > 0): DT kF32, v an fp32 value: the bf16 rounding of
// the fp32 x_q; DT kBF16, v a bf16 value: the bf16 x_q.  The same bits as slow_elem (then f2bf for
// kF32).  tab: LDS with the encode table at [kTabLo, kTabHi] and the state's bf16 decode table at
// kLdsLutBf16.  The magnitude bits of x * s, truncated to bf16 for fp32, index the encode table:
// HiF8 keeps at most 3 mantissa bits and rounds half away from zero, so the dropped bits never
// change the rounding.  nan_guard (the state did not prove the tensor finite): NaN takes the NaN
// code.  The torch semantics differ from the table only below 2^-22 (non-zero) and from 40960 up.
template <int DT>
__device__ __forceinline__ uint32_t fast_elem_bf16(float v, float s, int sem, const uint8_t *tab, bool nan_guard)
{
    uint32_t xs, u, full;
    if (DT == kF32) {
        xs = f2u(v * s);
        u = (xs >> 16) & 0x7FFFu;
        full = xs & 0x7FFFFFFFu;
    } else {
        xs = f2bf(v * s);
        u = xs & 0x7FFFu;
        full = u;
    }
    const uint32_t mag = tab[clampu(u)];
    const uint32_t sign = (DT == kF32 ? xs >> 24 : xs >> 8) & 0x80u;
    uint32_t code = mag ? (mag | sign) : 0u;   // magnitude 0 stays 0x00 (0x80 is NaN)
    if (nan_guard && u > 0x7F80u) code = kNanCode;
    uint32_t y = ((const uint16_t *)(tab + kLdsLutBf16))[code];
    if (sem == kSemTorch && ((full != 0u && u < 0x3480u) || u >= 0x4720u)) {
        const float q = qdq_torch(DT == kF32 ? u2f(xs) : bf2f(xs));
        y = DT == kF32 ? f2bf(q / s) : f2bf(bf2f(f2bf(q)) / s);
    }
    return y;
}

// Sign fix-up for 4 magnitude codes: a code of magnitude 0 stays 0x00 (0x80 is NaN).
__device__ __forceinline__ uint32_t apply_signs(uint32_t mags, uint32_t signs80)
{
    return mags | ((mags + 0x7F7F7F7Fu) & signs80);
}

}  // namespace hif8
