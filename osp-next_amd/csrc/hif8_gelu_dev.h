// GELU (tanh approximation) of the DiT block's FFN -- nn.GELU(approximate="tanh") between the
// up- and down-projections, osp_next.py:873-877 -- and the statistic that gives amax|GELU(y)| of
// the up-projection's output without a pass over it.  Shared by the GEMM epilogues (which fold
// the statistic) and the codec (which applies GELU in the down-projection's quantisation pass),
// so both evaluate GELU with the same roundings.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"
#include "hif8_state_dev.h"

namespace hif8 {

// GELU in fp32 as the reference evaluates it on a bf16 tensor:
//   u = sqrt(2/pi) (x + 0.044715 x^3),   y = 0.5 x (1 + tanh(u)).
// tanh(u) = sign(u) (1 - d) with d = 2 / (1 + e^(2|u|)), from the hardware exp2 and reciprocal;
// forming 1 - d in fp32 rounds it to the fp32 grid next to +-1 as an fp32 tanh does, so the
// cancellation in 1 + tanh(u) for u << 0 (the result's tail) behaves as in the reference.  The
// product-sum in u is one fused multiply-add and nothing else is contracted, whatever the
// translation unit's contraction setting.
__device__ __forceinline__ float gelu_tanh(float x)
{
#pragma clang fp contract(off)
    const float u = 0.7978845608028654f * __builtin_fmaf(0.044715f, x * x * x, x);
    const float e = __builtin_amdgcn_exp2f(__builtin_fabsf(u) * 2.8853900817779268f);  // e^(2|u|)
    const float d = 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
    const float th = __builtin_copysignf(1.0f - d, u);
    return 0.5f * x * (1.0f + th);
}

// Packed RNE conversion of two floats to bf16 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t gelu_pk_cvt(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// GELU of the two bf16 values of a word, each rounded to bf16: the GELU layer's bf16 output.
__device__ __forceinline__ uint32_t gelu_bf16x2(uint32_t w)
{
    return gelu_pk_cvt(gelu_tanh(bf2f(w & 0xFFFFu)), gelu_tanh(bf2f(w >> 16)));
}
__device__ __forceinline__ uint32_t gelu_bf16(uint32_t b) { return gelu_bf16x2(b & 0xFFFFu) & 0xFFFFu; }

// gelu_bf16 over all finite inputs from a window table of 2 x 1440 values.  Outside the window
// of magnitudes [kGeluWinLo, kGeluWinHi) the rounded GELU has a closed form:
//   |x| < kGeluWinLo (0.0024):  GELU(x) = rnd(x * 0.5) -- 0.5 x (1 + tanh(u)) = 0.5 x + 0.399 x^2
//                               + ..., whose x^2 term is below half a bf16 unit of 0.5 x there;
//   x >= kGeluWinHi (6.0):      GELU(x) = x -- 1 - tanh(u) < 2^-34 rounds to 1 in fp32;
//   x <= -kGeluWinHi:           GELU(x) = -0 -- likewise tanh(u) = -1 and 1 + tanh(u) = 0
// (torch's tanh GELU of a bf16 tensor meets them from 0x3B4B, 2.75 and -5.06 on; the window is
// wider, and a test compares the window route with torch's GELU for every bf16 input).  Inside
// the window, entry 2 * (|x| bits - kGeluWinLo) + sign is gelu_bf16 of that input, so the
// magnitude -kGeluWinHi + 1 unit (entry 2 * (kGeluWinN - 1) + 1) holds the -0 that every larger
// negative magnitude takes.
constexpr uint32_t kGeluWinLo = 0x3B20u, kGeluWinHi = 0x40C0u;
constexpr uint32_t kGeluWinN = kGeluWinHi - kGeluWinLo;   // 1440 magnitudes per sign

// The window table (2 * kGeluWinN values, interleaved by sign) from gelu_bf16; threads tid of
// nthreads share the work.
__device__ __forceinline__ void gelu_win_fill(uint16_t *tab, uint32_t tid, uint32_t nthreads)
{
    for (uint32_t i = tid; i < kGeluWinN; i += nthreads) {
        const uint32_t b = kGeluWinLo + i;
        *(uint32_t *)(tab + 2 * i) = gelu_bf16x2(b | ((b | 0x8000u) << 16));   // (+x, -x) in one word
    }
}

// gelu_bf16x2(w) for a word of two FINITE bf16 values through the window table at LDS byte
// address tab, with packed 16-bit arithmetic and no branches: ~20 VALU operations and two
// lookups per word, against the evaluation's 26 and four transcendentals.
__device__ __forceinline__ uint32_t gelu_win_bf16x2(uint32_t w, const uint16_t *tab)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    typedef short i16x2 __attribute__((ext_vector_type(2)));
    const u16x2 lo2 = {uint16_t(kGeluWinLo), uint16_t(kGeluWinLo)};
    const u16x2 m = __builtin_bit_cast(u16x2, w & 0x7FFF7FFFu);
    // index i = min(max(m - lo, 0), N - 1), byte offset 4 i + 2 sign
    const u16x2 i0 = __builtin_elementwise_sub_sat(m, lo2);
    const u16x2 i1 = __builtin_elementwise_min(i0, u16x2{uint16_t(kGeluWinN - 1), uint16_t(kGeluWinN - 1)});
    const uint32_t off = (__builtin_bit_cast(uint32_t, i1 << u16x2{2, 2})) | ((w >> 14) & 0x00020002u);
    const uint8_t *tb = (const uint8_t *)tab;
    const uint32_t t0 = *(const uint16_t *)(tb + (off & 0xFFFFu));
    const uint32_t t1 = *(const uint16_t *)(tb + (off >> 16));
    const uint32_t t = t0 | (t1 << 16);
    // masks per half (all ones where true): below the window (m < lo); and the table, not the
    // positive tail (m < hi, or negative).  m - lo and m - hi fit in int16.
    const i16x2 ms = __builtin_bit_cast(i16x2, m);
    const uint32_t tiny = __builtin_bit_cast(uint32_t, (ms - i16x2{short(kGeluWinLo), short(kGeluWinLo)}) >> i16x2{15, 15});
    const uint32_t neg = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, w) >> i16x2{15, 15});
    const uint32_t below_hi = __builtin_bit_cast(uint32_t, (ms - i16x2{short(kGeluWinHi), short(kGeluWinHi)}) >> i16x2{15, 15}) | neg;
    const uint32_t halves = gelu_pk_cvt(__builtin_bit_cast(float, w << 16) * 0.5f,
                                        __builtin_bit_cast(float, w & 0xFFFF0000u) * 0.5f);
    const uint32_t r = (below_hi & t) | (~below_hi & w);      // the table, or the positive tail x
    return (tiny & halves) | (~tiny & r);
}

// The GELU statistic of a set of bf16 outputs: the largest non-negative value (bf16 bits, 0 when
// there is none) or kGeluNonFinite when any output is Inf or NaN (GELU(-Inf) and GELU(NaN) are
// NaN: the amax then needs the full pass).  Accumulated two outputs per 32-bit word, one packed
// max each, on the raw bits:
//   smax_i: signed 16-bit max -- a negative bf16 is a negative int16 and a non-negative one keeps
//           its numeric order, so this is the largest non-negative output, and +Inf / +NaN
//           (0x7F80 .. 0x7FFF) are the largest int16 values of all;
//   smax_u: unsigned 16-bit max -- -Inf / -NaN (0xFF80 .. 0xFFFF) are the largest uint16 values.
constexpr uint32_t kGeluNonFinite = 0x10000u;
__device__ __forceinline__ void gelu_stat_pk(uint32_t &smax_i, uint32_t &smax_u, uint32_t w0, uint32_t w1)
{
    typedef short i16x2 __attribute__((ext_vector_type(2)));
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const i16x2 p = __builtin_elementwise_max(__builtin_bit_cast(i16x2, w0), __builtin_bit_cast(i16x2, w1));
    smax_i = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(i16x2, smax_i), p));
    const u16x2 q = __builtin_elementwise_max(__builtin_bit_cast(u16x2, w0), __builtin_bit_cast(u16x2, w1));
    smax_u = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, smax_u), q));
}
// One lane's statistic from its packed maxima (both start at 0; as an unsigned value, maxima of
// these over lanes and workgroups are the statistic of the union).
__device__ __forceinline__ uint32_t gelu_stat_final(uint32_t smax_i, uint32_t smax_u)
{
    const int lo = int(short(smax_i & 0xFFFFu)), hi = int(short(smax_i >> 16));
    const int p = lo > hi ? lo : hi;
    if (p >= 0x7F80 || max(smax_u & 0xFFFFu, smax_u >> 16) >= 0xFF80u) return kGeluNonFinite;
    return p > 0 ? uint32_t(p) : 0u;
}

// |GELU(y)| for y <= 0 is at most 0.16997 (near y = -0.7518): 0x3E2E (0.16992) once rounded to
// bf16, with every y <= 0 mapping at or below it.  GELU increases on y >= 0, so when GELU(ymax)
// rounds above 0x3E2E the largest |GELU(y)| over a tensor is GELU(ymax) itself.
constexpr uint32_t kGeluNegAmaxBits = 0x3E2Eu;

// Fold one wave's statistic (the max of gelu_stat_final over its lanes) into st->amax_acc: a
// relaxed atomic max with no return value and no fence, so the wave ends without waiting for its
// output stores to complete (a release at agent scope would wait for them and write back the
// XCD's L2 in every workgroup).  gelu_stat_settle reads the maximum in a kernel launched after the
// GEMM on the same stream.
__device__ __forceinline__ void fold_gelu_stat(State *st, uint32_t m)
{
    __hip_atomic_fetch_max(&st->amax_acc, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Settle the state after a GEMM that folded the statistic of its output y into st (one workgroup
// of 256 threads): reset the accumulator and, when max y settles the amax, write
// amax = GELU(max y), the scale for smax, the flags and the decode tables, as hif8_absmax_scale of
// GELU(y) would; otherwise mark the state pending (the down-projection's quantisation then runs
// the amax pass first).  lds is two words of LDS.
__device__ __forceinline__ void gelu_stat_settle(State *st, float smax, uint32_t *lds)
{
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        const uint32_t a = st->amax_acc;
        st->amax_acc = 0u;
        uint32_t g = 0;
        bool settled = false;
        if (a < kGeluNonFinite) {
            g = gelu_bf16(a);                                  // a: the largest output, non-negative
            settled = g > kGeluNegAmaxBits && g < 0x7F80u;   // positive, finite, above every y <= 0
        }
        bool fast = false;
        float s = 0.0f;
        if (settled) s = scale_from_amax(g, kBF16, smax, fast);
        st->amax_bits = settled ? g : 0u;
        st->scale = s;
        st->fast = fast ? 1u : 0u;
        st->finite = fast ? 1u : 0u;
        st->dtype = uint32_t(kBF16);
        st->pending = settled ? 0u : 1u;
        lds[0] = settled ? 1u : 0u;
        lds[1] = f2u(s);
    }
    __syncthreads();
    if (lds[0]) fill_luts(st, u2f(lds[1]), tid);
}

}  // namespace hif8
