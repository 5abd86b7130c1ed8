// Shared HiF8 arithmetic for the MI355X kernels (host + device, constexpr).
//
// HiF8 value set: 0, +-2^e * 1.m with 3 mantissa bits for |e| <= 3, 2 for
// |e| <= 7, 1 for |e| <= 15, and the powers 2^-22 .. 2^-16; +-Inf; NaN.
// Code layout (HiFloat8, Luo et al. 2024): sign | dot | exponent | mantissa,
//   0000 MMM  : M = 0 -> zero, else 2^(M-23)
//   0001 mmm  : e = 0
//   001 S mmm : |e| = 1
//   01 S f mmm: |e| = 2 + f
//   10 S ff mm: |e| = 4 + ff
//   11 S fff m: |e| = 8 + fff
// S = 1 for negative exponents.  0x80 = NaN, 0x6F/0xEF = +-Inf (the 1.5*2^15
// slot), so the largest finite magnitude is 2^15.
#pragma once

#include <stdint.h>

#if !defined(__HIP__) && !defined(__host__)
#define __host__
#define __device__
#endif

namespace hif8 {

// Magnitude code of 2^e * (1 + m3/8); m3 must already fit the precision of e.
__host__ __device__ constexpr uint32_t enc_mag(int e, uint32_t m3)
{
    int ae = e < 0 ? -e : e;
    uint32_t S = e < 0 ? 1u : 0u;
    if (e == 0) return 0x08u | m3;
    if (ae == 1) return 0x10u | (S << 3) | m3;
    if (ae <= 3) return 0x20u | (S << 4) | (uint32_t(ae - 2) << 3) | m3;
    if (ae <= 7) return 0x40u | (S << 4) | (uint32_t(ae - 4) << 2) | (m3 >> 1);
    if (ae <= 15) return 0x60u | (S << 4) | (uint32_t(ae - 8) << 1) | (m3 >> 2);
    return uint32_t(e + 23);  // e in [-22, -16]
}

__host__ __device__ constexpr int mant_bits(int e)
{
    int ae = e < 0 ? -e : e;
    return ae <= 3 ? 3 : ae <= 7 ? 2 : ae <= 15 ? 1 : 0;
}

// HiF8 code of the NPU-semantics qdq of the fp32 value with bit pattern xb
// (ospnext/quant_cy_npu/base/cusrc/hif8_quant_op.h:88-151):
//   |x| < 2^-23 -> 0;  [2^-23, 2^-22) -> 2^-22;  |x| >= 40960 -> Inf;
//   otherwise round-half-away to the tapered grid of x's binade.
// Only the top 16 bits of xb matter (the rounding bit sits at mantissa bit
// 22-mb >= 19 and every threshold has zero low bits), so the same function
// serves bf16 and fp32 inputs.  NaN -> 0xEF (-Inf), as the reference kernel:
// NaN fails both of its range compares (x < 40960, x > -40960), so its +Inf
// select and then its -Inf select apply (hif8_quant_op.h:109-110,143-150).
constexpr uint32_t kNanCode = 0xEFu;

__host__ __device__ constexpr uint32_t encode_npu_bits(uint32_t xb)
{
    uint32_t s = xb >> 31;
    uint32_t a = xb & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return kNanCode;
    if (a >= 0x47200000u) return s ? 0xEFu : 0x6Fu;       // |x| >= 40960
    int E = int(a >> 23);
    if (E < 104) return 0x00u;                             // |x| < 2^-23, incl. +-0
    if (E == 104) return (s << 7) | 0x01u;                 // -> 2^-22
    int e = E - 127;
    int mb = mant_bits(e);
    uint32_t sh = uint32_t(23 - mb);
    uint32_t r = (((a & 0x7FFFFFu) | 0x800000u) + (1u << (sh - 1))) >> sh;  // half away
    uint32_t m3 = 0;
    if (r == (2u << mb)) {  // carried into the next binade: value 2^(e+1)
        e += 1;
    } else {
        m3 = (r - (1u << mb)) << (3 - mb);
    }
    return (s << 7) | enc_mag(e, m3);
}

// fp32 bit pattern of the value of a code.
__host__ __device__ constexpr uint32_t decode_bits(uint32_t c)
{
    if (c == 0x80u) return 0x7FC00000u;
    if (c == 0x6Fu) return 0x7F800000u;
    if (c == 0xEFu) return 0xFF800000u;
    uint32_t s = c >> 7, u = c & 0x7Fu;
    int e = 0;
    uint32_t m = 0;
    if (u == 0) return 0u;
    if (u < 0x08u) { e = int(u) - 23; m = 0; }
    else if (u < 0x10u) { e = 0; m = u & 7u; }
    else if (u < 0x20u) { e = ((u >> 3) & 1u) ? -1 : 1; m = u & 7u; }
    else if (u < 0x40u) { int ae = 2 + int((u >> 3) & 1u); e = ((u >> 4) & 1u) ? -ae : ae; m = u & 7u; }
    else if (u < 0x60u) { int ae = 4 + int((u >> 2) & 3u); e = ((u >> 4) & 1u) ? -ae : ae; m = (u & 3u) << 1; }
    else { int ae = 8 + int((u >> 1) & 7u); e = ((u >> 4) & 1u) ? -ae : ae; m = (u & 1u) << 2; }
    return (s << 31) | (uint32_t(e + 127) << 23) | (m << 20);
}

// Encode table, indexed by the bf16 magnitude bits u of the scaled value,
// clamped to [kTabLo, kTabHi].  Entry = magnitude code (sign applied apart).
//   u <= 0x3380 (|x| <= 2^-24) -> 0,  u >= 0x4800 (|x| >= 2^17) -> Inf.
constexpr uint32_t kTabLo = 0x3380u;
constexpr uint32_t kTabHi = 0x4800u;
constexpr uint32_t kTabSize = kTabHi - kTabLo + 1;

struct EncTable {
    uint8_t v[(kTabSize + 15) & ~15u];
};

__host__ __device__ constexpr EncTable make_enc_table()
{
    EncTable t{};
    for (uint32_t i = 0; i < sizeof(t.v); ++i) {
        uint32_t u = kTabLo + (i < kTabSize ? i : kTabSize - 1);
        t.v[i] = uint8_t(encode_npu_bits(u << 16) & 0x7Fu);
    }
    return t;
}

}  // namespace hif8
