// Producer fusion for the modulated LayerNorm in front of the self-attention q/k/v and FFN-up
// projections (ospnext/modules/osp_next.py:941,954):
//
//   y   = rnd(rnd(n * rnd(1 + scale)) + shift),   n = rnd(LN(x))            (bf16 ops)
//   x_q = qdq(rnd(y * s)) / s,   s from amax|y|                              (_quant, hif8_linear.py:42-50)
//
// with LN the WanLayerNorm (ospnext/modules/want2v.py:96-106: fp32 layer norm without affine,
// eps 1e-6, cast back to bf16) and shift = e[0] / e[3], scale = e[1] / e[4] of the block's
// modulation.  The reference materialises n, rnd(1 + scale), the product and y as full
// tensors and then runs _quant(y) once per consuming linear (three times for q, k, v).
//
// Two passes over x, 6 bytes per element in total:
//   hif8_modln_amax         reads x, writes each row's (mean, rstd) and folds amax|y| into the
//                           state (its last workgroup computes the scale and decode tables);
//                           with one modulation row, amax|y| comes from per-column extremes of
//                           n (k_modln_amax_ext below), without y per element;
//   hif8_modln_fake_quant   reads x again, recomputes y from the stored statistics (the same
//                           instructions, so the same bits) and writes x_q (and y if asked).
//
// One wavefront per row: lane l holds the 16-byte chunks l, l + 64, ... of the row in
// registers, so mean and variance are two-pass sums over registers (no re-read), reduced
// across the wavefront, and the loads of the wavefront's next row are in flight meanwhile.
// Rows are strided over a grid of 2-3 workgroups x 4 wavefronts per CU.  With one modulation
// row, rnd(1 + scale) and shift are computed once per workgroup into LDS as fp32.
//
// The same two passes serve the affine LayerNorm in front of the cross-attention's q projection
// (norm3, osp_next.py:860-864 and 949-951: WanLayerNorm with elementwise_affine, fp32 weight and bias):
//   y = rnd(w * ((x - mean) * rstd) + b)    (fp32, the product-sum fused, then RNE to bf16)
// as torch's layer-norm kernel evaluates gamma * (rstd * (x - mean)) + beta on the fp32 copy of
// x; w and b sit in LDS where the modulation would (hif8_ln_affine_amax / _fake_quant).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "hif8_common.h"
#include "hif8_internal.h"
#include "hif8_state_dev.h"
#include "hif8_qdq_dev.h"

namespace hif8 {
namespace norm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTPB = 256;
constexpr int kWaves = kTPB / 64;
constexpr int kMaxChunks = 16;   // 16-B chunks per lane: dim <= 16 * 64 * 8 = 8192
constexpr int kWgPerCu = 3;     // pass 1 (157 VGPRs at dim 5120: 3 wavefronts per SIMD)
constexpr int kExtWgPerCu = 2;  // pass 1 from per-column extremes (k_modln_amax_ext)
constexpr int kQdqWgPerCu = 2;  // pass 2 (2 workgroups per CU streamed 1.2-1.4 % faster than 3 at 14B 720P)

// Sum over the wavefront, returned to every lane: DPP steps within each row of 16 lanes
// (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the four row sums.
template <int CTRL> __device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <typename T> __device__ __forceinline__ T ld_stream(const T *p) { return __builtin_nontemporal_load(p); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x2 as_bf2(uint32_t u) { return __builtin_bit_cast(bf16x2, u); }

// v_dot2_f32_bf16 (three-operand form) computes lo * b.lo + hi * b.hi + c in fp32.  With
// b = (1, 0) or (0, 1) it is one bf16 half of a plus c; with b = (t, 0) or (0, t) the exact
// product of that half with the bf16 t.  The other half enters as a product with 0, which
// differs from 0 only when that half is Inf or NaN.
//
// The three steps of the chain are asm blocks of 8 dot2 followed by their consumers because a
// VALU read of a DOT result needs 3 wait states, which the compiler cannot see inside asm: in
// each block every consumer is at least 3 instructions after the dot2 it reads, and every
// block ends with v_cvt_pk_bf16_f32 (not a DOT), so nothing after a block depends on a DOT
// inside it.  (The compiler's own dot2 builtin selects the two-operand accumulating form,
// which costs a copy of c per use.)

// n = rnd((x - mean) * rstd) for 4 words of x (8 elements), nmean = -mean
#define HIF8_DOT_SUB_MUL(n, w, one_lo, one_hi, nmean, rstd)                                                       \
    do {                                                                                                       \
        float d0_, d1_, d2_, d3_, d4_, d5_, d6_, d7_;                                                          \
        asm("v_dot2_f32_bf16 %[d0], %[w0], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d1], %[w0], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d2], %[w1], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d3], %[w1], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d4], %[w2], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d5], %[w2], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d6], %[w3], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d7], %[w3], %[hi], %[nm]\n\t"                                                   \
            "v_mul_f32 %[d0], %[d0], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d1], %[d1], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d2], %[d2], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d3], %[d3], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d4], %[d4], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d5], %[d5], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d6], %[d6], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d7], %[d7], %[rs]\n\t"                                                                \
            "v_cvt_pk_bf16_f32 %[n0], %[d0], %[d1]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n1], %[d2], %[d3]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n2], %[d4], %[d5]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n3], %[d6], %[d7]"                                                            \
            : [n0] "=&v"(n[0]), [n1] "=&v"(n[1]), [n2] "=&v"(n[2]), [n3] "=&v"(n[3]), [d0] "=&v"(d0_),         \
              [d1] "=&v"(d1_), [d2] "=&v"(d2_), [d3] "=&v"(d3_), [d4] "=&v"(d4_), [d5] "=&v"(d5_),             \
              [d6] "=&v"(d6_), [d7] "=&v"(d7_)                                                                 \
            : [w0] "v"(w[0]), [w1] "v"(w[1]), [w2] "v"(w[2]), [w3] "v"(w[3]), [lo] "s"(one_lo),                \
              [hi] "s"(one_hi), [nm] "v"(nmean), [rs] "v"(rstd));                                              \
    } while (0)

// r = rnd(a.lo * b0 + c0, a.hi * b1 + c1) per word: with b the (t, 0) / (0, t) words and c = 0 the
// products n * t; with b = (1, 0) / (0, 1) and c = shift the sums u + shift.
#define HIF8_DOT_PAIR8(r, a, B0, B1, B2, B3, B4, B5, B6, B7, C0, C1, C2, C3, C4, C5, C6, C7, BC, CC)            \
    do {                                                                                                       \
        float e0_, e1_, e2_, e3_, e4_, e5_, e6_, e7_;                                                          \
        asm("v_dot2_f32_bf16 %[e0], %[a0], %[b0], %[c0]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e1], %[a0], %[b1], %[c1]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e2], %[a1], %[b2], %[c2]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e3], %[a1], %[b3], %[c3]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e4], %[a2], %[b4], %[c4]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e5], %[a2], %[b5], %[c5]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e6], %[a3], %[b6], %[c6]\n\t"                                                   \
            "v_dot2_f32_bf16 %[e7], %[a3], %[b7], %[c7]\n\t"                                                   \
            "v_cvt_pk_bf16_f32 %[r0], %[e0], %[e1]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[r1], %[e2], %[e3]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[r2], %[e4], %[e5]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[r3], %[e6], %[e7]"                                                            \
            : [r0] "=&v"(r[0]), [r1] "=&v"(r[1]), [r2] "=&v"(r[2]), [r3] "=&v"(r[3]), [e0] "=&v"(e0_),         \
              [e1] "=&v"(e1_), [e2] "=&v"(e2_), [e3] "=&v"(e3_), [e4] "=&v"(e4_), [e5] "=&v"(e5_),             \
              [e6] "=&v"(e6_), [e7] "=&v"(e7_)                                                                 \
            : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [b0] BC(B0), [b1] BC(B1),        \
              [b2] BC(B2), [b3] BC(B3), [b4] BC(B4), [b5] BC(B5), [b6] BC(B6), [b7] BC(B7), [c0] CC(C0),       \
              [c1] CC(C1), [c2] CC(C2), [c3] CC(C3), [c4] CC(C4), [c5] CC(C5), [c6] CC(C6), [c7] CC(C7));      \
    } while (0)

// HIF8_DOT_SUB_MUL folded into running per-column extremes: n = rnd((x - mean) * rstd) of 4 words
// (8 columns), then mx = max(mx, n) and mn = min(mn, n) per 16-bit half with v_pk_max_f16 /
// v_pk_min_f16 on the bf16 bit patterns.  Read as fp16, bf16 bit patterns keep their order
// (both are sign-magnitude with the magnitude monotone in the low 15 bits) wherever neither
// is an fp16 NaN, i.e. for |n| < 2^121; the caller only folds rows whose n are all finite
// and far below that.  One asm block, so the n temporaries end inside it.
#define HIF8_DOT_SUB_MUL_EXT(w, one_lo, one_hi, nmean, rstd, mx, mn)                                           \
    do {                                                                                                       \
        float d0_, d1_, d2_, d3_, d4_, d5_, d6_, d7_;                                                          \
        uint32_t n0_, n1_, n2_, n3_;                                                                           \
        asm("v_dot2_f32_bf16 %[d0], %[w0], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d1], %[w0], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d2], %[w1], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d3], %[w1], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d4], %[w2], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d5], %[w2], %[hi], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d6], %[w3], %[lo], %[nm]\n\t"                                                   \
            "v_dot2_f32_bf16 %[d7], %[w3], %[hi], %[nm]\n\t"                                                   \
            "v_mul_f32 %[d0], %[d0], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d1], %[d1], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d2], %[d2], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d3], %[d3], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d4], %[d4], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d5], %[d5], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d6], %[d6], %[rs]\n\t"                                                                \
            "v_mul_f32 %[d7], %[d7], %[rs]\n\t"                                                                \
            "v_cvt_pk_bf16_f32 %[n0], %[d0], %[d1]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n1], %[d2], %[d3]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n2], %[d4], %[d5]\n\t"                                                        \
            "v_cvt_pk_bf16_f32 %[n3], %[d6], %[d7]\n\t"                                                        \
            "v_pk_max_f16 %[x0], %[x0], %[n0]\n\t"                                                             \
            "v_pk_min_f16 %[m0], %[m0], %[n0]\n\t"                                                             \
            "v_pk_max_f16 %[x1], %[x1], %[n1]\n\t"                                                             \
            "v_pk_min_f16 %[m1], %[m1], %[n1]\n\t"                                                             \
            "v_pk_max_f16 %[x2], %[x2], %[n2]\n\t"                                                             \
            "v_pk_min_f16 %[m2], %[m2], %[n2]\n\t"                                                             \
            "v_pk_max_f16 %[x3], %[x3], %[n3]\n\t"                                                             \
            "v_pk_min_f16 %[m3], %[m3], %[n3]"                                                                 \
            : [n0] "=&v"(n0_), [n1] "=&v"(n1_), [n2] "=&v"(n2_), [n3] "=&v"(n3_), [d0] "=&v"(d0_),             \
              [d1] "=&v"(d1_), [d2] "=&v"(d2_), [d3] "=&v"(d3_), [d4] "=&v"(d4_), [d5] "=&v"(d5_),             \
              [d6] "=&v"(d6_), [d7] "=&v"(d7_), [x0] "+v"(mx[0]), [x1] "+v"(mx[1]), [x2] "+v"(mx[2]),          \
              [x3] "+v"(mx[3]), [m0] "+v"(mn[0]), [m1] "+v"(mn[1]), [m2] "+v"(mn[2]), [m3] "+v"(mn[3])         \
            : [w0] "v"(w[0]), [w1] "v"(w[1]), [w2] "v"(w[2]), [w3] "v"(w[3]), [lo] "s"(one_lo),                \
              [hi] "s"(one_hi), [nm] "v"(nmean), [rs] "v"(rstd));                                              \
    } while (0)

// The bf16 pairs (1, 0) and (0, 1).  They are passed in SGPRs set up by sgpr_word: as an
// immediate, 0x3F800000 is the bit pattern of fp32 1.0 and gets encoded as the inline
// constant 1.0, which a packed-bf16 operand does not read as (0, 1).
constexpr uint32_t kOneLo = 0x00003F80u, kOneHi = 0x3F800000u;

// An offset of 0 the compiler cannot see through: keeps the per-row reads of the (row
// invariant) modulation in LDS inside the row loop instead of hoisting 16 registers per chunk.
__device__ __forceinline__ uint32_t opaque_zero()
{
    uint32_t z = 0;
    asm volatile("" : "+s"(z));
    return z;
}

__device__ __forceinline__ uint32_t sgpr_word(uint32_t v)
{
    uint32_t r;
    asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}

// Modulation of the lane's 8 columns of chunk c: t = rnd(1 + scale) as bf16 placed in the low
// (even column) or high (odd column) half of a word whose other half is 0, and shift as fp32.
// With MODL (one modulation row for every row of x) both live in LDS, written once per
// workgroup (t words at [0, 4*dim), shift at [4*dim, 8*dim) bytes); otherwise they are read
// per row.
template <bool MODL>
__device__ __forceinline__ void load_mod(const uint32_t *lmod, const uint16_t *shift, const uint16_t *scale,
                                         int64_t moff, int c, int dim, uint32_t (&tw)[8], float (&sh)[8])
{
    if (MODL) {
        const u32x4 *tp = (const u32x4 *)(lmod + 8 * c), *sp = (const u32x4 *)(lmod + dim + 8 * c);
        const u32x4 t0 = tp[0], t1 = tp[1], s0 = sp[0], s1 = sp[1];
        tw[0] = t0.x; tw[1] = t0.y; tw[2] = t0.z; tw[3] = t0.w; tw[4] = t1.x; tw[5] = t1.y; tw[6] = t1.z; tw[7] = t1.w;
        sh[0] = u2f(s0.x); sh[1] = u2f(s0.y); sh[2] = u2f(s0.z); sh[3] = u2f(s0.w);
        sh[4] = u2f(s1.x); sh[5] = u2f(s1.y); sh[6] = u2f(s1.z); sh[7] = u2f(s1.w);
    } else {
        const u32x4 a = shift ? *(const u32x4 *)(shift + moff + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        const u32x4 b = scale ? *(const u32x4 *)(scale + moff + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sh[2 * k] = bf2f(aw[k] & 0xFFFFu);
            sh[2 * k + 1] = u2f(aw[k] & 0xFFFF0000u);
            const uint32_t tt = f2bf_pk(1.0f + bf2f(bw[k] & 0xFFFFu), 1.0f + u2f(bw[k] & 0xFFFF0000u));
            tw[2 * k] = tt & 0xFFFFu;
            tw[2 * k + 1] = tt & 0xFFFF0000u;
        }
    }
}

template <bool MODL>
__device__ __forceinline__ void fill_mod(uint32_t *lmod, const uint16_t *shift, const uint16_t *scale, int dim)
{
    if (!MODL) return;
    for (int c = threadIdx.x; c < (dim >> 3); c += kTPB) {
        uint32_t tw[8];
        float sh[8];
        load_mod<false>(nullptr, shift, scale, 0, c, dim, tw, sh);
        u32x4 *tp = (u32x4 *)(lmod + 8 * c), *sp = (u32x4 *)(lmod + dim + 8 * c);
        tp[0] = u32x4{tw[0], tw[1], tw[2], tw[3]};
        tp[1] = u32x4{tw[4], tw[5], tw[6], tw[7]};
        sp[0] = u32x4{f2u(sh[0]), f2u(sh[1]), f2u(sh[2]), f2u(sh[3])};
        sp[1] = u32x4{f2u(sh[4]), f2u(sh[5]), f2u(sh[6]), f2u(sh[7])};
    }
}

// y of the 8 elements of one chunk (4 packed words in, 4 packed words out):
//   n = rnd((x - mean) * rstd),  u = rnd(n * t),  y = rnd(u + shift),
// each an fp32 operation rounded to bf16 as the reference's ops are, on the dot2 blocks above.
// (x - mean) is exact for a constant row, whose n is then exactly 0.  A non-finite half
// pollutes its neighbour only where the row statistics are NaN (x) or where the modulation
// itself overflows or is NaN (u); both make amax|y| non-finite, so x_q is all NaN there as in
// the reference, and only the diagnostic y differs.
// u = rnd(n * t) and y = rnd(u + shift) of 4 words of n: the modulation half of the chain.
__device__ __forceinline__ void uy8(const uint32_t (&n)[4], const uint32_t (&tw)[8], const float (&sh)[8],
                                    uint32_t one_lo, uint32_t one_hi, uint32_t (&y)[4])
{
    uint32_t u[4];
#define HIF8_Z(v) "i"(0)
    HIF8_DOT_PAIR8(u, n, tw[0], tw[1], tw[2], tw[3], tw[4], tw[5], tw[6], tw[7], 0, 0, 0, 0, 0, 0, 0, 0, "v", HIF8_Z);
#undef HIF8_Z
    HIF8_DOT_PAIR8(y, u, one_lo, one_hi, one_lo, one_hi, one_lo, one_hi, one_lo, one_hi, sh[0], sh[1], sh[2], sh[3],
                   sh[4], sh[5], sh[6], sh[7], "s", "v");
}

__device__ __forceinline__ void modln8(const u32x4 &xv, float nmean, float rstd, const uint32_t (&tw)[8],
                                       const float (&sh)[8], uint32_t one_lo, uint32_t one_hi, uint32_t (&y)[4])
{
    const uint32_t w[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t n[4];
    HIF8_DOT_SUB_MUL(n, w, one_lo, one_hi, nmean, rstd);
    uy8(n, tw, sh, one_lo, one_hi, y);
}

// Affine LayerNorm of the 8 elements of one chunk: y = rnd(fma(w, (x - mean) * rstd, b)).
// wb holds the fp32 bits of w, bb the fp32 b (the LDS slots of t and shift).
__device__ __forceinline__ void lnaff8(const u32x4 &xv, float mean, float rstd, const uint32_t (&wb)[8],
                                       const float (&bb)[8], uint32_t (&y)[4])
{
    const uint32_t w[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float t0 = (bf2f(w[k] & 0xFFFFu) - mean) * rstd;
        const float t1 = (u2f(w[k] & 0xFFFF0000u) - mean) * rstd;
        y[k] = f2bf_pk(__builtin_fmaf(u2f(wb[2 * k]), t0, bb[2 * k]), __builtin_fmaf(u2f(wb[2 * k + 1]), t1, bb[2 * k + 1]));
    }
}

// w and b of the affine LayerNorm into the LDS slots of t and shift (fp32 bits).
__device__ __forceinline__ void fill_aff(uint32_t *lmod, const float *lw, const float *lb, int dim)
{
    for (int c = threadIdx.x; c < (dim >> 3); c += kTPB) {
        const u32x4 *wp = (const u32x4 *)(lw + 8 * c), *bp = (const u32x4 *)(lb + 8 * c);
        u32x4 *tp = (u32x4 *)(lmod + 8 * c), *sp = (u32x4 *)(lmod + dim + 8 * c);
        tp[0] = wp[0];
        tp[1] = wp[1];
        sp[0] = bp[0];
        sp[1] = bp[1];
    }
}

// Row statistics of the wavefront's row, chunks in registers.  sum(x) and sum(x^2) come from
// the bf16 dot product (v_dot2_f32_bf16: the products of bf16 values are exact in fp32), so
// var = sum(x^2) / dim - mean^2.  When that difference could cancel (mean^2 > var, or a
// non-finite sum) the variance is recomputed two-pass as sum((x - mean)^2) / dim.
// rstd = 1 / sqrt(var + eps).
template <int NCH, bool FULL>
__device__ __forceinline__ void row_stats(const u32x4 (&xv)[NCH], int lane, int nch_row, int dim, float eps,
                                          float &mean, float &rstd)
{
    const bf16x2 ones = as_bf2(0x3F803F80u);
    float s = 0.0f, q = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        if (FULL || lane + 64 * j < nch_row) {
            const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bf16x2 v = as_bf2(w[k]);
                s = __builtin_amdgcn_fdot2_f32_bf16(v, ones, s, false);
                q = __builtin_amdgcn_fdot2_f32_bf16(v, v, q, false);
            }
        }
    }
    mean = wave_sum(s) / float(dim);
    float var = wave_sum(q) / float(dim) - mean * mean;
    if (!(mean * mean <= var)) {
        float q2 = 0.0f;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (FULL || lane + 64 * j < nch_row) {
                const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float d0 = bf2f(w[k] & 0xFFFFu) - mean, d1 = u2f(w[k] & 0xFFFF0000u) - mean;
                    q2 = __builtin_fmaf(d0, d0, q2);
                    q2 = __builtin_fmaf(d1, d1, q2);
                }
            }
        }
        var = wave_sum(q2) / float(dim);
    }
    rstd = 1.0f / __builtin_sqrtf(var + eps);
}

template <int NCH, bool FULL>
__device__ __forceinline__ void load_row(const uint16_t *x, int64_t row, int dim, int lane, int nch_row,
                                         u32x4 (&xv)[NCH])
{
    const u32x4 *xr = (const u32x4 *)(x + row * dim);
#pragma unroll
    for (int j = 0; j < NCH; ++j)
        xv[j] = (FULL || lane + 64 * j < nch_row) ? ld_stream(xr + lane + 64 * j) : u32x4{0u, 0u, 0u, 0u};
}

// Pass 1.  Each wavefront streams its rows with the next row's loads in flight while the
// current row is reduced.
template <int NCH, bool MODL, bool FULL, bool AFF>
__global__ __launch_bounds__(kTPB) void k_modln_amax(const uint16_t *__restrict__ x, const uint16_t *__restrict__ shift,
                                                      const uint16_t *__restrict__ scale, const float *__restrict__ lw,
                                                      const float *__restrict__ lb, int64_t rows, int dim,
                                                      int64_t rows_per_batch, float eps, float *__restrict__ stats,
                                                      State *__restrict__ st, float smax)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lmod[];
    __shared__ uint32_t red[kWaves + 2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch_row = dim >> 3;
    if (AFF) fill_aff(lmod, lw, lb, dim);
    else fill_mod<MODL>(lmod, shift, scale, dim);
    __syncthreads();
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m2 = {0, 0};
    const int64_t step = int64_t(gridDim.x) * kWaves;
    int64_t row = int64_t(blockIdx.x) * kWaves + wave;
    const uint32_t one_lo = sgpr_word(kOneLo), one_hi = sgpr_word(kOneHi);
    auto body = [&](const u32x4 (&xv)[NCH], int64_t r) {
        float mean, rstd;
        row_stats<NCH, FULL>(xv, lane, nch_row, dim, eps, mean, rstd);
        const int64_t moff = MODL ? 0 : (r / rows_per_batch) * dim;
        const uint32_t *lm = lmod + opaque_zero();
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (FULL || lane + 64 * j < nch_row) {
                uint32_t tw[8];
                float sh[8];
                load_mod<MODL>(lm, shift, scale, moff, lane + 64 * j, dim, tw, sh);
                uint32_t y[4];
                if (AFF) lnaff8(xv[j], mean, rstd, tw, sh, y);
                else modln8(xv[j], -mean, rstd, tw, sh, one_lo, one_hi, y);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, y[k] & 0x7FFF7FFFu));
            }
        }
        if (lane == 0) {
            stats[2 * r] = mean;
            stats[2 * r + 1] = rstd;
        }
    };
    // two register buffers in turn: the next row's loads are in flight during a row's work
    u32x4 xa[NCH], xb[NCH];
    if (row < rows) load_row<NCH, FULL>(x, row, dim, lane, nch_row, xa);
    while (row < rows) {
        if (row + step < rows) load_row<NCH, FULL>(x, row + step, dim, lane, nch_row, xb);
        body(xa, row);
        row += step;
        if (row >= rows) break;
        if (row + step < rows) load_row<NCH, FULL>(x, row + step, dim, lane, nch_row, xa);
        body(xb, row);
        row += step;
    }
    uint32_t m = m2.x > m2.y ? m2.x : m2.y;
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    fold_amax(st, m, gridDim.x, kBF16, smax, red + kWaves);
}

// Pass 1 with one modulation row (MODL) and at most 10 chunks per lane (dim <= 5120).
// y = rnd(rnd(n * t) + shift) is, for each column, a monotone function of n (non-decreasing
// for t >= 0, non-increasing for t < 0: every step is a monotone fp32 operation followed by a
// monotone rounding), so over all rows max|y| of a column is |y| at the column's largest or
// smallest n.  The row loop computes n and folds it into the lane's per-column max and min
// (two packed ops per word instead of the modulation, the magnitude and the max); after the
// loop y is evaluated at the 2 x 8 extremes per chunk with the instructions pass 2 uses, so
// the amax is the same bits as the max over pass 2's y.
// Rows whose n could be non-finite (mean or rstd non-finite, or rstd = 0 from an overflowed
// variance, where (x - mean) * 0 can be NaN) are not folded: a wavefront that meets one
// re-reads all its rows after the loop and takes every y through the full chain, as the
// per-element pass does, so NaN rows give the same NaN bits.  One row in registers at a time:
// 151 VGPRs, 3 wavefronts per SIMD; 2 workgroups per CU stream x faster than 3 here.
template <int NCH>
__global__ __launch_bounds__(kTPB) __attribute__((amdgpu_waves_per_eu(3))) void k_modln_amax_ext(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ shift, const uint16_t *__restrict__ scale,
    int64_t rows, int dim, float eps, float *__restrict__ stats, State *__restrict__ st, float smax)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lmod[];
    __shared__ uint32_t red[kWaves + 2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch_row = dim >> 3;
    fill_mod<true>(lmod, shift, scale, dim);
    __syncthreads();
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m2 = {0, 0};
    const int64_t step = int64_t(gridDim.x) * kWaves;
    const int64_t row0 = int64_t(blockIdx.x) * kWaves + wave;
    const uint32_t one_lo = sgpr_word(kOneLo), one_hi = sgpr_word(kOneHi);
    uint32_t mx[NCH][4], mn[NCH][4];           // fp16 -Inf / +Inf patterns: replaced by the first row
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            mx[j][k] = 0xFC00FC00u;
            mn[j][k] = 0x7C007C00u;
        }
    bool folded = false, redo = false;         // wavefront-uniform
    for (int64_t row = row0; row < rows; row += step) {
        u32x4 xv[NCH];
        load_row<NCH, false>(x, row, dim, lane, nch_row, xv);
        float mean, rstd;
        row_stats<NCH, false>(xv, lane, nch_row, dim, eps, mean, rstd);
        if (lane == 0) {
            stats[2 * row] = mean;
            stats[2 * row + 1] = rstd;
        }
        if (__builtin_isfinite(mean) && __builtin_isfinite(rstd) && rstd > 0.0f) {
            folded = true;
            const float nmean = -mean;
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                if (lane + 64 * j < nch_row) {
                    const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
                    HIF8_DOT_SUB_MUL_EXT(w, one_lo, one_hi, nmean, rstd, mx[j], mn[j]);
                }
            }
        } else {
            redo = true;
        }
    }
    if (folded) {
        const uint32_t *lm = lmod + opaque_zero();
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (lane + 64 * j < nch_row) {
                uint32_t tw[8];
                float sh[8];
                load_mod<true>(lm, shift, scale, 0, lane + 64 * j, dim, tw, sh);
                uint32_t y[4], z[4];
                uy8(mx[j], tw, sh, one_lo, one_hi, y);
                uy8(mn[j], tw, sh, one_lo, one_hi, z);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, y[k] & 0x7FFF7FFFu));
                    m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, z[k] & 0x7FFF7FFFu));
                }
            }
            __builtin_amdgcn_sched_barrier(0);   // one chunk's modulation in registers at a time
        }
    }
    if (redo) {
        for (int64_t row = row0; row < rows; row += step) {
            u32x4 xv[NCH];
            load_row<NCH, false>(x, row, dim, lane, nch_row, xv);
            float mean, rstd;
            row_stats<NCH, false>(xv, lane, nch_row, dim, eps, mean, rstd);
            const uint32_t *lm = lmod + opaque_zero();
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                if (lane + 64 * j < nch_row) {
                    uint32_t tw[8];
                    float sh[8];
                    load_mod<true>(lm, shift, scale, 0, lane + 64 * j, dim, tw, sh);
                    uint32_t y[4];
                    modln8(xv[j], -mean, rstd, tw, sh, one_lo, one_hi, y);
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, y[k] & 0x7FFF7FFFu));
                }
            }
        }
    }
    uint32_t m = m2.x > m2.y ? m2.x : m2.y;
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    fold_amax(st, m, gridDim.x, kBF16, smax, red + kWaves);
}

// qdq of 8 bf16 values y through the codec's LDS tables (encode table + decode table), with
// the torch-semantics fix-ups (SEM_TORCH) or the scalar reference route (!FAST: a degenerate
// scale or a tensor not proven finite).
template <bool FAST>
__device__ __forceinline__ void qdq8_codec(const uint32_t (&y)[4], float s, int sem, const uint8_t *enc,
                                           const uint16_t *lut16, uint32_t (&out)[4])
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t r[2];
        if (FAST) {
            const uint32_t xs = f2bf_pk(bf2f(y[k] & 0xFFFFu) * s, u2f(y[k] & 0xFFFF0000u) * s);   // y * scale (bf16)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t xb = h ? (xs >> 16) : (xs & 0xFFFFu);
                const uint32_t u = xb & 0x7FFFu;
                uint32_t code = uint32_t(enc[clampu(u) - kTabLo]);
                code |= (code + 0x7Fu) & (xb >> 8) & 0x80u;                // sign; magnitude 0 stays 0
                uint32_t q = lut16[code];
                if (sem == kSemTorch && ((u != 0u && u < 0x3480u) || u >= 0x4720u))
                    q = f2bf(bf2f(f2bf(qdq_torch(bf2f(xb)))) / s);
                r[h] = q;
            }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t code;
                slow_elem<kBF16>(h ? (y[k] >> 16) : (y[k] & 0xFFFFu), s, sem, r[h], code);
            }
        }
        out[k] = r[0] | (r[1] << 16);
    }
}

// NPU semantics with a finite state: x_q as a function of y's magnitude bits alone.  The table
// holds |x_q| for the kYTab magnitudes ylo .. ylo + kYTab - 1; every smaller magnitude has
// y * s below the encode table (code 0, x_q = 0) and every larger one at or above its top
// (code Inf), which the builder checks, so clamping into the window is exact.
constexpr uint32_t kYTab = 5376;

__device__ __forceinline__ void qdq8_ytab(const uint32_t (&y)[4], uint32_t ylo, uint32_t yhi,
                                          const uint16_t *ytab, uint32_t (&out)[4])
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = min(max(y[k] & 0x7FFFu, ylo), yhi);
        const uint32_t b = min(max((y[k] >> 16) & 0x7FFFu, ylo), yhi);
        const uint32_t qq = uint32_t(ytab[a - ylo]) | (uint32_t(ytab[b - ylo]) << 16);
        out[k] = qq | ((qq + 0x7FFF7FFFu) & y[k] & 0x80008000u);       // sign; magnitude 0 stays +0
    }
}

// LDS of pass 2: the y-table, or the codec's decode table (512 B at kQdqLut) and encode table
// (indexed by clamped magnitude - kTabLo, at kQdqEnc).
constexpr uint32_t kQdqLut = 0;
constexpr uint32_t kQdqEnc = 512;
constexpr uint32_t kQdqLds = (kQdqEnc + sizeof(EncTable) > 2 * kYTab) ? kQdqEnc + sizeof(EncTable) : 2 * kYTab;

// MODE 0: y-table (NPU, finite); 1: codec tables (FAST); 2: scalar reference route.
template <int NCH, bool MODL, bool FULL, bool AFF, int MODE>
__device__ __forceinline__ void qdq_rows(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows,
                                         int dim, int64_t rows_per_batch, const float *stats, float s, int sem,
                                         uint16_t *xq, uint16_t *yout, const uint32_t *lmod, const uint8_t *lds,
                                         uint32_t ylo)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nch_row = dim >> 3;
    const uint16_t *lut16 = (const uint16_t *)(lds + kQdqLut);
    const uint8_t *enc = lds + kQdqEnc;
    const uint16_t *ytab = (const uint16_t *)lds;
    const uint32_t yhi = ylo + kYTab - 1;
    const int64_t step = int64_t(gridDim.x) * kWaves;
    int64_t row = int64_t(blockIdx.x) * kWaves + wave;
    const uint32_t one_lo = sgpr_word(kOneLo), one_hi = sgpr_word(kOneHi);
    auto body = [&](const u32x4 (&xv)[NCH], int64_t r) {
        const float mean = stats[2 * r], rstd = stats[2 * r + 1];
        const int64_t moff = MODL ? 0 : (r / rows_per_batch) * dim;
        const uint32_t *lm = lmod + opaque_zero();
        u32x4 *xo = (u32x4 *)(xq + r * dim);
        u32x4 *yo = yout ? (u32x4 *)(yout + r * dim) : nullptr;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (FULL || lane + 64 * j < nch_row) {
                const int c = lane + 64 * j;
                uint32_t tw[8];
                float sh[8];
                load_mod<MODL>(lm, shift, scale, moff, c, dim, tw, sh);
                uint32_t y[4], o[4];
                if (AFF) lnaff8(xv[j], mean, rstd, tw, sh, y);
                else modln8(xv[j], -mean, rstd, tw, sh, one_lo, one_hi, y);
                if (MODE == 0) qdq8_ytab(y, ylo, yhi, ytab, o);
                else qdq8_codec<MODE == 1>(y, s, sem, enc, lut16, o);
                // non-temporal: x_q is not read again here (8 % on the 14B producer's pass 2)
                __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, &xo[c]);
                if (yo) __builtin_nontemporal_store(u32x4{y[0], y[1], y[2], y[3]}, &yo[c]);
            }
        }
    };
    u32x4 xa[NCH], xb[NCH];
    if (row < rows) load_row<NCH, FULL>(x, row, dim, lane, nch_row, xa);
    while (row < rows) {
        if (row + step < rows) load_row<NCH, FULL>(x, row + step, dim, lane, nch_row, xb);
        body(xa, row);
        row += step;
        if (row >= rows) break;
        if (row + step < rows) load_row<NCH, FULL>(x, row + step, dim, lane, nch_row, xa);
        body(xb, row);
        row += step;
    }
}

// Pass 2: the same rows, statistics from pass 1, y recomputed and quantised.
// 3 wavefronts per SIMD (<= 168 VGPRs) where that fits without spills: enough rows in flight
// to stream at HBM rate.
template <int NCH, bool MODL> constexpr int qdq_waves() { return NCH > 10 ? 1 : (MODL ? 3 : 2); }

template <int NCH, bool MODL, bool FULL, bool AFF>
__global__ __launch_bounds__(kTPB) __attribute__((amdgpu_waves_per_eu(qdq_waves<NCH, MODL>()))) void k_modln_qdq(const uint16_t *__restrict__ x, const uint16_t *__restrict__ shift,
                                                     const uint16_t *__restrict__ scale, const float *__restrict__ lw,
                                                     const float *__restrict__ lb, int64_t rows, int dim,
                                                     int64_t rows_per_batch, const float *__restrict__ stats,
                                                     const State *__restrict__ st, int sem, uint16_t *__restrict__ xq,
                                                     uint16_t *__restrict__ yout)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[kQdqLds];
    __shared__ uint32_t ok;
    extern __shared__ __attribute__((aligned(16))) uint32_t lmod[];
    const int tid = threadIdx.x;
    const float s = st->scale;
    const bool fast = st->fast != 0 && st->finite != 0;
    if (AFF) fill_aff(lmod, lw, lb, dim);
    else fill_mod<MODL>(lmod, shift, scale, dim);
    uint32_t ylo = 0;
    bool use_ytab = fast && sem == kSemNpu;
    if (use_ytab) {
        // window start: a few magnitudes below the smallest y with y * s >= the table's bottom
        const uint32_t y0 = f2bf(bf2f(kTabLo) / s) & 0x7FFFu;
        ylo = y0 > 8u ? y0 - 8u : 0u;
        if (tid == 0) {
            const uint32_t top = ylo + kYTab - 1;
            const uint32_t top_xs = top < 0x7F80u ? (f2bf(bf2f(top) * s) & 0x7FFFu) : 0x7F80u;
            const uint32_t bot_xs = f2bf(bf2f(ylo) * s) & 0x7FFFu;
            ok = (top_xs >= kTabHi && bot_xs <= kTabLo) ? 1u : 0u;
        }
        uint16_t *ytab = (uint16_t *)lds;
        for (uint32_t i = tid; i < kYTab; i += kTPB) {
            const uint32_t ym = ylo + i < 0x7F80u ? ylo + i : 0x7F80u;
            const uint32_t u = f2bf(bf2f(ym) * s) & 0x7FFFu;
            ytab[i] = st->lut_bf16[kEncTable.v[clampu(u) - kTabLo]];
        }
        __syncthreads();
        use_ytab = ok != 0;
        __syncthreads();
    }
    if (!use_ytab) {
        ((uint16_t *)(lds + kQdqLut))[tid] = st->lut_bf16[tid];
        const uint4 *src = (const uint4 *)&kEncTable;
        uint4 *dst = (uint4 *)(lds + kQdqEnc);
        for (uint32_t i = tid; i < sizeof(EncTable) / 16; i += kTPB) dst[i] = src[i];
    }
    __syncthreads();
    if (use_ytab)
        qdq_rows<NCH, MODL, FULL, AFF, 0>(x, shift, scale, rows, dim, rows_per_batch, stats, s, sem, xq, yout, lmod, lds, ylo);
    else if (fast)
        qdq_rows<NCH, MODL, FULL, AFF, 1>(x, shift, scale, rows, dim, rows_per_batch, stats, s, sem, xq, yout, lmod, lds, ylo);
    else
        qdq_rows<NCH, MODL, FULL, AFF, 2>(x, shift, scale, rows, dim, rows_per_batch, stats, s, sem, xq, yout, lmod, lds, ylo);
}

static int cu_count()
{
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

static inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int check_args(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows, int64_t dim,
                      int64_t rows_per_batch, const void *stats, const void *state)
{
    if (!x || !stats || !state || rows <= 0 || dim <= 0 || rows_per_batch <= 0) return HIF8_ERR_ARG;
    if (dim % 8 != 0 || dim > 64 * 8 * kMaxChunks) return HIF8_ERR_SHAPE;
    if (rows > (int64_t(1) << 40)) return HIF8_ERR_SHAPE;
    if (!aligned16(x) || (shift && !aligned16(shift)) || (scale && !aligned16(scale))) return HIF8_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(stats) & 7u) != 0) return HIF8_ERR_ALIGN;
    return HIF8_OK;
}

// One modulation row for all of x (batch 1, the inference case) and dim <= 6144: t and shift
// as fp32 in LDS (8 * dim bytes, written once per workgroup); otherwise read per row.
static bool use_lds_modulation(int64_t rows, int64_t dim, int64_t rows_per_batch)
{
    return rows_per_batch >= rows && dim <= 6144;
}

static int grid_for_rows(int64_t rows, int wg_per_cu)
{
    const int64_t need = (rows + kWaves - 1) / kWaves;
    const int64_t cap = int64_t(cu_count()) * wg_per_cu;
    return int(need < cap ? need : cap);
}

// Instantiations: the model widths 1536 and 5120 without per-chunk bounds checks (FULL), any
// other width with the chunk count rounded up to a power of two; LDS modulation (MODL) only
// where it fits (dim <= 6144).
template <int NCH, bool FULL>
static void launch_amax(bool modl, int grid, hipStream_t s, const uint16_t *x, const uint16_t *shift,
                        const uint16_t *scale, int64_t rows, int dim, int64_t rpb, float eps, float *stats,
                        State *st, float smax)
{
    if constexpr (NCH <= 10) {
        if (modl) {
            const int g = grid_for_rows(rows, kExtWgPerCu);
            hipLaunchKernelGGL((k_modln_amax_ext<NCH>), dim3(g), dim3(kTPB), size_t(8 * dim), s, x, shift, scale,
                               rows, dim, eps, stats, st, smax);
            return;
        }
    } else if constexpr (NCH * 512 <= 6144) {
        if (modl) {
            hipLaunchKernelGGL((k_modln_amax<NCH, true, FULL, false>), dim3(grid), dim3(kTPB), size_t(8 * dim), s, x,
                               shift, scale, nullptr, nullptr, rows, dim, rpb, eps, stats, st, smax);
            return;
        }
    }
    hipLaunchKernelGGL((k_modln_amax<NCH, false, FULL, false>), dim3(grid), dim3(kTPB), 0, s, x, shift, scale,
                       nullptr, nullptr, rows, dim, rpb, eps, stats, st, smax);
}

template <int NCH, bool FULL>
static void launch_qdq(bool modl, int grid, hipStream_t s, const uint16_t *x, const uint16_t *shift,
                       const uint16_t *scale, int64_t rows, int dim, int64_t rpb, const float *stats, const State *st,
                       int sem, uint16_t *xq, uint16_t *y)
{
    if constexpr (NCH * 512 <= 6144) {
        if (modl) {
            hipLaunchKernelGGL((k_modln_qdq<NCH, true, FULL, false>), dim3(grid), dim3(kTPB), size_t(8 * dim), s, x,
                               shift, scale, nullptr, nullptr, rows, dim, rpb, stats, st, sem, xq, y);
            return;
        }
    }
    hipLaunchKernelGGL((k_modln_qdq<NCH, false, FULL, false>), dim3(grid), dim3(kTPB), 0, s, x, shift, scale,
                       nullptr, nullptr, rows, dim, rpb, stats, st, sem, xq, y);
}

// The affine LayerNorm: w and b in LDS (8 * dim bytes, sized at launch), dim <= kAffMaxDim
// (checked by the entry points; dims above 4096 other than 5120 take the 16-chunk instantiation).
constexpr int64_t kAffMaxDim = 6144;

template <int NCH, bool FULL>
static void launch_amax_aff(int grid, hipStream_t s, const uint16_t *x, const float *lw, const float *lb, int64_t rows,
                            int dim, float eps, float *stats, State *st, float smax)
{
    hipLaunchKernelGGL((k_modln_amax<NCH, true, FULL, true>), dim3(grid), dim3(kTPB), size_t(8 * dim), s, x, nullptr,
                       nullptr, lw, lb, rows, dim, rows, eps, stats, st, smax);
}

template <int NCH, bool FULL>
static void launch_qdq_aff(int grid, hipStream_t s, const uint16_t *x, const float *lw, const float *lb, int64_t rows,
                           int dim, const float *stats, const State *st, int sem, uint16_t *xq, uint16_t *y)
{
    hipLaunchKernelGGL((k_modln_qdq<NCH, true, FULL, true>), dim3(grid), dim3(kTPB), size_t(8 * dim), s, x, nullptr,
                       nullptr, lw, lb, rows, dim, rows, stats, st, sem, xq, y);
}

// Calls F<NCH, FULL>::run(args...) for the instantiation covering dim.
template <template <int, bool> class F, typename... A> static int dispatch_dim(int64_t dim, A... args)
{
    const int64_t nch = (dim / 8 + 63) / 64;
    if (dim == 1536) F<3, true>::run(args...);
    else if (dim == 5120) F<10, true>::run(args...);
    else if (nch <= 1) F<1, false>::run(args...);
    else if (nch <= 2) F<2, false>::run(args...);
    else if (nch <= 4) F<4, false>::run(args...);
    else if (nch <= 8) F<8, false>::run(args...);
    else if (nch <= 16) F<16, false>::run(args...);
    else return HIF8_ERR_SHAPE;
    return HIF8_OK;
}

// Pass 1 keeps the bounds-checked body at every width: without the checks the compiler
// schedules the whole row at once and needs more than 256 VGPRs.
template <int NCH, bool FULL> struct AmaxL {
    template <typename... A> static void run(A... a) { launch_amax<NCH, false>(a...); }
};
template <int NCH, bool FULL> struct QdqL {
    template <typename... A> static void run(A... a) { launch_qdq<NCH, FULL>(a...); }
};
template <int NCH, bool FULL> struct AmaxAffL {
    template <typename... A> static void run(A... a) { launch_amax_aff<NCH, false>(a...); }
};
template <int NCH, bool FULL> struct QdqAffL {
    template <typename... A> static void run(A... a) { launch_qdq_aff<NCH, FULL>(a...); }
};

// ---------------------------------------------------------------------------
// Workspace of hif8_modln_quant_static: the per-row statistics and the quantisation state of the
// modulated-LayerNorm producer in one file-scope device array instead of caller buffers, for
// callers that cannot allocate.  Each GPU holds its own copy until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a stand-in for the symbol):
// it uses the per-device address hipGetSymbolAddress returns.
constexpr int64_t kStaticMaxRows = 131072;                                  // 14B at 768P: 84672 rows
constexpr size_t kScratchStats = size_t(kStaticMaxRows) * 2 * sizeof(float);  // (mean, rstd) per row: 1 MiB
constexpr size_t kScratchBytes = kScratchStats + sizeof(State);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Clears the counters and scalars of the state in the workspace (the previous call leaves them
// zero unless it was interrupted); a fill kernel, so a captured graph holds no memset node.
__global__ void k_scratch_state_clear(State *st)
{
    if (threadIdx.x == 0) {
        st->counter = 0;
        st->amax_acc = 0;
        st->amax_bits = 0;
        st->scale = 0.0f;
        st->fast = 0;
        st->dtype = 0;
        st->finite = 0;
        st->pending = 0;
    }
}

static std::mutex g_scratch_mu;
static uint8_t *g_scratch_dev[64];

// The current device's address of the workspace, looked up once per device.
static int scratch_base(uint8_t **base)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return HIF8_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return HIF8_ERR_HIP;
        g_scratch_dev[dev] = (uint8_t *)p;
    }
    *base = g_scratch_dev[dev];
    return HIF8_OK;
}

}  // namespace norm
}  // namespace hif8

using namespace hif8;
using namespace hif8::norm;

extern "C" {

int hif8_modln_amax(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows, int64_t dim,
                    int64_t rows_per_batch, float eps, float *stats, float scale_max, void *state,
                    hif8_stream_t stream)
{
    const int rc = check_args(x, shift, scale, rows, dim, rows_per_batch, stats, state);
    if (rc != HIF8_OK) return rc;
    const bool modl = use_lds_modulation(rows, dim, rows_per_batch);
    const int st = dispatch_dim<AmaxL>(dim, modl, grid_for_rows(rows, kWgPerCu), (hipStream_t)stream, x, shift,
                                       scale, rows, int(dim), rows_per_batch, eps, stats, (State *)state, scale_max);
    if (st != HIF8_OK) return st;
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

int hif8_modln_fake_quant(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows, int64_t dim,
                          int64_t rows_per_batch, const float *stats, const void *state, int semantics,
                          uint16_t *x_q, uint16_t *y, hif8_stream_t stream)
{
    const int rc = check_args(x, shift, scale, rows, dim, rows_per_batch, stats, state);
    if (rc != HIF8_OK) return rc;
    if (!x_q || (semantics != HIF8_SEM_NPU && semantics != HIF8_SEM_TORCH)) return HIF8_ERR_ARG;
    if (!aligned16(x_q) || (y && !aligned16(y))) return HIF8_ERR_ALIGN;
    const bool modl = use_lds_modulation(rows, dim, rows_per_batch);
    const int st = dispatch_dim<QdqL>(dim, modl, grid_for_rows(rows, kQdqWgPerCu), (hipStream_t)stream, x, shift,
                                      scale, rows, int(dim), rows_per_batch, stats, (const State *)state, semantics,
                                      x_q, y);
    if (st != HIF8_OK) return st;
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

int hif8_modln_quant_static(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows,
                            int64_t dim, int64_t rows_per_batch, float eps, float scale_max, int semantics,
                            uint16_t *x_q, hif8_stream_t stream)
{
    if (!x || !x_q || rows <= 0 || dim <= 0 || rows_per_batch <= 0) return HIF8_ERR_ARG;
    if (semantics != HIF8_SEM_NPU && semantics != HIF8_SEM_TORCH) return HIF8_ERR_ARG;
    if (rows > kStaticMaxRows) return HIF8_ERR_SCRATCH;
    if (dim % 8 != 0 || dim > 64 * 8 * kMaxChunks) return HIF8_ERR_SHAPE;
    if (!aligned16(x) || !aligned16(x_q) || (shift && !aligned16(shift)) || (scale && !aligned16(scale)))
        return HIF8_ERR_ALIGN;
    uint8_t *base = nullptr;
    int rc = scratch_base(&base);
    if (rc != HIF8_OK) return rc;
    float *stats = (float *)base;
    State *st = (State *)(base + kScratchStats);
    rc = check_args(x, shift, scale, rows, dim, rows_per_batch, stats, st);
    if (rc != HIF8_OK) return rc;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_scratch_state_clear, dim3(1), dim3(64), 0, s, st);
    const bool modl = use_lds_modulation(rows, dim, rows_per_batch);
    rc = dispatch_dim<AmaxL>(dim, modl, grid_for_rows(rows, kWgPerCu), s, x, shift, scale, rows, int(dim),
                             rows_per_batch, eps, stats, st, scale_max);
    if (rc != HIF8_OK) return rc;
    rc = dispatch_dim<QdqL>(dim, modl, grid_for_rows(rows, kQdqWgPerCu), s, x, shift, scale, rows, int(dim),
                            rows_per_batch, (const float *)stats, (const State *)st, semantics, x_q,
                            (uint16_t *)nullptr);
    if (rc != HIF8_OK) return rc;
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

static int check_aff(const uint16_t *x, const float *weight, const float *bias, int64_t rows, int64_t dim,
                     const void *stats, const void *state)
{
    const int rc = check_args(x, nullptr, nullptr, rows, dim, rows, stats, state);
    if (rc != HIF8_OK) return rc;
    if (!weight || !bias) return HIF8_ERR_ARG;
    if (dim > kAffMaxDim) return HIF8_ERR_SHAPE;
    if (!aligned16(weight) || !aligned16(bias)) return HIF8_ERR_ALIGN;
    return HIF8_OK;
}

int hif8_ln_affine_amax(const uint16_t *x, const float *weight, const float *bias, int64_t rows, int64_t dim,
                        float eps, float *stats, float scale_max, void *state, hif8_stream_t stream)
{
    const int rc = check_aff(x, weight, bias, rows, dim, stats, state);
    if (rc != HIF8_OK) return rc;
    const int st = dispatch_dim<AmaxAffL>(dim, grid_for_rows(rows, kWgPerCu), (hipStream_t)stream, x, weight, bias,
                                          rows, int(dim), eps, stats, (State *)state, scale_max);
    if (st != HIF8_OK) return st;
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

int hif8_ln_affine_fake_quant(const uint16_t *x, const float *weight, const float *bias, int64_t rows, int64_t dim,
                              const float *stats, const void *state, int semantics, uint16_t *x_q, uint16_t *y,
                              hif8_stream_t stream)
{
    const int rc = check_aff(x, weight, bias, rows, dim, stats, state);
    if (rc != HIF8_OK) return rc;
    if (!x_q || (semantics != HIF8_SEM_NPU && semantics != HIF8_SEM_TORCH)) return HIF8_ERR_ARG;
    if (!aligned16(x_q) || (y && !aligned16(y))) return HIF8_ERR_ALIGN;
    const int st = dispatch_dim<QdqAffL>(dim, grid_for_rows(rows, kQdqWgPerCu), (hipStream_t)stream, x, weight, bias,
                                         rows, int(dim), stats, (const State *)state, semantics, x_q, y);
    if (st != HIF8_OK) return st;
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

}  // extern "C"
