// HiF8 per-tensor quantisation kernels for MI355X (gfx950): amax + scale,
// encode to 8-bit codes, fake-quant (qdq) and decode.  C ABI at the bottom;
// declarations and reference citations in include/hif8_mi355x.h.
//
// Data layout: a quantised tensor is its original buffer plus a State (device
// memory, caller-owned) holding amax, scale and two 256-entry decode tables
// x_q(code).  Codes are one byte per element in the input's element order.
//
// Bandwidth design: each thread moves 16 elements per step with 128-bit loads
// and stores (bf16: 2 x 16 B in, 16 B of codes out); the code of an element is
// an LDS table lookup indexed by the bf16 magnitude bits of x*scale, so the
// per-element ALU work is a multiply, a packed bf16 convert, a clamp and one
// ds_read_u8.  amax is one read pass with packed u16 max and one atomic per
// workgroup; the last workgroup computes the scale and the decode tables.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_common.h"
#include "hif8_internal.h"
#include "hif8_state_dev.h"
#include "hif8_qdq_dev.h"
#include "hif8_gelu_dev.h"

namespace hif8 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- kernels

__global__ void k_state_init(State *st)
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

__global__ __launch_bounds__(256) void k_set_scale(State *st, int dtype, float s)
{
    uint32_t c = threadIdx.x;
    if (c == 0) {
        st->scale = s;
        st->dtype = uint32_t(dtype);
        st->fast = (__builtin_isfinite(s) && s > 0.0f) ? 1u : 0u;
        st->finite = 0;   // no amax pass: inputs may hold NaN
        st->amax_bits = 0;
        st->pending = 0;
    }
    fill_luts(st, s, c);
}

constexpr int kTPB = 256;

// Streaming access: the codec reads each input element once, so its global loads carry
// the non-temporal hint (measured on the 774 MB 14B activation: amax 4.98 -> 6.5 TB/s).
// Code output (1 B/element) is stored the same way; bf16/fp32 qdq output is stored
// normally, which measured faster for it.
template <typename T> __device__ __forceinline__ T ld_stream(const T *p)
{
    return __builtin_nontemporal_load(p);
}
template <typename T> __device__ __forceinline__ void st_stream(T *p, const T &v)
{
    __builtin_nontemporal_store(v, p);
}

// One pass of |x| max.  Magnitude bit patterns order like the values and put
// NaN above Inf, so an unsigned max propagates NaN as torch's amax does.
template <int DT>
__global__ __launch_bounds__(kTPB) void k_absmax(const void *__restrict__ xv, int64_t n,
                                                  State *__restrict__ st, float smax)
{
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    const int tid = threadIdx.x;
    uint32_t m = 0;
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    if (DT != kF32) {
        const uint16_t *x = (const uint16_t *)xv;
        const int64_t nvec = n >> 3;                       // uint4 = 8 bf16
        const u32x4 *xq = (const u32x4 *)x;
        u16x2 acc = {0, 0};
        int64_t i = int64_t(blockIdx.x) * kTPB + tid;
        for (; i + 7 * stride < nvec; i += 8 * stride) {
            u32x4 v0 = ld_stream(&xq[i]);
            u32x4 v1 = ld_stream(&xq[i + stride]);
            u32x4 v2 = ld_stream(&xq[i + 2 * stride]);
            u32x4 v3 = ld_stream(&xq[i + 3 * stride]);
            u32x4 v4 = ld_stream(&xq[i + 4 * stride]);
            u32x4 v5 = ld_stream(&xq[i + 5 * stride]);
            u32x4 v6 = ld_stream(&xq[i + 6 * stride]);
            u32x4 v7 = ld_stream(&xq[i + 7 * stride]);
#define HIF8_ACC(v)                                                                          \
    acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, (v).x & 0x7FFF7FFFu));   \
    acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, (v).y & 0x7FFF7FFFu));   \
    acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, (v).z & 0x7FFF7FFFu));   \
    acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, (v).w & 0x7FFF7FFFu));
            HIF8_ACC(v0) HIF8_ACC(v1) HIF8_ACC(v2) HIF8_ACC(v3)
            HIF8_ACC(v4) HIF8_ACC(v5) HIF8_ACC(v6) HIF8_ACC(v7)
        }
        for (; i < nvec; i += stride) {
            u32x4 v0 = xq[i];
            HIF8_ACC(v0)
        }
#undef HIF8_ACC
        m = acc.x > acc.y ? acc.x : acc.y;
        for (int64_t j = (nvec << 3) + int64_t(blockIdx.x) * kTPB + tid; j < n; j += stride) {
            uint32_t b = x[j] & 0x7FFFu;
            m = b > m ? b : m;
        }
    } else {
        const uint32_t *x = (const uint32_t *)xv;
        const int64_t nvec = n >> 2;
        const u32x4 *xq = (const u32x4 *)x;
        int64_t i = int64_t(blockIdx.x) * kTPB + tid;
        uint32_t m0 = 0, m1 = 0;
        for (; i + 3 * stride < nvec; i += 4 * stride) {
            u32x4 v0 = ld_stream(&xq[i]);
            u32x4 v1 = ld_stream(&xq[i + stride]);
            u32x4 v2 = ld_stream(&xq[i + 2 * stride]);
            u32x4 v3 = ld_stream(&xq[i + 3 * stride]);
            m0 = max(m0, max(max(v0.x & 0x7FFFFFFFu, v0.y & 0x7FFFFFFFu), max(v0.z & 0x7FFFFFFFu, v0.w & 0x7FFFFFFFu)));
            m1 = max(m1, max(max(v1.x & 0x7FFFFFFFu, v1.y & 0x7FFFFFFFu), max(v1.z & 0x7FFFFFFFu, v1.w & 0x7FFFFFFFu)));
            m0 = max(m0, max(max(v2.x & 0x7FFFFFFFu, v2.y & 0x7FFFFFFFu), max(v2.z & 0x7FFFFFFFu, v2.w & 0x7FFFFFFFu)));
            m1 = max(m1, max(max(v3.x & 0x7FFFFFFFu, v3.y & 0x7FFFFFFFu), max(v3.z & 0x7FFFFFFFu, v3.w & 0x7FFFFFFFu)));
        }
        for (; i < nvec; i += stride) {
            u32x4 v0 = xq[i];
            m0 = max(m0, max(max(v0.x & 0x7FFFFFFFu, v0.y & 0x7FFFFFFFu), max(v0.z & 0x7FFFFFFFu, v0.w & 0x7FFFFFFFu)));
        }
        m = max(m0, m1);
        for (int64_t j = (nvec << 2) + int64_t(blockIdx.x) * kTPB + tid; j < n; j += stride)
            m = max(m, x[j] & 0x7FFFFFFFu);
    }
    // wavefront reduction, then across the 4 waves through LDS
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
    __shared__ uint32_t red[kTPB / 64 + 2];
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    // bf16 held as fp32: the fp32 magnitude bits of the same value (NaN stays above Inf)
    if (DT == kBF16F32) fold_amax(st, m << 16, gridDim.x, kF32, smax, red + kTPB / 64);
    else fold_amax(st, m, gridDim.x, DT, smax, red + kTPB / 64);
}

// Element j of k_quant through the scalar reference route.
template <int DT, int MODE>
__device__ __forceinline__ void scalar_elem(const void *xv, void *outv, int64_t j, float s, int sem)
{
    uint32_t xb, yb, code;
    if (DT == kBF16) {
        xb = ((const uint16_t *)xv)[j];
        slow_elem<kBF16>(xb, s, sem, yb, code);
    } else {
        xb = DT == kF32 ? ((const uint32_t *)xv)[j] : uint32_t(((const uint16_t *)xv)[j]) << 16;
        slow_elem<kF32>(xb, s, sem, yb, code);
        if (MODE == 3) yb = f2bf(u2f(yb));
    }
    if (MODE == 0) ((uint8_t *)outv)[j] = uint8_t(code);
    else if (DT == kBF16 || MODE == 3) ((uint16_t *)outv)[j] = uint16_t(yb);
    else ((uint32_t *)outv)[j] = yb;
}

// MODE 0: codes, MODE 1: qdq in the arithmetic dtype (bf16 for kBF16, fp32 otherwise),
// MODE 2: decode codes -> x_q, MODE 3: qdq rounded to the bf16 GEMM operand.
// DT kBF16F32 loads bf16 and computes as kF32 on the exact fp32 values.
// span > 0: workgroup b quantises the span * TPB consecutive 16-element groups from
// b * span * TPB on (the grid covers the tensor once, in dispatch order, so the groups in flight
// at any time lie in one moving window of memory); span 0: a grid-stride loop.
template <int DT, int MODE, int TPB = kTPB>
__global__ __launch_bounds__(TPB) void k_quant(const void *__restrict__ xv, int64_t n,
                                                 const State *__restrict__ st, void *__restrict__ outv,
                                                 int sem, int use_state, int span)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    const int tid = threadIdx.x;
    const int64_t ngrp = n >> 4;  // 16 elements per step
    const int64_t stride = int64_t(gridDim.x) * TPB;
    // This workgroup's iterations: base G0 (a multiple of 256 groups) from i0 in steps of istep
    // while G0 < iend.  In the quantise modes thread tid's input chunk j (16 bytes) of an iteration
    // is chunk G0 * kVec + j * 256 + tid of the tensor, so every load and store instruction of a
    // wave covers one contiguous span (the operation is elementwise: which 16 elements a thread
    // holds does not matter); chunks past the last whole group are masked.  The decode mode keeps
    // one 16-code group per thread (g = G0 + tid).
    const int64_t i0 = span ? int64_t(blockIdx.x) * span * TPB : int64_t(blockIdx.x) * TPB;
    const int64_t istep = span ? int64_t(TPB) : stride;
    const int64_t iend = span ? (i0 + int64_t(span) * TPB < ngrp ? i0 + int64_t(span) * TPB : ngrp) : ngrp;
    constexpr int kVec = DT == kF32 ? 4 : 2;      // 16-byte input chunks per 16 elements
    constexpr int kIpc = 16 / kVec;              // elements per input chunk
    const int64_t nchunk = ngrp * kVec;
    const u32x4 *xq = (const u32x4 *)xv;
    // the first iteration's input is requested before the tables are set up, so its latency
    // overlaps the table loads and the barrier
    u32x4 pre[4] = {};
    if (MODE != 2 && i0 < iend) {
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            const int64_t c = i0 * kVec + j * TPB + tid;
            if (c < nchunk) pre[j] = ld_stream(&xq[c]);
        }
    }
    float s = use_state ? st->scale : 1.0f;
    bool fast = use_state ? (st->fast != 0) : true;
    // NaN inputs map to the +Inf entry of the table; unless an amax pass proved
    // the tensor finite, each 16-element group is checked and patched to kNanCode.
    const bool nan_guard = use_state ? (st->finite == 0) : true;
    // decode tables for this scale
    if (tid < 256) {
        uint32_t c = uint32_t(tid);
        float y;
        if (use_state) y = st->lut_f32[c];
        else y = u2f(decode_bits(c));
        ((float *)(lds + kLdsLutF32))[c] = y;
        ((uint16_t *)(lds + kLdsLutBf16))[c] = use_state ? st->lut_bf16[c] : uint16_t(f2bf(y));
    }
    if (MODE != 2) {
        const uint4 *src = (const uint4 *)&kEncTable;
        uint4 *dst = (uint4 *)(lds + kTabLo);
        for (uint32_t i = tid; i < sizeof(EncTable) / 16; i += TPB) dst[i] = src[i];
    }
    __syncthreads();
    const uint16_t *lut16 = (const uint16_t *)(lds + kLdsLutBf16);
    const float *lut32 = (const float *)(lds + kLdsLutF32);

    if (MODE == 2) {
        // decode: 16 codes -> 16 outputs per thread and iteration, in chunks of 8 codes (bf16
        // out, 16 bytes each) or 4 codes (fp32 out), chunk j at G0 * kOc + j * TPB + tid so that
        // the loads and stores of a wave are contiguous
        constexpr int kOc = DT == kBF16 ? 2 : 4;     // output chunks of 16 bytes per 16 codes
        const int64_t noc = ngrp * kOc;
        for (int64_t G0 = i0; G0 < iend; G0 += istep) {
#pragma unroll
            for (int j = 0; j < kOc; ++j) {
                const int64_t c = G0 * kOc + j * TPB + tid;
                if (c >= noc) continue;
                if (DT == kBF16) {
                    const u32x2 cw = ((const u32x2 *)xv)[c];
                    uint32_t o[4];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t d = cw[h];
                        o[2 * h] = uint32_t(lut16[d & 0xFF]) | (uint32_t(lut16[(d >> 8) & 0xFF]) << 16);
                        o[2 * h + 1] = uint32_t(lut16[(d >> 16) & 0xFF]) | (uint32_t(lut16[d >> 24]) << 16);
                    }
                    st_stream(&((u32x4 *)outv)[c], u32x4{o[0], o[1], o[2], o[3]});
                } else {
                    const uint32_t d = ((const uint32_t *)xv)[c];
                    st_stream(&((u32x4 *)outv)[c], u32x4{f2u(lut32[d & 0xFF]), f2u(lut32[(d >> 8) & 0xFF]),
                                                         f2u(lut32[(d >> 16) & 0xFF]), f2u(lut32[d >> 24])});
                }
            }
        }
        for (int64_t j = (ngrp << 4) + int64_t(blockIdx.x) * TPB + tid; j < n; j += stride) {
            uint32_t c = ((const uint8_t *)xv)[j];
            if (DT == kBF16) ((uint16_t *)outv)[j] = lut16[c];
            else ((float *)outv)[j] = lut32[c];
        }
        return;
    }

    const bool out16 = DT == kBF16 || MODE == 3;  // bf16 output (MODE 1/3)
    if (fast) {
        // the next iteration's input is loaded one iteration ahead (two in flight)
        for (int64_t G0 = i0; G0 < iend; G0 += istep) {
            uint32_t codes[4];
            uint32_t wide[16];   // per element: magnitude bits of xs, and the full bits for fp32
            uint32_t xs_full[16];
            u32x4 cur[4] = {pre[0], pre[1], pre[2], pre[3]};
            if (G0 + istep < iend) {
#pragma unroll
                for (int j = 0; j < kVec; ++j) {
                    const int64_t c = (G0 + istep) * kVec + j * TPB + tid;
                    pre[j] = c < nchunk ? ld_stream(&xq[c]) : u32x4{0u, 0u, 0u, 0u};
                }
            }
            if (DT == kBF16F32) {
                // the 16 bf16 values as the fp32 words x.float() holds
                const uint32_t p[8] = {cur[0].x, cur[0].y, cur[0].z, cur[0].w, cur[1].x, cur[1].y, cur[1].z, cur[1].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    cur[j] = u32x4{p[2 * j] << 16, p[2 * j] & 0xFFFF0000u, p[2 * j + 1] << 16, p[2 * j + 1] & 0xFFFF0000u};
            }
            if (DT == kBF16) {
                u32x4 a = cur[0];
                u32x4 b = cur[1];
                uint32_t p[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t p0 = p[2 * j], p1 = p[2 * j + 1];
                    uint32_t q01 = f2bf_pk(u2f(p0 << 16) * s, u2f(p0 & 0xFFFF0000u) * s);
                    uint32_t q23 = f2bf_pk(u2f(p1 << 16) * s, u2f(p1 & 0xFFFF0000u) * s);
                    uint32_t u0 = q01 & 0x7FFFu, u1 = (q01 >> 16) & 0x7FFFu;
                    uint32_t u2 = q23 & 0x7FFFu, u3 = (q23 >> 16) & 0x7FFFu;
                    wide[4 * j] = u0; wide[4 * j + 1] = u1; wide[4 * j + 2] = u2; wide[4 * j + 3] = u3;
                    xs_full[4 * j] = q01 & 0xFFFFu; xs_full[4 * j + 1] = q01 >> 16;
                    xs_full[4 * j + 2] = q23 & 0xFFFFu; xs_full[4 * j + 3] = q23 >> 16;
                    uint32_t mags = uint32_t(lds[clampu(u0)]) | (uint32_t(lds[clampu(u1)]) << 8) |
                                    (uint32_t(lds[clampu(u2)]) << 16) | (uint32_t(lds[clampu(u3)]) << 24);
                    uint32_t signs = __builtin_amdgcn_perm(p1, p0, 0x07050301u) & 0x80808080u;
                    codes[j] = apply_signs(mags, signs);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x4 a = cur[j];
                    uint32_t v[4] = {a.x, a.y, a.z, a.w};
                    uint32_t mags = 0;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        uint32_t xs = f2u(u2f(v[t]) * s);
                        xs_full[4 * j + t] = xs;
                        uint32_t u = (xs >> 16) & 0x7FFFu;
                        wide[4 * j + t] = u;
                        mags |= uint32_t(lds[clampu(u)]) << (8 * t);
                    }
                    uint32_t signs = __builtin_amdgcn_perm(v[3], v[2], 0x07030C0Cu) & 0x80800000u;
                    signs |= (__builtin_amdgcn_perm(v[1], v[0], 0x0C0C0703u) & 0x00008080u);
                    codes[j] = apply_signs(mags, signs);
                }
            }
            if (nan_guard) {
                uint32_t mx = 0;
#pragma unroll
                for (int t = 0; t < 16; ++t) mx = wide[t] > mx ? wide[t] : mx;
                if (mx > 0x7F80u) {
#pragma unroll
                    for (int t = 0; t < 16; ++t)
                        if (wide[t] > 0x7F80u) codes[t >> 2] = (codes[t >> 2] & ~(0xFFu << (8 * (t & 3)))) | (kNanCode << (8 * (t & 3)));
                }
            }
            if (MODE == 0) {
                // chunk j's kIpc codes are bytes j * kIpc .. of codes[]
#pragma unroll
                for (int j = 0; j < kVec; ++j) {
                    const int64_t c = G0 * kVec + j * TPB + tid;
                    if (c >= nchunk) continue;
                    if (kIpc == 8) st_stream(&((u32x2 *)outv)[c], u32x2{codes[2 * j], codes[2 * j + 1]});
                    else st_stream(&((uint32_t *)outv)[c], codes[j]);
                }
                continue;
            }
            // qdq output through the decode table
            uint32_t y[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t d = codes[j];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint32_t c = (d >> (8 * t)) & 0xFF;
                    y[4 * j + t] = out16 ? uint32_t(lut16[c]) : f2u(lut32[c]);
                }
            }
            if (sem == kSemTorch) {
                // the torch route differs only below 2^-22 (non-zero) and from 40960 up
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    uint32_t u = wide[t];
                    uint32_t full = DT == kBF16 ? (xs_full[t] & 0x7FFFu) : (xs_full[t] & 0x7FFFFFFFu);
                    if ((full != 0u && u < 0x3480u) || u >= 0x4720u) {
                        float xs = DT == kBF16 ? bf2f(xs_full[t]) : u2f(xs_full[t]);
                        float q = qdq_torch(xs);
                        if (DT == kBF16) y[t] = f2bf(bf2f(f2bf(q)) / s);
                        else if (MODE == 3) y[t] = f2bf(q / s);
                        else y[t] = f2u(q / s);
                    }
                }
            }
            // chunk j's outputs are y[j * kIpc ..], at chunk c of the output's own element size
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                const int64_t c = G0 * kVec + j * TPB + tid;
                if (c >= nchunk) continue;
                const uint32_t *yj = y + j * kIpc;
                if (out16 && kIpc == 8) {
                    st_stream(&((u32x4 *)outv)[c], u32x4{yj[0] | (yj[1] << 16), yj[2] | (yj[3] << 16),
                                                         yj[4] | (yj[5] << 16), yj[6] | (yj[7] << 16)});
                } else if (out16) {
                    st_stream(&((u32x2 *)outv)[c], u32x2{yj[0] | (yj[1] << 16), yj[2] | (yj[3] << 16)});
                } else if (kIpc == 4) {
                    st_stream(&((u32x4 *)outv)[c], u32x4{yj[0], yj[1], yj[2], yj[3]});
                } else {
                    st_stream(&((u32x4 *)outv)[2 * c], u32x4{yj[0], yj[1], yj[2], yj[3]});
                    st_stream(&((u32x4 *)outv)[2 * c + 1], u32x4{yj[4], yj[5], yj[6], yj[7]});
                }
            }
        }
    } else {
        // degenerate scale (amax Inf/NaN, scale 0/Inf/NaN): element-wise reference route, a
        // grid-stride loop over the elements (each visited once whatever the grid)
        for (int64_t j = int64_t(blockIdx.x) * TPB + tid; j < (ngrp << 4); j += stride)
            scalar_elem<DT, MODE>(xv, outv, j, s, sem);
    }
    // tail (n % 16) through the scalar route
    for (int64_t j = (ngrp << 4) + int64_t(blockIdx.x) * TPB + tid; j < n; j += stride)
        scalar_elem<DT, MODE>(xv, outv, j, s, sem);
}

// QFuncs/hif8.py:6-23 evaluated on a bf16 tensor without force_fp32 (quant_dequant_float with
// force_py=True, force_fp32=False, QTensor.py:99-102,118-119): each torch op on bf16 computes in
// fp32 and rounds its result to bf16.  bf16 bits in, bf16 bits out.  Roundings that can change
// the result are those of |x| + 2^-45, of log2 and of x * 2^(mb - e) + 0.5 (below 2^-43 only);
// the other ops are exact in bf16.  For every bf16 input, log2 of the rounded |x| + 2^-45 lies at
// least 10 fp32 ulps from a bf16 rounding boundary, so any faithfully rounded log2f gives the
// bf16 value torch's log2 gives.
static __device__ uint32_t qdq_torch_bf16(uint32_t xb)
{
    const float x = bf2f(xb);
    const float xu = fabsf(x);
    if (!(xu <= 3.402823466e38f)) return 0x7FC0u;                  // NaN, Inf -> NaN
    const float sign = float(x > 0.0f) - float(x < 0.0f);
    const float t = bf2f(f2bf(xu + 0x1p-45f));                      // x_unsigned + 2**-45
    const int e = int(__builtin_floorf(bf2f(f2bf(log2f(t)))));     // floor(log2(.))
    const int ae = e < 0 ? -e : e;
    const int mb = ae <= 3 ? 3 : ae <= 7 ? 2 : ae <= 15 ? 1 : 0;
    const float m = bf2f(f2bf(xu * __builtin_ldexpf(1.0f, mb - e)));    // x_unsigned * 2**(-e + mb)
    const float f = __builtin_floorf(bf2f(f2bf(m + 0.5f)));             // floor(. + 0.5)
    const float r = bf2f(f2bf(f * __builtin_ldexpf(1.0f, e - mb)));     // * 2**(e - mb)
    return f2bf(r * sign);                                              // * sign
}

// amax|GELU(y)| of a bf16 tensor folded into st with the scale rule for smax: hif8_absmax_scale
// of the GELU layer's output, without writing it.  With only_pending, a state whose GELU
// statistic settled the amax (pending == 0, written by the up-projection's GEMM) is left as it
// is and every workgroup returns at once; all workgroups read the same flag before any of them
// folds, so they all take the same branch.
__global__ __launch_bounds__(kTPB) void k_gelu_absmax(const uint16_t *__restrict__ y, int64_t n,
                                                      State *__restrict__ st, float smax, int only_pending)
{
    if (only_pending && st->pending == 0) return;
    const int tid = threadIdx.x;
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    const int64_t nvec = n >> 3;
    const u32x4 *yq = (const u32x4 *)y;
    uint32_t m = 0;
    for (int64_t i = int64_t(blockIdx.x) * kTPB + tid; i < nvec; i += stride) {
        const u32x4 v = ld_stream(&yq[i]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = gelu_bf16x2(v[t]) & 0x7FFF7FFFu;
            m = max(m, max(w & 0xFFFFu, w >> 16));
        }
    }
    for (int64_t j = (nvec << 3) + int64_t(blockIdx.x) * kTPB + tid; j < n; j += stride)
        m = max(m, gelu_bf16(y[j]) & 0x7FFFu);
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
    __shared__ uint32_t red[kTPB / 64 + 2];
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    fold_amax(st, m, gridDim.x, kBF16, smax, red + kTPB / 64);
}

// The state after a GELU-statistic GEMM: amax|GELU(y)| from max y, or pending.
// g = GELU(y) through the window table, 8 values per thread and step.
__global__ __launch_bounds__(kTPB) void k_gelu_bf16(const uint16_t *__restrict__ y, uint16_t *__restrict__ g, int64_t n)
{
    __shared__ __attribute__((aligned(16))) uint16_t win[2 * kGeluWinN];
    gelu_win_fill(win, threadIdx.x, kTPB);
    __syncthreads();
    const int64_t n8 = n >> 3;
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    auto gel = [&](uint32_t w) {   // words with an Inf or NaN take the evaluation itself
        const uint32_t e = ((w & 0x7F807F80u) + 0x00800080u) & 0x80008000u;
        return e ? gelu_bf16x2(w) : gelu_win_bf16x2(w, win);
    };
    for (int64_t i = int64_t(blockIdx.x) * kTPB + threadIdx.x; i < n8; i += stride) {
        const u32x4 v = ld_stream(&((const u32x4 *)y)[i]);
        ((u32x4 *)g)[i] = u32x4{gel(v.x), gel(v.y), gel(v.z), gel(v.w)};
    }
    for (int64_t j = (n8 << 3) + int64_t(blockIdx.x) * kTPB + threadIdx.x; j < n; j += stride)
        g[j] = uint16_t(gel(y[j]) & 0xFFFFu);
}

// ---------------------------------------------------------------------------------------------
// x_q = qdq(GELU(y) * s) / s of a bf16 y (the down-projection's _quant of the GELU layer's
// output) through a table of x_q over y.  For a state with a finite scale, proven finite by its
// amax pass (GELU(y) finite, hence y finite), x_q is a function of y's 16 bits; per sign it is
// constant below the smallest magnitude whose GELU quantises to a non-zero code and above the
// magnitude where it saturates (and, for y < 0, from -6 on, where GELU(y) is -0), so over the
// HiF8 range -- about 39 binades, some 5000 magnitudes -- it is tabled, with one entry for
// y = +-0 and one for the constant run below.  k_gelu_quant_prep (one workgroup, launched before
// every pass) finds the bounds -- a parallel search over the binades, then within one: x_q is
// monotone in |y| there -- and fills the table into the state with the per-element route (GELU
// through its window table, then the codec's table route: the bits of slow_elem).  k_gelu_quant
// copies it to LDS and maps 16 inputs per thread and step with a clamp and a lookup each, about
// 6 VALU operations per element against the 25 of GELU plus the codec.  States without a proven
// finite input, or a degenerate scale, take the per-element reference route.
constexpr uint32_t kGqWinOff = 2048;   // gelu_bf16 window table, in the gap of the codec's LDS map
static_assert(kGqWinOff + 4 * kGeluWinN <= kTabLo, "GELU window table overlaps the encode table");
// GELU(y) = -0 for y <= -6 (0xC0C0): the window table's edge, checked for every input by a test
// (torch's CPU evaluation reaches -0 from -5.06, the device's rounding of 1 + tanh(u) later)
constexpr uint32_t kGeluNegZero = kGeluWinHi;
constexpr int kGqPrepTPB = 1024;

// x_q(GELU(y)) of one finite bf16 input, through the window table and the codec's table route
__device__ __forceinline__ uint32_t gq_eval(uint32_t yb, float s, int sem, const uint8_t *lds)
{
    const uint32_t g = gelu_win_bf16x2(yb, (const uint16_t *)(lds + kGqWinOff)) & 0xFFFFu;
    return fast_elem_bf16<kBF16>(bf2f(g), s, sem, lds, false);
}

// The state's table for its scale and sem (one workgroup of kGqPrepTPB threads).
__global__ __launch_bounds__(kGqPrepTPB) void k_gelu_quant_prep(State *__restrict__ st, int sem)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    __shared__ uint32_t bnd[8];
    const uint32_t tid = threadIdx.x;
    const float s = st->scale;
    if (!(st->fast != 0 && st->finite != 0)) {
        if (tid == 0) st->gq[0] = 0u;
        return;
    }
    // codec tables (bf16 decode table and encode table) and the GELU window table
    if (tid < 256) ((uint16_t *)(lds + kLdsLutBf16))[tid] = st->lut_bf16[tid];
    {
        const uint4 *src = (const uint4 *)&kEncTable;
        uint4 *dst = (uint4 *)(lds + kTabLo);
        for (uint32_t i = tid; i < sizeof(EncTable) / 16; i += kGqPrepTPB) dst[i] = src[i];
    }
    gelu_win_fill((uint16_t *)(lds + kGqWinOff), tid, kGqPrepTPB);
    if (tid == 0) {
        bnd[0] = 0x7F80u;   // T: first binade start m = 128 t with f+(m) != f+(1)
        bnd[1] = 0u;        // U: last binade start with f+(m) != f+(0x7F7F)
        bnd[2] = 0x3B01u;   // V: first binade start up to 0x3B00 with f-(m) != f-(1) (none: 0x3B01)
    }
    __syncthreads();
    // f+(m) = x_q(GELU(m)), f-(m) = x_q(GELU(-m)).  f+ is monotone in m; so is f- below the GELU
    // window, where GELU(-m) = rnd(-m / 2); f-(m) = x_q(-0) from kGeluNegZero on.
    const uint32_t f1p = gq_eval(1u, s, sem, lds), ftp = gq_eval(0x7F7Fu, s, sem, lds);
    const uint32_t f1n = gq_eval(0x8001u, s, sem, lds);
    if (tid >= 1 && tid < 255) {
        const uint32_t m = tid << 7;
        const uint32_t v = gq_eval(m, s, sem, lds);
        if (v != f1p) atomicMin(&bnd[0], m);
        if (v != ftp) atomicMax(&bnd[1], m);
    } else if (tid >= 257 && tid <= 256 + 0x3B00u / 128u) {
        const uint32_t m = (tid - 256u) << 7;
        if (gq_eval(0x8000u | m, s, sem, lds) != f1n) atomicMin(&bnd[2], m);
    }
    __syncthreads();
    const uint32_t T = bnd[0], U = bnd[1], V = bnd[2];
    if (tid == 0) {
        bnd[4] = T;                                           // lo+ <= T (T differs, or is the top)
        bnd[5] = U + 128u < 0x7F7Fu ? U + 128u : 0x7F7Fu;     // hi+ <= U + 128 (equal to f+(top))
        bnd[6] = V;                                           // lo- <= V
    }
    __syncthreads();
    // within one binade: lo+ in (T - 128, T], hi+ in (U, U + 128], lo- in (V - 128, V]
    if (tid < 128) {
        const uint32_t m = T - 127u + tid;
        if (m < T && m <= 0x7F7Fu && gq_eval(m, s, sem, lds) != f1p) atomicMin(&bnd[4], m);
    } else if (tid < 256) {
        const uint32_t m = U + 1u + (tid - 128u);
        if (m < bnd[5] && gq_eval(m, s, sem, lds) == ftp) atomicMin(&bnd[5], m);
    } else if (tid < 384 && V < 0x3B01u) {
        const uint32_t m = V - 127u + (tid - 256u);
        if (m < V && gq_eval(0x8000u | m, s, sem, lds) != f1n) atomicMin(&bnd[6], m);
    }
    __syncthreads();
    // table over [lo, hi]: entry 0 is m = 0, entry 1 every 0 < m < lo, entry 2 + k m = lot + k.
    // A range past the table's capacity (scales far outside the model's) tables its top part from
    // lot, and the pass evaluates inputs in [lo, lot) element by element.
    uint32_t lo = bnd[4] < bnd[6] ? bnd[4] : bnd[6];
    lo = lo > 2u ? lo : 2u;
    const uint32_t hi = bnd[5] > kGeluNegZero ? bnd[5] : kGeluNegZero;
    const uint32_t lot = hi + 3u - lo > kGqCap ? hi + 3u - kGqCap : lo;
    const uint32_t top = 2u + hi - lot;
    for (uint32_t e = tid; e <= top; e += kGqPrepTPB) {
        const uint32_t m = e < 2u ? e : lot + e - 2u;
        // GELU of +m and -m in one packed evaluation, then the codec on each
        const uint32_t g2 = gelu_win_bf16x2(m | ((m | 0x8000u) << 16), (const uint16_t *)(lds + kGqWinOff));
        st->gq_tab[e] = fast_elem_bf16<kBF16>(bf2f(g2 & 0xFFFFu), s, sem, lds, false) |
                        (fast_elem_bf16<kBF16>(bf2f(g2 >> 16), s, sem, lds, false) << 16);
    }
    if (tid == 0) {
        st->gq[0] = 1u;
        st->gq[1] = lo;
        st->gq[2] = lot;
        st->gq[3] = top;
    }
}

// x_q of the two bf16 values of a word through the table: entry max(sat(m - (lot - 2)), min(m, 1))
// clamped to top, byte 4 * entry + 2 * sign
__device__ __forceinline__ uint32_t gq_word(uint32_t w, const uint32_t *tab, uint32_t lom2, uint32_t top)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 m = __builtin_bit_cast(u16x2, w & 0x7FFF7FFFu);
    const u16x2 l2 = {uint16_t(lom2), uint16_t(lom2)}, t2 = {uint16_t(top), uint16_t(top)};
    const u16x2 i = __builtin_elementwise_min(
        __builtin_elementwise_max(__builtin_elementwise_sub_sat(m, l2), __builtin_elementwise_min(m, u16x2{1, 1})), t2);
    const uint32_t off = __builtin_bit_cast(uint32_t, i << u16x2{2, 2}) | ((w >> 14) & 0x00020002u);
    const uint8_t *tb = (const uint8_t *)tab;
    return uint32_t(*(const uint16_t *)(tb + (off & 0xFFFFu))) | (uint32_t(*(const uint16_t *)(tb + (off >> 16))) << 16);
}

// x_q of one bf16 input through the reference route (GELU evaluated, then slow_elem)
__device__ __forceinline__ uint32_t gq_ref(uint32_t yb, float s, int sem)
{
    uint32_t o, code;
    slow_elem<kBF16>(gelu_bf16(yb), s, sem, o, code);
    return o;
}

__global__ __launch_bounds__(kTPB) void k_gelu_quant(const uint16_t *__restrict__ y, int64_t n,
                                                     const State *__restrict__ st, uint16_t *__restrict__ xq, int sem,
                                                     int span)
{
    __shared__ __attribute__((aligned(16))) uint32_t tab[kGqCap];
    const uint32_t tid = threadIdx.x;
    const int64_t ngrp = n >> 4;
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    const int64_t i0 = span ? int64_t(blockIdx.x) * span * kTPB : int64_t(blockIdx.x) * kTPB;
    const int64_t istep = span ? int64_t(kTPB) : stride;
    const int64_t iend = span ? (i0 + int64_t(span) * kTPB < ngrp ? i0 + int64_t(span) * kTPB : ngrp) : ngrp;
    const int64_t nchunk = ngrp * 2;
    const u32x4 *yq = (const u32x4 *)y;
    // chunk j (16 bytes) of an iteration G0 is chunk G0 * 2 + j * 256 + tid: each load and store
    // instruction of a wave covers one contiguous run.  The first iteration's input is requested
    // before the table is copied.
    u32x4 pre[2] = {};
    if (i0 < iend) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t c = i0 * 2 + j * kTPB + tid;
            if (c < nchunk) pre[j] = ld_stream(&yq[c]);
        }
    }
    const float s = st->scale;
    if (st->gq[0] == 0u) {
        // the per-element reference route (this workgroup's span, or its grid-stride share)
        const int64_t j0 = span ? i0 * 16 + tid : int64_t(blockIdx.x) * kTPB + tid;
        for (int64_t j = j0; j < (iend << 4); j += span ? int64_t(kTPB) : stride) xq[j] = uint16_t(gq_ref(y[j], s, sem));
        for (int64_t j = (ngrp << 4) + int64_t(blockIdx.x) * kTPB + tid; j < n; j += stride)
            xq[j] = uint16_t(gq_ref(y[j], s, sem));
        return;
    }
    const uint32_t lo = st->gq[1], lot = st->gq[2], top = st->gq[3];
    {
        const u32x4 *src = (const u32x4 *)st->gq_tab;
        for (uint32_t i = tid; i <= top / 4u; i += kTPB) ((u32x4 *)tab)[i] = src[i];
    }
    __syncthreads();
    const uint32_t lom2 = lot - 2u;
    const bool split = lot > lo;
    for (int64_t G0 = i0; G0 < iend; G0 += istep) {
        const u32x4 cur[2] = {pre[0], pre[1]};
        if (G0 + istep < iend) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t c = (G0 + istep) * 2 + j * kTPB + tid;
                pre[j] = c < nchunk ? ld_stream(&yq[c]) : u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t c = G0 * 2 + j * kTPB + tid;
            const uint32_t w[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = gq_word(w[k], tab, lom2, top);
            if (split) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t b = (w[k] >> (16 * h)) & 0xFFFFu, m = b & 0x7FFFu;
                        if (m >= lo && m < lot)
                            o[k] = (o[k] & (0xFFFF0000u >> (16 * h))) | (gq_ref(b, s, sem) << (16 * h));
                    }
                }
            }
            if (c < nchunk) st_stream(&((u32x4 *)xq)[c], u32x4{o[0], o[1], o[2], o[3]});
        }
    }
    // tail (n % 16)
    for (int64_t j = (ngrp << 4) + int64_t(blockIdx.x) * kTPB + tid; j < n; j += stride) {
        const uint32_t b = y[j], m = b & 0x7FFFu;
        xq[j] = uint16_t((split && m >= lo && m < lot) ? gq_ref(b, s, sem) : (gq_word(b, tab, lom2, top) & 0xFFFFu));
    }
}

__global__ __launch_bounds__(kTPB) void k_gelu_stat_settle(State *__restrict__ st, float smax)
{
    __shared__ uint32_t lds[2];
    gelu_stat_settle(st, smax, lds);
}

// Unscaled qdq of a bf16 tensor with QFuncs/hif8.py evaluated in bf16 arithmetic (the
// HIF8_SEM_TORCH_BF16 route of hif8_quant_bf16): elementwise, off the linear's path.
__global__ __launch_bounds__(kTPB) void k_qdq_torch_bf16(const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                         int64_t n)
{
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    for (int64_t i = int64_t(blockIdx.x) * kTPB + threadIdx.x; i < n; i += stride)
        y[i] = uint16_t(qdq_torch_bf16(x[i]));
}

// fp16 <-> fp32: exact widening; narrowing by v_cvt_f16_f32, round-to-nearest-even with fp16
// subnormals and overflow to Inf (the fp16 denormal mode is on), as c10::Half rounds.
__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }
__device__ __forceinline__ uint32_t f2h(float f) { return __builtin_bit_cast(uint16_t, _Float16(f)); }
__device__ __forceinline__ float rh(float f) { return h2f(f2h(f)); }

// QFuncs/hif8.py:6-23 on one fp16 value in fp16 arithmetic (the fp16 branch of :10-11, offset
// 2^-14): each op computed in fp32 and rounded to fp16, as torch's fp16 ops compute.  The floor
// of the fp16-rounded log2 is unchanged by a log2 error of 32 float32 ulps on every input, so
// log2f gives torch's exponent.  2^(e - mb) is Inf for e = 16 (|x| >= 57344 gives Inf).  The
// final "* sign" sets the sign bit of the non-negative fp16 result r (r * -1 is -r exactly, -0
// for r = 0): written as a float product narrowed to fp16, it is compiled to an fma_mix with a
// +0 addend, which turns -0 into +0.
static __device__ uint32_t qdq_torch_f16(uint32_t xh)
{
    const float x = h2f(xh);
    const float xu = fabsf(x);
    if (!(xu <= 65504.0f)) return 0x7E00u;                          // NaN, Inf -> NaN
    const float t = rh(xu + 0x1p-14f);                              // x_unsigned + 2**-14
    const int e = int(__builtin_floorf(rh(log2f(t))));              // floor(log2(.))
    const int ae = e < 0 ? -e : e;
    const int mb = ae <= 3 ? 3 : ae <= 7 ? 2 : ae <= 15 ? 1 : 0;
    const float m = rh(xu * rh(__builtin_ldexpf(1.0f, mb - e)));     // x_unsigned * 2**(-e + mb)
    const float f = __builtin_floorf(rh(m + 0.5f));                 // floor(. + 0.5)
    const uint32_t r = f2h(f * rh(__builtin_ldexpf(1.0f, e - mb))); // * 2**(e - mb), >= 0
    return x < 0.0f ? (r | 0x8000u) : r;                            // * sign (0 for x = +-0)
}

// quant_dequant_float of an fp16 tensor (hif8_quant_f16): the fp32 kernels' element routes on
// x.float() with the result cast back, or the fp16-arithmetic torch route.  Elementwise, off the
// linear's path.
__global__ __launch_bounds__(kTPB) void k_qdq_f16(const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                  int64_t n, int sem)
{
    const int64_t stride = int64_t(gridDim.x) * kTPB;
    for (int64_t i = int64_t(blockIdx.x) * kTPB + threadIdx.x; i < n; i += stride) {
        const uint32_t h = x[i];
        uint32_t r;
        if (sem == HIF8_SEM_TORCH_F16) {
            r = qdq_torch_f16(h);
        } else {
            // the empty asm keeps the fp32 result (and the sign of a zero) apart from the
            // narrowing, which would otherwise absorb qdq_torch's last product into an fma_mix
            float q = sem == kSemTorch ? qdq_torch(h2f(h)) : qdq_npu(h2f(h));
            asm volatile("" : "+v"(q));
            r = f2h(q);
        }
        y[i] = uint16_t(r);
    }
}

// Byte-matrix transpose, codes [R][C] -> [C][R]: the packed weight W^T that the fused GEMM
// reads as its weight operand for dgrad (grad_q @ w_q, hif8_linear.py:97).  64 x 64 tiles
// through LDS; interior tiles of 16-byte aligned matrices move 16 bytes per lane.
__global__ __launch_bounds__(kTPB) void k_transpose_codes(const uint8_t *__restrict__ in, int64_t R, int64_t C,
                                                          uint8_t *__restrict__ out, int64_t tiles_c, int vec)
{
    __shared__ uint32_t tile[64][17];  // 64 rows x 64 bytes, one pad dword per row
    const int64_t t = blockIdx.x;
    const int64_t tr = t / tiles_c, tc = t - tr * tiles_c;
    const int64_t r0 = tr * 64, c0 = tc * 64;
    const int tid = threadIdx.x;
    const int rr = tid >> 2, q = tid & 3;  // this lane: row rr of the tile, bytes 16q .. 16q+15
    const bool full = vec && r0 + 64 <= R && c0 + 64 <= C;
    {
        const int64_t r = r0 + rr, c = c0 + 16 * q;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (full) {
            const uint4 v = *(const uint4 *)(in + r * C + c);
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else if (r < R) {
            for (int j = 0; j < 16; ++j)
                if (c + j < C) w[j >> 2] |= uint32_t(in[r * C + c + j]) << (8 * (j & 3));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[rr][4 * q + j] = w[j];
    }
    __syncthreads();
    // output row c0 + rr holds input column rr: bytes from input rows 16q .. 16q+15
    uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int src_row = 16 * q + j;
        const uint32_t b = (tile[src_row][rr >> 2] >> (8 * (rr & 3))) & 0xFFu;
        o[j >> 2] |= b << (8 * (j & 3));
    }
    const int64_t orow = c0 + rr, ocol = r0 + 16 * q;
    if (full) {
        *(uint4 *)(out + orow * R + ocol) = make_uint4(o[0], o[1], o[2], o[3]);
    } else if (orow < C) {
        for (int j = 0; j < 16; ++j)
            if (ocol + j < R) out[orow * R + ocol + j] = uint8_t(o[j >> 2] >> (8 * (j & 3)));
    }
}

// bf16 transpose with zero padding, [R][C] -> [C][Rp]: out[c][r] = in[r][c] for r < R and 0 for
// R <= r < Rp.  The wgrad operands g_q^T and x_q^T (hif8_linear.py:104), with the token
// dimension padded to the GEMM's k-step.  64 x 64 tiles through LDS; rows of 66 elements put the
// 8 rows a wavefront reads together in 8 different banks.
__global__ __launch_bounds__(kTPB) void k_transpose_bf16(const uint16_t *__restrict__ in, int64_t R, int64_t C,
                                                         int64_t Rp, uint16_t *__restrict__ out, int64_t tiles_c,
                                                         int vec)
{
    __shared__ uint32_t tile[64 * 33];   // 64 rows (r) x 66 bf16 (c), dword-aligned rows
    uint16_t *t16 = (uint16_t *)tile;
    const int64_t t = blockIdx.x;
    const int64_t tr = t / tiles_c, tc = t - tr * tiles_c;
    const int64_t r0 = tr * 64, c0 = tc * 64;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ch = tid + kTPB * k;
        const int rr = ch >> 3, cq = ch & 7;            // tile row, 8-element column chunk
        const int64_t r = r0 + rr, c = c0 + 8 * cq;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (r < R) {
            if (vec && c + 8 <= C) {
                const uint4 v = *(const uint4 *)(in + r * C + c);
                w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
            } else {
                for (int j = 0; j < 8; ++j)
                    if (c + j < C) w[j >> 1] |= uint32_t(in[r * C + c + j]) << (16 * (j & 1));
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[rr * 33 + 4 * cq + j] = w[j];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ch = tid + kTPB * k;
        const int cc = ch >> 3, rq = ch & 7;            // output row (column of in), 8-element chunk of r
        const int64_t c = c0 + cc, r = r0 + 8 * rq;
        if (c >= C || r >= Rp) continue;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = uint32_t(t16[(8 * rq + 2 * j) * 66 + cc]) | (uint32_t(t16[(8 * rq + 2 * j + 1) * 66 + cc]) << 16);
        if (vec && r + 8 <= Rp) {
            *(uint4 *)(out + c * Rp + r) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int j = 0; j < 8 && r + j < Rp; ++j) out[c * Rp + r + j] = uint16_t(w[j >> 1] >> (16 * (j & 1)));
        }
    }
}

// ---------------------------------------------------------------- launch

// Workgroups per CU (measured on the 14B activation): amax streams best with one
// (4 waves per CU, 8 x 16 B loads in flight per lane); encode with 4, qdq with 8.
// k_quant's span (groups of 16 elements per thread, per workgroup): a one-pass grid of spans in
// dispatch order streams at copy speed, where a grid-stride loop over the whole tensor spreads
// the workgroups' accesses over it (copy probe, 774 MB in + out: 6.2-6.5 TB/s against 4.4-5.3
// at 4-8 workgroups per CU).  0 selects the grid-stride loop everywhere.
#ifndef HIF8_QUANT_SPAN
#define HIF8_QUANT_SPAN 4
#endif
constexpr int kQuantSpan = HIF8_QUANT_SPAN;
constexpr int kAmaxWgPerCu = 1;
constexpr int kEncodeWgPerCu = 4;
constexpr int kQdqWgPerCu = 8;
constexpr int kGeluAmaxWgPerCu = 4;   // the GELU amax pass is VALU-bound: more waves per CU

static int grid_for(int64_t units, int max_blocks)
{
    int64_t b = (units + kTPB - 1) / kTPB;
    if (b < 1) b = 1;
    return int(b < max_blocks ? b : max_blocks);
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

static int last_launch() { return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP; }

int launch_gelu_stat_settle(State *y_st, float y_smax, hif8_stream_t stream)
{
    hipLaunchKernelGGL(k_gelu_stat_settle, dim3(1), dim3(kTPB), 0, (hipStream_t)stream, y_st, y_smax);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

}  // namespace hif8

using namespace hif8;

// Workgroups of one k_quant instantiation that fit on a CU at once (its registers decide: 65 or
// more VGPRs allow 7 or fewer waves per SIMD), read once from the runtime.  A grid of more
// workgroups per CU than fit would run the excess as a second, partial wave.
template <int DT, int MODE> static int resident_wgs()
{
    static int wgs = 0;
    if (wgs == 0) {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_quant<DT, MODE>, kTPB, 0) != hipSuccess || b <= 0)
            b = 1;
        wgs = b;
    }
    return wgs;
}

template <int DT, int MODE>
static void launch_k_quant(const void *x, int64_t n, const State *st, void *out, int sem, int use_state, int wg_per_cu,
                           hipStream_t s)
{
    const int64_t ngrp = (n + 15) / 16;
    int grid, span = 0;
    if (kQuantSpan > 0 && ngrp >= int64_t(kQuantSpan) * kTPB * cu_count()) {
        // one pass of spans over the tensor (at least a workgroup per CU)
        const int64_t blocks = (ngrp + int64_t(kQuantSpan) * kTPB - 1) / (int64_t(kQuantSpan) * kTPB);
        grid = int(blocks);
        span = kQuantSpan;
    } else {
        const int fit = resident_wgs<DT, MODE>();
        grid = grid_for(ngrp, cu_count() * (wg_per_cu < fit ? wg_per_cu : fit));
    }
    hipLaunchKernelGGL((k_quant<DT, MODE>), dim3(grid), dim3(kTPB), 0, s, x, n, st, out, sem, use_state, span);
}

// The GELU route: the prep kernel, then spans of HIF8_GELU_SPAN x 256 groups per workgroup
// (each copies the table from the state first), or a grid-stride loop over a grid of resident
// workgroups for tensors under one span per CU.  On the 14B FFN-down input a sweep of the span
// gave 846 / 696 / 718 / 715 / 748 / 795 / 803 / 815 us for 1 / 2 / 3 / 4 / 8 / 16 / 32 / 64.
#ifndef HIF8_GELU_SPAN
#define HIF8_GELU_SPAN 2
#endif
constexpr int kGeluSpan = HIF8_GELU_SPAN;
static void launch_gelu_quant(const void *x, int64_t n, const State *st, void *out, int sem, hipStream_t s)
{
    const int64_t ngrp = (n + 15) / 16;
    int grid, span = 0;
    if (ngrp >= int64_t(kGeluSpan) * kTPB * cu_count()) {
        grid = int((ngrp + int64_t(kGeluSpan) * kTPB - 1) / (int64_t(kGeluSpan) * kTPB));
        span = kGeluSpan;
    } else {
        static int fit = 0;
        if (fit == 0) {
            int b = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_gelu_quant, kTPB, 0) != hipSuccess || b <= 0) b = 1;
            fit = b;
        }
        grid = grid_for(ngrp, cu_count() * fit);
    }
    hipLaunchKernelGGL(k_gelu_quant_prep, dim3(1), dim3(kGqPrepTPB), 0, s, (State *)st, sem);
    hipLaunchKernelGGL(k_gelu_quant, dim3(grid), dim3(kTPB), 0, s, (const uint16_t *)x, n, st, (uint16_t *)out, sem,
                       span);
}

extern "C" {

const char *hif8_strerror(int status)
{
    switch (status) {
    case HIF8_OK: return "ok";
    case HIF8_ERR_ARG: return "invalid argument (null pointer, empty or negative size, or bad enum)";
    case HIF8_ERR_SHAPE: return "unsupported shape";
    case HIF8_ERR_ALIGN: return "pointer not 16-byte aligned";
    case HIF8_ERR_HIP: return "HIP launch or runtime failure";
    case HIF8_ERR_SCRATCH: return "input larger than the static workspace of an allocation-free entry point";
    default: return "unknown hif8 status";
    }
}

size_t hif8_state_size(void) { return sizeof(State); }

int hif8_state_init(void *state, hif8_stream_t stream)
{
    if (!state) return HIF8_ERR_ARG;
    hipLaunchKernelGGL(k_state_init, dim3(1), dim3(64), 0, (hipStream_t)stream, (State *)state);
    return last_launch();
}

int hif8_state_read(const void *state, uint32_t *amax_bits, float *scale, hif8_stream_t stream)
{
    if (!state) return HIF8_ERR_ARG;
    State h;
    if (hipMemcpyAsync(&h, state, 32, hipMemcpyDeviceToHost, (hipStream_t)stream) != hipSuccess) return HIF8_ERR_HIP;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return HIF8_ERR_HIP;
    if (amax_bits) *amax_bits = h.amax_bits;
    if (scale) *scale = h.scale;
    return HIF8_OK;
}

int hif8_absmax_scale(const void *x, int dtype, int64_t n, float scale_max, void *state,
                      hif8_stream_t stream)
{
    if (!x || !state || n <= 0 || (dtype != HIF8_DTYPE_BF16 && dtype != HIF8_DTYPE_F32 && dtype != kBF16F32))
        return HIF8_ERR_ARG;
    if (!aligned16(x)) return HIF8_ERR_ALIGN;
    const int per_thread_vec = dtype == HIF8_DTYPE_F32 ? 4 : 8;
    int grid = grid_for((n + per_thread_vec * 8 - 1) / (per_thread_vec * 8), cu_count() * kAmaxWgPerCu);
    if (dtype == HIF8_DTYPE_BF16)
        hipLaunchKernelGGL(k_absmax<kBF16>, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, x, n, (State *)state, scale_max);
    else if (dtype == kBF16F32)
        hipLaunchKernelGGL(k_absmax<kBF16F32>, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, x, n, (State *)state,
                           scale_max);
    else
        hipLaunchKernelGGL(k_absmax<kF32>, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, x, n, (State *)state, scale_max);
    return last_launch();
}

int hif8_set_scale(void *state, int dtype, float scale, hif8_stream_t stream)
{
    if (!state || (dtype != HIF8_DTYPE_BF16 && dtype != HIF8_DTYPE_F32)) return HIF8_ERR_ARG;
    hipLaunchKernelGGL(k_set_scale, dim3(1), dim3(256), 0, (hipStream_t)stream, (State *)state, dtype, scale);
    return last_launch();
}

static int launch_quant(const void *x, int dtype, int64_t n, const void *state, void *out, int mode,
                        int sem, int use_state, hif8_stream_t stream, bool gelu = false)
{
    if (!x || !out || n <= 0 || (use_state && !state)) return HIF8_ERR_ARG;
    if (dtype != HIF8_DTYPE_BF16 && dtype != HIF8_DTYPE_F32 && !(dtype == kBF16F32 && mode != 2)) return HIF8_ERR_ARG;
    if (sem != HIF8_SEM_NPU && sem != HIF8_SEM_TORCH) return HIF8_ERR_ARG;
    if (!aligned16(x) || !aligned16(out)) return HIF8_ERR_ALIGN;
    const int wpc = mode == 0 ? kEncodeWgPerCu : kQdqWgPerCu;
    hipStream_t s = (hipStream_t)stream;
    const State *st = (const State *)state;
#define HIF8_LAUNCH(DT, MODE) launch_k_quant<DT, MODE>(x, n, st, out, sem, use_state, wpc, s)
    if (gelu) {
        if (dtype != HIF8_DTYPE_BF16 || mode != 1 || !use_state) return HIF8_ERR_ARG;
        launch_gelu_quant(x, n, st, out, sem, s);
    } else if (dtype == HIF8_DTYPE_BF16) {
        if (mode == 0) HIF8_LAUNCH(kBF16, 0);
        else if (mode == 1 || mode == 3) HIF8_LAUNCH(kBF16, 1);
        else HIF8_LAUNCH(kBF16, 2);
    } else if (dtype == HIF8_DTYPE_F32) {
        if (mode == 0) HIF8_LAUNCH(kF32, 0);
        else if (mode == 1) HIF8_LAUNCH(kF32, 1);
        else if (mode == 2) HIF8_LAUNCH(kF32, 2);
        else HIF8_LAUNCH(kF32, 3);
    } else {
        if (mode == 0) HIF8_LAUNCH(kBF16F32, 0);
        else if (mode == 1) HIF8_LAUNCH(kBF16F32, 1);
        else HIF8_LAUNCH(kBF16F32, 3);
    }
#undef HIF8_LAUNCH
    return last_launch();
}

int hif8_encode(const void *x, int dtype, int64_t n, const void *state, uint8_t *codes, hif8_stream_t stream)
{
    return launch_quant(x, dtype, n, state, codes, 0, HIF8_SEM_NPU, 1, stream);
}

int hif8_fake_quant(const void *x, int dtype, int64_t n, const void *state, void *y, int semantics,
                    hif8_stream_t stream)
{
    return launch_quant(x, dtype, n, state, y, 1, semantics, 1, stream);
}

int hif8_fake_quant_to_bf16(const void *x, int dtype, int64_t n, const void *state, uint16_t *y, int semantics,
                            hif8_stream_t stream)
{
    return launch_quant(x, dtype, n, state, y, 3, semantics, 1, stream);
}

int hif8_decode(const uint8_t *codes, int64_t n, const void *state, int out_dtype, void *y, hif8_stream_t stream)
{
    return launch_quant(codes, out_dtype, n, state, y, 2, HIF8_SEM_NPU, 1, stream);
}

int hif8_quant_f32(const float *x, float *y, int64_t n, int semantics, hif8_stream_t stream)
{
    return launch_quant(x, HIF8_DTYPE_F32, n, nullptr, y, 1, semantics, 0, stream);
}

int hif8_quant_bf16(const uint16_t *x, uint16_t *y, int64_t n, int semantics, hif8_stream_t stream)
{
    if (semantics == HIF8_SEM_TORCH_BF16) {
        if (!x || !y || n <= 0) return HIF8_ERR_ARG;
        const int grid = grid_for(n, cu_count() * kQdqWgPerCu);
        hipLaunchKernelGGL(k_qdq_torch_bf16, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, x, y, n);
        return last_launch();
    }
    return launch_quant(x, HIF8_DTYPE_BF16, n, nullptr, y, 1, semantics, 0, stream);
}

int hif8_quant_f16(const uint16_t *x, uint16_t *y, int64_t n, int semantics, hif8_stream_t stream)
{
    if (!x || !y || n <= 0) return HIF8_ERR_ARG;
    if (semantics != HIF8_SEM_NPU && semantics != HIF8_SEM_TORCH && semantics != HIF8_SEM_TORCH_F16)
        return HIF8_ERR_ARG;
    const int grid = grid_for(n, cu_count() * kQdqWgPerCu);
    hipLaunchKernelGGL(k_qdq_f16, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, x, y, n, semantics);
    return last_launch();
}

int hif8_gelu_absmax_scale(const uint16_t *y, int64_t n, float scale_max, void *state, hif8_stream_t stream)
{
    if (!y || !state || n <= 0) return HIF8_ERR_ARG;
    if (!aligned16(y)) return HIF8_ERR_ALIGN;
    const int grid = grid_for((n + 7) / 8, cu_count() * kGeluAmaxWgPerCu);
    hipLaunchKernelGGL(k_gelu_absmax, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, y, n, (State *)state,
                       scale_max, 0);
    return last_launch();
}

int hif8_gelu_bf16(const uint16_t *y, uint16_t *g, int64_t n, hif8_stream_t stream)
{
    if (!y || !g || n <= 0) return HIF8_ERR_ARG;
    if (!aligned16(y) || !aligned16(g)) return HIF8_ERR_ALIGN;
    const int grid = grid_for((n + 7) / 8, cu_count() * kQdqWgPerCu);
    hipLaunchKernelGGL(k_gelu_bf16, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, y, g, n);
    return last_launch();
}

int hif8_gelu_fake_quant(const uint16_t *y, int64_t n, void *state, float scale_max, uint16_t *x_q, int semantics,
                         hif8_stream_t stream)
{
    if (!y || !state || !x_q || n <= 0) return HIF8_ERR_ARG;
    if (semantics != HIF8_SEM_NPU && semantics != HIF8_SEM_TORCH) return HIF8_ERR_ARG;
    if (!aligned16(y) || !aligned16(x_q)) return HIF8_ERR_ALIGN;
    const int grid = grid_for((n + 7) / 8, cu_count() * kGeluAmaxWgPerCu);
    hipLaunchKernelGGL(k_gelu_absmax, dim3(grid), dim3(kTPB), 0, (hipStream_t)stream, y, n, (State *)state,
                       scale_max, 1);
    const int rc = last_launch();
    if (rc != HIF8_OK) return rc;
    return launch_quant(y, HIF8_DTYPE_BF16, n, state, x_q, 1, semantics, 1, stream, true);
}

int hif8_transpose_bf16(const uint16_t *x, int64_t rows, int64_t cols, int64_t rows_pad, uint16_t *out,
                        hif8_stream_t stream)
{
    if (!x || !out || rows <= 0 || cols <= 0 || rows_pad < rows) return HIF8_ERR_ARG;
    if (rows_pad >= (int64_t(1) << 40) || cols >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    const int64_t tiles_r = (rows_pad + 63) / 64, tiles_c = (cols + 63) / 64;
    if (tiles_r * tiles_c >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    const int vec = (cols % 8 == 0 && rows_pad % 8 == 0 && aligned16(x) && aligned16(out)) ? 1 : 0;
    hipLaunchKernelGGL(k_transpose_bf16, dim3(unsigned(tiles_r * tiles_c)), dim3(kTPB), 0, (hipStream_t)stream, x,
                       rows, cols, rows_pad, out, tiles_c, vec);
    return last_launch();
}

int hif8_transpose_codes(const uint8_t *codes, int64_t rows, int64_t cols, uint8_t *out, hif8_stream_t stream)
{
    if (!codes || !out || rows <= 0 || cols <= 0) return HIF8_ERR_ARG;
    if (rows >= (int64_t(1) << 31) || cols >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    const int64_t tiles_r = (rows + 63) / 64, tiles_c = (cols + 63) / 64;
    if (tiles_r * tiles_c >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    const int vec = (rows % 16 == 0 && cols % 16 == 0 && aligned16(codes) && aligned16(out)) ? 1 : 0;
    hipLaunchKernelGGL(k_transpose_codes, dim3(unsigned(tiles_r * tiles_c)), dim3(kTPB), 0, (hipStream_t)stream,
                       codes, rows, cols, out, tiles_c, vec);
    return last_launch();
}

}  // extern "C"
