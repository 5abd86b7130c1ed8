// q/k normalisation and rotary embedding of the DiT's attention in one pass (MI355X, gfx950).
//
// The reference computes, on the bf16 output of the q (or k) projection x [rows, dim]:
//   WanRMSNorm with an fp32 weight and a bf16 output (want2v.py:77-93 under the model's
//   high-precision norm policy):
//     y1 = rnd_bf16(x * rsqrt(mean(x^2) + eps))      _norm(x.float()).type_as(x)
//     y2 = rnd_bf16(rnd_f32(y1 * w))                  * weight (fp32), .to(bf16)
//   then, for self-attention, the 3-D RoPE (osp_next.py:596-644) on pairs (2i, 2i+1) of each
//   head, in fp32, with the token's angles:
//     o1 = x1 * cos - x2 * sin,  o2 = x1 * sin + x2 * cos
//   and the attention's cast of the fp32 result to bf16 (attention.py:460-518): out = rnd_bf16(o).
// As torch ops that is about fifteen passes over fp32 and bf16 copies of the tensor; here it is
// one read and one write of bf16 per element.  Every rounding point above is kept (products and
// sums in fp32, -ffp-contract=off for this file); the mean's sum is taken in this kernel's own
// order, so y1 can differ from torch's by one bf16 step where x * rsqrt lands next to a rounding
// boundary.
//
// One wavefront per row: lane l holds elements c*512 + 8l .. +7 of each 512-element chunk c, as
// one 16-byte load; with 512 % head_dim == 0 its four rope pairs have the same in-head index in
// every chunk, so each lane loads its 4 cosines and 4 sines once per row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"
#include "hif8_qdq_dev.h"

namespace hif8 {
namespace dit {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxChunks = 16;  // dim <= 8192

__device__ __forceinline__ float lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
__device__ __forceinline__ float hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xFFFF0000u); }
// Round-to-nearest-even to bf16 of two floats in one v_cvt_pk_bf16_f32 (f2bf_pk): the same bits
// as the integer RNE for every finite value, as the codec relies on; NaN stays NaN.
__device__ __forceinline__ uint32_t pack(float a, float b) { return f2bf_pk(a, b); }

// MODE 0: out = the bf16 output.  MODE 1: no output; the amax of the output before that rounding
// -- the fp32 rope output, or without rope the bf16 norm output -- folded into st with the scale
// rule for smax (fp32 with rope, bf16 without), the last workgroup settling st: the _quant amax of
// the q or k the reference hands hif8_attention_with_mask (hif8_attention.py:60-74).  MODE 2:
// out = bf16 of that output's HiF8 fake quant with st's scale (the attention's bf16 cast of
// _quant(q)), and y_out, if not null, the output itself (fp32 with rope, bf16 without).  For a
// state with a finite scale the fake quant is the codec's table route (the encode table and the
// state's bf16 decode table in LDS, fast_elem_bf16), otherwise the scalar route; the same bits.
template <int NC, bool ROPE, int MODE>
__global__ __launch_bounds__(kThreads) void k_rms_norm_rope(const uint16_t *__restrict__ x, const float *__restrict__ w,
                                                            const float *__restrict__ cs, const float *__restrict__ sn,
                                                            uint16_t *__restrict__ out, int64_t rows, int dim,
                                                            int head_dim, int64_t seq, int64_t rep, float eps,
                                                            State *__restrict__ st, float smax, int sem,
                                                            void *__restrict__ y_out)
{
    const int lane = threadIdx.x & 63;
    uint32_t amax = 0;
    const float qs = MODE == 2 ? st->scale : 0.0f;
    // MODE 2: the tables of the table route (one lut entry per thread)
    static_assert(kThreads == 256, "one decode-table entry per thread");
    __shared__ __attribute__((aligned(16))) uint8_t qtab[MODE == 2 ? kLdsBytes : 16];
    const bool qfast = MODE == 2 && st->fast != 0;
    const bool nan_guard = MODE == 2 && st->finite == 0;
    if (MODE == 2) {
        if (qfast) {
            ((uint16_t *)(qtab + kLdsLutBf16))[threadIdx.x] = st->lut_bf16[threadIdx.x];
            const uint4 *src = (const uint4 *)&kEncTable;
            uint4 *dst = (uint4 *)(qtab + kTabLo);
            for (uint32_t i = threadIdx.x; i < sizeof(EncTable) / 16; i += kThreads) dst[i] = src[i];
        }
        __syncthreads();
    }
    const int64_t wstride = int64_t(gridDim.x) * (kThreads / 64);
    const float inv_dim = 1.0f / float(dim);
    for (int64_t row = int64_t(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6); row < rows; row += wstride) {
        const u32x4 *xr = (const u32x4 *)(x + row * dim);
        u32x4 v[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] = __builtin_nontemporal_load(&xr[c * 64 + lane]);
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float a = lo(v[c][t]), b = hi(v[c][t]);
                ss += a * a;
                ss += b * b;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float r = rsqrtf(ss * inv_dim + eps);
        f32x4 ca = {}, sa = {};
        if (ROPE) {
            const int64_t s = row % seq;
            const int64_t cr = (row / seq / rep) * seq + s;
            const int pair = ((lane * 8) % head_dim) / 2;
            const int d = head_dim / 2;
            ca = *(const f32x4 *)(cs + cr * d + pair);
            sa = *(const f32x4 *)(sn + cr * d + pair);
        }
        u32x4 *orow = (u32x4 *)(out + row * dim);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int e0 = c * 512 + lane * 8;
            const f32x4 w0 = *(const f32x4 *)(w + e0);
            const f32x4 w1 = *(const f32x4 *)(w + e0 + 4);
            const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
            float y[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                y[2 * t] = lo(v[c][t]);
                y[2 * t + 1] = hi(v[c][t]);
            }
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const uint32_t y1 = pack(y[e] * r, y[e + 1] * r);
                const uint32_t y2 = pack(lo(y1) * wv[e], hi(y1) * wv[e + 1]);
                y[e] = lo(y2);
                y[e + 1] = hi(y2);
            }
            float f[8];
            if (ROPE) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float x1 = y[2 * t], x2 = y[2 * t + 1];
                    const float p1 = x1 * ca[t], p2 = x2 * sa[t], p3 = x1 * sa[t], p4 = x2 * ca[t];
                    f[2 * t] = p1 - p2;
                    f[2 * t + 1] = p3 + p4;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = y[e];   // bf16 values
            }
            if (MODE == 0) {
                u32x4 o;
#pragma unroll
                for (int t = 0; t < 4; ++t) o[t] = pack(f[2 * t], f[2 * t + 1]);
                orow[c * 64 + lane] = o;
            } else if (MODE == 1) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    // without rope f[e] is a bf16 value: its top half is its bf16 bits
                    const uint32_t mb = __builtin_bit_cast(uint32_t, f[e]) & 0x7FFFFFFFu;
                    const uint32_t m = ROPE ? mb : (mb >> 16);
                    amax = m > amax ? m : amax;
                }
            } else {
                uint32_t qb[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (qfast) {
                        qb[e] = fast_elem_bf16<ROPE ? kF32 : kBF16>(f[e], qs, sem, qtab, nan_guard);
                    } else {
                        uint32_t yb, code;
                        if (ROPE) {
                            slow_elem<kF32>(__builtin_bit_cast(uint32_t, f[e]), qs, sem, yb, code);
                            qb[e] = f2bf(u2f(yb));
                        } else {
                            slow_elem<kBF16>(__builtin_bit_cast(uint32_t, f[e]) >> 16, qs, sem, yb, code);
                            qb[e] = yb;
                        }
                    }
                }
                orow[c * 64 + lane] = u32x4{qb[0] | (qb[1] << 16), qb[2] | (qb[3] << 16), qb[4] | (qb[5] << 16),
                                            qb[6] | (qb[7] << 16)};
                if (y_out) {
                    if (ROPE) {
                        f32x4 *yr = (f32x4 *)((float *)y_out + row * dim + c * 512 + lane * 8);
                        yr[0] = f32x4{f[0], f[1], f[2], f[3]};
                        yr[1] = f32x4{f[4], f[5], f[6], f[7]};
                    } else {
                        u32x4 o;
#pragma unroll
                        for (int t = 0; t < 4; ++t) o[t] = pack(f[2 * t], f[2 * t + 1]);
                        ((u32x4 *)((uint16_t *)y_out + row * dim))[c * 64 + lane] = o;
                    }
                }
            }
        }
    }
    if (MODE == 1) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, o, 64));
        __shared__ uint32_t red[kThreads / 64 + 2];
        if (lane == 0) red[threadIdx.x >> 6] = amax;
        __syncthreads();
        amax = max(max(red[0], red[1]), max(red[2], red[3]));
        fold_amax(st, amax, gridDim.x, ROPE ? kF32 : kBF16, smax, red + kThreads / 64);
    }
}

// Gated residual of the block (osp_next.py:947, :955): out = x + y * gate as torch's bf16 ops
// compute it, t = rnd_bf16(y * g) then out = rnd_bf16(x + t), each in fp32 (no fused
// multiply-add; this file is built with -ffp-contract=off).  gate is one bf16 row of dim per
// batch of rows_per_batch rows; with no gate, out = rnd_bf16(x + y) (osp_next.py:949).  Each
// thread takes 8 elements (16 bytes) per step.
// RNE to bf16 as torch's software conversion does it, NaN as the canonical 0x7FC0.
__device__ __forceinline__ uint32_t bf_t(float f)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t pack_t(float a, float b) { return bf_t(a) | (bf_t(b) << 16); }

// out may be x (an in-place residual update): x, y and out are not restrict-qualified.  Each
// element is loaded before its own store and no other element reads it.
template <bool GATE>
__global__ __launch_bounds__(kThreads) void k_gated_residual(const u32x4 *x, const u32x4 *y,
                                                             const uint16_t *__restrict__ gate, u32x4 *out,
                                                             int64_t nvec, int64_t dim, int64_t rows_per_batch)
{
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < nvec; i += stride) {
        const u32x4 xv = __builtin_nontemporal_load(&x[i]);
        const u32x4 yv = __builtin_nontemporal_load(&y[i]);
        u32x4 o;
        if (GATE) {
            const int64_t e0 = i * 8;
            const int64_t row = e0 / dim, col = e0 - row * dim;
            const u32x4 gv = *(const u32x4 *)(gate + (row / rows_per_batch) * dim + col);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t tp = pack_t(lo(yv[t]) * lo(gv[t]), hi(yv[t]) * hi(gv[t]));
                o[t] = pack_t(lo(xv[t]) + lo(tp), hi(xv[t]) + hi(tp));
            }
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) o[t] = pack_t(lo(xv[t]) + lo(yv[t]), hi(xv[t]) + hi(yv[t]));
        }
        __builtin_nontemporal_store(o, &out[i]);
    }
}

// The block's layout changes as one row gather: the Skiparse rearranges (skiparse_func.py:18-52)
// and the padding and cropping around them (SkiparseRearrange.forward, osp_next.py:239-283) each
// send every token row to one output row and fill the padding rows with zeros.  out[r] = x[src[r]]
// for 0 <= src[r] < in_rows, a zero row otherwise; rows of vpr 16-byte vectors.  Each thread
// moves one vector per step, kGatherU steps in flight; n = rows * vpr < 2^31.
constexpr int kGatherU = 4;
__global__ __launch_bounds__(kThreads) void k_gather_rows(const u32x4 *__restrict__ x, const int32_t *__restrict__ src,
                                                          uint32_t n, uint32_t vpr, int64_t in_rows,
                                                          u32x4 *__restrict__ out)
{
    const uint32_t stride = gridDim.x * uint32_t(kThreads);
    for (uint32_t base = blockIdx.x * uint32_t(kThreads) + threadIdx.x; base < n; base += stride * kGatherU) {
        u32x4 v[kGatherU];
#pragma unroll
        for (int u = 0; u < kGatherU; ++u) {
            const uint32_t i = base + uint32_t(u) * stride;
            v[u] = u32x4{0u, 0u, 0u, 0u};
            if (i < n) {
                const uint32_t r = i / vpr, c = i - r * vpr;
                const int32_t sr = src[r];
                if (sr >= 0 && sr < in_rows) v[u] = __builtin_nontemporal_load(&x[int64_t(sr) * vpr + c]);
            }
        }
#pragma unroll
        for (int u = 0; u < kGatherU; ++u) {
            const uint32_t i = base + uint32_t(u) * stride;
            if (i < n) out[i] = v[u];
        }
    }
}

}  // namespace dit
}  // namespace hif8

using namespace hif8;

namespace {

// Checks and launches k_rms_norm_rope<., ., MODE> (see hif8_rms_norm_rope and its quantising forms).
int launch_rms_norm_rope(int mode, const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t,
                         uint16_t *out, int64_t rows, int64_t dim, int64_t head_dim, int64_t seq, int64_t rep,
                         float eps, State *st, float smax, int sem, void *y_out, hif8_stream_t stream)
{
    if (!x || !weight || rows <= 0) return HIF8_ERR_ARG;
    if ((mode != 1 && !out) || (mode != 0 && !st)) return HIF8_ERR_ARG;
    if (mode == 1 && !(smax > 0.0f)) return HIF8_ERR_ARG;
    if (mode == 2 && sem != kSemNpu && sem != kSemTorch) return HIF8_ERR_ARG;
    if ((cos_t == nullptr) != (sin_t == nullptr)) return HIF8_ERR_ARG;
    if (dim <= 0 || dim % 512 != 0 || dim > 512 * dit::kMaxChunks) return HIF8_ERR_SHAPE;
    const bool rope = cos_t != nullptr;
    if (rope && (head_dim < 8 || head_dim % 8 != 0 || 512 % head_dim != 0 || dim % head_dim != 0 || seq <= 0 ||
                 rep <= 0 || rows % seq != 0))
        return HIF8_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)out | (uintptr_t)weight | (uintptr_t)y_out) & 15u) return HIF8_ERR_ALIGN;
    if (rope && (((uintptr_t)cos_t | (uintptr_t)sin_t) & 15u)) return HIF8_ERR_ALIGN;
    if (rows >= (int64_t(1) << 40)) return HIF8_ERR_SHAPE;
    static int cu_cache[64] = {0};
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
        if (cu_cache[dev] == 0) {
            int c = 0;
            if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
            cu_cache[dev] = c;
        }
        cus = cu_cache[dev];
    }
    const int64_t want = (rows + 3) / 4;
    const int grid = int(want < int64_t(cus) * 8 ? want : int64_t(cus) * 8);
    hipStream_t s = (hipStream_t)stream;
    const int nc = int(dim / 512);
    const int hd = rope ? int(head_dim) : 8;
    const int64_t sq = rope ? seq : 1, rp = rope ? rep : 1;
#define HIF8_RN_MODE(NC, R, M)                                                                                            hipLaunchKernelGGL((dit::k_rms_norm_rope<NC, R, M>), dim3(grid), dim3(dit::kThreads), 0, s, x, weight, cos_t,                           sin_t, out, rows, int(dim), hd, sq, rp, eps, st, smax, sem, y_out)
#define HIF8_RN(NC)                                                                                                       case NC:                                                                                                                  if (mode == 0) {                                                                                                          if (rope) HIF8_RN_MODE(NC, true, 0);                                                                                  else HIF8_RN_MODE(NC, false, 0);                                                                                  } else if (mode == 1) {                                                                                                   if (rope) HIF8_RN_MODE(NC, true, 1);                                                                                  else HIF8_RN_MODE(NC, false, 1);                                                                                  } else {                                                                                                                  if (rope) HIF8_RN_MODE(NC, true, 2);                                                                                  else HIF8_RN_MODE(NC, false, 2);                                                                                  }                                                                                                                     break;
    switch (nc) {
        HIF8_RN(1) HIF8_RN(2) HIF8_RN(3) HIF8_RN(4) HIF8_RN(5) HIF8_RN(6) HIF8_RN(7) HIF8_RN(8)
        HIF8_RN(9) HIF8_RN(10) HIF8_RN(11) HIF8_RN(12) HIF8_RN(13) HIF8_RN(14) HIF8_RN(15) HIF8_RN(16)
    default:
        return HIF8_ERR_SHAPE;
    }
#undef HIF8_RN
#undef HIF8_RN_MODE
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

}  // namespace

extern "C" int hif8_rms_norm_rope(const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t,
                                  uint16_t *out, int64_t rows, int64_t dim, int64_t head_dim, int64_t seq,
                                  int64_t rep, float eps, hif8_stream_t stream)
{
    return launch_rms_norm_rope(0, x, weight, cos_t, sin_t, out, rows, dim, head_dim, seq, rep, eps, nullptr, 0.0f,
                                kSemNpu, nullptr, stream);
}

extern "C" int hif8_rms_norm_rope_amax(const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t,
                                       int64_t rows, int64_t dim, int64_t head_dim, int64_t seq, int64_t rep,
                                       float eps, float scale_max, void *state, hif8_stream_t stream)
{
    return launch_rms_norm_rope(1, x, weight, cos_t, sin_t, nullptr, rows, dim, head_dim, seq, rep, eps,
                                (State *)state, scale_max, kSemNpu, nullptr, stream);
}

extern "C" int hif8_rms_norm_rope_fake_quant(const uint16_t *x, const float *weight, const float *cos_t,
                                             const float *sin_t, int64_t rows, int64_t dim, int64_t head_dim,
                                             int64_t seq, int64_t rep, float eps, const void *state, int semantics,
                                             uint16_t *x_q, void *y, hif8_stream_t stream)
{
    return launch_rms_norm_rope(2, x, weight, cos_t, sin_t, x_q, rows, dim, head_dim, seq, rep, eps,
                                (State *)state, 0.0f, semantics, y, stream);
}

extern "C" int hif8_gated_residual(const uint16_t *x, const uint16_t *y, const uint16_t *gate, uint16_t *out,
                                   int64_t rows, int64_t dim, int64_t rows_per_batch, hif8_stream_t stream)
{
    if (!x || !y || !out || rows <= 0 || dim <= 0) return HIF8_ERR_ARG;
    if (dim % 8 != 0 || rows >= (int64_t(1) << 40) || dim >= (int64_t(1) << 24)) return HIF8_ERR_SHAPE;
    if (gate && (rows_per_batch <= 0 || rows % rows_per_batch != 0)) return HIF8_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)out | (uintptr_t)gate) & 15u) return HIF8_ERR_ALIGN;
    const int64_t nvec = rows * dim / 8;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const int64_t want = (nvec + dit::kThreads - 1) / dit::kThreads;
    const int grid = int(want < int64_t(cus) * 8 ? want : int64_t(cus) * 8);
    hipStream_t s = (hipStream_t)stream;
    typedef dit::u32x4 V;
    if (gate)
        hipLaunchKernelGGL(dit::k_gated_residual<true>, dim3(grid), dim3(dit::kThreads), 0, s, (const V *)x,
                           (const V *)y, gate, (V *)out, nvec, dim, rows_per_batch);
    else
        hipLaunchKernelGGL(dit::k_gated_residual<false>, dim3(grid), dim3(dit::kThreads), 0, s, (const V *)x,
                           (const V *)y, (const uint16_t *)nullptr, (V *)out, nvec, dim, int64_t(1));
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

extern "C" int hif8_gather_rows(const uint16_t *x, int64_t in_rows, const int32_t *src_row, int64_t rows,
                                int64_t cols, uint16_t *out, hif8_stream_t stream)
{
    if (!x || !src_row || !out || in_rows <= 0 || rows <= 0 || cols <= 0) return HIF8_ERR_ARG;
    if (cols % 8 != 0 || rows * (cols / 8) >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)out) & 15u || ((uintptr_t)src_row & 3u)) return HIF8_ERR_ALIGN;
    const int64_t vpr = cols / 8, n = rows * vpr;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const int64_t want = (n + int64_t(dit::kThreads) * dit::kGatherU - 1) / (int64_t(dit::kThreads) * dit::kGatherU);
    const int grid = int(want < int64_t(cus) * 8 ? want : int64_t(cus) * 8);
    typedef dit::u32x4 V;
    hipLaunchKernelGGL(dit::k_gather_rows, dim3(grid), dim3(dit::kThreads), 0, (hipStream_t)stream, (const V *)x,
                       src_row, uint32_t(n), uint32_t(vpr), in_rows, (V *)out);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}
