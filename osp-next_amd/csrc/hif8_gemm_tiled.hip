// Fused HiF8 dequant-GEMM on the GEMM-native operand layouts (MI355X, gfx950):
//   Y[M,N] = X_q[M,K] . W_q[N,K]^T + bias[N]          (hif8_linear.py:86)
// X_q arrives in the "XT" tile layout (bf16, written by hif8_fake_quant_tiled),
// W as packed 8-bit HiF8 codes in the "WT" tile layout (hif8_tile_weight_codes).
//
// Design (4 waves, one per SIMD, workgroup tile 256 x 256 x 64)
//   - Each wave owns a 128 (n) x 128 (m) output block: 4 x 4 tiles of
//     v_mfma_f32_32x32x16_bf16, 256 fp32 accumulators per lane (AGPRs).
//   - X operands never touch LDS: XT stores every 32-row x 16-k MFMA operand as
//     1 KB in lane order, so each operand is one coalesced global_load_dwordx4
//     per lane, fetched one k-step ahead into registers.
//   - W codes (16 KB per k-step) are loaded two k-steps ahead, decoded once per
//     workgroup through a 256-entry LDS table (x_q(code) = rnd(decode(code) /
//     scale_w), the reference's exact operand) and written to LDS in lane order,
//     so every W operand read is one contiguous, conflict-free ds_read_b128.
//   - LDS traffic per k-step: 32 KB of decoded W written, 64 KB read, 16 K table
//     lookups; two LDS stages, one barrier per k-step.  The decode of step k+1
//     is interleaved with the MFMAs of step k.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"

namespace hif8 {
namespace tiled {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kStageBytes = 8 * 4096;           // 8 n-blocks x 4 KB of decoded bf16
constexpr int kLdsBytes = 2 * kStageBytes + 512;
constexpr int kGroupM = 8;

__device__ __forceinline__ uint32_t f2bf_pk(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// 16 codes -> 16 bf16 through the LDS table; two lanes' operand pieces.
__device__ __forceinline__ void decode16(const u32x4 &c, const uint16_t *lut, u32x4 &lo, u32x4 &hi)
{
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t d = c[j];
        o[2 * j] = uint32_t(lut[d & 0xFFu]) | (uint32_t(lut[(d >> 8) & 0xFFu]) << 16);
        o[2 * j + 1] = uint32_t(lut[(d >> 16) & 0xFFu]) | (uint32_t(lut[d >> 24]) << 16);
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

__global__ __launch_bounds__(kThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_linear_tiled(const uint8_t *__restrict__ XT, const uint8_t *__restrict__ WT, const State *__restrict__ w_st,
                    const uint16_t *__restrict__ bias, uint16_t *__restrict__ Y, int M, int N, int K,
                    int tiles_m, int tiles_n)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[kLdsBytes];
    uint16_t *lut = (uint16_t *)(smem + 2 * kStageBytes);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;

    // tile id: a contiguous range per XCD (workgroups go round-robin over the 8
    // XCDs), grouped kGroupM m-tiles at a time
    const int nb_all = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3;
    const int per = nb_all >> 3, rem = nb_all & 7;
    const int t = xcd * per + (xcd < rem ? xcd : rem) + local;
    const int group = t / (kGroupM * tiles_n);
    const int first_m = group * kGroupM;
    const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int within = t - group * kGroupM * tiles_n;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int m0 = tm * kBM, n0 = tn * kBN;

    lut[tid] = w_st->lut_bf16[tid];

    const int KS = K / kBK;
    // X operand streams: row-block (m0/32 + wm*4 + j), 4 KB per k-step
    const uint8_t *xrow = XT + (size_t(m0 / 32 + wm * 4) * KS) * 4096 + lane * 16;
    const size_t xrb_stride = size_t(KS) * 4096;
    // W code stream: thread loads 16-B chunk q = tid + 256 i (i < 4) of the 16 KB step
    // tile: n-block q/128, chunk c = q%128 -> kk = c/32, lanes 2(c%32), 2(c%32)+1
    const uint8_t *wrow[4];
    uint32_t wdst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = tid + 256 * i;
        const int nbk = q >> 7, c = q & 127;
        wrow[i] = WT + (size_t(n0 / 32 + nbk) * KS) * 2048 + c * 16;
        wdst[i] = uint32_t(nbk * 4096 + (c >> 5) * 1024 + (c & 31) * 32);
    }

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    bf16x8 xf[2][4][4];   // [buffer][m-block j][kk]
    u32x4 wc[2][4];       // [buffer][chunk]

    auto load_x = [&](int ks, bf16x8 (&dst)[4][4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                dst[j][kk] = *(const bf16x8 *)(xrow + j * xrb_stride + size_t(ks) * 4096 + kk * 1024);
    };
    auto load_w = [&](int ks, u32x4 (&dst)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = *(const u32x4 *)(wrow[i] + size_t(ks) * 2048);
    };
    auto store_w = [&](const u32x4 (&src)[4], int stage, int part) {
        uint8_t *base = smem + stage * kStageBytes;
        u32x4 lo, hi;
        decode16(src[part], lut, lo, hi);
        *(u32x4 *)(base + wdst[part]) = lo;
        *(u32x4 *)(base + wdst[part] + 16) = hi;
    };
    auto compute = [&](int stage, const bf16x8 (&x)[4][4], const u32x4 (&wsrc)[4], bool do_store) {
        const uint8_t *base = smem + stage * kStageBytes + (wn * 4) * 4096 + lane * 16;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8 wf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) wf[i] = *(const bf16x8 *)(base + i * 4096 + kk * 1024);
            if (do_store) store_w(wsrc, stage ^ 1, kk);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], x[j][kk], acc[i][j], 0, 0, 0);
        }
    };

    // prologue: codes for steps 0 and 1, X for step 0, decode step 0
    load_w(0, wc[0]);
    if (KS > 1) load_w(1, wc[1]);
    load_x(0, xf[0]);
    __syncthreads();  // decode table
#pragma unroll
    for (int part = 0; part < 4; ++part) store_w(wc[0], 0, part);
    __syncthreads();

    // steady state, unrolled by two so every register buffer index is static
    int ks = 0;
    for (; ks + 1 < KS; ks += 2) {
        // even step: stage 0, X buffer 0, decode codes of ks+1 (wc[1]) into stage 1
        load_x(ks + 1, xf[1]);
        if (ks + 2 < KS) load_w(ks + 2, wc[0]);
        compute(0, xf[0], wc[1], true);
        __syncthreads();
        // odd step: stage 1, X buffer 1, decode codes of ks+2 (wc[0]) into stage 0
        const bool more = ks + 2 < KS;
        if (more) load_x(ks + 2, xf[0]);
        if (ks + 3 < KS) load_w(ks + 3, wc[1]);
        compute(1, xf[1], wc[0], more);
        __syncthreads();
    }
    if (ks < KS) {  // odd KS: last step on stage 0
        compute(0, xf[0], wc[1], false);
    }

    // epilogue: lane holds D[n][m] with n = 8*(r/4) + 4*(lane/32) + r%4, m = lane%32
    const int fhalf = lane >> 5, frow = lane & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * 128 + i * 32 + 8 * g + 4 * fhalf;
            if (n >= N) continue;
            float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
            if (bias) {
                uint2 bb = *(const uint2 *)(bias + n);
                b0 = __builtin_bit_cast(float, bb.x << 16);
                b1 = __builtin_bit_cast(float, bb.x & 0xFFFF0000u);
                b2 = __builtin_bit_cast(float, bb.y << 16);
                b3 = __builtin_bit_cast(float, bb.y & 0xFFFF0000u);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + wm * 128 + j * 32 + frow;
                if (m >= M) continue;
                const f32x16 &a = acc[i][j];
                uint2 v;
                v.x = f2bf_pk(a[4 * g] + b0, a[4 * g + 1] + b1);
                v.y = f2bf_pk(a[4 * g + 2] + b2, a[4 * g + 3] + b3);
                *(uint2 *)(Y + size_t(m) * size_t(N) + n) = v;
            }
        }
    }
}

}  // namespace tiled
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_linear_fwd_tiled(const uint16_t *xt, const uint8_t *wt, const void *w_state,
                                     const uint16_t *bias, uint16_t *y, int64_t M, int64_t N, int64_t K,
                                     hif8_stream_t stream)
{
    if (!xt || !wt || !w_state || !y) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    if (K % tiled::kBK != 0 || N % 8 != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)xt | (uintptr_t)wt | (uintptr_t)y) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    const int tiles_m = int((M + tiled::kBM - 1) / tiled::kBM);
    const int tiles_n = int((N + tiled::kBN - 1) / tiled::kBN);
    const int64_t tiles = int64_t(tiles_m) * tiles_n;
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    hipLaunchKernelGGL(tiled::k_linear_tiled, dim3(unsigned(tiles)), dim3(tiled::kThreads), 0, (hipStream_t)stream,
                       (const uint8_t *)xt, wt, (const State *)w_state, bias, y, int(M), int(N), int(K), tiles_m,
                       tiles_n);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}
