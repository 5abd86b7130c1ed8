// Fused HiF8 dequant-GEMM for MI355X (gfx950):
//   Y[M,N] = X_q[M,K] . W_q[N,K]^T + bias[N]
// the F.linear(x_q, w_q, bias) of ospnext/modules/hif8_linear.py:86, with W
// stored as packed 8-bit HiF8 codes.  hif8_linear_fwd runs bf16 activations on
// k_linear_dtl (hif8_gemm_dtl.hip); this kernel serves activations given as
// HiF8 codes (HIF8_A_CODES), which it decodes like W.
//
// Design
//   - Workgroup tile 256 (m) x 256 (n) x 64 (k), 512 threads = 8 waves, two per
//     SIMD, wave grid 2 (n) x 4 (m); each wave owns a 128 (n) x 64 (m) block as
//     4 x 2 v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators, 128 per lane).
//   - W code tiles (16 KB per k-step) come from HBM as bytes, are decoded in
//     registers through a 256-entry LDS table (x_q(code) = rnd(decode(code) /
//     scale_w), the reference's exact dequantised operand) and stored to LDS as
//     bf16.  Activations arrive as bf16 (or as codes decoded the same way).
//   - Two LDS stages; global loads for step k+1 are in flight while the MFMAs of
//     step k run; one barrier per k-step.  LDS rows are 128 B; 16-byte chunks
//     are XOR-swizzled so the MFMA fragment reads (32 rows x one chunk) hit
//     distinct banks for both 32- and 64-bank LDS.
//   - The MFMA A operand is the W tile and B the X tile, so each lane's
//     accumulators hold 4 consecutive output features: the epilogue adds bias in
//     fp32, rounds to bf16 (RNE) and stores 8 bytes per group.
//   - Tiles are ordered per XCD (8 contiguous ranges, one per XCD's L2) and in
//     groups of 8 m-tiles so concurrently running workgroups share W and X panels.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"

namespace hif8 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kThreads = 512;
constexpr int kTileBytes = 256 * kBK * 2;        // one bf16 operand tile, 32 KB
constexpr int kLdsBytes = 4 * kTileBytes + 1024;  // 2 stages x (W, X) + two decode tables
constexpr int kGroupM = 8;

__device__ __forceinline__ uint32_t tile_off(uint32_t row, uint32_t chunk)
{
    return row * 128u + ((chunk ^ ((row & 7u) ^ ((row >> 3) & 1u))) << 4);
}

// 16 codes -> 16 bf16 (8 dwords) through an LDS table.
__device__ __forceinline__ void decode16(const u32x4 &c, const uint16_t *lut, uint32_t o[8])
{
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t d = c[j];
        o[2 * j] = uint32_t(lut[d & 0xFFu]) | (uint32_t(lut[(d >> 8) & 0xFFu]) << 16);
        o[2 * j + 1] = uint32_t(lut[(d >> 16) & 0xFFu]) | (uint32_t(lut[d >> 24]) << 16);
    }
}

__device__ __forceinline__ uint32_t f2bf_pk(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <int AFMT>
__global__ __launch_bounds__(kThreads, 1) void k_linear(
    const void *__restrict__ A, const State *__restrict__ a_st, const uint8_t *__restrict__ Wc,
    const State *__restrict__ w_st, const uint16_t *__restrict__ bias, uint16_t *__restrict__ Y, int M,
    int N, int K, int tiles_m, int tiles_n)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[kLdsBytes];
    uint16_t *lutW = (uint16_t *)(smem + 4 * kTileBytes);
    uint16_t *lutA = lutW + 256;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1;   // 2 waves along n
    const int wm = wave >> 1;  // 4 waves along m

    // ---- tile id: contiguous range per XCD, grouped along m
    const int nb = gridDim.x;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3;
    const int per = nb >> 3, rem = nb & 7;
    const int t = xcd * per + (xcd < rem ? xcd : rem) + local;
    const int group = t / (kGroupM * tiles_n);
    const int first_m = group * kGroupM;
    const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int within = t - group * kGroupM * tiles_n;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int m0 = tm * kBM, n0 = tn * kBN;

    if (tid < 256) lutW[tid] = w_st->lut_bf16[tid];
    else if (AFMT == HIF8_A_CODES) lutA[tid - 256] = a_st->lut_bf16[tid - 256];

    // ---- global -> register staging
    constexpr int kXChunks = AFMT == HIF8_A_BF16 ? 4 : 2;  // 16-B chunks per thread per k-step
    u32x4 xr[kXChunks];
    u32x4 wr[2];
    const uint8_t *xbase[kXChunks];
    uint32_t xoff[kXChunks];
    const uint8_t *wbase[2];
    uint32_t woff[2];
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
        int q = tid + kThreads * i;
        int row, col_bytes;
        if (AFMT == HIF8_A_BF16) { row = q >> 3; col_bytes = (q & 7) * 16; }
        else { row = q >> 2; col_bytes = (q & 3) * 16; }
        int gr = m0 + row;
        gr = gr < M ? gr : M - 1;
        size_t row_bytes = AFMT == HIF8_A_BF16 ? size_t(K) * 2 : size_t(K);
        xbase[i] = (const uint8_t *)A + size_t(gr) * row_bytes + col_bytes;
        xoff[i] = AFMT == HIF8_A_BF16 ? tile_off(uint32_t(row), uint32_t(q & 7)) : uint32_t(q);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int q = tid + kThreads * i;
        int row = q >> 2;
        int gr = n0 + row;
        gr = gr < N ? gr : N - 1;
        wbase[i] = Wc + size_t(gr) * size_t(K) + (q & 3) * 16;
        woff[i] = uint32_t(q);
    }

    auto load_global = [&](int kt) {
        const size_t kx = AFMT == HIF8_A_BF16 ? size_t(kt) * kBK * 2 : size_t(kt) * kBK;
#pragma unroll
        for (int i = 0; i < kXChunks; ++i) xr[i] = *(const u32x4 *)(xbase[i] + kx);
        const size_t kw = size_t(kt) * kBK;
#pragma unroll
        for (int i = 0; i < 2; ++i) wr[i] = *(const u32x4 *)(wbase[i] + kw);
    };

    auto store_lds = [&](int stage) {
        uint8_t *sW = smem + stage * kTileBytes;
        uint8_t *sX = smem + (2 + stage) * kTileBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t o[8];
            decode16(wr[i], lutW, o);
            uint32_t q = woff[i], row = q >> 2, c = (q & 3) * 2;
            *(u32x4 *)(sW + tile_off(row, c)) = u32x4{o[0], o[1], o[2], o[3]};
            *(u32x4 *)(sW + tile_off(row, c + 1)) = u32x4{o[4], o[5], o[6], o[7]};
        }
        if (AFMT == HIF8_A_BF16) {
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) *(u32x4 *)(sX + xoff[i]) = xr[i];
        } else {
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) {
                uint32_t o[8];
                decode16(xr[i], lutA, o);
                uint32_t q = xoff[i], row = q >> 2, c = (q & 3) * 2;
                *(u32x4 *)(sX + tile_off(row, c)) = u32x4{o[0], o[1], o[2], o[3]};
                *(u32x4 *)(sX + tile_off(row, c + 1)) = u32x4{o[4], o[5], o[6], o[7]};
            }
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    const int nk = K / kBK;
    load_global(0);
    __syncthreads();  // decode tables
    store_lds(0);
    __syncthreads();

    const uint32_t frow = uint32_t(lane & 31);
    const uint32_t fhalf = uint32_t(lane >> 5);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_global(kt + 1);
        const uint8_t *sW = smem + cur * kTileBytes;
        const uint8_t *sX = smem + (2 + cur) * kTileBytes;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const uint32_t chunk = uint32_t(2 * kk) + fhalf;
            bf16x8 fw[4], fx[2];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fw[i] = *(const bf16x8 *)(sW + tile_off(uint32_t(wn * 128 + i * 32) + frow, chunk));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fx[j] = *(const bf16x8 *)(sX + tile_off(uint32_t(wm * 64 + j * 32) + frow, chunk));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fw[i], fx[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds D[n][m], n = 8*(r/4) + 4*(lane/32) + r%4, m = lane%32
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * 128 + i * 32 + 8 * g + 4 * int(fhalf);
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
            for (int j = 0; j < 2; ++j) {
                const int m = m0 + wm * 64 + j * 32 + int(frow);
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

}  // namespace hif8

using namespace hif8;

extern "C" int hif8_linear_fwd_gelu_amax(const void *a, const uint8_t *w_codes, const void *w_state,
                                         const uint16_t *bias, uint16_t *y, int64_t M, int64_t N, int64_t K,
                                         float scale_max, void *y_state, hif8_stream_t stream)
{
    if (!a || !w_codes || !w_state || !y || !y_state) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    if (K % kBK != 0 || N % 8 != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)w_codes | (uintptr_t)y) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    return launch_linear_dtl((const uint16_t *)a, w_codes, (const State *)w_state, bias, y, M, N, K, stream,
                             (State *)y_state, scale_max);
}

extern "C" int hif8_linear_fwd_grouped(const void *a, const uint8_t *w_codes, const void *const *w_states,
                                       const uint16_t *bias, uint16_t *const *ys, const int64_t *ns, int groups,
                                       int64_t M, int64_t K, hif8_stream_t stream)
{
    if (!a || !w_codes || !w_states || !ys || !ns || groups < 1) return HIF8_ERR_ARG;
    if (groups > kMaxGroups) return HIF8_ERR_SHAPE;
    if (M <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || K >= (int64_t(1) << 22) || K % kBK != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)w_codes) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    Groups g{};
    g.n = groups;
    int64_t N = 0;
    for (int i = 0; i < groups; ++i) {
        if (!w_states[i] || !ys[i] || ns[i] <= 0) return HIF8_ERR_ARG;
        if (ns[i] % 8 != 0 || (i + 1 < groups && ns[i] % kBN != 0)) return HIF8_ERR_SHAPE;
        if ((uintptr_t)ys[i] & 15u) return HIF8_ERR_ALIGN;
        N += ns[i];
        if (N >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
        g.tile_end[i] = int((N + kBN - 1) / kBN);
        g.cols[i] = int(ns[i]);
        g.st[i] = (const State *)w_states[i];
        g.y[i] = ys[i];
    }
    const int64_t tiles = int64_t((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    return launch_linear_dtl_groups((const uint16_t *)a, w_codes, g, bias, M, N, K, stream);
}

extern "C" int hif8_linear_fwd(const void *a, int a_fmt, const void *a_state, const uint8_t *w_codes,
                               const void *w_state, const uint16_t *bias, uint16_t *y, int64_t M, int64_t N,
                               int64_t K, hif8_stream_t stream)
{
    if (!a || !w_codes || !w_state || !y) return HIF8_ERR_ARG;
    if (a_fmt != HIF8_A_BF16 && a_fmt != HIF8_A_CODES) return HIF8_ERR_ARG;
    if (a_fmt == HIF8_A_CODES && !a_state) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    if (K % kBK != 0 || N % 8 != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)w_codes | (uintptr_t)y) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    const int tiles_m = int((M + kBM - 1) / kBM);
    const int tiles_n = int((N + kBN - 1) / kBN);
    const int64_t tiles = int64_t(tiles_m) * tiles_n;
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (a_fmt == HIF8_A_BF16)
        return launch_linear_dtl((const uint16_t *)a, w_codes, (const State *)w_state, bias, y, M, N, K, stream);
    else
        hipLaunchKernelGGL(k_linear<HIF8_A_CODES>, dim3(unsigned(tiles)), dim3(kThreads), 0, s, a,
                           (const State *)a_state, w_codes, (const State *)w_state, bias, y, int(M), int(N),
                           int(K), tiles_m, tiles_n);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}
