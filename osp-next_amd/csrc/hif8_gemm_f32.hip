// The GEMMs of HIF8Linear off the bf16 MFMA path (MI355X, gfx950):
//   - k_gemm_f32: C = A . B with fp32 accumulation on strided bf16 or fp32 operands -- the
//     backward's grad_q @ w_q and grad_q^T @ x_q (ospnext/modules/hif8_linear.py:97,104) of a
//     layer that computes in fp32 (the reference's matmuls run in the saved tensors' dtype);
//   - k_pad_2d: zero padding (or cropping) of a row-major matrix, so that shapes outside the
//     MFMA kernels' tiles (in_features % 64 != 0, out_features % 8 != 0) run on those kernels
//     over zero-padded operands (zero codes decode to 0, zero rows and columns add nothing).
// Neither is on the 14B/1.3B shapes; both are plain LDS-tiled kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"

namespace hif8 {
namespace f32g {

constexpr int kTM = 64, kTN = 64, kTK = 16, kThreads = 256;

template <int DT> __device__ __forceinline__ float ld(const void *p, int64_t i)
{
    if (DT == kBF16) return __builtin_bit_cast(float, uint32_t(((const uint16_t *)p)[i]) << 16);
    return ((const float *)p)[i];
}

__device__ __forceinline__ uint16_t f2bf(float f)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// C[m][n] = sum_k A[m*sam + k*sak] * B[k*sbk + n*sbn], C row-major [M][N] in fp32 or bf16 (RNE).
// One workgroup per 64 x 64 tile of C, 16 x 16 threads of 4 x 4 outputs; A and B k-slices of 16
// through LDS, loaded along whichever index of the operand is contiguous.  Out-of-range elements
// read as zero.
template <int AT, int BT, int CT>
__global__ __launch_bounds__(kThreads) void k_gemm_f32(const void *__restrict__ A, const void *__restrict__ B,
                                                       void *__restrict__ C, int64_t M, int64_t N, int64_t K,
                                                       int64_t sam, int64_t sak, int64_t sbk, int64_t sbn)
{
    __shared__ float As[kTK][kTM + 4];
    __shared__ float Bs[kTK][kTN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int64_t m0 = int64_t(blockIdx.y) * kTM, n0 = int64_t(blockIdx.x) * kTN;
    const bool a_m_fast = sam == 1 && sak != 1;
    const bool b_n_fast = sbn == 1;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += kTK) {
        for (int e = tid; e < kTM * kTK; e += kThreads) {
            const int mm = a_m_fast ? e % kTM : e / kTK, kk = a_m_fast ? e / kTM : e % kTK;
            const int64_t m = m0 + mm, k = k0 + kk;
            As[kk][mm] = (m < M && k < K) ? ld<AT>(A, m * sam + k * sak) : 0.0f;
        }
        for (int e = tid; e < kTN * kTK; e += kThreads) {
            const int nn = b_n_fast ? e % kTN : e / kTK, kk = b_n_fast ? e / kTN : e % kTK;
            const int64_t n = n0 + nn, k = k0 + kk;
            Bs[kk][nn] = (n < N && k < K) ? ld<BT>(B, k * sbk + n * sbn) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kTK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n >= N) continue;
            if (CT == kBF16) ((uint16_t *)C)[m * N + n] = f2bf(acc[i][j]);
            else ((float *)C)[m * N + n] = acc[i][j];
        }
    }
}

// dst[r][c] = src[r][c] for r < sr, c < sc; 0 elsewhere in [dr][dc] (both row-major, contiguous)
template <typename T>
__global__ __launch_bounds__(kThreads) void k_pad_2d(const T *__restrict__ src, int64_t sr, int64_t sc,
                                                     T *__restrict__ dst, int64_t dr, int64_t dc)
{
    const int64_t total = dr * dc;
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / dc, c = i - r * dc;
        dst[i] = (r < sr && c < sc) ? src[r * sc + c] : T(0);
    }
}

template <int AT, int BT>
static void launch_gemm(const void *a, const void *b, void *c, int c_dtype, int64_t M, int64_t N, int64_t K,
                        int64_t sam, int64_t sak, int64_t sbk, int64_t sbn, hipStream_t s)
{
    const dim3 grid(unsigned((N + kTN - 1) / kTN), unsigned((M + kTM - 1) / kTM));
    if (c_dtype == kBF16)
        hipLaunchKernelGGL((k_gemm_f32<AT, BT, kBF16>), grid, dim3(kThreads), 0, s, a, b, c, M, N, K, sam, sak, sbk, sbn);
    else
        hipLaunchKernelGGL((k_gemm_f32<AT, BT, kF32>), grid, dim3(kThreads), 0, s, a, b, c, M, N, K, sam, sak, sbk, sbn);
}

}  // namespace f32g
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_gemm_f32(const void *a, int a_dtype, const void *b, int b_dtype, void *c, int c_dtype, int64_t M,
                             int64_t N, int64_t K, int64_t sa_m, int64_t sa_k, int64_t sb_k, int64_t sb_n,
                             hif8_stream_t stream)
{
    if (!a || !b || !c || M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    for (int dt : {a_dtype, b_dtype, c_dtype})
        if (dt != HIF8_DTYPE_BF16 && dt != HIF8_DTYPE_F32) return HIF8_ERR_ARG;
    if (sa_m < 0 || sa_k < 0 || sb_k < 0 || sb_n < 0) return HIF8_ERR_ARG;
    if ((M + f32g::kTM - 1) / f32g::kTM >= 65536 || (N + f32g::kTN - 1) / f32g::kTN >= (int64_t(1) << 31))
        return HIF8_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (a_dtype == kBF16 && b_dtype == kBF16) f32g::launch_gemm<kBF16, kBF16>(a, b, c, c_dtype, M, N, K, sa_m, sa_k, sb_k, sb_n, s);
    else if (a_dtype == kBF16) f32g::launch_gemm<kBF16, kF32>(a, b, c, c_dtype, M, N, K, sa_m, sa_k, sb_k, sb_n, s);
    else if (b_dtype == kBF16) f32g::launch_gemm<kF32, kBF16>(a, b, c, c_dtype, M, N, K, sa_m, sa_k, sb_k, sb_n, s);
    else f32g::launch_gemm<kF32, kF32>(a, b, c, c_dtype, M, N, K, sa_m, sa_k, sb_k, sb_n, s);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

extern "C" int hif8_pad_2d(const void *src, int64_t src_rows, int64_t src_cols, void *dst, int64_t dst_rows,
                           int64_t dst_cols, int elem_bytes, hif8_stream_t stream)
{
    if (!src || !dst || src_rows <= 0 || src_cols <= 0 || dst_rows <= 0 || dst_cols <= 0) return HIF8_ERR_ARG;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) return HIF8_ERR_ARG;
    const int64_t total = dst_rows * dst_cols;
    int64_t blocks = (total + f32g::kThreads - 1) / f32g::kThreads;
    if (blocks > 65536) blocks = 65536;
    hipStream_t s = (hipStream_t)stream;
    if (elem_bytes == 1)
        hipLaunchKernelGGL(f32g::k_pad_2d<uint8_t>, dim3(unsigned(blocks)), dim3(f32g::kThreads), 0, s,
                           (const uint8_t *)src, src_rows, src_cols, (uint8_t *)dst, dst_rows, dst_cols);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(f32g::k_pad_2d<uint16_t>, dim3(unsigned(blocks)), dim3(f32g::kThreads), 0, s,
                           (const uint16_t *)src, src_rows, src_cols, (uint16_t *)dst, dst_rows, dst_cols);
    else
        hipLaunchKernelGGL(f32g::k_pad_2d<uint32_t>, dim3(unsigned(blocks)), dim3(f32g::kThreads), 0, s,
                           (const uint32_t *)src, src_rows, src_cols, (uint32_t *)dst, dst_rows, dst_cols);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}
