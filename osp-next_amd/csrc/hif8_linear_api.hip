// C-ABI entry points of the fused HiF8 dequant-GEMM (k_linear_dtl, hif8_gemm_dtl.hip):
//   Y[M,N] = X_q[M,K] . W_q[N,K]^T + bias[N]
// the F.linear(x_q, w_q, bias) of ospnext/modules/hif8_linear.py:86 with bf16 activations x_q
// and W held as packed 8-bit HiF8 codes, plus its GELU-statistic epilogue and grouped forms.
// Shapes and alignment are checked here; the kernels assume them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"

namespace hif8 {

constexpr int kBM = 256;   // the fused kernel's workgroup tile: 256 rows x 256 features x 64 k
constexpr int kBN = 256;
constexpr int kBK = 64;

}  // namespace hif8

using namespace hif8;

extern "C" int hif8_linear_fwd_gelu_stat(const void *a, const uint8_t *w_codes, const void *w_state,
                                         const uint16_t *bias, uint16_t *y, int64_t M, int64_t N, int64_t K,
                                         float scale_max, void *y_state, hif8_stream_t stream)
{
    if (!a || !w_codes || !w_state || !y || !y_state) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 22)) return HIF8_ERR_SHAPE;
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

extern "C" int hif8_linear_fwd(const uint16_t *a, const uint8_t *w_codes, const void *w_state, const uint16_t *bias,
                               uint16_t *y, int64_t M, int64_t N, int64_t K, hif8_stream_t stream)
{
    if (!a || !w_codes || !w_state || !y) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 22)) return HIF8_ERR_SHAPE;
    if (K % kBK != 0 || N % 8 != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)w_codes | (uintptr_t)y) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    return launch_linear_dtl(a, w_codes, (const State *)w_state, bias, y, M, N, K, stream);
}
