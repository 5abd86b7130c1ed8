// Internal declarations shared by the codec and GEMM translation units.
#pragma once

#include <stdint.h>

#include "../../include/hif8_mi355x.h"

namespace hif8 {

constexpr int kBF16 = HIF8_DTYPE_BF16;
constexpr int kF32 = HIF8_DTYPE_F32;
constexpr int kBF16F32 = HIF8_DTYPE_BF16_AS_F32;   // bf16 storage, fp32 arithmetic and state
constexpr int kSemNpu = HIF8_SEM_NPU;
constexpr int kSemTorch = HIF8_SEM_TORCH;

// Entries of the GELU quantisation pass's table of x_q over y (hif8_codec.hip, k_gelu_quant).
constexpr uint32_t kGqCap = 5248;

// Per-tensor quantisation state (device memory, hif8_state_size() bytes).
struct alignas(256) State {
    uint32_t counter;      // workgroups finished in the running amax pass (reset by the last)
    uint32_t amax_acc;     // running max of magnitude bits (reset by the last workgroup)
    uint32_t amax_bits;    // amax of the last pass: bf16 or fp32 magnitude bits
    float scale;           // scale in the tensor dtype's rounding, held as fp32
    uint32_t fast;         // 1 when amax and scale are finite and scale > 0
    uint32_t dtype;        // HIF8_DTYPE_* the tables were built for
    uint32_t finite;       // 1 when an amax pass proved every input element finite
    uint32_t pending;      // 1 when a GEMM's GELU statistic left amax|GELU(y)| to an amax pass
    uint16_t lut_bf16[256];  // bf16 bits of x_q(code) = rnd(decode(code) / scale)
    float lut_f32[256];      // fp32 decode(code) / scale
    // For the GELU quantisation pass of the tensor this state scales (written by its prep kernel
    // before every pass): x_q over y for y = +-0, the run 0 < |y| < lo, and |y| = lot .. hi
    // (entry e: x_q of +|y| in the low half, of -|y| in the high half); gq[0..3] = valid, lo, lot,
    // top (the last entry).
    uint32_t gq[4];
    uint32_t gq_tab[kGqCap];
};

static_assert(sizeof(State) % 256 == 0, "state size");

// The output features of a fused GEMM as consecutive groups, each its own weight (codes
// concatenated along N, one state each) and output buffer [M, cols]: several linears on the
// same activation in one launch.  Every group but the last covers whole 256-wide tiles.
constexpr int kMaxGroups = 8;
struct Groups {
    int n;                        // number of groups (1 for a single linear)
    int tile_end[kMaxGroups];     // exclusive end of each group in 256-wide n-tiles
    int cols[kMaxGroups];         // output features of each group (its output row stride)
    const State *st[kMaxGroups];  // decode state of each group's weight
    uint16_t *y[kMaxGroups];      // output of each group
};

// Fused GEMM for bf16 activations (hif8_gemm_dtl.hip); the caller has checked shapes and
// alignment as hif8_linear_fwd documents.  With y_st, the epilogue also folds the GELU
// statistic of its output (max y, hif8_gelu_dev.h) into y_st, and the settle kernel
// (launch_gelu_stat_settle) follows it on the stream.
int launch_linear_dtl(const uint16_t *x, const uint8_t *w_codes, const State *w_st, const uint16_t *bias,
                      uint16_t *y, int64_t M, int64_t N, int64_t K, hif8_stream_t stream, State *y_st = nullptr,
                      float y_smax = 0.0f);
// The decode-free twin (hif8_gemm_w16.hip): W given as dequantised bf16 [N, K].
int launch_linear_w16(const uint16_t *x, const uint16_t *w_q, const uint16_t *bias, uint16_t *y, int64_t M,
                      int64_t N, int64_t K, hif8_stream_t stream, State *y_st, float y_smax);
int launch_linear_w16_groups(const uint16_t *x, const uint16_t *w_q, const Groups &g, const uint16_t *bias,
                             int64_t M, int64_t N, int64_t K, hif8_stream_t stream);
// The grouped form: N is the total of the groups' features.
int launch_linear_dtl_groups(const uint16_t *x, const uint8_t *w_codes, const Groups &g, const uint16_t *bias,
                             int64_t M, int64_t N, int64_t K, hif8_stream_t stream);

// One workgroup that settles y_st after a GELU-statistic GEMM (gelu_stat_settle, hif8_codec.hip).
int launch_gelu_stat_settle(State *y_st, float y_smax, hif8_stream_t stream);

}  // namespace hif8
