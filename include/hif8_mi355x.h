/*
 * hif8_mi355x.h -- C ABI of the MI355X (gfx950) HiF8 fake-quant linear library.
 *
 * Drop-in boundary for OSP-Next's per-tensor HiF8 quantized linear path.  Every
 * entry point names the reference interface it replaces (paths relative to the
 * OSP-Next tree).
 *
 * Conventions
 *   - Every function returns an int status: HIF8_OK (0) or a negative HIF8_ERR_*.
 *     hif8_strerror() turns it into text; a HIP launch failure is HIF8_ERR_HIP.
 *   - All pointers are device pointers the caller owns (no allocation inside any
 *     entry point), already offset to the first element.  Element counts are
 *     int64_t.  bf16 tensors are passed as uint16_t bit patterns.
 *   - Work is enqueued on the given HIP stream (NULL = legacy default stream) and
 *     is stream-ordered; no entry point synchronises the host.
 *   - Per-tensor quantisation state (amax, scale, decode tables) lives in a
 *     caller-allocated device buffer of hif8_state_size() bytes ("state").  A
 *     state must be initialised once with hif8_state_init() and must not be used
 *     by two streams at the same time.
 *
 * Semantics of the two HiF8 qdq flavours the reference has:
 *   HIF8_SEM_NPU   -- ospnext/quant_cy_npu/base/cusrc/hif8_quant_op.h:88-151, the
 *                     path taken when quant_dequant_float is called without
 *                     force_py (QTensor.py:115-117): a true 8-bit format (flush
 *                     below 2^-23, 2^-22 for [2^-23,2^-22), +-Inf from |x|>=40960).
 *   HIF8_SEM_TORCH -- ospnext/quant_cy_npu/base/QFuncs/hif8.py:6-23, the
 *                     force_py=True path (no flush, no saturation).
 *   They agree exactly on {0} U [2^-22, 40960).  Codes always follow HIF8_SEM_NPU.
 */
#ifndef HIF8_MI355X_H
#define HIF8_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *hif8_stream_t; /* == hipStream_t */

enum {
    HIF8_OK = 0,
    HIF8_ERR_ARG = -1,       /* null pointer, negative or empty size, bad enum */
    HIF8_ERR_SHAPE = -2,     /* shape the kernel does not support (see each call) */
    HIF8_ERR_ALIGN = -3,     /* pointer alignment the kernel needs is not met */
    HIF8_ERR_HIP = -4,       /* a HIP runtime call or kernel launch failed */
    HIF8_ERR_SCRATCH = -5,   /* input larger than an allocation-free entry point's static workspace */
};

enum { HIF8_DTYPE_BF16 = 0, HIF8_DTYPE_F32 = 1, HIF8_DTYPE_BF16_AS_F32 = 2 };
/* HIF8_DTYPE_BF16_AS_F32: a bf16 tensor quantised as the fp32 tensor x.float() holds it --
 * fp32 amax, scale and arithmetic, an fp32 state.  This is the self-attention o input of the
 * reference, whose fp32 values are the bf16 attention output cast up
 * (ospnext/modules/attention.py:473,518 and osp_next.py:644): quantising the bf16 tensor
 * directly gives the same x_q without materialising the fp32 copy.  Taken by
 * hif8_absmax_scale, hif8_encode, hif8_fake_quant (y fp32) and hif8_fake_quant_to_bf16. */
enum { HIF8_SEM_NPU = 0, HIF8_SEM_TORCH = 1, HIF8_SEM_TORCH_BF16 = 2, HIF8_SEM_TORCH_F16 = 3 };
/* HIF8_SEM_TORCH_BF16: QFuncs/hif8.py:6-23 evaluated in bf16 arithmetic, every op rounded to bf16
 * -- quant_dequant_float(x, QType('hif8'), force_py=True, force_fp32=False) of a bf16 tensor
 * (QTensor.py:99-102 skipped).  It differs from HIF8_SEM_TORCH only for |x| < 2^-43.  Taken by
 * hif8_quant_bf16 only.
 * HIF8_SEM_TORCH_F16: the same for an fp16 tensor -- the fp16 branch of QFuncs/hif8.py:10-11
 * (offset 2^-14) with every op rounded to fp16.  Taken by hif8_quant_f16 only. */

/* Text for a status code (static storage). */
const char *hif8_strerror(int status);

/* ---------------------------------------------------------------------------
 * Per-tensor state.  Holds the reduction counter, amax, scale and the two
 * 256-entry decode tables x_q(code) of one quantised tensor.
 * Replaces the scalar tensors x_max / scale of _quant
 * (ospnext/modules/hif8_linear.py:45-46), which the reference keeps on device.
 */
size_t hif8_state_size(void);
/* Clear the counters of a fresh state (a fill kernel, no hipMemset). */
int hif8_state_init(void *state, hif8_stream_t stream);
/* Host-readable copy of a state's scalars: amax bits, scale (fp32 value). */
int hif8_state_read(const void *state, uint32_t *amax_bits, float *scale, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * amax + scale: hif8_linear.py:45-46
 *   x_max = x.abs().amax().clamp(min=1e-8);  scale = scale_max / x_max
 * with torch's rounding: scale = rnd(rnd(1/x_max) * scale_max), rnd = the input
 * dtype.  One pass over x; the last workgroup also fills the decode tables.
 * dtype: HIF8_DTYPE_BF16, HIF8_DTYPE_F32 or HIF8_DTYPE_BF16_AS_F32 (an fp32 state).  n >= 1.
 */
int hif8_absmax_scale(const void *x, int dtype, int64_t n, float scale_max, void *state,
                      hif8_stream_t stream);

/* Set a state's scale directly (no amax): used for the unscaled qdq drop-ins and
 * for callers that carry their own scale. */
int hif8_set_scale(void *state, int dtype, float scale, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Encode: HiF8 codes of qdq(x * scale), NPU semantics (hif8_linear.py:47-48 with
 * QTensor.py:94-128 -> hif8_quant_op.h:88-151).  codes: n bytes.
 */
int hif8_encode(const void *x, int dtype, int64_t n, const void *state, uint8_t *codes,
                hif8_stream_t stream);

/* Fake quant: y = quant_dequant_float(x * scale, QType('hif8'), force_fp32=True) / scale
 * (hif8_linear.py:47-48).  y has the dtype of x (fp32 for HIF8_DTYPE_BF16_AS_F32).
 * semantics: HIF8_SEM_*. */
int hif8_fake_quant(const void *x, int dtype, int64_t n, const void *state, void *y,
                    int semantics, hif8_stream_t stream);

/* Fake quant into the bf16 GEMM operand: y = bf16(x_q), the rounding torch.autocast(bf16)
 * applies to x_q when F.linear(x_q, w_q, bias) runs (hif8_linear.py:86 under the pipeline's
 * autocast, ospnext/schedulers/flow_matching.py:108).  For a bf16 x this is hif8_fake_quant;
 * for an fp32 x (or HIF8_DTYPE_BF16_AS_F32) it quantises in fp32 and writes 2 bytes per
 * element, so the fp32 x_q is never stored.  y: n bf16. */
int hif8_fake_quant_to_bf16(const void *x, int dtype, int64_t n, const void *state, uint16_t *y,
                            int semantics, hif8_stream_t stream);

/* The FFN's GELU layer (nn.GELU(approximate="tanh") on a bf16 tensor, osp_next.py:875) folded
 * into the next linear's _quant (hif8_linear.py:42-50), so its output is never written:
 *   hif8_gelu_absmax_scale: amax|GELU(y)| and its scale for scale_max into state, as
 *     hif8_absmax_scale of GELU(y) would (one read of y);
 *   hif8_gelu_fake_quant: x_q = qdq(GELU(y) * s) / s in bf16 with state's scale -- first running
 *     the amax of GELU(y) when state is pending (hif8_linear_fwd[_wq]_gelu_stat could not settle
 *     it), otherwise reading y once.  A one-workgroup kernel first tables x_q over y's 16 bits
 *     into state (for a state whose amax pass proved the input finite), and the pass maps y
 *     through that table; other states take the per-element evaluation.
 * GELU(y) = bf16(0.5 y (1 + tanh(sqrt(2/pi) (y + 0.044715 y^3)))) in fp32, the same evaluation
 * in every kernel.  y: n bf16, x_q: n bf16, 16-byte aligned.  No counterpart of its own in the
 * reference, which runs GELU, amax and the fake quant as separate tensor ops. */
int hif8_gelu_absmax_scale(const uint16_t *y, int64_t n, float scale_max, void *state, hif8_stream_t stream);
/* The GELU those kernels apply, written out: g = GELU(y) for n bf16 values (nn.GELU(approximate=
 * "tanh") on a bf16 tensor, osp_next.py:875), through the window table the quantisation pass uses
 * (closed forms outside |y| in [0.0024, 6)).  y and g 16-byte aligned. */
int hif8_gelu_bf16(const uint16_t *y, uint16_t *g, int64_t n, hif8_stream_t stream);
int hif8_gelu_fake_quant(const uint16_t *y, int64_t n, void *state, float scale_max, uint16_t *x_q, int semantics,
                         hif8_stream_t stream);

/* Decode codes to x_q = decode(code) / scale in out_dtype (bf16 x_q of a bf16
 * tensor, or fp32 x_q of an fp32 tensor). */
int hif8_decode(const uint8_t *codes, int64_t n, const void *state, int out_dtype, void *y,
                hif8_stream_t stream);

/* Unscaled qdq drop-ins for the reference's pybind entry points
 * npu_quant.hif8_quant(x, y) and npu_quant.hif8_quant_bf16(x, y)
 * (ospnext/quant_cy_npu/base/cusrc/npu_quant.cpp:19-33 -> run_hif8_kernel[_bf16],
 * hif8_quant_op.h:208-214).  Unlike the reference, n is 64-bit, every length is
 * handled (no 512-element batches past the end) and semantics is selectable
 * (HIF8_SEM_TORCH gives QFuncs/hif8.py:6-23 in fp32; hif8_quant_bf16 also takes
 * HIF8_SEM_TORCH_BF16, the same function in bf16 arithmetic). */
int hif8_quant_f32(const float *x, float *y, int64_t n, int semantics, hif8_stream_t stream);
int hif8_quant_bf16(const uint16_t *x, uint16_t *y, int64_t n, int semantics,
                    hif8_stream_t stream);
/* quant_dequant_float(x, QType('hif8'), force_py, force_fp32) of an fp16 tensor, fp16 in and
 * out (QTensor.py:94-128 with its dtype routing at :66-79): HIF8_SEM_NPU -- the reference has no
 * fp16 NPU kernel, so the fp32 kernel runs on x.float() and the result is cast back to fp16
 * (QTensor.py:72-79,126-127); HIF8_SEM_TORCH -- force_py with force_fp32: QFuncs/hif8.py:6-23 in
 * fp32, then the cast; HIF8_SEM_TORCH_F16 -- force_py alone: the function in fp16 arithmetic
 * (QFuncs/hif8.py:10-11).  Any alignment; n >= 1. */
int hif8_quant_f16(const uint16_t *x, uint16_t *y, int64_t n, int semantics, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Fused HiF8 linear forward: hif8_linear.py:68-86
 *   y[M,N] = F.linear(x_q, w_q, bias) = x_q @ w_q^T + bias
 * with x_q the bf16 quantised activation (hif8_fake_quant, or hif8_fake_quant_to_bf16 for an
 * fp32 input) and w_q = decode(w_codes)/scale_w taken from w_state's table: the packed 8-bit
 * weight is decoded inside the GEMM.  bf16 MFMA, fp32 accumulation, bias added in fp32, bf16
 * output (RNE).
 *   a: [M,K] row-major bf16; w_codes: [N,K] row-major bytes; bias: [N] bf16 or NULL;
 *   y: [M,N] row-major bf16.
 * Shapes: K % 64 == 0, N % 8 == 0; M, N >= 1 and < 2^31, 1 <= K < 2^22.  16-byte aligned
 * a, w_codes and y; 8-byte aligned bias.
 */
int hif8_linear_fwd(const uint16_t *a, const uint8_t *w_codes, const void *w_state, const uint16_t *bias,
                    uint16_t *y, int64_t M, int64_t N, int64_t K, hif8_stream_t stream);

/* Several HIF8Linear layers on the same quantised input in one launch: the self-attention
 * q, k, v projections of osp_next.py:742-744 (each an F.linear(x_q, w_q, b) of
 * hif8_linear.py:86 on the same x_q), or any such set.  Each group i is its own weight
 * (its own state, hence its own scale) and output:
 *     ys[i][M, ns[i]] = x_q[M, K] . w_q_i[ns[i], K]^T + bias_i
 * a is bf16 x_q; w_codes holds the groups' codes concatenated along the output features
 * ([sum ns, K]); bias is NULL or the groups' biases concatenated ([sum ns]).  w_states, ys
 * and ns are host arrays of `groups` entries (1 <= groups <= 8).  Every ns[i] is a multiple
 * of 8 and, except the last, of 256 (a tile never spans two groups).  K % 64 == 0,
 * K < 2^22; a, w_codes and each ys[i] 16-byte aligned, bias 8-byte aligned.  The result of
 * each group equals hif8_linear_fwd of that group alone, bit for bit.
 * No single reference function: it merges the reference's separate linears of one input. */
int hif8_linear_fwd_grouped(const void *a, const uint8_t *w_codes, const void *const *w_states,
                            const uint16_t *bias, uint16_t *const *ys, const int64_t *ns, int groups,
                            int64_t M, int64_t K, hif8_stream_t stream);

/* Producer fusion for nn.Sequential(HIF8Linear, GELU(tanh), HIF8Linear) (osp_next.py:873-877),
 * the up-projection's half: hif8_linear_fwd with bf16 activations, the same y, whose epilogue
 * also folds the GELU statistic of y (its max, or a non-finite flag) into y_state.  When max y
 * settles amax|GELU(y)| (GELU(max y) above 0.1699, the largest |GELU| of a non-positive input;
 * GELU increases on y >= 0), y_state then holds that amax, its scale for scale_max and the
 * decode tables, as hif8_absmax_scale(GELU(y)) would; otherwise it is marked pending.  The
 * down-projection's _quant (hif8_linear.py:45-48) of the GELU layer's output is then
 * hif8_gelu_fake_quant(y, y_state), which applies GELU itself: the GELU output is never
 * written and no amax pass runs unless the state is pending.  y_state must have been
 * initialised (hif8_state_init); shapes as hif8_linear_fwd.  Two launches on the stream: the GEMM
 * (each wave folds its maximum with one relaxed atomic) and a one-workgroup kernel that settles
 * y_state from it.
 * No single reference function: it fuses three reference steps. */
int hif8_linear_fwd_gelu_stat(const void *a, const uint8_t *w_codes, const void *w_state, const uint16_t *bias,
                              uint16_t *y, int64_t M, int64_t N, int64_t K, float scale_max, void *y_state,
                              hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Decode-once route of hif8_linear_fwd for many rows: the same linear
 *   y[M,N] = x_q[M,K] @ w_q[N,K]^T + bias
 * (hif8_linear.py:86) with w_q given already dequantised, bf16 [N, K] -- hif8_decode of the
 * packed codes with the weight's state, into a caller buffer, once per call.  The fused kernel
 * decodes each weight element once per 256-row tile of x (M/256 times); this route decodes it
 * once and streams bf16 W.  The same 16x16x32 MFMA products in the same k order: the outputs
 * equal hif8_linear_fwd's bit for bit.  Shapes, alignment and the GELU-statistic and grouped variants
 * as for hif8_linear_fwd / _gelu_stat / _grouped (w_q concatenated along N for groups).
 * No counterpart of its own in the reference: it is F.linear on the dequantised operands. */
int hif8_linear_fwd_wq(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *y, int64_t M,
                       int64_t N, int64_t K, hif8_stream_t stream);

/* hif8_linear_fwd_wq with a split tail, for the backward's GEMMs (dgrad on the decode-once
 * route, wgrad): when a grid of fewer than 8 waves of 256 x 256 output tiles (one workgroup per
 * CU) ends in a partial wave that would leave over half the CUs idle, each of those tail tiles
 * is computed as 2-8 workgroups over
 * consecutive k ranges (at least 8 k-steps each), whose fp32 sums a second kernel adds in a fixed
 * order and rounds once: deterministic, and within fp32 rounding of the unsplit sums (the tail
 * tiles' outputs may differ from hif8_linear_fwd_wq's in the last bf16 bit).  The workspace is
 * hif8_linear_split_workspace_bytes(M, N, K) bytes of device memory, 16-byte aligned (at most
 * 64 MiB on 256 CUs; 0 when no split applies, e.g. whole waves); with workspace NULL every tile
 * is computed whole.  Shapes and alignment as hif8_linear_fwd_wq.  No counterpart of its own in
 * the reference: F.linear's and the backward matmuls' tiling is the library's choice. */
int64_t hif8_linear_split_workspace_bytes(int64_t M, int64_t N, int64_t K);
int hif8_linear_fwd_wq_split(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *y, int64_t M,
                             int64_t N, int64_t K, void *workspace, int64_t workspace_bytes, hif8_stream_t stream);
int hif8_linear_fwd_wq_gelu_stat(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *y,
                                 int64_t M, int64_t N, int64_t K, float scale_max, void *y_state,
                                 hif8_stream_t stream);
int hif8_linear_fwd_wq_grouped(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *const *ys,
                               const int64_t *ns, int groups, int64_t M, int64_t K, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * The DiT block's q/k normalisation and rotary embedding in one pass (the harness around the
 * path: the q/k projections' outputs on their way into attention).  x and out are bf16
 * [rows, dim], weight fp32 [dim]:
 *   y = rnd_bf16(rnd_f32(rnd_bf16(x * rsqrt(mean(x^2) + eps)) * weight))
 * is WanRMSNorm with an fp32 weight and a bf16 output (want2v.py:77-93 as osp_next.py:666-667
 * runs it under the high-precision norm policy).  With cos_t/sin_t (fp32 [cos batches, seq,
 * head_dim / 2]) each head's pairs (y[2i], y[2i+1]) are then rotated in fp32 by the angle of
 * the row's token (osp_next.py:596-644; row r is token r % seq of batch r / seq, which uses cos
 * batch r / seq / rep) and rounded to bf16 as the attention casts them (attention.py:460-518);
 * with NULL tables out = y (the cross-attention's norms, osp_next.py:794-796).  Shapes:
 * dim % 512 == 0, dim <= 8192; with rope 512 % head_dim == 0, dim % head_dim == 0 and
 * rows % seq == 0.  16-byte aligned pointers.  No counterpart of its own in the reference,
 * which runs these as about fifteen torch ops. */
int hif8_rms_norm_rope(const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t, uint16_t *out,
                       int64_t rows, int64_t dim, int64_t head_dim, int64_t seq, int64_t rep, float eps,
                       hif8_stream_t stream);
/* The same pass as producers of quant_attn="hif8" (hif8_attention.py:60-74): the reference
 * hands hif8_attention_with_mask the fp32 rope output of q and k (the norm's bf16 output when
 * there is no rope, the cross-attention's q) and quantises each with _quant before the
 * attention's bf16 cast.
 * hif8_rms_norm_rope_amax folds the amax of that output (fp32 with cos_t/sin_t, bf16 without)
 * into state with the scale rule for scale_max (fp32 rule with rope, bf16 rule without); the last
 * workgroup settles the state.  hif8_rms_norm_rope_fake_quant writes x_q, bf16 [rows, dim]: the
 * bf16 value of the output's fake quant with the state's scale (semantics HIF8_SEM_NPU or
 * HIF8_SEM_TORCH), and y, when not NULL, the output itself (fp32 [rows, dim] with rope, bf16
 * without; 16-byte aligned).  Shapes, tables and alignment as for hif8_rms_norm_rope. */
int hif8_rms_norm_rope_amax(const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t,
                            int64_t rows, int64_t dim, int64_t head_dim, int64_t seq, int64_t rep, float eps,
                            float scale_max, void *state, hif8_stream_t stream);
int hif8_rms_norm_rope_fake_quant(const uint16_t *x, const float *weight, const float *cos_t, const float *sin_t,
                                  int64_t rows, int64_t dim, int64_t head_dim, int64_t seq, int64_t rep, float eps,
                                  const void *state, int semantics, uint16_t *x_q, void *y, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Backward support.  The reference's dgrad is grad_q @ w_q (hif8_linear.py:97), a
 * product with the weight's [out, in] rows as the reduction dimension.  The fused
 * GEMM reduces over its weight operand's rows, so dgrad runs hif8_linear_fwd on
 * grad_q (bf16 [M, out]) and the transposed codes [in, out] with the weight's state.
 * This entry point has no reference counterpart (the reference never holds codes):
 * it writes out[c][r] = codes[r][c] for a [rows, cols] byte matrix.
 */
int hif8_transpose_codes(const uint8_t *codes, int64_t rows, int64_t cols, uint8_t *out, hif8_stream_t stream);

/* wgrad support.  The reference's weight gradient is grad_q^T @ x_q over the flattened tokens
 * (hif8_linear.py:100-105), a product whose reduction runs over the rows of both operands.  The
 * row-major decode-free GEMM reduces over its operands' rows of contiguous k, so the fallback
 * of hif8_linear_wgrad runs it on the two operands transposed, with the token dimension
 * padded with zeros to a multiple of 64 (zeros add nothing to the sums).  This entry point writes
 * out[c][r] = x[r][c] for r < rows and 0 for rows <= r < rows_pad: x bf16 [rows, cols],
 * out bf16 [cols, rows_pad].  Any shape and alignment; 16-byte aligned pointers, cols % 8 == 0
 * and rows_pad % 8 == 0 take the vector path.  No counterpart of its own in the reference. */
int hif8_transpose_bf16(const uint16_t *x, int64_t rows, int64_t cols, int64_t rows_pad, uint16_t *out,
                        hif8_stream_t stream);

/* The weight gradient of _HIF8LinearFunction.backward, grad_W = grad_q^T @ x_q
 * (hif8_linear.py:100-105), on the operands as the forward and the gradient quantisation leave
 * them, token-major:
 *   dw[n_out, k_in] = g[tokens, n_out]^T . x[tokens, k_in]     (fp32 sums, bf16 out)
 * The decode-free GEMM's tiles with both operands staged k-major in LDS and read with transposing
 * loads (ds_read_b64_tr_b16), so neither operand is transposed in memory; tokens need not be a
 * multiple of 64.  n_out % 8 == 0, k_in % 8 == 0, 16-byte aligned pointers, and
 * (tokens + 128) * n_out * 2 and (tokens + 128) * k_in * 2 below 2^32 (HIF8_ERR_SHAPE otherwise: the caller then
 * transposes both operands with hif8_transpose_bf16 and runs hif8_linear_fwd_wq_split).  The
 * split tail as for hif8_linear_fwd_wq_split, with
 * hif8_linear_split_workspace_bytes(n_out, k_in, tokens) bytes of workspace (or NULL): the
 * 1080 tiles over 75600 tokens of the 14B FFN-up weight split 56 tail tiles 4 ways.  The sums'
 * order differs from the reference's bf16 matmul (it does in any case).  No counterpart of its
 * own in the reference. */
int hif8_linear_wgrad(const uint16_t *g, const uint16_t *x, uint16_t *dw, int64_t tokens, int64_t n_out,
                      int64_t k_in, void *workspace, int64_t workspace_bytes, hif8_stream_t stream);

/* The backward's products for a layer that computes in fp32: grad_q @ w_q and grad_q^T @ x_q
 * (hif8_linear.py:97,104), which the reference evaluates as matmuls in the saved tensors' dtype.
 *   c[m][n] = sum_k a[m*sa_m + k*sa_k] * b[k*sb_k + n*sb_n]      (fp32 fused multiply-adds)
 * a, b: HIF8_DTYPE_BF16 or HIF8_DTYPE_F32 elements with any element strides (a transposed operand
 * is a stride pair); c: [M, N] row-major, HIF8_DTYPE_F32 or HIF8_DTYPE_BF16 (RNE).  M < 2^22.
 * An LDS-tiled fp32 kernel (the MFMA kernels take bf16 operands only); the sums' order differs
 * from the vendor matmul's. */
int hif8_gemm_f32(const void *a, int a_dtype, const void *b, int b_dtype, void *c, int c_dtype, int64_t M,
                  int64_t N, int64_t K, int64_t sa_m, int64_t sa_k, int64_t sb_k, int64_t sb_n,
                  hif8_stream_t stream);

/* Zero padding (or cropping) of a row-major matrix: dst[r][c] = src[r][c] for r < src_rows and
 * c < src_cols, 0 elsewhere in [dst_rows][dst_cols]; elem_bytes 1 (codes), 2 (bf16) or 4.  The
 * linears whose in_features is not a multiple of 64 or out_features not a multiple of 8 run the
 * MFMA GEMMs on operands padded with zeros (zero codes decode to 0, so the padding adds nothing)
 * and crop the output.  Any alignment.  No counterpart in the reference (its vendor GEMM takes
 * any shape). */
int hif8_pad_2d(const void *src, int64_t src_rows, int64_t src_cols, void *dst, int64_t dst_rows,
                int64_t dst_cols, int elem_bytes, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Producer fusion for the modulated LayerNorm in front of the self-attention q/k/v
 * and FFN-up projections: block_forward's
 *     y = norm(x) * (1 + scale) + shift                  (osp_next.py:941, :954)
 * with norm the WanLayerNorm (want2v.py:96-106: fp32 layer norm over the last dim,
 * no affine, eps, result cast to bf16), the product and sum bf16 tensor ops, and
 * then _quant(y) of each consuming HIF8Linear (hif8_linear.py:42-50).  No single
 * reference function: it fuses these steps, and the three identical _quant(y) of
 * q, k and v become one.
 *
 * x is bf16 [rows, dim] (dim % 8 == 0, dim <= 8192); shift and scale are bf16
 * [rows / rows_per_batch, dim] (row r uses modulation row r / rows_per_batch), or
 * NULL for zeros (then y = norm(x)).  stats is a float [rows * 2] buffer (8-byte
 * aligned) for each row's (mean, rstd); x, shift, scale, x_q and y are 16-byte
 * aligned.
 *
 * hif8_modln_amax: writes stats and folds amax|y| into state with the scale rule
 *   for scale_max, as hif8_absmax_scale(y) would (state initialised).
 * hif8_modln_fake_quant: x_q = qdq(y * s) / s in bf16 with that state, as
 *   hif8_fake_quant(y, state, semantics) would; y is also written when non-NULL.
 * The row statistics are fp32 two-pass sums, so y may differ from another fp32
 * layer norm's by one bf16 unit where the fp32 result rounds at a tie boundary;
 * x_q is exactly the qdq of the y this library computes.
 */
int hif8_modln_amax(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows, int64_t dim,
                    int64_t rows_per_batch, float eps, float *stats, float scale_max, void *state,
                    hif8_stream_t stream);
int hif8_modln_fake_quant(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows,
                          int64_t dim, int64_t rows_per_batch, const float *stats, const void *state,
                          int semantics, uint16_t *x_q, uint16_t *y, hif8_stream_t stream);

/* Allocation-free form of hif8_modln_amax + hif8_modln_fake_quant: the same x_q, bit for bit,
 * with the row statistics and the quantisation state held in a static device array of the
 * library (1 MiB + hif8_state_size() bytes per GPU, kept until the process ends) instead of
 * caller buffers: x, shift, scale and x_q as for those two entry points, no stats, no state, no
 * y.  It calls no allocation routine, so it serves callers that cannot allocate: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  rows <= 131072 (the 14B
 * model at 768P has 84672), else HIF8_ERR_SCRATCH before any work is enqueued.  Every call on a
 * GPU shares that GPU's array (the current device's; the stream must belong to it): calls that
 * overlap on one GPU -- two streams, or two host threads -- race, and must be serialised by the
 * caller.  The state's counters are cleared at the start of every call (a fill kernel, not a
 * memset).  No counterpart in the reference. */
int hif8_modln_quant_static(const uint16_t *x, const uint16_t *shift, const uint16_t *scale, int64_t rows,
                            int64_t dim, int64_t rows_per_batch, float eps, float scale_max, int semantics,
                            uint16_t *x_q, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * The block's residual updates (the harness around the path): x + y * e[2] and x + y * e[5]
 * (osp_next.py:947, :955) and x + cross_attn(...) (osp_next.py:949), as torch's bf16 ops
 * compute them: t = rnd_bf16(y * gate), out = rnd_bf16(x + t), each in fp32; with gate NULL,
 * out = rnd_bf16(x + y).  x, y, out bf16 [rows, dim]; gate bf16 [rows / rows_per_batch, dim]
 * (row r uses gate row r / rows_per_batch).  dim % 8 == 0, 16-byte aligned pointers; out may
 * be x.  No counterpart of its own in the reference, which runs them as two torch ops.
 */
int hif8_gated_residual(const uint16_t *x, const uint16_t *y, const uint16_t *gate, uint16_t *out, int64_t rows,
                        int64_t dim, int64_t rows_per_batch, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * The block's token layout changes (the harness around the path): the Skiparse rearranges
 * (skiparse_func.py:18-52: token, group, their reverses and token <-> group) with the zero padding
 * of a full -> Skiparse change and the cropping of a Skiparse -> full one (SkiparseRearrange.forward,
 * osp_next.py:239-283) are each one row permutation, run as a gather:
 *     out[r, :] = x[src_row[r], :]  for 0 <= src_row[r] < in_rows, zeros otherwise.
 * x bf16 [in_rows, cols], out bf16 [rows, cols], src_row int32 [rows]; cols % 8 == 0,
 * rows * cols / 8 < 2^31, 16-byte aligned x and out.  The reference runs them as einops / torch
 * permutes and pads; this replaces no reference interface of its own.
 */
int hif8_gather_rows(const uint16_t *x, int64_t in_rows, const int32_t *src_row, int64_t rows, int64_t cols,
                     uint16_t *out, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * Producer fusion for the affine LayerNorm in front of the cross-attention's q
 * projection:
 *     y = norm3(x)                                        (osp_next.py:949-951)
 * with norm3 the WanLayerNorm with elementwise_affine (osp_next.py:860-864,
 * want2v.py:96-106: fp32 layer norm with fp32 weight and bias, cast to bf16), then
 * _quant(y) of the q projection (hif8_linear.py:42-50).  No single reference
 * function: it fuses these steps.
 *
 * x is bf16 [rows, dim] (dim % 8 == 0, dim <= 6144); weight and bias are fp32 [dim];
 * stats, x_q, y, state and alignment as for hif8_modln_*, weight and bias 16-byte
 * aligned.  y = rnd_bf16(weight * ((x - mean) * rstd) + bias), the product-sum fused.
 * hif8_ln_affine_amax writes stats and folds amax|y| into state (scale rule for
 * scale_max); hif8_ln_affine_fake_quant writes x_q = qdq(y * s) / s (and y when
 * non-NULL).  As for hif8_modln_*, y may differ from another fp32 layer norm's by one
 * bf16 unit next to a rounding boundary; x_q is exactly the qdq of this y.
 */
int hif8_ln_affine_amax(const uint16_t *x, const float *weight, const float *bias, int64_t rows, int64_t dim,
                        float eps, float *stats, float scale_max, void *state, hif8_stream_t stream);
int hif8_ln_affine_fake_quant(const uint16_t *x, const float *weight, const float *bias, int64_t rows,
                              int64_t dim, const float *stats, const void *state, int semantics, uint16_t *x_q,
                              uint16_t *y, hif8_stream_t stream);

/* ---------------------------------------------------------------------------
 * The DiT's attention with the o projection's amax in its epilogue: attention_with_mask
 * (ospnext/modules/attention.py:460-518, the SDPA branch, attn_mask_kv as a list of the kept
 * keys) followed by the amax of _quant at the o projection (osp_next.py:777 ->
 * hif8_linear.py:42-46).
 *
 * out[b, i, h, :] = sum_j softmax_j(softmax_scale * q[b, i, h, :] . k[b, j, h, :]) v[b, j, h, :]
 * over the keys j kept for batch b; bf16 in and out, fp32 scores and accumulation.  q, k, v, out
 * are bf16 [batch][tokens][heads][head_dim] with token row strides row_strides[0..3] and batch
 * strides batch_strides[0..3] (elements, in the order q, k, v, out; a batch stride may be 0,
 * e.g. keys shared by every batch).  head_dim must be 128; strides multiples of 8, at least
 * heads * 128; for k and v, (n_kv - 1) * row stride * 2 + 256 below 2^31 and the row stride below
 * 2^23 elements; 16-byte aligned tensors.
 * key_idx NULL and key_count NULL: every key 0 .. n_kv - 1.  key_count [batch] alone: the first
 * key_count[b] keys.  key_idx [batch][idx_batch_stride] with key_count: the key rows
 * key_idx[b][0 .. key_count[b] - 1] (entries clamped to [0, n_kv)).  A query with no key gets
 * zeros (the reference raises for a sequence whose keys are all masked).
 * row_strides and batch_strides are host arrays of 4.
 * out_state NULL: attention only.  Otherwise the o projection's input state: the kernel folds the
 * amax of out and a one-workgroup kernel after it writes amax, scale (rule for scale_max) and
 * tables exactly as hif8_absmax_scale(out, out_state_dtype, ...) over out would, so the
 * quantisation of out needs no amax pass.  out_state_dtype HIF8_DTYPE_BF16_AS_F32: the o input
 * is out as fp32 values (the self-attention, whose q is fp32 after the rotary embedding);
 * HIF8_DTYPE_BF16: out itself (the cross-attention).
 */
int hif8_attention_fwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *out, int64_t batch,
                       int64_t n_q, int64_t n_kv, int64_t heads, int64_t head_dim, const int64_t *row_strides,
                       const int64_t *batch_strides, const int32_t *key_idx, int64_t idx_batch_stride,
                       const int32_t *key_count, float softmax_scale, void *out_state, int out_state_dtype,
                       float scale_max, hif8_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HIF8_MI355X_H */
