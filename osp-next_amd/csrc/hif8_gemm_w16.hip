// Decode-free twin of the fused HiF8 GEMM for MI355X (gfx950):
//   Y[M,N] = X_q[M,K] . W_q[N,K]^T + bias[N]
// with W_q already dequantised to bf16 (hif8_decode of the packed codes, once per call).  The
// fused kernel (hif8_gemm_dtl.hip) decodes every weight element once per 256-row tile of X:
// at M = 75600 that is 296 decodes per element, about a tenth of its cycles and of its energy
// at the board's power limit.  Decoding W once into a workspace and streaming bf16 W costs one
// pass over the codes and twice the weight bytes through L2; for a few thousand rows and more
// it is the faster route.  The products are the same v_mfma_f32_16x16x32_bf16 on the same
// operand values, in the same k order, so the two kernels agree bit for bit.
//
// Design (shared with k_linear_dtl except for W, the wave quadrants and the LDS ring):
//   - One workgroup per 256 x 256 output tile, 4 waves; wave w owns the 128 x 128 quadrant of
//     rows 128 (w & 1) .. +127 and output features 128 (w >> 1) .. +127: 8 x 8 tiles of
//     v_mfma_f32_16x16x32_bf16.  At the board's power limit the 16x16x32 form sustains about
//     13 % more bf16 throughput than 32x32x16 on the same operand data (it moves fewer
//     accumulator bytes per flop).  (k_linear_dtl gives each wave 64 features for all 256
//     rows because a wave decodes the W rows it uses.)
//   - X and W (bf16) go global -> LDS with buffer_load ... lds.  LDS is a ring of five 32 KB
//     operand stages (one operand, 256 rows x 64 k each; 160 KB): k-step j's X and W take
//     stages 2j and 2j + 1.  Each k-step has one barrier (in its second phase); the X loads of
//     k-step j + 2 are issued in the first phase of k-step j and the W loads right after the
//     barrier, so they have three and two phases to land.  With two 64 KB stages (128 KB) the
//     last loads of a k-step had less than one phase, and the loop waited for the misses of
//     every panel that L2 does not hold.
//   - The main loop is the fixed schedule in hif8_gemm_schedule_w16.inc (gen_gemm_schedule.py).
//   - Epilogue: bias, RNE to bf16, staged through LDS into whole 512-byte row stores, non-temporal
//     (the output is not read again here; it should not displace operand panels from L2); the
//     GELU-statistic variant and grouped outputs as in k_linear_dtl.
//   - Tile order: groups of group_m m-tiles, n-tiles outer within a group.  Workgroups go to the
//     8 XCDs round robin, so each XCD runs (group_m / 8) m-tiles x (256 / group_m) n-tiles of
//     every 256 consecutive tiles and its L2 fetches that many X and W panels.  Measured on the
//     14B shapes (ms, groups of 16 / 32 / 64 m-tiles): FFN up 7.37 / 7.22 / 7.17, FFN down
//     (N = 5120) 7.22 / 7.19 / 7.30, o 2.74 / 2.74 / 2.71; 128 was 10 % slower on FFN up.
//   - Token-major operands (TR, the weight gradient grad_q^T x_q on the tensors as they lie):
//     the same loop with k-major LDS stages and fragments built by transposing reads
//     (ds_read_b64_tr_b16), the same products in the same order.
//   - Split tail: for a grid of a few waves whose last one would leave most CUs idle, the tail
//     tiles are computed over k ranges into fp32 partials (EPI 2) that k_split_reduce adds in a
//     fixed order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"
#include "hif8_gelu_dev.h"
#include "hif8_state_dev.h"

namespace hif8 {
namespace w16 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 256;
constexpr int kBK = 64;
constexpr int kThreads = 256;
// m-tiles per group of the tile order: wide output (>= 32 n-tiles) / narrow output
constexpr int kGroupWide = 64;
constexpr int kGroupNarrow = 32;

// LDS map (bytes): operand stage s (0..4) at s * 32K, 256 rows x 128 B (64 k) with the 16-B
// chunks of row m XOR-swizzled by f(m) = (m & 7) ^ ((m >> 3) & 1): the 32 rows of a fragment
// read hit distinct banks.  The epilogue reuses the first 132 KB.
constexpr uint32_t kSlot = 32768;
constexpr uint32_t kSlots = 5;
constexpr uint32_t kOutRow = 528;  // epilogue: padded LDS row of the 256-wide output tile
constexpr uint32_t kLds = kSlots * kSlot;
static_assert(kLds >= 256 * kOutRow, "the epilogue staging fits in the ring");

#define ASMV asm volatile

template <int OFF> __device__ __forceinline__ void ldsb128(u32x4 &d, uint32_t a)
{
    ASMV("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(a), "i"(OFF));
}
__device__ __forceinline__ void mfma(f32x4 &c, const u32x4 &a, const u32x4 &b)
{
    ASMV("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
template <int N> __device__ __forceinline__ void wait_lgkm() { ASMV("s_waitcnt lgkmcnt(%0)" ::"i"(N)); }
template <int N> __device__ __forceinline__ void wait_vm() { ASMV("s_waitcnt vmcnt(%0)" ::"i"(N)); }
__device__ __forceinline__ void barrier() { ASMV("s_barrier" ::: "memory"); }
// 64 lanes x 16 B from the buffer (voffset per lane) into LDS at m0v + lane*16
__device__ __forceinline__ void dtl_load(uint32_t m0v, uint32_t voff, const u32x4 &rs)
{
    ASMV("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(rs) : "memory", "m0");
}
__device__ __forceinline__ void tie(u32x4 &a) { ASMV("" : "+v"(a)); }

__device__ __forceinline__ uint32_t f2bf_pk(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Per-wave loop state.  Fragment sets alternate between phases: set 0 is consumed in the even
// phase (first 32 k of a k-step) and filled in the odd one, set 1 the other way round.
// TR: the operands are k-major (token-major) in memory and in LDS, read with transposing loads
// (the K-major layout below).
template <bool TR> struct Ctx {
    u32x4 B[2][8];    // [set][j]  X fragments (m-tile j)
    u32x4 A[2][8];    // [set][i]  W fragments (n-tile i)
    uint32_t xb[2], wb[2];  // fragment read bases in stage 0: [phase p]; TR: [parity of the tile]
    uint32_t xr, wr;        // the same in the stages read this phase (TR: even tiles)
    uint32_t xr1, wr1;      // TR: odd tiles
    uint32_t xstep, wstep;  // TR: source bytes per k-step of X and W (uniform)
    f32x4 acc[8][8];
    u32x4 rx, rw, ex, ew;  // buffer resources: X, W, and the effective ones (size 0 past the end)
    uint32_t xoff[8], woff[8];  // DTL source offsets of the next X and W stage to load
    uint32_t xs, ws, ls;  // LDS offsets of the X and W stages read and of the stage loaded this phase
    uint32_t wave;
};

// K-major stage (TR): 64 k-rows x 256 columns of one operand in 128-byte blocks of 4 k-rows x
// 16 columns (the width of an MFMA tile); block (q, P) -- k-rows 4q .. 4q + 3, columns
// 16P .. 16P + 15 -- at (16 q + (P ^ ((q >> 1) & 1))) * 128, k-row 4q + e at +32 e.  A
// ds_read_b64_tr_b16 gives lane l of each 16-lane group element j of the 4 loaded by lane
// 4 j + (l % 16) / 4 of the group, at position (l % 4): with lane 4 j + u of group g loading
// columns 4u .. 4u + 3 of k-row 8 g + j (+ 4 for the second read), lane (r, g) receives k-rows
// 8 g .. 8 g + 7 of column r -- the operand layout of v_mfma_f32_16x16x32_bf16.  The XOR puts
// the k-rows 8 g + 0..3 of groups g and g + 1, read in the same cycle, in opposite halves of the
// 64 banks; within a block the 4 k-rows cover 32 distinct banks.  A DTL item (1 KB) is the 8
// blocks of one 4-k-row group and one half of the columns.

__device__ __forceinline__ uint32_t ring(uint32_t off, uint32_t n) { return off + n * kSlot >= kLds ? off + n * kSlot - kLds : off + n * kSlot; }
// before the reads of phase P: the even phase reads the second half of its own k-step, the odd
// phase the first half of the next one, whose stages are two further along the ring
template <int P, bool TR> __device__ __forceinline__ void read_bases(Ctx<TR> &c)
{
    if (P == 1) {
        c.xs = ring(c.xs, 2);
        c.ws = ring(c.ws, 2);
    }
    constexpr int p = 1 - P;
    if (TR) {
        // k-rows 32 p .. of the stage: 8 blocks of 4 k-rows further
        c.xr = c.xb[0] + c.xs + uint32_t(p) * 16384u;
        c.xr1 = c.xb[1] + c.xs + uint32_t(p) * 16384u;
        c.wr = c.wb[0] + c.ws + uint32_t(p) * 16384u;
        c.wr1 = c.wb[1] + c.ws + uint32_t(p) * 16384u;
    } else {
        c.xr = c.xb[p] + c.xs;
        c.wr = c.wb[p] + c.ws;
    }
}
template <bool TR> __device__ __forceinline__ void rotate(Ctx<TR> &c) { c.ls = ring(c.ls, 1); }
// a k-step further in the source: 64 k (128 bytes) along a row, or 64 k-rows (TR)
template <int I, bool TR> __device__ __forceinline__ void adv(Ctx<TR> &c)
{
    if (TR) {
        if (I < 8) ASMV("v_add_u32 %0, %1, %0" : "+v"(c.xoff[I]) : "s"(c.xstep));
        else ASMV("v_add_u32 %0, %1, %0" : "+v"(c.woff[I - 8]) : "s"(c.wstep));
    } else {
        if (I < 8) ASMV("v_add_u32 %0, 0x80, %0" : "+v"(c.xoff[I]));
        else ASMV("v_add_u32 %0, 0x80, %0" : "+v"(c.woff[I - 8]));
    }
}

// DTL item i of the X (OP 0) or W (OP 1) stage at the current source offsets, into the stage at
// `stage`: 1 KB at (8 wave + i) KB, rows (8 wave + i) * 8 .. + 7 x 128 B, or (TR) one half of the
// columns of 4 k-rows.
template <int OP, bool TR> __device__ __forceinline__ void issue_dtl(Ctx<TR> &c, uint32_t stage, int i)
{
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(stage + (c.wave * 8u + uint32_t(i)) * 1024u);
    if (OP == 0) dtl_load(m0v, c.xoff[i], c.ex);
    else dtl_load(m0v, c.woff[i], c.ew);
}
template <int OP, bool TR> __device__ __forceinline__ void issue_dtl(Ctx<TR> &c, int i) { issue_dtl<OP>(c, c.ls, i); }

// two transposing reads (TR): k-rows 8 g + 0..3 and 8 g + 4..7 of a 16-column tile
template <int OFF> __device__ __forceinline__ void ldstr(u32x4 &d, uint32_t a)
{
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 lo, hi;
    ASMV("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo) : "v"(a), "i"(OFF));
    ASMV("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(hi) : "v"(a), "i"(OFF + 2048));
    d = u32x4{lo.x, lo.y, hi.x, hi.y};
}
// one of the two transposing reads of a fragment (TR): H = 0 its k-rows 8 g + 0..3, H = 1 the
// next four, into the fragment's low or high half
template <int OFF, int H> __device__ __forceinline__ void ldstr_half(u32x4 &d, uint32_t a)
{
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 v;
    ASMV("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF + H * 2048));
    if (H == 0) d = u32x4{v.x, v.y, d.z, d.w};
    else d = u32x4{d.x, d.y, v.x, v.y};
}
template <int NXT, int J, int H, bool TR> __device__ __forceinline__ void rd_x_half(Ctx<TR> &c)
{
    ldstr_half<(J & ~1) * 128, H>(c.B[NXT][J], (J & 1) ? c.xr1 : c.xr);
}
template <int NXT, int I, int H, bool TR> __device__ __forceinline__ void rd_w_half(Ctx<TR> &c)
{
    ldstr_half<(I & ~1) * 128, H>(c.A[NXT][I], (I & 1) ? c.wr1 : c.wr);
}
// fragment reads: 16 rows x 128 B per m- or n-tile, or (TR) a 16-column block column
template <int NXT, int J, bool TR> __device__ __forceinline__ void rd_x(Ctx<TR> &c)
{
    if (TR) ldstr<(J & ~1) * 128>(c.B[NXT][J], (J & 1) ? c.xr1 : c.xr);
    else ldsb128<J * 2048>(c.B[NXT][J], c.xr);
}
template <int NXT, int I, bool TR> __device__ __forceinline__ void rd_w(Ctx<TR> &c)
{
    if (TR) ldstr<(I & ~1) * 128>(c.A[NXT][I], (I & 1) ? c.wr1 : c.wr);
    else ldsb128<I * 2048>(c.A[NXT][I], c.wr);
}
// Issue order of a phase's 64 MFMAs over the 8 x 8 tiles (i: W fragment, j: X fragment): 2 x 2
// blocks, (2bi, 2bj), (2bi + 1, 2bj), (2bi + 1, 2bj + 1), (2bi, 2bj + 1), the blocks in a snake
// along j.  Each fragment register pair feeds two MFMAs in a row before the next one switches in,
// and at the board's power limit that cost less: against the row order (A fixed for 8 MFMAs, B
// changing every MFMA) 1.3-2.6 % on the 14B shapes; a plain snake 0.3-1.7 %, 4 x 4 blocks 0.4-1.7 %,
// 2 x 4 or 4 x 2 blocks 1.0-1.4 %, a Hilbert curve 0.9-2.4 % (A/B of builds on one box).  Every
// accumulator still receives its products in k order, so the outputs do not change.
constexpr int blk2_order(int m)
{
    const int q = m / 4, r = m % 4, bi = q / 4, bj = (q / 4) % 2 ? 3 - q % 4 : q % 4;
    return 8 * (2 * bi + ((r == 1 || r == 2) ? 1 : 0)) + 2 * bj + (r >= 2 ? 1 : 0);
}
template <int CUR, int MI, bool TR> __device__ __forceinline__ void mm(Ctx<TR> &c)
{
    constexpr int i = blk2_order(MI) / 8, j = blk2_order(MI) % 8;
    mfma(c.acc[i][j], c.A[CUR][i], c.B[CUR][j]);
}
// after the wait covering the fragments of set SET
template <int SET, bool TR> __device__ __forceinline__ void tie_set(Ctx<TR> &c)
{
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        tie(c.B[SET][j]);
        tie(c.A[SET][j]);
    }
}

#include "hif8_gemm_schedule_w16.inc"

// Tile t of the order: groups of group_m m-tiles, n-tiles outer within a group.
__device__ __forceinline__ void tile_origin(int t, int tiles_m, int tiles_n, int group_m, int &m0, int &n0)
{
    const int group = t / (group_m * tiles_n);
    const int first_m = group * group_m;
    const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
    const int within = t - group * group_m * tiles_n;
    m0 = (first_m + within % gm) * kTile;
    n0 = (within / gm) * kTile;
}

// EPI 0: y = rnd(acc + bias).  EPI 1: the same y, and the GELU statistic of y (its max, or a
// non-finite flag) folded into y_st's accumulator; the settle kernel launched after it turns that
// into amax|GELU(y)| and its scale when max y settles it (hif8_gelu_dev.h).  The output features
// are G.n groups, each with its output buffer.
// EPI 2, the split tail: workgroup w computes k range w % splits (consecutive k-steps) of tile
// tile0 + w / splits and writes its fp32 sums to part (256 KB per workgroup, in the accumulators'
// lane order) for k_split_reduce.  (A separate instantiation: in the same kernel as the bf16
// epilogue, the register allocator moved all accumulators to VGPRs ahead of the branch and
// spilled.)
// TR: X and Wq are k-major, X^T [K][M] and Wq^T [K][N] (contiguous rows of M and N elements):
// the weight gradient's grad_q [tokens][out] and x_q [tokens][in] as they are, K = tokens.  Rows
// past K read as zero through the buffers' ranges; columns past M or N read other data, which
// only reaches outputs that are not stored.
template <int EPI, bool TR = false>
__global__ __launch_bounds__(kThreads, 1) void k_linear_w16(const uint16_t *__restrict__ X, const uint16_t *__restrict__ Wq,
                                                            const Groups G, const uint16_t *__restrict__ bias,
                                                            int M, int N, int K, int tiles_m, int tiles_n,
                                                            int group_m, State *__restrict__ y_st, int tile0,
                                                            int splits, float *__restrict__ part)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];
    ASMV("; lds base %0" ::"v"(uint32_t(uintptr_t(smem))) : "memory");
    Ctx<TR> c;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t r = lane & 15u, g = lane >> 4;

    int t = blockIdx.x;
    int nk = TR ? (K + kBK - 1) / kBK : K / kBK, kb = 0;
    if (EPI == 2) {
        t = tile0 + int(blockIdx.x) / splits;
        const int per = (nk + splits - 1) / splits;
        kb = (int(blockIdx.x) % splits) * per;
        nk = (nk - kb < per ? nk - kb : per);
    }
    int m0, n0;
    tile_origin(t, tiles_m, tiles_n, group_m, m0, n0);
    int gi = 0;
    while (gi + 1 < G.n && n0 / kTile >= G.tile_end[gi]) ++gi;
    uint16_t *__restrict__ Y = G.y[gi];
    const int col0 = gi == 0 ? 0 : G.tile_end[gi - 1] * kTile;
    const int ycols = G.cols[gi];

    if (!TR) {
        // the buffers start at k-step kb of row 0; rows past M or N lie past the range
        const uint32_t kofs = uint32_t(kb) * uint32_t(kBK) * 2u;
        const uint64_t xa = uint64_t(X) + uint64_t(m0) * uint64_t(K) * 2u + kofs;
        const uint32_t xrows = uint32_t(M - m0 < kTile ? M - m0 : kTile);
        c.rx = u32x4{uint32_t(xa), uint32_t(xa >> 32), xrows * uint32_t(K) * 2u - kofs, 0x00020000u};
        const uint64_t wa = uint64_t(Wq) + uint64_t(n0) * uint64_t(K) * 2u + kofs;
        const uint32_t wrows = uint32_t(N - n0 < kTile ? N - n0 : kTile);
        c.rw = u32x4{uint32_t(wa), uint32_t(wa >> 32), wrows * uint32_t(K) * 2u - kofs, 0x00020000u};
    } else {
        // the buffers start at column m0 (n0) of k-row 64 kb and end with the matrix: k-rows past
        // K lie past the range (the caller keeps K * M * 2 and K * N * 2 below 2^32)
        const uint64_t xofs = uint64_t(kb) * uint64_t(kBK) * uint64_t(M) * 2u + uint64_t(m0) * 2u;
        const uint64_t xa = uint64_t(X) + xofs;
        c.rx = u32x4{uint32_t(xa), uint32_t(xa >> 32), uint32_t(uint64_t(K) * uint64_t(M) * 2u - xofs), 0x00020000u};
        const uint64_t wofs = uint64_t(kb) * uint64_t(kBK) * uint64_t(N) * 2u + uint64_t(n0) * 2u;
        const uint64_t wa = uint64_t(Wq) + wofs;
        c.rw = u32x4{uint32_t(wa), uint32_t(wa >> 32), uint32_t(uint64_t(K) * uint64_t(N) * 2u - wofs), 0x00020000u};
        c.xstep = __builtin_amdgcn_readfirstlane(uint32_t(kBK) * uint32_t(M) * 2u);
        c.wstep = __builtin_amdgcn_readfirstlane(uint32_t(kBK) * uint32_t(N) * 2u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c.rx[i] = __builtin_amdgcn_readfirstlane(c.rx[i]);
        c.rw[i] = __builtin_amdgcn_readfirstlane(c.rw[i]);
    }
    const uint32_t wm = (c.wave & 1u) * 128u, wn = (c.wave >> 1) * 128u;
    if (!TR) {
        // DTL source offsets of k-step 0.  LDS 16-B slot s of a stage is written by lane s%64 of
        // load s/64; its source chunk is the slot's chunk un-swizzled (the XOR is an involution).
        // X and W rows share the layout.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = (c.wave * 8u + i) * 8u + (lane >> 3);
            const uint32_t ch = (lane & 7u) ^ (lane >> 3) ^ uint32_t(i & 1);
            c.xoff[i] = row * uint32_t(K) * 2u + ch * 16u;
            c.woff[i] = c.xoff[i];
        }
        // Fragment read bases.  Lane (r, g) = (lane & 15, lane >> 4) holds k = 32p + 8g .. +7 of
        // phase p for row r of its 16-row tile, for both operands: chunk 4p + g of rows wm + 16j + r
        // (X) and wn + 16i + r (W); f(row) = f(r).
        const uint32_t fr = (r & 7u) ^ ((r >> 3) & 1u);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t ch = ((4u * p + g) ^ fr) << 4;
            c.xb[p] = (wm + r) * 128u + ch;
            c.wb[p] = (wn + r) * 128u + ch;
        }
    } else {
        // DTL item it = 8 wave + i: 4-k-row group q = it / 2, column half it % 2; lane s writes
        // block P' = 8 (it % 2) + s / 8, k-row e = (s % 8) / 2, bytes 16 (s % 2) .. of its 32; the
        // source is column block P = P' ^ ((q >> 1) & 1) of k-row 4 q + e.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t it = c.wave * 8u + uint32_t(i), q = it >> 1;
            const uint32_t pb = ((it & 1u) * 8u + (lane >> 3)) ^ ((q >> 1) & 1u);
            const uint32_t krow = 4u * q + ((lane & 7u) >> 1);
            const uint32_t col = pb * 32u + (lane & 1u) * 16u;
            c.xoff[i] = krow * uint32_t(M) * 2u + col;
            c.woff[i] = krow * uint32_t(N) * 2u + col;
        }
        // Fragment read bases: lane (L, g) = (lane & 15, lane >> 4) reads k-rows 8 g + L / 4 (and
        // + 4) of the stage, columns 4 (L % 4) .. of a 16-column block: block group q = 2 g (+ 1),
        // XOR bit s = g & 1.  Even tiles J sit at J * 128 + s * 128, odd ones at (J - 1) * 128 +
        // 128 - s * 128 from the quadrant's first block (wm / 16 or wn / 16).
        const uint32_t sx = g & 1u;
        const uint32_t common = g * 4096u + (r >> 2) * 32u + (r & 3u) * 8u;
        c.xb[0] = common + (wm / 16u) * 128u + sx * 128u;
        c.xb[1] = common + (wm / 16u) * 128u + 128u - sx * 128u;
        c.wb[0] = common + (wn / 16u) * 128u + sx * 128u;
        c.wb[1] = common + (wn / 16u) * 128u + 128u - sx * 128u;
    }

    // The bias words of this lane's output features (4 per MFMA tile row i), loaded ahead of the
    // operand loads: they land during the main loop (in-order completion puts them before every
    // operand wait), where in the epilogue each was a global load waited for on its own.
    uint2 bw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int n = n0 + int(wn + uint32_t(i * 16) + 4u * (lane >> 4));
        bw[i] = (bias && n < N) ? *(const uint2 *)(bias + n) : uint2{0u, 0u};
    }

    // Prologue: X and W of k-steps 0 and 1 into stages 0..3; wait for k-step 0.
    c.ex = c.rx;
    c.ew = c.rw;
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_dtl<0>(c, 0u, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_dtl<1>(c, kSlot, i);
    c.ex[2] = nk > 1 ? c.rx[2] : 0u;
    c.ew[2] = nk > 1 ? c.rw[2] : 0u;
    adv<0>(c); adv<1>(c); adv<2>(c); adv<3>(c); adv<4>(c); adv<5>(c); adv<6>(c); adv<7>(c);
    adv<8>(c); adv<9>(c); adv<10>(c); adv<11>(c); adv<12>(c); adv<13>(c); adv<14>(c); adv<15>(c);
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_dtl<0>(c, 2u * kSlot, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_dtl<1>(c, 3u * kSlot, i);
    adv<0>(c); adv<1>(c); adv<2>(c); adv<3>(c); adv<4>(c); adv<5>(c); adv<6>(c); adv<7>(c);
    adv<8>(c); adv<9>(c); adv<10>(c); adv<11>(c); adv<12>(c); adv<13>(c); adv<14>(c); adv<15>(c);
    wait_vm<16>();
    barrier();
    // reads for the first phase (k-step 0, first half) into set 0
    c.xs = 0;
    c.ws = kSlot;
    c.xr = c.xb[0];
    c.wr = c.wb[0] + kSlot;
    c.xr1 = c.xb[1];  // TR: the odd tiles' bases
    c.wr1 = c.wb[1] + kSlot;
    rd_w<0, 0>(c); rd_x<0, 0>(c); rd_x<0, 1>(c); rd_x<0, 2>(c); rd_x<0, 3>(c);
    rd_x<0, 4>(c); rd_x<0, 5>(c); rd_x<0, 6>(c); rd_x<0, 7>(c);
    rd_w<0, 1>(c); rd_w<0, 2>(c); rd_w<0, 3>(c); rd_w<0, 4>(c); rd_w<0, 5>(c); rd_w<0, 6>(c); rd_w<0, 7>(c);
    c.ls = 4u * kSlot;  // the first phase loads X of k-step 2
    read_bases<0>(c);

#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) c.acc[i][j] = f32x4{};
    // One k-step per iteration.  The loads of k-step kk + 2 use the resources with size 0 past
    // the end: they read nothing and nothing consumes them.
    for (int kk = 0; kk < nk; ++kk) {
        c.ex[2] = kk + 2 < nk ? c.rx[2] : 0u;
        c.ew[2] = kk + 2 < nk ? c.rw[2] : 0u;
        if (TR) {
            phase0_tr(c);
            phase1_tr(c);
        } else {
            phase0(c);
            phase1(c);
        }
    }
    // no load may still target LDS when it is reused or released
    wait_vm<0>();
    wait_lgkm<0>();
    // the last MFMAs' results must be complete before the accumulators are read
    ASMV("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) ASMV("" : "+a"(c.acc[i][j]));

    if (EPI == 2) {
        // a k range of a split tile: the fp32 sums, 1 KB per store instruction
        f32x4 *P = (f32x4 *)part + size_t(blockIdx.x) * 16384u + c.wave * 4096u + lane;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) P[(i * 8 + j) * 64] = c.acc[i][j];
        return;
    }

    // Epilogue.  acc[i][j] lane (r, g), element e: D[n][m] with n = wn + 16i + 4g + e,
    // m = wm + 16j + r.  Rows go to LDS (padded), then each wave stores 2 rows x 512 B per
    // instruction.
    __syncthreads();
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            {
                const uint32_t nl = wn + uint32_t(i * 16) + 4u * g;
                const uint2 bb = bw[i];
                const float b0 = __builtin_bit_cast(float, bb.x << 16);
                const float b1 = __builtin_bit_cast(float, bb.x & 0xFFFF0000u);
                const float b2 = __builtin_bit_cast(float, bb.y << 16);
                const float b3 = __builtin_bit_cast(float, bb.y & 0xFFFF0000u);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const f32x4 &a = c.acc[i][j];
                    uint2 v;
                    v.x = f2bf_pk(a[0] + b0, a[1] + b1);
                    v.y = f2bf_pk(a[2] + b2, a[3] + b3);
                    *(uint2 *)(smem + (wm + uint32_t(j * 16) + r) * kOutRow + nl * 2u) = v;
                }
            }
        }
    }
    __syncthreads();
    // EPI 1: packed running maxima of the in-range outputs this lane stores (the GELU statistic)
    uint32_t smax_i = 0, smax_u = 0;
    {
        const uint32_t colb = (lane & 31u) * 16u, h = lane >> 5;
        const int n = n0 + int(colb / 2u);
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            u32x4 v[8];
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const uint32_t row = c.wave * 64u + uint32_t(blk * 8 + it) * 2u + h;
                v[it] = *(const u32x4 *)(smem + row * kOutRow + colb);
            }
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int m = m0 + int(c.wave * 64u + uint32_t(blk * 8 + it) * 2u + h);
                if (m < M && n - col0 < ycols) {
                    __builtin_nontemporal_store(v[it], (u32x4 *)(Y + size_t(m) * size_t(ycols) + (n - col0)));
                    if (EPI == 1) {
                        gelu_stat_pk(smax_i, smax_u, v[it][0], v[it][1]);
                        gelu_stat_pk(smax_i, smax_u, v[it][2], v[it][3]);
                    }
                }
            }
        }
    }
    if (EPI == 1) {
        uint32_t ystat = gelu_stat_final(smax_i, smax_u);
        for (int o = 32; o > 0; o >>= 1) ystat = max(ystat, (uint32_t)__shfl_xor((int)ystat, o, 64));
        if (lane == 0) fold_gelu_stat(y_st, ystat);
    }
}

// The split tiles' outputs: workgroup b sums the splits fp32 partials of tile full_tiles + b / 8,
// MFMA tile row i = b % 8 of each wave quadrant, in split order (a fixed order: the result does
// not depend on timing), adds the bias, rounds to bf16 and stores the in-range outputs.  One lane
// per 4 consecutive outputs of a row; 8 workgroups per tile so that the reads fill the chip.
__global__ __launch_bounds__(kThreads) void k_split_reduce(const float *__restrict__ part, int splits, int full_tiles,
                                                            int tiles_m, int tiles_n, int group_m, int M, int N,
                                                            const uint16_t *__restrict__ bias, uint16_t *__restrict__ Y)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t r = lane & 15u, g = lane >> 4;
    int m0, n0;
    const uint32_t tile = blockIdx.x >> 3;
    const int i = int(blockIdx.x & 7u);
    tile_origin(full_tiles + int(tile), tiles_m, tiles_n, group_m, m0, n0);
    const uint32_t wm = (wave & 1u) * 128u, wn = (wave >> 1) * 128u;
    const f32x4 *P = (const f32x4 *)part + size_t(tile) * size_t(splits) * 16384u + wave * 4096u + lane;
    {
        const int n = n0 + int(wn) + i * 16 + int(4u * g);
        if (n >= N) return;
        float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
        if (bias) {
            const uint2 bb = *(const uint2 *)(bias + n);
            b0 = __builtin_bit_cast(float, bb.x << 16);
            b1 = __builtin_bit_cast(float, bb.x & 0xFFFF0000u);
            b2 = __builtin_bit_cast(float, bb.y << 16);
            b3 = __builtin_bit_cast(float, bb.y & 0xFFFF0000u);
        }
        for (int j = 0; j < 8; ++j) {
            const int m = m0 + int(wm) + j * 16 + int(r);
            if (m >= M) continue;
            f32x4 a = P[(i * 8 + j) * 64];
            for (int sp = 1; sp < splits; ++sp) {
                const f32x4 q = P[size_t(sp) * 16384u + (i * 8 + j) * 64];
                a[0] = a[0] + q[0];
                a[1] = a[1] + q[1];
                a[2] = a[2] + q[2];
                a[3] = a[3] + q[3];
            }
            uint2 v;
            v.x = f2bf_pk(a[0] + b0, a[1] + b1);
            v.y = f2bf_pk(a[2] + b2, a[3] + b3);
            *(uint2 *)(Y + size_t(m) * size_t(N) + n) = v;
        }
    }
}

}  // namespace w16

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

// Split of the last, partial wave of tiles (one workgroup per CU): for grids of fewer than 8
// waves whose tail (tiles % CUs) fills at most half the CUs, each tail tile runs as `splits`
// workgroups over consecutive k ranges (at least 8 k-steps each), so the last wave takes about
// 1/splits of a tile's time.  Measured on MI355X: the 14B FFN-up wgrad (1080 tiles, 4.2 waves)
// 8.08-8.19 -> 7.22-7.26 ms; its dgrad (5920 tiles, 23.1 waves) 7.35 ms either way -- after
// many waves the CUs' tile boundaries have drifted apart and the tail tiles start as CUs free up.
struct SplitPlan {
    int full;     // tiles computed whole
    int tail;     // tiles computed in k ranges
    int splits;   // k ranges per tail tile (1: no split)
    int64_t bytes() const { return splits > 1 ? int64_t(tail) * splits * w16::kTile * w16::kTile * 4 : 0; }
};
static SplitPlan plan_split(int64_t tiles, int64_t K)
{
    const int cus = cu_count();
    const int tail = int(tiles % cus);
    const int64_t nk = (K + w16::kBK - 1) / w16::kBK;
    SplitPlan p{int(tiles), 0, 1};
    if (tiles < cus || tiles >= 8 * int64_t(cus) || tail == 0 || tail > cus / 2) return p;
    int sp = cus / tail;
    if (sp > 8) sp = 8;
    while (sp > 1 && nk < 8 * int64_t(sp)) --sp;
    if (sp < 2) return p;
    return SplitPlan{int(tiles) - tail, tail, sp};
}

// Shapes: K % 64 == 0, N % 8 == 0, 16-byte aligned X, W_q and Y, 8-byte aligned bias (checked
// by the caller).  M, N < 2^31, K < 2^22.  y_st != NULL selects the GELU-statistic epilogue and the
// settle kernel (scale for y_smax).  part != NULL (one output group, no y_st) splits the tail as
// plan_split says, with part holding plan_split(...).bytes() bytes.  tr: x and w_q are k-major
// (one output group, no y_st).
static int launch_w16(const uint16_t *x, const uint16_t *w_q, const Groups &g, const uint16_t *bias, int64_t M,
                      int64_t N, int64_t K, hif8_stream_t stream, State *y_st, float y_smax, float *part = nullptr,
                      bool tr = false)
{
    hipStream_t s = (hipStream_t)stream;
    if (K >= (int64_t(1) << 22)) return HIF8_ERR_SHAPE;
    const int tiles_m = int((M + w16::kTile - 1) / w16::kTile);
    const int tiles_n = int((N + w16::kTile - 1) / w16::kTile);
    const int64_t tiles = int64_t(tiles_m) * tiles_n;
    const int group_m = tiles_n >= 32 ? w16::kGroupWide : w16::kGroupNarrow;
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    SplitPlan sp{int(tiles), 0, 1};
    if (tr && (y_st || g.n != 1)) return HIF8_ERR_ARG;
    if (part) {
        if (y_st || g.n != 1) return HIF8_ERR_ARG;
        sp = plan_split(tiles, K);
    }
    if (y_st)
        hipLaunchKernelGGL(w16::k_linear_w16<1>, dim3(unsigned(sp.full)), dim3(w16::kThreads), 0, s, x, w_q, g, bias,
                           int(M), int(N), int(K), tiles_m, tiles_n, group_m, y_st, 0, 1, (float *)nullptr);
    else if (sp.full > 0 && tr)
        hipLaunchKernelGGL((w16::k_linear_w16<0, true>), dim3(unsigned(sp.full)), dim3(w16::kThreads), 0, s, x, w_q, g,
                           bias, int(M), int(N), int(K), tiles_m, tiles_n, group_m, (State *)nullptr, 0, 1,
                           (float *)nullptr);
    else if (sp.full > 0)
        hipLaunchKernelGGL(w16::k_linear_w16<0>, dim3(unsigned(sp.full)), dim3(w16::kThreads), 0, s, x, w_q, g, bias,
                           int(M), int(N), int(K), tiles_m, tiles_n, group_m, (State *)nullptr, 0, 1,
                           (float *)nullptr);
    if (hipGetLastError() != hipSuccess) return HIF8_ERR_HIP;
    if (sp.splits > 1) {
        // after the whole tiles on the stream: they fill whole waves, so the split workgroups
        // start as the last of them end
        if (tr)
            hipLaunchKernelGGL((w16::k_linear_w16<2, true>), dim3(unsigned(sp.tail * sp.splits)), dim3(w16::kThreads), 0,
                               s, x, w_q, g, bias, int(M), int(N), int(K), tiles_m, tiles_n, group_m, (State *)nullptr,
                               sp.full, sp.splits, part);
        else
            hipLaunchKernelGGL(w16::k_linear_w16<2>, dim3(unsigned(sp.tail * sp.splits)), dim3(w16::kThreads), 0, s, x,
                               w_q, g, bias, int(M), int(N), int(K), tiles_m, tiles_n, group_m, (State *)nullptr,
                               sp.full, sp.splits, part);
        if (hipGetLastError() != hipSuccess) return HIF8_ERR_HIP;
        hipLaunchKernelGGL(w16::k_split_reduce, dim3(unsigned(sp.tail) * 8u), dim3(w16::kThreads), 0, s, part, sp.splits,
                           sp.full, tiles_m, tiles_n, group_m, int(M), int(N), bias, g.y[0]);
        if (hipGetLastError() != hipSuccess) return HIF8_ERR_HIP;
    }
    return y_st ? launch_gelu_stat_settle(y_st, y_smax, stream) : HIF8_OK;
}

int launch_linear_w16(const uint16_t *x, const uint16_t *w_q, const uint16_t *bias, uint16_t *y, int64_t M,
                      int64_t N, int64_t K, hif8_stream_t stream, State *y_st, float y_smax)
{
    Groups g{};
    g.n = 1;
    g.tile_end[0] = int((N + w16::kTile - 1) / w16::kTile);
    g.cols[0] = int(N);
    g.y[0] = y;
    return launch_w16(x, w_q, g, bias, M, N, K, stream, y_st, y_smax);
}

int launch_linear_w16_groups(const uint16_t *x, const uint16_t *w_q, const Groups &g, const uint16_t *bias,
                             int64_t M, int64_t N, int64_t K, hif8_stream_t stream)
{
    return launch_w16(x, w_q, g, bias, M, N, K, stream, nullptr, 0.0f);
}

}  // namespace hif8

using namespace hif8;

static int check_w16(const void *a, const void *w_q, const uint16_t *bias, const void *y, int64_t M, int64_t N,
                     int64_t K)
{
    if (!a || !w_q || !y) return HIF8_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return HIF8_ERR_ARG;
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 22)) return HIF8_ERR_SHAPE;
    if (K % w16::kBK != 0 || N % 8 != 0) return HIF8_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)w_q | (uintptr_t)y) & 15u) return HIF8_ERR_ALIGN;
    if (bias && ((uintptr_t)bias & 7u)) return HIF8_ERR_ALIGN;
    const int64_t tiles = ((M + w16::kTile - 1) / w16::kTile) * ((N + w16::kTile - 1) / w16::kTile);
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    return HIF8_OK;
}

extern "C" int hif8_linear_fwd_wq(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *y,
                                  int64_t M, int64_t N, int64_t K, hif8_stream_t stream)
{
    const int rc = check_w16(a, w_q, bias, y, M, N, K);
    return rc != HIF8_OK ? rc : launch_linear_w16(a, w_q, bias, y, M, N, K, stream, nullptr, 0.0f);
}

extern "C" int64_t hif8_linear_split_workspace_bytes(int64_t M, int64_t N, int64_t K)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int64_t tiles = ((M + w16::kTile - 1) / w16::kTile) * ((N + w16::kTile - 1) / w16::kTile);
    return plan_split(tiles, K).bytes();
}

static int split_part(void *workspace, int64_t workspace_bytes, int64_t M, int64_t N, int64_t K, float **part)
{
    *part = nullptr;
    const int64_t need = hif8_linear_split_workspace_bytes(M, N, K);
    if (!workspace || need == 0) return HIF8_OK;
    if (workspace_bytes < need) return HIF8_ERR_ARG;
    if ((uintptr_t)workspace & 15u) return HIF8_ERR_ALIGN;
    *part = (float *)workspace;
    return HIF8_OK;
}

extern "C" int hif8_linear_fwd_wq_split(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias, uint16_t *y,
                                        int64_t M, int64_t N, int64_t K, void *workspace, int64_t workspace_bytes,
                                        hif8_stream_t stream)
{
    int rc = check_w16(a, w_q, bias, y, M, N, K);
    if (rc != HIF8_OK) return rc;
    float *part = nullptr;
    rc = split_part(workspace, workspace_bytes, M, N, K, &part);
    if (rc != HIF8_OK) return rc;
    Groups g{};
    g.n = 1;
    g.tile_end[0] = int((N + w16::kTile - 1) / w16::kTile);
    g.cols[0] = int(N);
    g.y[0] = y;
    return launch_w16(a, w_q, g, bias, M, N, K, stream, nullptr, 0.0f, part);
}

extern "C" int hif8_linear_wgrad(const uint16_t *g, const uint16_t *x, uint16_t *dw, int64_t tokens, int64_t n_out,
                                 int64_t k_in, void *workspace, int64_t workspace_bytes, hif8_stream_t stream)
{
    if (!g || !x || !dw) return HIF8_ERR_ARG;
    if (tokens <= 0 || n_out <= 0 || k_in <= 0) return HIF8_ERR_ARG;
    if (n_out % 8 != 0 || k_in % 8 != 0) return HIF8_ERR_SHAPE;
    if (n_out >= (int64_t(1) << 31) || k_in >= (int64_t(1) << 31) || tokens >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    // the k-major buffers address g and x with 32-bit offsets, including the k-rows of the last
    // k-step past the tokens (which must fall past the buffers' ranges, not wrap into them)
    if ((tokens + 128) * n_out * 2 >= (int64_t(1) << 32) || (tokens + 128) * k_in * 2 >= (int64_t(1) << 32))
        return HIF8_ERR_SHAPE;
    if (((uintptr_t)g | (uintptr_t)x | (uintptr_t)dw) & 15u) return HIF8_ERR_ALIGN;
    const int64_t tiles = ((n_out + w16::kTile - 1) / w16::kTile) * ((k_in + w16::kTile - 1) / w16::kTile);
    if (tiles >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
    float *part = nullptr;
    const int rc = split_part(workspace, workspace_bytes, n_out, k_in, tokens, &part);
    if (rc != HIF8_OK) return rc;
    Groups gr{};
    gr.n = 1;
    gr.tile_end[0] = int((k_in + w16::kTile - 1) / w16::kTile);
    gr.cols[0] = int(k_in);
    gr.y[0] = dw;
    return launch_w16(g, x, gr, nullptr, n_out, k_in, tokens, stream, nullptr, 0.0f, part, true);
}

extern "C" int hif8_linear_fwd_wq_gelu_stat(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias,
                                            uint16_t *y, int64_t M, int64_t N, int64_t K, float scale_max,
                                            void *y_state, hif8_stream_t stream)
{
    if (!y_state) return HIF8_ERR_ARG;
    const int rc = check_w16(a, w_q, bias, y, M, N, K);
    return rc != HIF8_OK ? rc : launch_linear_w16(a, w_q, bias, y, M, N, K, stream, (State *)y_state, scale_max);
}

extern "C" int hif8_linear_fwd_wq_grouped(const uint16_t *a, const uint16_t *w_q, const uint16_t *bias,
                                          uint16_t *const *ys, const int64_t *ns, int groups, int64_t M, int64_t K,
                                          hif8_stream_t stream)
{
    if (!ys || !ns || groups < 1) return HIF8_ERR_ARG;
    if (groups > kMaxGroups) return HIF8_ERR_SHAPE;
    Groups g{};
    g.n = groups;
    int64_t N = 0;
    for (int i = 0; i < groups; ++i) {
        if (!ys[i] || ns[i] <= 0) return HIF8_ERR_ARG;
        if (ns[i] % 8 != 0 || (i + 1 < groups && ns[i] % w16::kTile != 0)) return HIF8_ERR_SHAPE;
        if ((uintptr_t)ys[i] & 15u) return HIF8_ERR_ALIGN;
        N += ns[i];
        if (N >= (int64_t(1) << 31)) return HIF8_ERR_SHAPE;
        g.tile_end[i] = int((N + w16::kTile - 1) / w16::kTile);
        g.cols[i] = int(ns[i]);
        g.y[i] = ys[i];
    }
    const int rc = check_w16(a, w_q, bias, ys[0], M, N, K);
    return rc != HIF8_OK ? rc : launch_linear_w16_groups(a, w_q, g, bias, M, N, K, stream);
}
