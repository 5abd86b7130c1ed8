// Attention forward of the DiT block for MI355X (gfx950), with the HiF8 amax of its output folded
// into the o projection's quantisation state.
//
// The reference's attention (attention_with_mask, attention.py:460-518, SDPA branch) computes, per
// batch b, head h and query i,
//   out[b, i, h] = sum_j softmax_j(q[b, i, h] . k[b, j, h] / sqrt(128)) v[b, j, h]
// over the keys j its key mask keeps, in bf16 with fp32 accumulation, and the o projection then
// runs _quant on that output (hif8_linear.py:42-50 via osp_next.py:777): a full pass for amax|out|
// before the quantisation pass.  Here the attention kernel's epilogue keeps the max of the
// magnitudes it stores, so the amax pass is not needed.
//
// Design (flash attention, online softmax; head_dim 128):
//   - One workgroup per 384 queries of one (batch, head); 12 waves, three per SIMD (at most 168
//     VGPRs each), each owning 32 queries.  Keys go in tiles of 64: K and V tiles (16 KB each) are loaded
//     global -> LDS with buffer_load ... lds into one of two buffers while the other is computed;
//     every wave reads the whole tile from LDS, so more waves per tile mean fewer tile loads per
//     flop and more waves to cover each other's waits (measured at the 720P block's shape: 8 waves
//     1000 TFLOP/s, 12 waves 1090).
//   - Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_bf16: the A operand is
//     a K fragment from LDS, the B operand the wave's Q fragments, held in registers for the whole
//     kernel.  In the accumulator layout a lane holds one query and 4 keys of each 16 x 16 block,
//     which is exactly the B-operand layout of P^T for O^T = V^T P^T (the key order inside an MFMA's
//     reduction is free, and both operands use the same one), so P goes from the softmax to the
//     matrix cores without leaving the lane.  The V^T fragments come from LDS through
//     ds_read_b64_tr_b16 (transposing reads).
//   - Online softmax in the log2 domain with a lazily moved reference: the running max a tile's
//     exponentials are taken against only moves when a tile's max exceeds it by more than 8 (the
//     exponentials stay below 2^8 in between), so the O accumulators are rescaled a handful of times
//     per query instead of at every tile.  Row sums are per-lane partials of the bf16 probabilities
//     the P.V products take (v_dot2c_f32_bf16 with (1, 1): two per instruction), reduced once at
//     the end.  The row max is a tree of v_maximum3_f32 (fmaxf adds a canonicalising v_max per
//     input), and fragment addresses are one lane base per operand with the tile, key-block and
//     dim-block parts as immediate offsets: 115 VALU per wave and tile besides the exponentials
//     and their fmas, against 177 before (4 % of the kernel's time).
//   - Keys: an optional per-batch list of key rows (the rows the key mask keeps) and count; tiles
//     past the count are masked to -inf.  The whole key tensor is never gathered.  The list's
//     entries reach LDS like K and V (a ring of three 256-byte slots, two tiles ahead), so the loop
//     has no load of its own to wait for: a wait for a global load issued after a tile's K/V loads
//     would also wait for those (the counter completes in order), 14 % of the kernel's time.
//   - The exponentials are about 7 % of the time and the K/V loads after the prologue 12 %, of
//     which the traffic is 2 % (a copy loading the same 64 L2-resident rows every tile) and the
//     rest their issue and LDS writes: loading two tiles ahead into three buffers was slower, and
//     without the per-tile barrier the kernel ran the same (measured by removing each).
//   - Tile order: workgroup w runs on XCD w % 8; consecutive query tiles of one head are given to
//     one XCD, so the CUs of an XCD stream the same K/V tiles through its L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_internal.h"
#include "hif8_state_dev.h"

namespace hif8 {
namespace attn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;                  // head dim
constexpr int kBN = 64;                  // keys per tile
constexpr int kWaves = 12;
constexpr int kThreads = kWaves * 64;
constexpr int kQW = 32;                  // queries per wave
constexpr int kBM = kWaves * kQW;        // queries per workgroup
constexpr uint32_t kTile = kBN * kD * 2;  // bytes of one K or V tile
constexpr uint32_t kList = 4 * kTile;     // key-list ring: 3 slots of one tile's 64 entries
constexpr uint32_t kLds = kList + 3 * kBN * 4;
constexpr float kLazy = 8.0f;             // log2 headroom before the reference max moves

struct Params {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int64_t q_rs, k_rs, v_rs, o_rs;  // token row strides (elements)
    int64_t q_bs, k_bs, v_bs, o_bs;  // batch strides (elements)
    const int32_t *key_idx;          // [batch][idx_bs] key rows, or null (all n_kv keys in order)
    const int32_t *key_count;        // [batch] keys used, or null (n_kv)
    int64_t idx_bs;
    int n_q, n_kv, heads, q_tiles;
    float c;                         // softmax scale * log2(e)
    State *o_st;                     // amax of the output folded here, or null
    uint32_t o_shift;                // 16: folded as fp32 magnitude bits, 0: as bf16 bits
};

#define ASMV asm volatile

// 64 lanes x 16 B from the buffer (voffset per lane) into LDS at m0v + lane * 16
__device__ __forceinline__ void dtl_load(uint32_t m0v, uint32_t voff, const u32x4 &rs)
{
    ASMV("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(rs) : "memory", "m0");
}

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 ld_tr(const uint8_t *lds_base, uint32_t off)
{
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(lds_base + off));
    return __builtin_bit_cast(u32x2, v);
}

// 64 lanes x 4 B from the buffer (voffset per lane) into LDS at m0v + lane * 4
__device__ __forceinline__ void dtl_load_b32(uint32_t m0v, uint32_t voff, const u32x4 &rs)
{
    ASMV("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(rs) : "memory", "m0");
}

// max over the 4 lanes holding the same query (lanes l, l ^ 16, l ^ 32, l ^ 48): permlane32_swap
// of (m, m) gives lane l the pair m[l % 32], m[l % 32 + 32]; permlane16_swap the pair of rows 2k,
// 2k + 1 at lane l % 16.  The elements are copied out before the casts: a bit cast of a vector
// element reads element 0.
__device__ __forceinline__ float max_over_groups(float m)
{
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m),
                                                    false, false);
    const uint32_t p0 = p[0], p1 = p[1];
    m = __builtin_elementwise_maximum(__builtin_bit_cast(float, p0), __builtin_bit_cast(float, p1));
    const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m),
                                                    false, false);
    const uint32_t q0 = q[0], q1 = q[1];
    return __builtin_elementwise_maximum(__builtin_bit_cast(float, q0), __builtin_bit_cast(float, q1));
}

// LDS layout of a tile (64 keys x 128 dims, bf16):
//   K: key row r at r * 256, its 16-byte chunk c (dims 8c .. 8c + 7) at ((c ^ (r & 15)) * 16): the
//      16 rows an MFMA fragment read takes hit 16 distinct chunk positions, all 64 banks.
//   V: 128-byte blocks of 4 keys x 16 dims; block (q, P) -- keys 4q .. 4q + 3, dims 16P .. 16P + 15
//      -- at (8q + (P ^ (q & 1))) * 128, key 4q + e at +32e.  A ds_read_b64_tr_b16 gives lane l of
//      each 16-lane group element j of the four values loaded by lane 4j + (l % 16) / 4 of the group,
//      at position l % 4: lane 4j + u of group g loading dims 16P + 4u .. +3 of key 4g + j gives
//      lane (d, g) the keys 4g .. 4g + 3 of dim 16P + d.  Groups g and g + 1 (read in the same
//      cycle) read blocks of opposite parity, opposite halves of the banks.
//   A DTL instruction writes 1 KB: 4 K rows, or the 8 V blocks of one 4-key group.
// LIST: the keys are p.key_idx[b][0 .. count - 1]; otherwise keys 0 .. count - 1.  Key-list
// entries reach LDS the way K and V do (wave 0 loads a tile's 64 entries two tiles ahead into a
// ring of three slots), so the loop holds no global load whose wait would also wait for the
// K and V loads of the next tile.
template <bool LIST> __global__ __launch_bounds__(kThreads, 1) void k_attn_fwd(const Params p)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cq = lane & 15u, g = lane >> 4;

    // workgroup -> (batch, head, query tile), consecutive query tiles of a head on one XCD
    const int nwg = gridDim.x, w = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = w & 7, slot = w >> 3;
    const int L = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    const int qt = L % p.q_tiles, bh = L / p.q_tiles;
    const int h = bh % p.heads, b = bh / p.heads;

    int nk = p.n_kv;
    if (p.key_count) {
        nk = p.key_count[b];
        nk = nk < 0 ? 0 : (nk > p.n_kv ? p.n_kv : nk);
        if (p.key_idx && int64_t(nk) > p.idx_bs) nk = int(p.idx_bs);
    }
    nk = __builtin_amdgcn_readfirstlane(nk);
    const int ntiles = (nk + kBN - 1) / kBN;

    // buffer resources of this (batch, head)'s K and V: rows of 256 bytes at the row stride; the
    // range ends with the last key row
    u32x4 rk, rv, rl;
    {
        const uint64_t ka = uint64_t(p.k + int64_t(b) * p.k_bs + int64_t(h) * kD);
        const uint64_t va = uint64_t(p.v + int64_t(b) * p.v_bs + int64_t(h) * kD);
        const uint32_t kn = uint32_t(int64_t(p.n_kv - 1) * p.k_rs * 2 + kD * 2);
        const uint32_t vn = uint32_t(int64_t(p.n_kv - 1) * p.v_rs * 2 + kD * 2);
        rk = u32x4{uint32_t(ka), uint32_t(ka >> 32), kn, 0x00020000u};
        rv = u32x4{uint32_t(va), uint32_t(va >> 32), vn, 0x00020000u};
        // the key list's range is the batch's count: entries past it read as 0
        const uint64_t la = LIST ? uint64_t(p.key_idx + int64_t(b) * p.idx_bs) : 0;
        rl = u32x4{uint32_t(la), uint32_t(la >> 32), uint32_t(nk) * 4u, 0x00020000u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rk[i] = __builtin_amdgcn_readfirstlane(rk[i]);
            rv[i] = __builtin_amdgcn_readfirstlane(rv[i]);
            rl[i] = __builtin_amdgcn_readfirstlane(rl[i]);
        }
    }
    const uint32_t krs = uint32_t(p.k_rs * 2), vrs = uint32_t(p.v_rs * 2);
    // contiguous keys: a DTL item's lane offset inside its tile is the same for every tile (the
    // tile's first row goes into the buffer resource's base, rows past the tensor read as zero)
    uint32_t voffc[3] = {0u, 0u, 0u};
    if (!LIST) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint32_t item = wave + uint32_t(j) * kWaves;
            if (item < 16) {
                const uint32_t r = 4u * item + (lane >> 4);
                voffc[j] = r * krs + ((lane & 15u) ^ (r & 15u)) * 16u;
            } else if (item < 32) {
                const uint32_t it = item - 16u, r = 4u * it + ((lane & 7u) >> 1);
                voffc[j] = r * vrs + (16u * (((lane >> 3) ^ (it & 1u))) + 8u * (lane & 1u)) * 2u;
            }
        }
    }
    const uint32_t lds0 = uint32_t(uintptr_t(smem));
    // the key-list entries of tile t into ring slot t % 3 (wave 0)
    auto list_dtl = [&](int t) {
        if (LIST && wave == 0)
            dtl_load_b32(__builtin_amdgcn_readfirstlane(lds0 + kList + uint32_t(t % 3) * (kBN * 4)),
                         (uint32_t(t) * kBN + lane) * 4u, rl);
    };
    // the DTL of tile t: list entries are clamped into the tensor (keys past the count read row 0);
    // contiguous keys past the tensor read as zero through the buffer's range; keys past the count
    // are masked
    auto issue_tile = [&](int t) {
        const uint32_t buf = uint32_t(t & 1);
        if (!LIST) {
            // tile t's first row is row 64 t: base + 64 t rows, range less the same (t * 64 < n_kv)
            const uint32_t ko = uint32_t(t) * (uint32_t(kBN) * krs), vo = uint32_t(t) * (uint32_t(kBN) * vrs);
            const uint64_t kb = ((uint64_t(rk[1]) << 32) | rk[0]) + ko, vb = ((uint64_t(rv[1]) << 32) | rv[0]) + vo;
            const u32x4 rkt = u32x4{uint32_t(kb), uint32_t(kb >> 32), rk[2] - ko, rk[3]};
            const u32x4 rvt = u32x4{uint32_t(vb), uint32_t(vb >> 32), rv[2] - vo, rv[3]};
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const uint32_t item = wave + uint32_t(j) * kWaves;
                if (item < 16)
                    dtl_load(__builtin_amdgcn_readfirstlane(lds0 + buf * kTile + item * 1024u), voffc[j], rkt);
                else if (item < 32)
                    dtl_load(__builtin_amdgcn_readfirstlane(lds0 + 2u * kTile + buf * kTile + (item - 16u) * 1024u),
                             voffc[j], rvt);
            }
            return;
        }
        const int *slot = (const int *)(smem + kList + uint32_t(t % 3) * (kBN * 4));
        // 32 DTL items per tile (16 of K, 16 of V) over the waves: items wave, wave + 12, ...
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint32_t item = wave + uint32_t(j) * kWaves;
            if (item < 16) {
                const uint32_t it = item, r = 4u * it + (lane >> 4);
                const int raw = LIST ? slot[r] : t * kBN + int(r);
                const uint32_t row = uint32_t(min(max(raw, 0), p.n_kv - 1));
                dtl_load(__builtin_amdgcn_readfirstlane(lds0 + buf * kTile + it * 1024u),
                         __umul24(row, krs) + ((lane & 15u) ^ (r & 15u)) * 16u, rk);
            } else if (item < 32) {
                const uint32_t it = item - 16u, r = 4u * it + ((lane & 7u) >> 1);
                const int raw = LIST ? slot[r] : t * kBN + int(r);
                const uint32_t row = uint32_t(min(max(raw, 0), p.n_kv - 1));
                dtl_load(__builtin_amdgcn_readfirstlane(lds0 + 2u * kTile + buf * kTile + it * 1024u),
                         __umul24(row, vrs) + (16u * (((lane >> 3) ^ (it & 1u))) + 8u * (lane & 1u)) * 2u, rv);
            }
        }
    };

    if (ntiles > 0) {
        if (LIST) {
            list_dtl(0);
            if (ntiles > 1) list_dtl(1);
            ASMV("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        issue_tile(0);
    }

    // Q fragments: lane (cq, g) holds dims 32 pp + 8 g .. +7 of query 16 qb + cq of the wave's 32
    const int qbase = qt * kBM + int(wave) * kQW;
    u32x4 qf[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int row = qbase + 16 * qb + int(cq);
        const uint16_t *qr = p.q + int64_t(b) * p.q_bs + int64_t(row < p.n_q ? row : 0) * p.q_rs + int64_t(h) * kD;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            qf[qb][pp] = *(const u32x4 *)(qr + 32 * pp + 8 * g);
            if (row >= p.n_q) qf[qb][pp] = u32x4{0u, 0u, 0u, 0u};
        }
    }

    f32x4 o[8][2];
#pragma unroll
    for (int d = 0; d < 8; ++d)
        o[d][0] = o[d][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mref[2] = {-__builtin_inff(), -__builtin_inff()};
    float lsum[2] = {0.f, 0.f};
    const float c = p.c;

    // fragment read offsets (bytes) inside a tile
    const uint32_t kfrag = cq * 256u;                       // + kb * 4096, chunk ((4 pp + g) ^ cq) * 16
    const uint32_t vfrag = (8u * g) * 128u + 32u * ((lane & 15u) >> 2) + 8u * (lane & 3u);  // + block

    // lane parts of the fragment addresses (the tile, key block and dim block parts are immediates):
    // K chunk ((4 pp + g) ^ cq) of row cq; V block d ^ (g & 1) is d + (g & 1) for even d, d - (g & 1)
    // for odd d
    uint32_t ka[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) ka[pp] = kfrag + (((4u * pp + g) ^ cq) << 4);
    const uint32_t va_e = vfrag + (g & 1u) * 128u, va_o = vfrag - (g & 1u) * 128u;
    for (int t = 0; t < ntiles; ++t) {
        ASMV("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t + 1 < ntiles) issue_tile(t + 1);
        if (t + 2 < ntiles) list_dtl(t + 2);
        const uint8_t *ks = smem + uint32_t(t & 1) * kTile;
        const uint8_t *vs = smem + 2u * kTile + uint32_t(t & 1) * kTile;

        // S^T = K Q^T for the 64 keys x 32 queries of this wave
        f32x4 s[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            s[kb][0] = s[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                const u32x4 kf = *(const u32x4 *)(ks + ka[pp] + kb * 4096);
                s[kb][0] = mfma(kf, qf[0][pp], s[kb][0]);
                s[kb][1] = mfma(kf, qf[1][pp], s[kb][1]);
            }
        }
        // keys past the count (last tile only)
        if ((t + 1) * kBN > nk) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (t * kBN + 16 * kb + 4 * int(g) + i >= nk) s[kb][0][i] = s[kb][1][i] = -__builtin_inff();
        }

        u32x4 pf[2][2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = s[i >> 2][qb][i & 3];
#define MAX3(a, b, c) __builtin_elementwise_maximum(a, __builtin_elementwise_maximum(b, c))
            const float m0 = MAX3(v[0], v[1], v[2]), m1 = MAX3(v[3], v[4], v[5]), m2 = MAX3(v[6], v[7], v[8]);
            const float m3 = MAX3(v[9], v[10], v[11]), m4 = MAX3(v[12], v[13], v[14]);
            float mx = __builtin_elementwise_maximum(MAX3(m0, m1, m2), MAX3(m3, m4, v[15]));
#undef MAX3
            // this lane's scaled maximum: a query's tile maximum exceeds the reference by more than
            // kLazy if one of its four lanes' does, and the reduction over the lanes (scaling by
            // c > 0 commutes with it) is only needed when the reference moves
            const float mt = mx * c;
            if (__builtin_amdgcn_ballot_w64(mt > mref[qb] + kLazy)) {
                const float mn = __builtin_fmaxf(mref[qb], max_over_groups(mt));
                const float alpha = __builtin_amdgcn_exp2f(mref[qb] - mn);
                lsum[qb] *= alpha;
#pragma unroll
                for (int d = 0; d < 8; ++d) o[d][qb] *= alpha;
                mref[qb] = mn;
            }
            const float nm = -mref[qb];
            float e[4][4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    e[kb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][i], c, nm));
                }
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
                pf[qb][kc] = u32x4{pk_bf16(e[2 * kc][0], e[2 * kc][1]), pk_bf16(e[2 * kc][2], e[2 * kc][3]),
                                   pk_bf16(e[2 * kc + 1][0], e[2 * kc + 1][1]),
                                   pk_bf16(e[2 * kc + 1][2], e[2 * kc + 1][3])};
            // the row sums of the bf16 probabilities the P.V products take, two per instruction
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = pf[qb][kc][j];  // a scalar copy: a bit cast of a vector element reads element 0
                    lsum[qb] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                                              __builtin_bit_cast(bf16x2, 0x3F803F80u), lsum[qb], false);
                }
        }

        // O^T += V^T P^T
#pragma unroll
        for (int d = 0; d < 8; ++d) {
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                const uint8_t *vb = vs + ((d & 1) ? va_o : va_e);
                const u32x2 lo = ld_tr(vb, 8192u * kc + 128u * d), hi = ld_tr(vb, 8192u * kc + 128u * d + 4096u);
                const u32x4 vf = u32x4{lo.x, lo.y, hi.x, hi.y};
                o[d][0] = mfma(vf, pf[0][kc], o[d][0]);
                o[d][1] = mfma(vf, pf[1][kc], o[d][1]);
            }
        }
    }

    // epilogue: O / l, rounded to bf16; lane (cq, g) holds dims 16 d + 4 g .. +3 of query 16 qb + cq
    uint32_t amax = 0;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float l = lsum[qb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        const int row = qbase + 16 * qb + int(cq);
        if (row < p.n_q) {
            uint16_t *orow = p.out + int64_t(b) * p.o_bs + int64_t(row) * p.o_rs + int64_t(h) * kD + 4 * g;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const u32x2 wv = u32x2{pk_bf16(o[d][qb][0] * inv, o[d][qb][1] * inv),
                                       pk_bf16(o[d][qb][2] * inv, o[d][qb][3] * inv)};
                *(u32x2 *)(orow + 16 * d) = wv;
                const uint32_t m0 = wv.x & 0x7FFF7FFFu, m1 = wv.y & 0x7FFF7FFFu;
                amax = max(amax, max(max(m0 & 0xFFFFu, m0 >> 16), max(m1 & 0xFFFFu, m1 >> 16)));
            }
        }
    }
    if (p.o_st) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, off, 64));
        // one atomic per workgroup: every wave of every workgroup on one address contended at the L2
        // (a short-key attention, 512 text keys: 1.36 ms with them, 1.03 ms without the state)
        __shared__ uint32_t wmax[kWaves];
        if (lane == 0) wmax[wave] = amax;
        __syncthreads();
        if (tid == 0) {
            uint32_t m = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) m = max(m, wmax[w]);
            // bf16 values the o projection takes as fp32: the fp32 magnitude bits of the same value
            __hip_atomic_fetch_max(&p.o_st->amax_acc, m << p.o_shift, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The o projection's state after the attention: amax of the output (bf16, or as fp32 values),
// its scale for smax and the tables.
__global__ __launch_bounds__(256) void k_attn_amax_settle(State *__restrict__ st, int dtype, float smax)
{
    __shared__ uint32_t lds[1];
    settle_amax(st, dtype, smax, lds);
}

}  // namespace attn

extern "C" int hif8_attention_fwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *out,
                                  int64_t batch, int64_t n_q, int64_t n_kv, int64_t heads, int64_t head_dim,
                                  const int64_t *row_strides, const int64_t *batch_strides, const int32_t *key_idx,
                                  int64_t idx_batch_stride, const int32_t *key_count, float softmax_scale,
                                  void *out_state, int out_state_dtype, float scale_max, hif8_stream_t stream)
{
    using namespace attn;
    if (!q || !k || !v || !out || !row_strides || !batch_strides) return HIF8_ERR_ARG;
    if (batch <= 0 || n_q <= 0 || n_kv <= 0 || heads <= 0 || !(softmax_scale > 0.0f)) return HIF8_ERR_ARG;
    if (key_idx && (!key_count || idx_batch_stride <= 0)) return HIF8_ERR_ARG;
    if (out_state && (!(scale_max > 0.0f) || (out_state_dtype != kBF16 && out_state_dtype != kBF16F32)))
        return HIF8_ERR_ARG;
    if (head_dim != kD) return HIF8_ERR_SHAPE;
    const int64_t q_tiles = (n_q + kBM - 1) / kBM;
    if (n_q >= (int64_t(1) << 30) || n_kv >= (int64_t(1) << 30) || batch * heads * q_tiles >= (int64_t(1) << 31))
        return HIF8_ERR_SHAPE;
    for (int i = 0; i < 4; ++i) {
        if (row_strides[i] < heads * kD || row_strides[i] % 8 != 0 || batch_strides[i] < 0 || batch_strides[i] % 8 != 0)
            return HIF8_ERR_SHAPE;
    }
    // key offsets are 32-bit inside the buffer of one (batch, head), formed as a 24 x 24-bit
    // product of the key row and the row stride in bytes
    if ((n_kv - 1) * row_strides[1] * 2 + kD * 2 >= (int64_t(1) << 31) ||
        (n_kv - 1) * row_strides[2] * 2 + kD * 2 >= (int64_t(1) << 31) ||
        row_strides[1] * 2 >= (int64_t(1) << 24) || row_strides[2] * 2 >= (int64_t(1) << 24))
        return HIF8_ERR_SHAPE;
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u) return HIF8_ERR_ALIGN;
    if (((uintptr_t)key_idx | (uintptr_t)key_count) & 3u) return HIF8_ERR_ALIGN;

    Params p;
    p.q = q;
    p.k = k;
    p.v = v;
    p.out = out;
    p.q_rs = row_strides[0];
    p.k_rs = row_strides[1];
    p.v_rs = row_strides[2];
    p.o_rs = row_strides[3];
    p.q_bs = batch_strides[0];
    p.k_bs = batch_strides[1];
    p.v_bs = batch_strides[2];
    p.o_bs = batch_strides[3];
    p.key_idx = key_idx;
    p.key_count = key_count;
    p.idx_bs = idx_batch_stride;
    p.n_q = int(n_q);
    p.n_kv = int(n_kv);
    p.heads = int(heads);
    p.q_tiles = int(q_tiles);
    p.c = float(double(softmax_scale) * 1.4426950408889634);
    p.o_st = (State *)out_state;
    p.o_shift = out_state_dtype == kBF16F32 ? 16u : 0u;
    hipStream_t s = (hipStream_t)stream;
    if (key_idx)
        hipLaunchKernelGGL(k_attn_fwd<true>, dim3(unsigned(batch * heads * q_tiles)), dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL(k_attn_fwd<false>, dim3(unsigned(batch * heads * q_tiles)), dim3(kThreads), 0, s, p);
    if (out_state)
        hipLaunchKernelGGL(k_attn_amax_settle, dim3(1), dim3(256), 0, s, (State *)out_state,
                           out_state_dtype == kBF16F32 ? kF32 : kBF16, scale_max);
    return hipGetLastError() == hipSuccess ? HIF8_OK : HIF8_ERR_HIP;
}

}  // namespace hif8
