// Device-side helpers shared by the codec and the GEMM: bit casts, bf16 rounding, the
// scale rule of hif8_linear.py:45-46 and the decode tables of a State.  The arithmetic
// here must stay IEEE-rounded op by op: every product and quotient is rounded before
// the next operation uses it (no contraction is possible in these expressions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_common.h"
#include "hif8_internal.h"

namespace hif8 {

__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ float bf2f(uint32_t b) { return u2f(b << 16); }

// float -> bf16 bits, round-to-nearest-even, NaN -> 0x7FC0 (c10::BFloat16).
__device__ __forceinline__ uint32_t f2bf(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Scale rule of hif8_linear.py:45-46 for the dtype; returns scale as fp32.
__device__ __forceinline__ float scale_from_amax(uint32_t amax_bits, int dtype, float smax, bool &fast)
{
    float a, s;
    if (dtype == kBF16) {
        uint32_t ab = amax_bits & 0x7FFFu;
        if (ab <= 0x7F80u) ab = ab > 0x322Cu ? ab : 0x322Cu;   // clamp(min=bf16(1e-8))
        a = bf2f(ab);
        float r = bf2f(f2bf(1.0f / a));                      // reciprocal()   (bf16)
        s = bf2f(f2bf(r * smax));                            // * scale_max    (bf16)
    } else {
        a = u2f(amax_bits & 0x7FFFFFFFu);
        if (!__builtin_isnan(a)) a = a > 1e-8f ? a : 1e-8f;
        float r = 1.0f / a;
        s = r * smax;
    }
    fast = __builtin_isfinite(a) && __builtin_isfinite(s) && s > 0.0f;
    return s;
}

// Fill the decode tables of st for scale s (one entry per thread, 256 threads).
// bf16 tensors: x_q = rnd_bf16(q / s) with q exact in bf16 (QTensor.py:126-127
// then the bf16 division of hif8_linear.py:48).  fp32 tensors: x_q = q / s in
// fp32, and the bf16 GEMM operand is its autocast rounding.
__device__ __forceinline__ void fill_luts(State *st, float s, uint32_t c)
{
    float y = u2f(decode_bits(c)) / s;
    st->lut_f32[c] = y;
    st->lut_bf16[c] = uint16_t(f2bf(y));
}

// Thread 0: amax a (magnitude bits) -> amax, scale, flags of st; returns the scale.
__device__ __forceinline__ float write_amax_state(State *st, uint32_t a, int dtype, float smax)
{
    bool fast;
    const float s = scale_from_amax(a, dtype, smax, fast);
    st->amax_bits = a;
    st->scale = s;
    st->fast = fast ? 1u : 0u;
    st->finite = fast ? 1u : 0u;   // amax finite => every element finite
    st->dtype = uint32_t(dtype);
    st->pending = 0u;
    return s;
}

// Fold one workgroup's amax (magnitude bits; NaN above every finite value) into st;
// the last of `nwg` workgroups resets the accumulators and writes amax, scale, flags
// and the tables.  Called by all 256 threads of the workgroup with `m` already reduced
// over it (only thread 0's value is used); `lds` is two words of LDS scratch.
__device__ __forceinline__ void fold_amax(State *st, uint32_t m, uint32_t nwg, int dtype, float smax,
                                          uint32_t *lds)
{
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        __hip_atomic_fetch_max(&st->amax_acc, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t prev = __hip_atomic_fetch_add(&st->counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        lds[0] = (prev == nwg - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!lds[0]) return;
    if (tid == 0) {
        const uint32_t a = __hip_atomic_exchange(&st->amax_acc, 0u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&st->counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds[1] = f2u(write_amax_state(st, a, dtype, smax));
    }
    __syncthreads();
    fill_luts(st, u2f(lds[1]), tid);
}

// Settle st after a kernel that folded the amax of its output into st->amax_acc with relaxed
// atomics (one workgroup of 256 threads, launched after it on the same stream): reset the
// accumulator and write amax, scale, flags and tables as an amax pass over that output would.
__device__ __forceinline__ void settle_amax(State *st, int dtype, float smax, uint32_t *lds)
{
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        const uint32_t a = st->amax_acc;
        st->amax_acc = 0u;
        lds[0] = f2u(write_amax_state(st, a, dtype, smax));
    }
    __syncthreads();
    fill_luts(st, u2f(lds[0]), tid);
}

}  // namespace hif8
