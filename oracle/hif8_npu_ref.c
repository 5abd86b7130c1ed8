/*
 * CPU restatement of OSP-Next's Ascend HiF8 quantize-dequantize kernel, plus the
 * HiF8 8-bit code table.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
 * library built from it.  Nothing on the product path links it.
 *
 * hif8_npu_qdq_f32 follows ospnext/quant_cy_npu/base/cusrc/hif8_quant_op.h:88-151
 * (Hif8Vec<float>::Compute) step by step, one element at a time:
 *   :89        E     = bits(x) & 0x7F800000                    (2^e, 0 for denormals)
 *   :95-101    eabs  = max(E, ((~E) & 0x7F800000) - 2^23)      (2^|e|)
 *   :106-108   le15/le7/le3 = eabs <= 32768 / 128 / 8          (|e| <= 15 / 7 / 3)
 *   :109-110   keep_hi = x < 40960, keep_lo = x > -40960
 *   :111-113   keep0 = E >= 2^-23
 *   :118       E     = max(E, 2^-22)
 *   :120-128   step  = E * (le3?.5:1) * (le15?.5:1) * (le7?.5:1)
 *   :131-133   out   = round_half_away(x / step)               (vdiv, vconv_f322f32a)
 *   :137       out   = keep0 ? out : 0
 *   :140       out   = out * step
 *   :145,150   out   = keep_hi ? out : +Inf ;  out = keep_lo ? out : -Inf
 * The CCE intrinsics (vdiv, vconv_f322f32a) are not vendored; "f322f32a" is read
 * as round-half-away-from-zero, which the torch path (QFuncs/hif8.py:22,
 * floor(|x|*2^k + 0.5)) fixes independently.  On {0} U [2^-22, 40960) both
 * semantics agree exactly; the tests check that over every bf16 input.
 *
 * The 8-bit code layout is the published HiFloat8 layout (Luo et al., "Ascend
 * HiFloat8 Format for Deep Learning", 2024): sign | dot prefix | exponent
 * (sign + magnitude with implicit leading 1) | mantissa.  The reference never
 * materialises codes, so codes are checked through decode(encode(x)) == qdq(x).
 *   dot 0000 : denormal, value 2^(M-23), M = 1..7   (M = 0 is zero)
 *   dot 0001 : e = 0,            3 mantissa bits
 *   dot 001  : |e| = 1,          S, 3 mantissa bits
 *   dot 01   : |e| = 2..3,       S f, 3 mantissa bits
 *   dot 10   : |e| = 4..7,       S ff, 2 mantissa bits
 *   dot 11   : |e| = 8..15,      S fff, 1 mantissa bit
 * Specials: 0x00 = 0, 0x80 = NaN, 0x6F / 0xEF = +/-Inf (the e = +15, m = 1 slot),
 * so the largest finite magnitude is 2^15, which matches the kernel's 40960 cut.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* vconv_f322f32a: round to integral, ties away from zero */
static inline float round_half_away(float v) { return roundf(v); }

float hif8_npu_qdq_f32(float x)
{
    uint32_t E = f2u(x) & 0x7F800000u;                         /* :89 */
    float e_f = u2f(E);
    uint32_t nb = ((~E) & 0x7F800000u) - 0x00800000u;          /* :95-99 */
    float eabs = fmaxf(e_f, u2f(nb));                          /* :101 */
    int le15 = eabs <= 32768.0f, le7 = eabs <= 128.0f, le3 = eabs <= 8.0f;
    int keep_hi = x < 40960.0f, keep_lo = x > -40960.0f;       /* :109-110 */
    int keep0 = e_f >= u2f(0x34000000u);                       /* :111-113 */
    float step = fmaxf(e_f, u2f(0x34800000u));                 /* :116-118 */
    float b1 = le15 ? 0.5f : 1.0f, b2 = le7 ? 0.5f : 1.0f, b3 = le3 ? 0.5f : 1.0f;
    b1 = b2 * b1;                                              /* :125 */
    step = b3 * step;                                          /* :126 */
    step = b1 * step;                                          /* :128 */
    float out = x / step;                                      /* :131 */
    out = round_half_away(out);                                /* :133 */
    out = keep0 ? out : 0.0f;                                  /* :137 */
    out = out * step;                                          /* :140 */
    out = keep_hi ? out : INFINITY;                            /* :145 */
    out = keep_lo ? out : -INFINITY;                           /* :150 */
    return out;
}

/* bf16 variant (hif8_quant_op.h:80-84,154-157): widen, compute in fp32, narrow
 * with round-half-away.  Every finite output has <= 4 significant bits, so the
 * narrowing is exact; Inf stays Inf. */
uint16_t hif8_npu_qdq_bf16(uint16_t xb)
{
    float y = hif8_npu_qdq_f32(u2f((uint32_t)xb << 16));
    uint32_t u = f2u(y);
    uint32_t r = (u + 0x8000u) >> 16;      /* half-away on the magnitude bits */
    if (isnan(y)) r = 0x7FC0u;
    return (uint16_t)r;
}

/* ---- code table ---------------------------------------------------------- */

static uint8_t enc_mag(int e, int m3)
{
    int ae = e < 0 ? -e : e, S = e < 0;
    if (e == 0) return (uint8_t)(0x08 | m3);
    if (ae == 1) return (uint8_t)(0x10 | (S << 3) | m3);
    if (ae <= 3) return (uint8_t)(0x20 | (S << 4) | ((ae - 2) << 3) | m3);
    if (ae <= 7) return (uint8_t)(0x40 | (S << 4) | ((ae - 4) << 2) | (m3 >> 1));
    if (ae <= 15) return (uint8_t)(0x60 | (S << 4) | ((ae - 8) << 1) | (m3 >> 2));
    return (uint8_t)(e + 23);              /* denormal, e in [-22,-16] */
}

/* Code of a value that lies in the HiF8 value set (an output of the NPU qdq).
 * Every byte is a valid code, so "not representable" is reported through *ok. */
uint8_t hif8_encode_value(float q, int *ok)
{
    *ok = 1;
    if (isnan(q)) return 0x80;
    if (q == 0.0f) return 0x00;
    if (isinf(q)) return q > 0 ? 0x6F : 0xEF;
    uint32_t u = f2u(q);
    int s = (int)(u >> 31);
    int e = (int)((u >> 23) & 0xFF) - 127;
    uint32_t man = u & 0x7FFFFF;
    int m3 = (int)(man >> 20);
    if ((man & 0xFFFFF) != 0 || e < -22 || e > 15) { *ok = 0; return 0; }
    int ae = e < 0 ? -e : e;
    int mb = ae <= 3 ? 3 : ae <= 7 ? 2 : ae <= 15 ? 1 : 0;
    if (m3 & ((1 << (3 - mb)) - 1)) { *ok = 0; return 0; }
    if (e == 15 && m3 != 0) { *ok = 0; return 0; }   /* 1.5*2^15 is the Inf slot */
    return (uint8_t)((s << 7) | enc_mag(e, m3));
}

float hif8_decode(uint8_t c)
{
    if (c == 0x80) return NAN;
    if (c == 0x6F) return INFINITY;
    if (c == 0xEF) return -INFINITY;
    int s = c >> 7, u = c & 0x7F, e, m;
    if (u == 0) return 0.0f;
    if (u < 0x08) { e = u - 23; m = 0; }
    else if (u < 0x10) { e = 0; m = u & 7; }
    else if (u < 0x20) { e = ((u >> 3) & 1) ? -1 : 1; m = u & 7; }
    else if (u < 0x40) { int ae = 2 + ((u >> 3) & 1); e = ((u >> 4) & 1) ? -ae : ae; m = u & 7; }
    else if (u < 0x60) { int ae = 4 + ((u >> 2) & 3); e = ((u >> 4) & 1) ? -ae : ae; m = (u & 3) << 1; }
    else { int ae = 8 + ((u >> 1) & 7); e = ((u >> 4) & 1) ? -ae : ae; m = (u & 1) << 2; }
    float v = ldexpf(1.0f + (float)m / 8.0f, e);
    return s ? -v : v;
}

/* ---- batch entry points (ctypes) ---------------------------------------- */

void hif8_npu_qdq_f32_n(const float *x, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) y[i] = hif8_npu_qdq_f32(x[i]);
}

void hif8_npu_qdq_bf16_n(const uint16_t *x, uint16_t *y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) y[i] = hif8_npu_qdq_bf16(x[i]);
}

/* codes of NPU-qdq'd fp32 values; returns the number of inputs whose qdq value
 * has no code (must be 0: every NPU output is in the HiF8 value set). */
int64_t hif8_npu_encode_f32_n(const float *x, uint8_t *c, int64_t n)
{
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        int ok;
        c[i] = hif8_encode_value(hif8_npu_qdq_f32(x[i]), &ok);
        bad += !ok;
    }
    return bad;
}

void hif8_decode_n(const uint8_t *c, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) y[i] = hif8_decode(c[i]);
}
