/*
 * Plain-C restatement of the FlashFFN v3 per-group absmax codec (CPU oracle).
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile into
 * oracle/_build/liboracle_codec.so and bound by oracle/c_codec.py so that the
 * numpy restatement (oracle/codec.py) can be cross-checked bit-exactly against
 * an implementation with its own bit-level float16/bfloat16 rounding.
 *
 * Restates src/flashffn.py:1055-1110 (reference repo SDMuhsin/CompAct):
 *   scale = fp16(fp32(absmax / qmax)); safe = scale > 0 ? scale : 1;
 *   code  = clamp(rint(fp32(v / safe)), -qmax, qmax);
 *   int4: byte = (code[2j] + 8) | (code[2j+1] + 8) << 4; int8: code as int8;
 *   dequant = bf16(fp32(code) * fp32(scale)).
 * Build flags must keep IEEE semantics: -O2 -ffp-contract=off, no fast-math.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float32 -> binary16 bits, round-to-nearest-even, subnormals, overflow->inf. */
static uint16_t f32_to_f16_bits(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);          /* NaN */
    if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);         /* inf */
    int e = (int)(a >> 23) - 127;                                     /* unbiased */
    uint32_t mant = (a & 0x7FFFFFu) | (a >= 0x00800000u ? 0x800000u : 0u);
    if (a < 0x00800000u) e = -126;                                    /* f32 subnormal */
    /* value = mant * 2^(e-23). binary16 quantum: 2^(max(e,-14) - 10). */
    int qexp = (e < -14 ? -14 : e) - 10;
    int shift = qexp - (e - 23);            /* bits of mant below the quantum */
    uint32_t m;
    if (shift >= 32) {
        m = 0;
        if (shift == 32 && mant > 0x80000000u) m = 1;                 /* unreachable for f32 */
    } else if (shift > 0) {
        uint32_t kept = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        m = kept;
        if (rem > half || (rem == half && (kept & 1u))) m++;
    } else {
        m = mant << (-shift);
    }
    /* m is the significand at quantum 2^qexp; renormalise into fields */
    int be = qexp + 10 + 15;               /* biased exponent if m in [2^10, 2^11) */
    if (m >= 0x800u) { m >>= 1; be++; }    /* rounding carried out of the significand */
    if (m < 0x400u) return (uint16_t)(sign | m);                      /* subnormal or zero */
    if (be >= 31) return (uint16_t)(sign | 0x7C00u);                  /* overflow */
    return (uint16_t)(sign | ((uint32_t)be << 10) | (m & 0x3FFu));
}

static float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {                                                     /* subnormal: m * 2^-24 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    uint64_t r = ((uint64_t)u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return (uint16_t)r;
}

static float rint_even(float x) {          /* round half to even, exact in f32 */
    float fl = floorf(x);
    float rem = x - fl;                    /* exact for |x| < 2^24 */
    if (fabsf(x) >= 8388608.0f) return x;  /* already an integer */
    if (rem > 0.5f) return fl + 1.0f;
    if (rem < 0.5f) return fl;
    return (fmodf(fl, 2.0f) == 0.0f) ? fl : fl + 1.0f;
}

/* t: float32 [n, d] row-major. payload: int8 [n, d] or uint8 [n, d/2].
 * scales: binary16 bits [n, d/group]. Returns 0, or -1 on a bad argument. */
int oracle_quantize(const float* t, int64_t n, int64_t d, int bits, int group,
                    void* payload, uint16_t* scales) {
    if ((bits != 4 && bits != 8) || group <= 0 || d % group) return -1;
    const float qmax = (float)((1 << (bits - 1)) - 1);
    const int64_t ng = d / group;
    volatile float qm = qmax;               /* keep the division a real f32 division */
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t g = 0; g < ng; ++g) {
            const float* v = t + r * d + g * group;
            float amax = 0.0f;
            for (int i = 0; i < group; ++i) {
                float a = fabsf(v[i]);
                if (a > amax || a != a) amax = a;
            }
            float s32 = amax / qm;
            uint16_t sh = f32_to_f16_bits(s32);
            scales[r * ng + g] = sh;
            float safe = f16_bits_to_f32(sh);
            if (!(safe > 0.0f)) safe = 1.0f;
            for (int i = 0; i < group; ++i) {
                float q = rint_even(v[i] / safe);
                if (q < -qmax) q = -qmax;
                if (q > qmax) q = qmax;
                int64_t col = g * group + i;
                if (bits == 8) {
                    ((int8_t*)payload)[r * d + col] = (int8_t)q;
                } else {
                    uint8_t c = (uint8_t)(int)(q + 8.0f);
                    uint8_t* p = (uint8_t*)payload + r * (d / 2) + col / 2;
                    if (col & 1) *p = (uint8_t)((*p & 0x0Fu) | (c << 4));
                    else *p = (uint8_t)((*p & 0xF0u) | c);
                }
            }
        }
    }
    return 0;
}

/* Dequantize to bf16 bits [n, d]. */
int oracle_dequantize_bf16(const void* payload, const uint16_t* scales, int64_t n,
                           int64_t d, int bits, int group, uint16_t* out) {
    if ((bits != 4 && bits != 8) || group <= 0 || d % group) return -1;
    const int64_t ng = d / group;
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t col = 0; col < d; ++col) {
            float q;
            if (bits == 8) {
                q = (float)((const int8_t*)payload)[r * d + col];
            } else {
                uint8_t b = ((const uint8_t*)payload)[r * (d / 2) + col / 2];
                q = (float)((col & 1) ? (b >> 4) : (b & 0x0F)) - 8.0f;
            }
            float s = f16_bits_to_f32(scales[r * ng + col / group]);
            out[r * d + col] = f32_to_bf16_bits(q * s);
        }
    }
    return 0;
}

/* Exposed for the oracle's own tests of the conversion routines. */
uint16_t oracle_f32_to_f16_bits(float f) { return f32_to_f16_bits(f); }
uint16_t oracle_f32_to_bf16_bits(float f) { return f32_to_bf16_bits(f); }
