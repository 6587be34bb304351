/*
 * oracle/fp8_e4m3.c -- TEST INFRASTRUCTURE ONLY (checker, never shipped or measured).
 *
 * From-spec OCP 8-bit floating point, E4M3 "FN" variant (OCP 8-bit Floating Point
 * Specification (OFP8) rev 1.0, 2023): 1 sign bit, 4 exponent bits (bias 7), 3 mantissa
 * bits; no infinities; S.1111.111 is the only NaN; largest finite 448 (0x7E);
 * subnormals are m * 2^-9 for m = 1..7.
 *
 * Encoding rounds to nearest, ties to even, in the "non-saturating" convention: a value
 * whose rounded magnitude would exceed 448 (|x| > 464), an infinity or a NaN encodes as
 * NaN (0x7F with the input's sign).  This is the conversion that the reference's
 * quantize_kv_fp8 reaches through `tensor.to(torch.float8_e4m3fn)`
 * (specdec/engine/model_self.py:312); the exhaustive test in tests/ checks every fp32
 * bit pattern against torch's CPU cast.
 *
 * The encoder works on the fp32 bit pattern with integers only, so it does not depend on
 * the host's floating-point rounding mode or denormal handling.
 */
#include <stdint.h>
#include <string.h>
#include <stddef.h>

static uint8_t rne_shift(uint32_t mant, int shift) {
    /* round mant / 2^shift to nearest integer, ties to even (shift >= 1) */
    if (shift >= 32) return 0; /* mant < 2^24 <= 2^(shift-1): strictly below one half */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint8_t)q;
}

uint8_t oracle_e4m3fn_encode(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    const uint32_t a = u & 0x7FFFFFFFu;
    const int biased = (int)(a >> 23);
    if (biased == 0xFF) return (uint8_t)(0x7Fu | sign);          /* Inf / NaN */
    if (biased == 0) return sign;                                /* fp32 zero/subnormal: < 2^-126 -> 0 */
    const int e = biased - 127;                                  /* |f| = mant * 2^(e-23) */
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;          /* 24-bit significand */
    if (e < -6) {
        /* E4M3 subnormal range: value in units of 2^-9 is mant * 2^(e-23+9) */
        uint8_t q = rne_shift(mant, 14 - e);                     /* shift >= 21 */
        return (uint8_t)(q | sign);                              /* q == 8 is the 2^-6 normal: same code */
    }
    /* normal: keep the hidden bit plus 3 fraction bits */
    uint32_t q = rne_shift(mant, 20);                            /* in [8, 16] */
    int ee = e;
    if (q == 16u) { q = 8u; ee += 1; }
    const int ebits = ee + 7;
    if (ebits > 15 || (ebits == 15 && (q - 8u) == 7u)) return (uint8_t)(0x7Fu | sign);
    return (uint8_t)((uint32_t)(ebits << 3) | (q - 8u) | sign);
}

float oracle_e4m3fn_decode(uint8_t b) {
    const int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
    float v;
    if (e == 15 && m == 7) {
        uint32_t nan = 0x7FC00000u | ((uint32_t)s << 31);
        memcpy(&v, &nan, sizeof v);
        return v;
    }
    if (e == 0) {
        v = (float)m / 512.0f;                                   /* m * 2^-9, exact */
    } else {
        float p = 1.0f;
        int k = e - 7;
        for (; k > 0; --k) p *= 2.0f;
        for (; k < 0; ++k) p *= 0.5f;
        v = (1.0f + (float)m / 8.0f) * p;                        /* exact */
    }
    return s ? -v : v;
}

/* bulk helpers for ctypes */
void oracle_e4m3fn_encode_n(const float* in, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_e4m3fn_encode(in[i]);
}

/* encode every fp32 bit pattern in [lo, lo + n) (as uint32) */
void oracle_e4m3fn_encode_range(uint32_t lo, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u = lo + (uint32_t)i;
        float f;
        memcpy(&f, &u, sizeof f);
        out[i] = oracle_e4m3fn_encode(f);
    }
}

void oracle_e4m3fn_decode_n(const uint8_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_e4m3fn_decode(in[i]);
}
