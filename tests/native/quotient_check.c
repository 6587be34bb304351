/*
 * Exhaustive check of the division route of kernel 1 (quotient_rn in
 * specdec-context-scaling_amd/csrc/sdv_quant.hip).
 *
 * The reference quantizes v / s in fp32 with s = max|v| / 448 (quantize_kv_fp8,
 * specdec/engine/model_self.py:304-314) and casts the quotient to E4M3FN.  The kernel
 * instead divides through r = RN(1/s), computed once per token:
 *     q0 = RN(|x| r);  e = fma(-q0, s, |x|) (exact);  q = RN(q0 + e r)
 * This program walks every BF16 max-abs m (0, and every finite m >= 2^-60: the kernel's
 * fast route) and every BF16 x with 0 <= x <= m, for both scale modes
 * (s = RN(m / 448) and s = RN(m * RN(1/448)); s == 0 -> 1), and compares the E4M3FN code
 * of q with the code of the IEEE quotient RN(x / s).  Negative x follow by symmetry: both
 * routes round symmetrically and the kernel copies the sign of x onto q.  It also counts
 * fp32 differences of q from RN(x / s) and how many of them are at |q| >= 2^-10 (where
 * a difference could change a code).  Exit status 0 iff no code differs.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t oracle_e4m3fn_encode(float f); /* oracle/fp8_e4m3.c */

static float f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(void) {
    unsigned long long pairs = 0, code_diff = 0, q_diff = 0, q_diff_big = 0;
    for (int mode = 0; mode < 2; ++mode) {
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, code_diff, q_diff, q_diff_big)
        for (uint32_t mb = 0; mb <= 0x7F7F; ++mb) {
            if (mb != 0 && mb < 0x2180) continue; /* 0 < m < 2^-60: the kernel divides exactly */
            const float m = f32(mb << 16);
            float s = mode == 0 ? m / 448.0f : m * (1.0f / 448.0f);
            if (s == 0.0f) s = 1.0f;
            const float r = 1.0f / s;
            for (uint32_t xb = 0; xb <= mb; ++xb) {
                const float x = f32(xb << 16);
                const float want = x / s;
                const float q0 = x * r;
                const float e = fmaf(-q0, s, x);
                const float q = fmaf(e, r, q0);
                ++pairs;
                if (bits(q) != bits(want)) {
                    ++q_diff;
                    if (want >= 0x1p-10f) ++q_diff_big;
                }
                if (oracle_e4m3fn_encode(q) != oracle_e4m3fn_encode(want)) ++code_diff;
            }
        }
    }
    printf("pairs %llu code_diff %llu q_diff %llu q_diff_at_or_above_2^-10 %llu\n", pairs, code_diff, q_diff,
           q_diff_big);
    return code_diff != 0;
}
