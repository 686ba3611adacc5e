/*
 * codec_arith_check.c -- exhaustive checks of the short arithmetic forms the
 * lane codec's band quantizer uses in place of IEEE division
 * (shannon-prime-llama_amd/csrc/sp_lane.h: div_by_level, rcp_f16_scale and the
 * summed code fields of rec_add_code). Each form must give bit-identical
 * results to the reference quantizer's float arithmetic
 * (kernel_band_quantize_simple, shannon_prime_cuda.cu:131-204):
 *
 *  1. a / m for a band's largest level m = 2^(bits-1) - 1, bits 2..8 (a 1-bit
 *     band has m = 0, whose non-finite scale always takes the exact path):
 *     q0 = a*r, rem = fma(-q0, m, a), q = fma(rem, r, q0) with r = fl(1/m),
 *     for every fp32 significand at two exponents (the steps scale exactly with
 *     the exponent while the quotient is normal).
 *  2. 1/s for s an fp16 value: r1 = fma(fma(-s, r0, 1), r0, r0) for every fp16
 *     significand and every start r0 within +-3 ulp of 1/s (v_rcp_f32 is
 *     specified to 1 ulp).
 *  3. the code field: bits(fl(v + 1.5*2^23)) + (m - 0x4B400000) == rint(v) + m
 *     for v = x*inv near every half-integer in [-m - 1/2, m + 1/2], and the
 *     shifted sum of a word's fields equals their bitwise insertion.
 *
 * Prints one line per check and exits non-zero on any mismatch.
 * Build: gcc -O2 -ffp-contract=off codec_arith_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float as_f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t as_u(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }

static long check_div_by_level(void) {
    long bad_total = 0;
    for (int bits = 2; bits <= 8; bits++) {
        const int mi = (1 << (bits - 1)) - 1;
        const float m = (float)mi, r = 1.0f / m;
        long bad = 0;
        for (uint32_t e = 0x3f800000u; e <= 0x40000000u; e += 0x00800000u) {
            for (uint32_t mant = 0; mant < 0x800000u; mant++) {
                const float a = as_f(e | mant);
                volatile float q0 = a * r;
                const float rem = fmaf(-q0, m, a);
                const float q = fmaf(rem, r, q0);
                if (as_u(q) != as_u(a / m)) bad++;
            }
        }
        printf("div_by_level m=%d: %ld mismatches over 2^24 dividends\n", mi, bad);
        bad_total += bad;
    }
    return bad_total;
}

static long check_rcp(void) {
    long bad = 0;
    for (int i = 0; i < 1024; i++) {
        const float s = 1.0f + (float)i / 1024.0f; /* every fp16 significand */
        const float t = 1.0f / s;
        for (int d = -3; d <= 3; d++) {
            const float r0 = as_f(as_u(t) + (uint32_t)d);
            const float e = fmaf(-s, r0, 1.0f);
            const float r1 = fmaf(e, r0, r0);
            if (as_u(r1) != as_u(t)) bad++;
        }
    }
    printf("rcp_f16_scale: %ld mismatches over 1024 significands x 7 starts\n", bad);
    return bad;
}

static long check_code_fields(void) {
    long bad = 0;
    for (int bits = 2; bits <= 8; bits++) {
        const int m = (1 << (bits - 1)) - 1;
        for (int h = -2 * m - 1; h <= 2 * m + 1; h++) { /* v around h/2 */
            for (int k = -4; k <= 4; k++) {
                float v = (float)h * 0.5f;
                for (int s = 0; s < (k < 0 ? -k : k); s++) v = nextafterf(v, k < 0 ? -INFINITY : INFINITY);
                if (fabsf(v) >= (float)m + 0.5f) continue;
                const float t = v + 12582912.0f;
                const uint32_t code = as_u(t) + ((uint32_t)m - 0x4B400000u);
                const int want = (int)rintf(v) + m;
                if (code != (uint32_t)want) bad++;
                /* the summed form of a field at every shift that keeps it in the word */
                for (int sh = 0; sh + bits <= 32; sh++) {
                    const uint32_t sum = (as_u(t) << sh) + (((uint32_t)m - 0x4B400000u) << sh);
                    if (sum != ((uint32_t)want << sh)) bad++;
                }
            }
        }
    }
    printf("code fields: %ld mismatches\n", bad);
    return bad;
}

int main(void) {
    const long bad = check_div_by_level() + check_rcp() + check_code_fields();
    printf("%s\n", bad ? "FAIL" : "OK");
    return bad != 0;
}
