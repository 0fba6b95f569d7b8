/* Exhaustive check of the quantisers' division for bf16 inputs (test support, built by
 * tests/test_quant_ratio.py): for every positive finite bf16 group absmax m and every finite bf16 a
 * with |a| <= m, scale = max(m, 1e-10) / 448 and rcp = 1 / scale (IEEE), the quotient
 *   q = a * rcp;  copysign(fma(fma(-q, scale, a), rcp, q), q)
 * clamped to +-448 has the same e4m3fn code as a / scale (IEEE) clamped alike. Prints the pair
 * count and the number of code mismatches, and exits 1 on any mismatch. The e4m3fn encoder is the
 * oracle's (pwo_encode_e4m3fn). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int pwo_encode_e4m3fn(float value, uint8_t *out);

static float from_bits(uint32_t b)
{
    float x;
    memcpy(&x, &b, 4);
    return x;
}

static float clamp448(float v) { return v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v); }

int main(void)
{
    long long pairs = 0, mismatches = 0;
#pragma omp parallel for reduction(+ : pairs, mismatches) schedule(dynamic, 64)
    for (uint32_t mb = 1; mb < 0x7F80; ++mb) {
        const float m = from_bits(mb << 16);
        const float scale = fmaxf(m, 1.0e-10f) / 448.0f;
        const float rcp = 1.0f / scale;
        for (uint32_t ab = 0; ab < 0x10000; ++ab) {
            const float a = from_bits(ab << 16);
            if (!(fabsf(a) <= m))
                continue;
            const float q = a * rcp;
            const float got = copysignf(fmaf(fmaf(-q, scale, a), rcp, q), q);
            const float want = a / scale;
            ++pairs;
            if (memcmp(&got, &want, 4) == 0)
                continue;  /* equal quotients, equal codes */
            uint8_t cg, cw;
            pwo_encode_e4m3fn(clamp448(got), &cg);
            pwo_encode_e4m3fn(clamp448(want), &cw);
            mismatches += cg != cw;
        }
    }
    printf("pairs %lld code_mismatches %lld\n", pairs, mismatches);
    return mismatches != 0;
}
