/* Exhaustive check of the product's bf16 rounding (test support, built by
 * tests/test_round_bf16.py): pw::round_bf16 from the shared host/device numerics header, the
 * select form every kernel inlines, equals the oracle's pwo_round_bf16 bit for bit on all 2^32 f32
 * bit patterns (NaN payloads, infinities, the overflow to infinity and every tie included). Prints
 * the input count and the number of mismatches, and exits 1 on any mismatch. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pw_numerics.h"

extern "C" float pwo_round_bf16(float value);

int main()
{
    long long inputs = 0, mismatches = 0;
#pragma omp parallel for reduction(+ : inputs, mismatches) schedule(static)
    for (long long i = 0; i < (1LL << 32); ++i) {
        const float x = pw::f32_from((uint32_t)i);
        const float got = pw::round_bf16(x), want = pwo_round_bf16(x);
        ++inputs;
        mismatches += memcmp(&got, &want, 4) != 0;
    }
    printf("inputs %lld mismatches %lld\n", inputs, mismatches);
    return mismatches != 0;
}
