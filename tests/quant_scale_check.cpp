/* Exhaustive check of the bf16 quantisers' scale (test support, built by
 * tests/test_quant_scale.py): pw::scale_of_bf16_max from the shared host/device numerics header,
 * which forms max(m, 1e-10) / 448 from a product and one fused-multiply-add correction, equals the
 * scale the oracle's quantiser (pwo_dynamic_fp8) gives a group whose absolute maximum is m, for
 * every non-negative finite bf16 m. Prints the count and the number of mismatches, and exits 1 on
 * any mismatch. */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pw_numerics.h"

extern "C" int pwo_dynamic_fp8(const float *input, size_t rows, size_t cols, uint8_t *codes, float *scales,
                               float *dequantized);

int main()
{
    long long maxima = 0, mismatches = 0;
    float group[128];
    for (uint32_t hi = 0; hi < 0x7f80u; ++hi) {  // +0 .. the largest finite bf16
        const float m = pw::f32_from(hi << 16);
        memset(group, 0, sizeof group);
        group[hi % 128] = (hi & 1) ? -m : m;  // the maximum at varying positions, either sign
        float want = 0.f;
        if (pwo_dynamic_fp8(group, 1, 128, nullptr, &want, nullptr) != 0)
            return 2;
        const float got = pw::scale_of_bf16_max(m);
        ++maxima;
        mismatches += memcmp(&got, &want, 4) != 0;
    }
    printf("maxima %lld mismatches %lld\n", maxima, mismatches);
    return mismatches != 0;
}
