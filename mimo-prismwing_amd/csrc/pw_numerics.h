// Scalar numerics shared by host and device code: bf16 rounding, e4m3fn decode and encode.
// These restate the reference semantics (src/text_endpoint.rs:2960-3006, src/lib.rs:7456-7467)
// in closed form so that the GPU can evaluate them without a lookup table or a search.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define PW_HD __host__ __device__ __forceinline__
#else
#define PW_HD static inline
#endif

namespace pw {

PW_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
PW_HD float f32_from(uint32_t u) { return __builtin_bit_cast(float, u); }
PW_HD bool finite_f32_bits(float v) { return (f32_bits(v) & 0x7f800000u) != 0x7f800000u; }

// f32 -> bf16 round-to-nearest-even, returned as the widened f32 value. NaNs keep their sign and
// high payload and get the quiet bit 0x40 (src/text_endpoint.rs:2960-2971); infinities pass (the
// rounding bias cannot carry out of a zero mantissa). Written as one select, not a branch: in
// GPU code a branch here becomes exec-mask control flow around every call.
PW_HD float round_bf16(float value)
{
    const uint32_t bits = f32_bits(value);
    const uint32_t rounded = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
    const uint32_t quiet = (bits | 0x00400000u) & 0xffff0000u;
    return f32_from((bits & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

PW_HD uint16_t bf16_bits(float value) { return (uint16_t)(f32_bits(round_bf16(value)) >> 16); }

// Quantiser scale of a group whose absolute maximum m is a bf16 value, max(m, 1e-10) / 448
// (src/text_endpoint.rs:3008-3051), without a division: the product with RN(1/448) corrected once
// by fused multiply-add (P. Markstein, IBM J. Res. Dev. 34(1), 1990). It equals the IEEE quotient
// for every non-negative finite bf16 m (all 32,640 of them, compared with the oracle on the CPU);
// groups of f32 values keep the division.
PW_HD float scale_of_bf16_max(float m)
{
    const float x = m > 1.0e-10f ? m : 1.0e-10f;
    const float r = 1.0f / 448.0f;
    const float q = x * r;
    return __builtin_fmaf(__builtin_fmaf(-q, 448.0f, x), r, q);
}

// e4m3fn byte -> f32: sign, 4-bit exponent (bias 7), 3-bit mantissa, subnormals m/8 * 2^-6,
// 0x7f / 0xff are NaN.
PW_HD float decode_e4m3fn(uint8_t b)
{
    const uint32_t sign = (uint32_t)(b & 0x80) << 24;
    const uint32_t e = (b >> 3) & 0xf, m = b & 7;
    if (e == 15 && m == 7)
        return f32_from(sign | 0x7fc00000u);
    if (e == 0) {
        // m * 2^-9, exact
        const float v = (float)m * 0.001953125f;
        return f32_from(f32_bits(v) | sign);
    }
    return f32_from(sign | ((e + 120u) << 23) | (m << 20));
}

// Nearest e4m3fn code of a finite value with |value| <= 448, ties to the even code, the input's
// sign bit carried (so -0.0 -> 0x80). Equivalent to the reference's 127-candidate search
// (src/text_endpoint.rs:2985-3006): adjacent codes are adjacent representable magnitudes, so the
// nearest candidate with even-code tie-break is round-half-to-even on the 3-bit mantissa, with
// the subnormal step 2^-9 below 2^-6.
PW_HD uint8_t encode_e4m3fn_rne(float value)
{
    const uint32_t bits = f32_bits(value);
    const uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag < 0x3c800000u) {  // |value| < 2^-6: subnormal step 2^-9
        const float scaled = f32_from(mag) * 512.0f;  // exact
        // round half to even of a value in [0, 8]
        const uint32_t whole = (uint32_t)scaled;
        const float frac = scaled - (float)whole;
        uint32_t q = whole;
        if (frac > 0.5f || (frac == 0.5f && (whole & 1u)))
            q += 1;
        return (uint8_t)(sign | q);  // q == 8 is code 0x08 = 2^-6
    }
    int32_t exponent = (int32_t)(mag >> 23) - 127;  // -6 .. 8
    uint32_t mantissa = mag & 0x7fffffu;
    uint32_t keep = mantissa >> 20;
    const uint32_t rest = mantissa & 0xfffffu;
    if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u)))
        keep += 1;
    if (keep == 8) {
        keep = 0;
        exponent += 1;
    }
    return (uint8_t)(sign | (uint32_t)((exponent + 7) << 3) | keep);
}

// sleef_expf_u10 (src/text_endpoint.rs:4511-4536), the PyTorch vectorised f32 exp.
PW_HD float sleef_expf_u10(float d)
{
    if (d < -104.0f)
        return 0.0f;
    if (d > 100.0f)
        return __builtin_inff();
    const int q = (int)__builtin_rintf(d * 1.44269504088896340736f);
    const float qf = (float)q;
    float s = __builtin_fmaf(qf, -0.69314575f, d);
    s = __builtin_fmaf(qf, -1.4286068e-6f, s);
    float u = 0.00019852762f;
    u = __builtin_fmaf(u, s, 0.0013930436f);
    u = __builtin_fmaf(u, s, 0.008333361f);
    u = __builtin_fmaf(u, s, 0.041666485f);
    u = __builtin_fmaf(u, s, 0.16666667f);
    u = __builtin_fmaf(u, s, 0.5f);
    u = __builtin_fmaf(s * s, u, s) + 1.0f;
    const int first_q = q >> 1;
    const int second_q = q - first_q;
    return (u * f32_from((uint32_t)(first_q + 127) << 23)) * f32_from((uint32_t)(second_q + 127) << 23);
}

// pytorch_sigmoid_f32 (src/text_endpoint.rs:4538-4540).
PW_HD float sigmoid_pytorch(float v) { return 1.0f / (1.0f + sleef_expf_u10(-v)); }

}  // namespace pw
