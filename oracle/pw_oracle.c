/*
 * CPU oracle (test infrastructure only; see pw_oracle.h). Plain C restatement of the reference
 * CPU numerics for the block-scaled FP8 projection and routed-MoE path. Deliberately scalar and
 * sequential: it is the readable checker, not a fast path.
 */
#include "pw_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* src/lib.rs:7456-7467 (decode_f8_e4m3fn); MSL twin kernels/block_fp8_gemv.metal:4-15. */
float pwo_decode_e4m3fn(uint8_t bits)
{
    const float sign = (bits & 0x80) == 0 ? 1.0f : -1.0f;
    const int exponent = (bits >> 3) & 0x0f;
    const int mantissa = bits & 0x07;
    if (exponent == 0)
        return sign * ldexpf(1.0f, -6) * ((float)mantissa / 8.0f);
    if (exponent == 15 && mantissa == 7)
        return f32_from_bits(((uint32_t)(bits & 0x80) << 24) | 0x7ff00000u);
    return sign * ldexpf(1.0f, exponent - 7) * (1.0f + (float)mantissa / 8.0f);
}

/* src/text_endpoint.rs:2960-2971 (round_bf16): RNE with bias 0x7fff + lsb; NaN payload | 0x40. */
float pwo_round_bf16(float value)
{
    const uint32_t bits = bits_from_f32(value);
    if ((bits & 0x7f800000u) == 0x7f800000u) {
        if ((bits & 0x007fffffu) == 0)
            return value;
        const uint16_t payload = (uint16_t)((bits >> 16) | 0x0040u);
        return f32_from_bits((uint32_t)payload << 16);
    }
    const uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
    return f32_from_bits((bits + bias) & 0xffff0000u);
}

/* src/text_endpoint.rs:2985-3006 (encode_f8_e4m3fn): nearest of the 127 non-negative finite
 * codes by f32 distance, ties to the even code, sign from the input's sign bit. */
int pwo_encode_e4m3fn(float value, uint8_t *out)
{
    if (!isfinite(value) || fabsf(value) > 448.0f)
        return -1;
    const int negative = signbit(value) != 0;
    if (value == 0.0f) {
        *out = negative ? 0x80 : 0x00;
        return 0;
    }
    const float magnitude = fabsf(value);
    uint8_t best = 0;
    float best_distance = INFINITY;
    for (unsigned candidate = 0; candidate <= 0x7e; ++candidate) {
        const float distance = fabsf(magnitude - pwo_decode_e4m3fn((uint8_t)candidate));
        if (distance < best_distance ||
            (distance == best_distance && (candidate & 1u) == 0 && (best & 1u) != 0)) {
            best = (uint8_t)candidate;
            best_distance = distance;
        }
    }
    *out = (uint8_t)(best | (negative ? 0x80 : 0x00));
    return 0;
}

/* src/text_endpoint.rs:3008-3051 (dynamic_fp8_activations): per row, per 128-column group,
 * scale = max(absmax, 1e-10) / 448, code = encode(clamp(x / scale, -448, 448)). */
int pwo_dynamic_fp8(const float *input, size_t rows, size_t cols, uint8_t *codes, float *scales,
                    float *dequantized)
{
    const size_t group = 128;
    const float epsilon = 1.0e-10f, fp8_max = 448.0f;
    if (rows == 0 || cols == 0 || cols % group != 0 || input == NULL)
        return -1;
    for (size_t i = 0; i < rows * cols; ++i)
        if (!isfinite(input[i]))
            return -2;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < cols / group; ++g) {
            const float *values = input + r * cols + g * group;
            float absmax = 0.0f;
            for (size_t i = 0; i < group; ++i)
                absmax = fmaxf(absmax, fabsf(values[i]));
            absmax = fmaxf(absmax, epsilon);
            const float scale = absmax / fp8_max;
            if (!isfinite(scale) || scale <= 0.0f)
                return -2;
            if (scales)
                scales[r * (cols / group) + g] = scale;
            for (size_t i = 0; i < group; ++i) {
                float normalized = values[i] / scale;
                if (normalized < -fp8_max) normalized = -fp8_max;
                if (normalized > fp8_max) normalized = fp8_max;
                uint8_t code;
                if (pwo_encode_e4m3fn(normalized, &code) != 0)
                    return -2;
                const size_t at = r * cols + g * group + i;
                if (codes)
                    codes[at] = code;
                if (dequantized)
                    dequantized[at] = pwo_decode_e4m3fn(code) * scale;
            }
        }
    }
    return 0;
}

static size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

static int weights_finite(const uint8_t *w, size_t count)
{
    for (size_t i = 0; i < count; ++i)
        if (w[i] == 0x7f || w[i] == 0xff)
            return 0;
    return 1;
}

/* bf16_linear (src/text_endpoint.rs:3347-3380): decode the BF16 tensor (bits << 16, exact), f32
 * GEMM, round every output to bf16; the GPU form execute_bf16_linear (src/wide_metal_moe.rs:
 * 728-834) checks the input is finite. The reference's SGEMM order is closed; this restatement
 * sums sequentially over columns with separate multiply and add (like mapped_fp8_gemv).
 * y_raw (optional) receives the sums before rounding. */
int pwo_bf16_linear(const uint16_t *w, size_t n, size_t k, const float *x, size_t rows, float *y,
                    float *y_raw)
{
    if (w == NULL || x == NULL || y == NULL || n == 0 || k == 0 || rows == 0)
        return -1;
    for (size_t i = 0; i < rows * k; ++i)
        if (!isfinite(x[i]))
            return -2;
    for (size_t p = 0; p < rows; ++p) {
        const float *input = x + p * k;
        for (size_t r = 0; r < n; ++r) {
            const uint16_t *row = w + r * k;
            float sum = 0.0f;
            for (size_t c = 0; c < k; ++c) {
                const uint32_t bits = (uint32_t)row[c] << 16;
                float wv;
                memcpy(&wv, &bits, 4);
                sum += wv * input[c];
            }
            if (y_raw)
                y_raw[p * n + r] = sum;
            const float rounded = pwo_round_bf16(sum);
            if (!isfinite(rounded))
                return -3;
            y[p * n + r] = rounded;
        }
    }
    return 0;
}

/* src/lib.rs:1272-1309 (mapped_fp8_gemv; fixture form block_fp8_gemv :7469-7493) generalised to
 * `rows` activation rows and a partial trailing 128-row block: sequential over columns,
 * sum += decoded * scale * activation, f32, no fused multiply-add. Validation follows
 * validate_fp8_views_internal (src/lib.rs:1217-1270). */
int pwo_gemm_mode_a(const uint8_t *w, const float *s, size_t n, size_t k, const float *x,
                    size_t rows, float *y)
{
    if (w == NULL || s == NULL || x == NULL || y == NULL || n == 0 || k == 0 || k % 128 != 0 ||
        rows == 0)
        return -1;
    const size_t scale_cols = k / 128;
    for (size_t i = 0; i < ceil_div(n, 128) * scale_cols; ++i)
        if (!isfinite(s[i]))
            return -2;
    for (size_t i = 0; i < rows * k; ++i)
        if (!isfinite(x[i]))
            return -2;
    if (!weights_finite(w, n * k))
        return -2;
    for (size_t p = 0; p < rows; ++p) {
        const float *input = x + p * k;
        for (size_t r = 0; r < n; ++r) {
            const uint8_t *row = w + r * k;
            const float *scale_row = s + (r / 128) * scale_cols;
            float sum = 0.0f;
            for (size_t c = 0; c < k; ++c)
                sum += pwo_decode_e4m3fn(row[c]) * scale_row[c / 128] * input[c];
            if (!isfinite(sum))
                return -3;
            y[p * n + r] = sum;
        }
    }
    return 0;
}

/* src/wide_metal_moe.rs:404-421 (CPU equation of the block-scaled probe) and the kernel
 * kernels/block_fp8_gemv.metal:935-1046: per 128-column block the code dot product, then
 * total += dot * weight_scale * input_scale, blocks ascending. */
int pwo_gemm_mode_b_equation(const uint8_t *w, const float *s, size_t n, size_t k,
                             const uint8_t *q, const float *a, size_t rows, float *y)
{
    if (w == NULL || s == NULL || q == NULL || a == NULL || y == NULL || n == 0 || k == 0 ||
        k % 128 != 0 || rows == 0)
        return -1;
    const size_t blocks = k / 128;
    for (size_t p = 0; p < rows; ++p) {
        for (size_t r = 0; r < n; ++r) {
            float total = 0.0f;
            for (size_t b = 0; b < blocks; ++b) {
                float dot = 0.0f;
                for (size_t i = 0; i < 128; ++i) {
                    const size_t c = b * 128 + i;
                    dot += pwo_decode_e4m3fn(w[r * k + c]) * pwo_decode_e4m3fn(q[p * k + c]);
                }
                total += dot * s[(r / 128) * blocks + b] * a[p * blocks + b];
            }
            y[p * n + r] = total;
        }
    }
    return 0;
}

/* src/text_endpoint.rs:3053-3108 (fp8_linear): dynamic_fp8_activations dequantised input,
 * decode_fp8_matrix_f32 (src/lib.rs:2003-2015) weights, f32 GEMM x * W^T, bf16 round. The
 * reference runs Apple Accelerate cblas_sgemm (src/lib.rs:2039-2074), whose summation order is
 * not published; this restatement declares sequential k. */
int pwo_fp8_linear_mode_b(const uint8_t *w, const float *s, size_t n, size_t k, const float *x,
                          size_t rows, float *y)
{
    if (w == NULL || s == NULL || x == NULL || y == NULL || n == 0 || k == 0 || k % 128 != 0 ||
        rows == 0)
        return -1;
    if (!weights_finite(w, n * k))
        return -2;
    const size_t scale_cols = k / 128;
    for (size_t i = 0; i < ceil_div(n, 128) * scale_cols; ++i)
        if (!isfinite(s[i]))
            return -2;
    float *xd = (float *)malloc(rows * k * sizeof(float));
    float *wd = (float *)malloc(k * sizeof(float));
    if (xd == NULL || wd == NULL) {
        free(xd);
        free(wd);
        return -4;
    }
    int status = pwo_dynamic_fp8(x, rows, k, NULL, NULL, xd);
    if (status != 0) {
        free(xd);
        free(wd);
        return -2;
    }
    for (size_t r = 0; r < n && status == 0; ++r) {
        for (size_t c = 0; c < k; ++c)
            wd[c] = pwo_decode_e4m3fn(w[r * k + c]) * s[(r / 128) * scale_cols + c / 128];
        for (size_t p = 0; p < rows; ++p) {
            float sum = 0.0f;
            for (size_t c = 0; c < k; ++c)
                sum += xd[p * k + c] * wd[c];
            if (!isfinite(sum))
                status = -3;
            y[p * n + r] = pwo_round_bf16(sum);
        }
    }
    free(xd);
    free(wd);
    return status;
}

/* Mode A SwiGLU: kernels/block_fp8_gemv.metal:241-252 (swiglu_f32) and src/lib.rs:5840-5844. */
void pwo_swiglu_f32(const float *gate, const float *up, float *out, size_t count)
{
    for (size_t i = 0; i < count; ++i) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* Mode B SwiGLU: kernels/block_fp8_gemv.metal:139-160 (bf16_staged_swiglu) and
 * src/text_endpoint.rs:5336-5343: round(g), round(u), s = round(g/(1+e^-g)), h = round(s*u). */
void pwo_swiglu_bf16_staged(const float *gate, const float *up, float *out, size_t count)
{
    for (size_t i = 0; i < count; ++i) {
        const float g = pwo_round_bf16(gate[i]);
        const float u = pwo_round_bf16(up[i]);
        const float silu = pwo_round_bf16(g / (1.0f + expf(-g)));
        out[i] = pwo_round_bf16(silu * u);
    }
}

/* src/text_endpoint.rs:4511-4536 (sleef_expf_u10): SLEEF's published expf_u10 with the
 * two-step exponent scaling; q = round-half-even(d * log2(e)). */
float pwo_sleef_expf_u10(float d)
{
    if (d < -104.0f)
        return 0.0f;
    if (d > 100.0f)
        return INFINITY;
    const int q = (int)rintf(d * 1.44269504088896340736f);
    const float qf = (float)q;
    float s = fmaf(qf, -0.69314575f, d);
    s = fmaf(qf, -1.4286068e-6f, s);
    float u = 0.00019852762f;
    u = fmaf(u, s, 0.0013930436f);
    u = fmaf(u, s, 0.008333361f);
    u = fmaf(u, s, 0.041666485f);
    u = fmaf(u, s, 0.16666667f);
    u = fmaf(u, s, 0.5f);
    u = fmaf(s * s, u, s) + 1.0f;
    const int first_q = q >> 1;
    const int second_q = q - first_q;
    const float first = f32_from_bits((uint32_t)(first_q + 127) << 23);
    const float second = f32_from_bits((uint32_t)(second_q + 127) << 23);
    return (u * first) * second;
}

/* src/text_endpoint.rs:4538-4540 (pytorch_sigmoid_f32). */
float pwo_sigmoid_f32(float value) { return 1.0f / (1.0f + pwo_sleef_expf_u10(-value)); }

/* ---- libc++ std::nth_element ---------------------------------------------------------------
 * src/pytorch_topk.cpp:8-30 calls std::nth_element(begin, begin + k - 1, end, greater-by-value)
 * on (value, index) pairs and returns the first k indices. The reference's golden orders were
 * produced by libc++ (LLVM), which is not part of the reference tree and whose headers are absent
 * here; libstdc++'s introselect yields different orders. What follows restates LLVM libc++'s
 * published __nth_element (include/__algorithm/nth_element.h: median-of-three via __sort3,
 * guarded Hoare partition keeping the pivot tracked, the equal-to-first fallback partition, the
 * already-partitioned sortedness shortcut, selection sort at length <= 7). */
typedef struct {
    float value;
    int64_t index;
} pwo_pair;

static int pair_greater(const pwo_pair *a, const pwo_pair *b) { return a->value > b->value; }

static void pair_swap(pwo_pair *a, pwo_pair *b)
{
    const pwo_pair t = *a;
    *a = *b;
    *b = t;
}

static unsigned sort3(pwo_pair *x, pwo_pair *y, pwo_pair *z)
{
    unsigned swaps = 0;
    if (!pair_greater(y, x)) {
        if (!pair_greater(z, y))
            return swaps;
        pair_swap(y, z);
        swaps = 1;
        if (pair_greater(y, x)) {
            pair_swap(x, y);
            swaps = 2;
        }
        return swaps;
    }
    if (pair_greater(z, y)) {
        pair_swap(x, z);
        return 1;
    }
    pair_swap(x, y);
    swaps = 1;
    if (pair_greater(z, y)) {
        pair_swap(y, z);
        swaps = 2;
    }
    return swaps;
}

static void selection_sort(pwo_pair *first, pwo_pair *last)
{
    pwo_pair *lm1 = last - 1;
    for (; first != lm1; ++first) {
        pwo_pair *smallest = first;
        for (pwo_pair *it = first + 1; it != last; ++it)
            if (pair_greater(it, smallest))
                smallest = it;
        if (smallest != first)
            pair_swap(first, smallest);
    }
}

static void nth_element_libcxx(pwo_pair *first, pwo_pair *nth, pwo_pair *last)
{
    const ptrdiff_t limit = 7;
    for (;;) {
        if (nth == last)
            return;
        const ptrdiff_t len = last - first;
        switch (len) {
        case 0:
        case 1:
            return;
        case 2:
            if (pair_greater(last - 1, first))
                pair_swap(first, last - 1);
            return;
        case 3:
            sort3(first, first + 1, last - 1);
            return;
        default:
            break;
        }
        if (len <= limit) {
            selection_sort(first, last);
            return;
        }
        pwo_pair *m = first + len / 2;
        pwo_pair *lm1 = last - 1;
        unsigned n_swaps = sort3(first, m, lm1);
        pwo_pair *i = first;
        pwo_pair *j = lm1;
        if (!pair_greater(i, m)) {
            /* *first is equivalent to the pivot: look for a guard below lm1 */
            int guarded = 0;
            for (;;) {
                if (i == --j)
                    break;
                if (pair_greater(j, m)) {
                    guarded = 1;
                    break;
                }
            }
            if (guarded) {
                pair_swap(i, j);
                ++n_swaps;
            } else {
                /* everything is <= *first: partition into == *first and > *first */
                ++i;
                j = last;
                if (!pair_greater(first, --j)) {
                    for (;;) {
                        if (i == j)
                            return;
                        if (pair_greater(first, i)) {
                            pair_swap(i, j);
                            ++n_swaps;
                            ++i;
                            break;
                        }
                        ++i;
                    }
                }
                if (i == j)
                    return;
                for (;;) {
                    while (!pair_greater(first, i))
                        ++i;
                    do {
                        --j;
                    } while (pair_greater(first, j));
                    if (i >= j)
                        break;
                    pair_swap(i, j);
                    ++n_swaps;
                    ++i;
                }
                if (nth < i)
                    return;
                first = i;
                continue;
            }
        }
        ++i;
        if (i < j) {
            for (;;) {
                while (pair_greater(i, m))
                    ++i;
                do {
                    --j;
                } while (!pair_greater(j, m));
                if (i >= j)
                    break;
                pair_swap(i, j);
                ++n_swaps;
                if (m == i)
                    m = j;
                ++i;
            }
        }
        if (i != m && pair_greater(m, i)) {
            pair_swap(i, m);
            ++n_swaps;
        }
        if (nth == i)
            return;
        if (n_swaps == 0) {
            /* a perfectly partitioned input: stop if the side holding nth is already sorted */
            pwo_pair *a = nth < i ? first : i;
            pwo_pair *end = nth < i ? i : last;
            pwo_pair *prev = a;
            int sorted = 1;
            for (;;) {
                if (++a == end)
                    break;
                if (pair_greater(a, prev)) {
                    sorted = 0;
                    break;
                }
                prev = a;
            }
            if (sorted)
                return;
        }
        if (nth < i)
            last = i;
        else
            first = i + 1;
    }
}

int pwo_topk_unsorted(const float *values, size_t count, size_t top_k, uint32_t *selected)
{
    if (values == NULL || selected == NULL || top_k == 0 || top_k >= count)
        return -1;
    pwo_pair *queue = (pwo_pair *)malloc(count * sizeof(pwo_pair));
    if (queue == NULL)
        return -2;
    for (size_t i = 0; i < count; ++i) {
        queue[i].value = values[i];
        queue[i].index = (int64_t)i;
    }
    nth_element_libcxx(queue, queue + top_k - 1, queue + count);
    for (size_t i = 0; i < top_k; ++i)
        selected[i] = (uint32_t)queue[i].index;
    free(queue);
    return 0;
}

/* src/text_endpoint.rs:4382-4390 (pytorch_sum_eight). */
static float sum_eight(const float v[8])
{
    const float lanes[4] = {v[0] + v[4], v[1] + v[5], v[2] + v[6], v[3] + v[7]};
    float sum = 0.0f;
    for (int i = 0; i < 4; ++i)
        sum = sum + lanes[i];
    return sum;
}

/* src/text_endpoint.rs:4394-4473 (pytorch_noaux_routes), TOP_K = 8. */
int pwo_noaux_routes(const float *scores, const float *bias, size_t rows, size_t experts,
                     uint32_t *selected, float *weights, uint64_t *tie_rows)
{
    const size_t top_k = 8;
    if (scores == NULL || bias == NULL || selected == NULL || weights == NULL || experts <= top_k)
        return -1;
    for (size_t i = 0; i < rows * experts; ++i)
        if (!isfinite(scores[i]))
            return -1;
    for (size_t i = 0; i < experts; ++i)
        if (!isfinite(bias[i]))
            return -1;
    float *corrected = (float *)malloc(experts * sizeof(float));
    unsigned char *chosen = (unsigned char *)malloc(experts);
    if (corrected == NULL || chosen == NULL) {
        free(corrected);
        free(chosen);
        return -4;
    }
    uint64_t ties = 0;
    int status = 0;
    for (size_t p = 0; p < rows && status == 0; ++p) {
        const float *row = scores + p * experts;
        for (size_t e = 0; e < experts; ++e)
            corrected[e] = row[e] + bias[e];
        uint32_t sel[8];
        if (pwo_topk_unsorted(corrected, experts, top_k, sel) != 0) {
            status = -2;
            break;
        }
        memset(chosen, 0, experts);
        for (size_t i = 0; i < top_k; ++i) {
            if (sel[i] >= experts || chosen[sel[i]]) {
                status = -2;
                break;
            }
            chosen[sel[i]] = 1;
        }
        if (status != 0)
            break;
        float boundary = INFINITY, rejected = -INFINITY;
        for (size_t i = 0; i < top_k; ++i)
            boundary = fminf(boundary, corrected[sel[i]]);
        for (size_t e = 0; e < experts; ++e)
            if (!chosen[e])
                rejected = fmaxf(rejected, corrected[e]);
        if (!isfinite(boundary) || boundary < rejected) {
            status = -3;
            break;
        }
        if (boundary == rejected)
            ++ties;
        float picked[8];
        for (size_t i = 0; i < top_k; ++i)
            picked[i] = row[sel[i]];
        const float denominator = sum_eight(picked) + 1.0e-20f;
        float weight_sum = 0.0f;
        for (size_t i = 0; i < top_k; ++i) {
            const float w = row[sel[i]] / denominator;
            if (!isfinite(w) || w < 0.0f)
                status = -3;
            weights[p * top_k + i] = w;
            selected[p * top_k + i] = sel[i];
            weight_sum += w;
        }
        if (fabsf(weight_sum - 1.0f) > 1.0e-6f)
            status = -3;
    }
    free(corrected);
    free(chosen);
    if (tie_rows)
        *tie_rows = ties;
    return status;
}

void pwo_router_logits_t256(const float *x, size_t rows, const float *router_w, size_t experts,
                            size_t k, float *logits)
{
    for (size_t p = 0; p < rows; ++p) {
        for (size_t e = 0; e < experts; ++e) {
            float partial[256];
            for (size_t g = 0; g < 256; ++g) {
                float acc = 0.0f;
                for (size_t c0 = 8 * g; c0 < k; c0 += 2048)
                    for (size_t j = 0; j < 8; ++j)
                        acc = fmaf(x[p * k + c0 + j], router_w[e * k + c0 + j], acc);
                partial[g] = acc;
            }
            float wave[4];
            for (size_t w = 0; w < 4; ++w) {
                float *lane = partial + 64 * w;
                for (size_t offset = 32; offset > 0; offset /= 2)
                    for (size_t l = 0; l < offset; ++l)
                        lane[l] = lane[l] + lane[l + offset];
                wave[w] = lane[0];
            }
            logits[p * experts + e] = (wave[0] + wave[1]) + (wave[2] + wave[3]);
        }
    }
}

/* src/text_endpoint.rs:4342-4380 (route_mlp): logits -> pytorch sigmoid -> noaux routes. */
int pwo_route(const float *x, size_t rows, const float *router_w, const float *bias,
              size_t experts, size_t k, float *logits, float *scores, uint32_t *selected,
              float *weights, uint64_t *tie_rows)
{
    pwo_router_logits_t256(x, rows, router_w, experts, k, logits);
    for (size_t i = 0; i < rows * experts; ++i)
        scores[i] = pwo_sigmoid_f32(logits[i]);
    return pwo_noaux_routes(scores, bias, rows, experts, selected, weights, tie_rows);
}

/* Schedule of src/text_endpoint.rs:4767-4775 / :5302-5310: BTreeMap<expert, [(position, w)]>,
 * filled position-major then slot, iterated in ascending expert id. Returned as placement
 * lists grouped by expert (ascending), positions ascending inside each expert. */
typedef struct {
    size_t count;
    size_t *positions;
    float *weights;
} expert_slot;

static int build_schedule(size_t rows, size_t n_experts, const uint32_t *selected,
                          const float *weights, size_t top_k, expert_slot *slots)
{
    for (size_t e = 0; e < n_experts; ++e)
        slots[e].count = 0;
    for (size_t i = 0; i < rows * top_k; ++i) {
        if (selected[i] >= n_experts || !isfinite(weights[i]))
            return -1;
        slots[selected[i]].count++;
    }
    /* A token naming one expert twice is not a placement bijection: the reference's routes never
     * hold one (pytorch_noaux_routes checks the selected set, src/text_endpoint.rs:4426-4432) and
     * reconstruct_routed_from_schedule rejects a repeated (position, expert) pair
     * (src/text_endpoint.rs:10681-10710). */
    for (size_t p = 0; p < rows; ++p)
        for (size_t s = 0; s < top_k; ++s)
            for (size_t t = s + 1; t < top_k; ++t)
                if (selected[p * top_k + s] == selected[p * top_k + t])
                    return -1;
    for (size_t e = 0; e < n_experts; ++e) {
        slots[e].positions = slots[e].count ? (size_t *)malloc(slots[e].count * sizeof(size_t)) : NULL;
        slots[e].weights = slots[e].count ? (float *)malloc(slots[e].count * sizeof(float)) : NULL;
        if (slots[e].count && (!slots[e].positions || !slots[e].weights))
            return -4;
        if (slots[e].count > rows)
            return -1;
        slots[e].count = 0;
    }
    for (size_t p = 0; p < rows; ++p)
        for (size_t s = 0; s < top_k; ++s) {
            expert_slot *slot = &slots[selected[p * top_k + s]];
            slot->positions[slot->count] = p;
            slot->weights[slot->count] = weights[p * top_k + s];
            slot->count++;
        }
    return 0;
}

static void free_schedule(expert_slot *slots, size_t n)
{
    for (size_t e = 0; e < n; ++e) {
        free(slots[e].positions);
        free(slots[e].weights);
    }
}

static int moe_layer(int mode_b, const float *x, size_t rows, size_t hidden, size_t inter,
                     const pwo_expert *experts, size_t n_experts, const uint32_t *selected,
                     const float *weights, size_t top_k, float *out, float *out_raw)
{
    if (x == NULL || experts == NULL || selected == NULL || weights == NULL || out == NULL ||
        rows == 0 || hidden % 128 != 0 || inter % 128 != 0)
        return -1;
    expert_slot *slots = (expert_slot *)calloc(n_experts, sizeof(expert_slot));
    if (slots == NULL)
        return -4;
    int status = build_schedule(rows, n_experts, selected, weights, top_k, slots);
    float *block = (float *)calloc(rows * hidden, sizeof(float));
    float *gathered = (float *)malloc(rows * hidden * sizeof(float));
    float *gate = (float *)malloc(rows * inter * sizeof(float));
    float *up = (float *)malloc(rows * inter * sizeof(float));
    float *act = (float *)malloc(rows * inter * sizeof(float));
    float *proj = (float *)malloc(rows * hidden * sizeof(float));
    if (!block || !gathered || !gate || !up || !act || !proj)
        status = -4;
    for (size_t e = 0; e < n_experts && status == 0; ++e) {
        const size_t count = slots[e].count;
        if (count == 0)
            continue;
        const pwo_expert *ex = &experts[e];
        if (!ex->gate_w || !ex->gate_s || !ex->up_w || !ex->up_s || !ex->down_w || !ex->down_s) {
            status = -1;
            break;
        }
        for (size_t l = 0; l < count; ++l)
            memcpy(gathered + l * hidden, x + slots[e].positions[l] * hidden, hidden * sizeof(float));
        if (mode_b) {
            status = pwo_fp8_linear_mode_b(ex->gate_w, ex->gate_s, inter, hidden, gathered, count, gate);
            if (status == 0)
                status = pwo_fp8_linear_mode_b(ex->up_w, ex->up_s, inter, hidden, gathered, count, up);
            if (status == 0) {
                /* src/text_endpoint.rs:5336-5343 on already bf16-rounded gate/up */
                pwo_swiglu_bf16_staged(gate, up, act, count * inter);
                status = pwo_fp8_linear_mode_b(ex->down_w, ex->down_s, hidden, inter, act, count, proj);
            }
        } else {
            status = pwo_gemm_mode_a(ex->gate_w, ex->gate_s, inter, hidden, gathered, count, gate);
            if (status == 0)
                status = pwo_gemm_mode_a(ex->up_w, ex->up_s, inter, hidden, gathered, count, up);
            if (status == 0) {
                pwo_swiglu_f32(gate, up, act, count * inter);
                status = pwo_gemm_mode_a(ex->down_w, ex->down_s, hidden, inter, act, count, proj);
            }
        }
        if (status != 0)
            break;
        /* src/text_endpoint.rs:5365-5369 / src/lib.rs:5853-5858: out[pos] += y * w, f32 */
        for (size_t l = 0; l < count; ++l) {
            float *dst = block + slots[e].positions[l] * hidden;
            const float w = slots[e].weights[l];
            for (size_t c = 0; c < hidden; ++c)
                dst[c] += proj[l * hidden + c] * w;
        }
    }
    if (status == 0)
        for (size_t i = 0; i < rows * hidden; ++i)
        {
            if (out_raw)
                out_raw[i] = block[i];
            out[i] = pwo_round_bf16(block[i]);
        }
    free(block);
    free(gathered);
    free(gate);
    free(up);
    free(act);
    free(proj);
    free_schedule(slots, n_experts);
    free(slots);
    return status;
}

int pwo_moe_layer_mode_a(const float *x, size_t rows, size_t hidden, size_t inter,
                         const pwo_expert *experts, size_t n_experts, const uint32_t *selected,
                         const float *weights, size_t top_k, float *out, float *out_raw)
{
    return moe_layer(0, x, rows, hidden, inter, experts, n_experts, selected, weights, top_k, out,
                     out_raw);
}

int pwo_moe_layer_mode_b(const float *x, size_t rows, size_t hidden, size_t inter,
                         const pwo_expert *experts, size_t n_experts, const uint32_t *selected,
                         const float *weights, size_t top_k, float *out, float *out_raw)
{
    return moe_layer(1, x, rows, hidden, inter, experts, n_experts, selected, weights, top_k, out,
                     out_raw);
}

int pwo_expert_mode_a(const float *x, size_t rows, size_t hidden, size_t inter,
                      const pwo_expert *expert, float *out_f32, float *out_bf16)
{
    float *gate = (float *)malloc(rows * inter * sizeof(float));
    float *up = (float *)malloc(rows * inter * sizeof(float));
    float *act = (float *)malloc(rows * inter * sizeof(float));
    float *proj = (float *)malloc(rows * hidden * sizeof(float));
    int status = (!gate || !up || !act || !proj) ? -4 : 0;
    if (status == 0)
        status = pwo_gemm_mode_a(expert->gate_w, expert->gate_s, inter, hidden, x, rows, gate);
    if (status == 0)
        status = pwo_gemm_mode_a(expert->up_w, expert->up_s, inter, hidden, x, rows, up);
    if (status == 0) {
        pwo_swiglu_f32(gate, up, act, rows * inter);
        status = pwo_gemm_mode_a(expert->down_w, expert->down_s, hidden, inter, act, rows, proj);
    }
    if (status == 0)
        for (size_t i = 0; i < rows * hidden; ++i) {
            if (out_f32)
                out_f32[i] = proj[i];
            if (out_bf16)
                out_bf16[i] = pwo_round_bf16(proj[i]);
        }
    free(gate);
    free(up);
    free(act);
    free(proj);
    return status;
}

/* src/text_endpoint.rs:3174-3198 (full_qkv_source_row): 64 heads x 192 Q rows in four TP
 * shards of [Q 3072, K 192, V 128]. */
int64_t pwo_full_qkv_source_row(int64_t logical_row)
{
    const int64_t q_rows = 64 * 192, k_rows = 4 * 192, v_rows = 4 * 128;
    const int64_t q_per_shard = q_rows / 4, shard_rows = q_per_shard + 192 + 128;
    if (logical_row < 0)
        return -1;
    if (logical_row < q_rows)
        return (logical_row / q_per_shard) * shard_rows + logical_row % q_per_shard;
    if (logical_row < q_rows + k_rows) {
        const int64_t local = logical_row - q_rows;
        return (local / 192) * shard_rows + q_per_shard + local % 192;
    }
    if (logical_row < q_rows + k_rows + v_rows) {
        const int64_t local = logical_row - q_rows - k_rows;
        return (local / 128) * shard_rows + q_per_shard + 192 + local % 128;
    }
    return -1;
}

/* src/text_endpoint.rs:3227-3242 (full_qkv_scale_row): 27 scale rows per shard. */
int64_t pwo_full_qkv_scale_row(int64_t logical_row)
{
    const int64_t source = pwo_full_qkv_source_row(logical_row);
    if (source < 0)
        return -1;
    const int64_t shard = source / 3392, local = source % 3392;
    int64_t local_scale;
    if (local < 3072)
        local_scale = local / 128;
    else if (local < 3072 + 192)
        local_scale = 24 + (local - 3072) / 128;
    else
        local_scale = 26;
    return shard * 27 + local_scale;
}

/* src/text_endpoint.rs:3200-3225 (swa_qkv_source_row): 4 shards of [Q 3072, K 384, V 256]. */
int64_t pwo_swa_qkv_source_row(int64_t logical_row)
{
    const int64_t q_rows = 64 * 192, k_rows = 8 * 192, v_rows = 8 * 128;
    const int64_t qs = q_rows / 4, ks = k_rows / 4, vs = v_rows / 4, shard_rows = qs + ks + vs;
    if (logical_row < 0)
        return -1;
    if (logical_row < q_rows)
        return logical_row / qs * shard_rows + logical_row % qs;
    if (logical_row < q_rows + k_rows) {
        const int64_t local = logical_row - q_rows;
        return local / ks * shard_rows + qs + local % ks;
    }
    if (logical_row < q_rows + k_rows + v_rows) {
        const int64_t local = logical_row - q_rows - k_rows;
        return local / vs * shard_rows + qs + ks + local % vs;
    }
    return -1;
}
