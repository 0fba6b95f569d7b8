/*
 * CPU oracle for the block-scaled FP8 projection and routed-MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain single-threaded C, the reference
 * (x3haloed/mimo-prismwing) CPU numerics for the path. It is the checker that the HIP product is
 * compared against: only the tests, the smoke check and the benchmark's CPU-baseline leg load it.
 * The product library never links, loads or calls it.
 *
 * Every function cites the reference file:line it follows. Build: `make -C oracle` (gcc,
 * -ffp-contract=off so that a*b+c is never fused, matching Rust's default semantics).
 *
 * Pinning status (what checks each function independently of a retyped formula):
 *   pwo_decode_e4m3fn        golden f8-e4m3fn-all-bytes.json (all 256 bytes) + real block fixture
 *   pwo_round_bf16           golden pw0054-bf16-boundary.json (532 inputs incl. NaN/Inf)
 *   pwo_encode_e4m3fn        golden pw0053 codes; brute-force nearest search near every midpoint
 *   pwo_dynamic_fp8          golden pw0053-dynamic-fp8-activation.json (scales, codes, dequant bits)
 *   pwo_gemm_mode_a          real mtp-gate-fp8-gemv.json (abs 2e-7), closed form 384/896, f64 brute force
 *   pwo_bf16_linear          closed forms (exact sums of powers of two, bf16 rounding of a tie), f64
 *                            brute force, equality with pwo_gemm_mode_a on e4m3 values with unit scales
 *   pwo_gemm_mode_b_equation closed-form probe inputs vs f64 brute force; equals mode A when the
 *                            activation codes are exact and scales are 1
 *   pwo_fp8_linear_mode_b    f64 brute force on tiny shapes; bf16-rounding idempotence
 *   pwo_swiglu_f32           golden swiglu-f32.json (f64 oracle)
 *   pwo_swiglu_bf16_staged   known answers where dropping any one of the four bf16 roundings changes
 *                            the bits (incl. the reference's gate 1.03125 / up 0.71484375 case and a
 *                            tie of the product)
 *   pwo_sleef_expf_u10       golden pw0068-sleef-boundaries.json; pw0062 via the sigmoid
 *   pwo_sigmoid_f32          golden pw0062-router-sigmoid.json, pw0068
 *   pwo_topk_unsorted        golden pw0063-topk-order.json + 5 tie cases of pw0157 (order and set)
 *   pwo_noaux_routes         pw0157 tie counting; selected set = top 8 of the corrected scores and
 *                            weights = uncorrected scores over their sum (f64), summing to 1 within 1e-6
 *   pwo_router_logits_t256   known-answer sums whose f32 value fixes the fma, the column order, the
 *                            lane tree and the wave order; f64 brute force (tolerance). The order is
 *                            this build's declared one; the reference's (Apple Accelerate SGEMM) is
 *                            closed
 *   pwo_moe_layer_mode_a/_b  the reference's tiny noaux-tc MoE fixture (moe-noaux-tc-swiglu.json,
 *                            each weight carried by its own 128x128 block); f64 brute force on tiny
 *                            FP8 shapes; bit equality with the routed composition of the pinned
 *                            projections and SwiGLU; one-hot route weights reproduce the expert bit
 *                            for bit; repeated (token, expert) pairs rejected
 *   pwo_expert_mode_a        f64 brute force; its bf16 output is the round of its f32 output
 *   pwo_full/swa_qkv_*       known-answer row/scale maps of src/text_endpoint.rs:13686-13732
 */
#ifndef PW_ORACLE_H
#define PW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar numerics ---------------------------------------------------------------------- */
float pwo_decode_e4m3fn(uint8_t bits);
float pwo_round_bf16(float value);
/* 0 on success, -1 when value is non-finite or |value| > 448 */
int pwo_encode_e4m3fn(float value, uint8_t *out);
float pwo_sleef_expf_u10(float d);
float pwo_sigmoid_f32(float value);

/* ---- dynamic activation quantiser (per row, per 128-column group) ------------------------- */
/* codes [rows*cols], scales [rows*cols/128], dequantized [rows*cols] (any may be NULL) */
int pwo_dynamic_fp8(const float *input, size_t rows, size_t cols, uint8_t *codes, float *scales,
                    float *dequantized);

/* ---- projections --------------------------------------------------------------------------- */
/* Mode A: y[p, r] = sum_c dec(W[r, c]) * S[r/128, c/128] * x[p, c], f32, sequential over c.
 * W [n x k] e4m3fn, S [ceil(n/128) x k/128] f32, x [rows x k] f32 -> y [rows x n] f32.
 * Returns -1 on shape error, -2 on non-finite input/scale/weight (0x7f/0xff), -3 non-finite out. */
int pwo_gemm_mode_a(const uint8_t *w, const float *s, size_t n, size_t k, const float *x,
                    size_t rows, float *y);
/* BF16 linear: y[p, r] = round_bf16(sum_c bf16(W[r, c]) * x[p, c]), f32, sequential over c.
 * W [n x k] bf16 bits, x [rows x k] f32 -> y [rows x n]; y_raw (may be NULL) gets the sums.
 * Returns -1 on shape error, -2 on non-finite input, -3 on a non-finite output. */
int pwo_bf16_linear(const uint16_t *w, size_t n, size_t k, const float *x, size_t rows, float *y,
                    float *y_raw);
/* Block-scaled equation of the GPU mode-B kernels:
 * y[p, r] = sum_b (sum_{c in b} dec(W) * dec(q[p, c])) * S[r/128, b] * a[p, b], blocks ascending. */
int pwo_gemm_mode_b_equation(const uint8_t *w, const float *s, size_t n, size_t k,
                             const uint8_t *q, const float *a, size_t rows, float *y);
/* fp8_linear: quantise->dequantise x per 128 group, dequantise W, f32 GEMM (sequential k), bf16. */
int pwo_fp8_linear_mode_b(const uint8_t *w, const float *s, size_t n, size_t k, const float *x,
                          size_t rows, float *y);

/* ---- SwiGLU --------------------------------------------------------------------------------- */
void pwo_swiglu_f32(const float *gate, const float *up, float *out, size_t count);
void pwo_swiglu_bf16_staged(const float *gate, const float *up, float *out, size_t count);

/* ---- router ---------------------------------------------------------------------------------- */
/* libc++ std::nth_element(first, first+k-1, last, greater-by-value) over (value, index) pairs,
 * returning the first k indices in partition order. -1 on bad arguments. */
int pwo_topk_unsorted(const float *values, size_t count, size_t top_k, uint32_t *selected);
/* noaux-tc routes: scores [rows x 256] (sigmoid outputs), bias [256] -> selected [rows x 8],
 * weights [rows x 8]; *tie_rows counts rows whose selected boundary equals the best rejected. */
int pwo_noaux_routes(const float *scores, const float *bias, size_t rows, size_t experts,
                     uint32_t *selected, float *weights, uint64_t *tie_rows);
/* Router logits in the declared 256-thread order (k a multiple of 8): for each (p, e) 256 partial
 * sums, partial g accumulating with fmaf over the 8-column groups c0 = 8g, 8g + 2048, ... (columns
 * c0 .. c0 + 7 in order); each 64-partial wave reduced by the halving tree 32,16,8,4,2,1 into
 * w0..w3; logit = (w0 + w1) + (w2 + w3). */
void pwo_router_logits_t256(const float *x, size_t rows, const float *router_w, size_t experts,
                            size_t k, float *logits);
/* Full route: logits (lane-64) -> sigmoid -> noaux routes. */
int pwo_route(const float *x, size_t rows, const float *router_w, const float *bias,
              size_t experts, size_t k, float *logits, float *scores, uint32_t *selected,
              float *weights, uint64_t *tie_rows);

/* ---- routed MoE layer ------------------------------------------------------------------------- */
typedef struct {
    const uint8_t *gate_w; const float *gate_s;  /* [inter x hidden], [inter/128 x hidden/128] */
    const uint8_t *up_w;   const float *up_s;
    const uint8_t *down_w; const float *down_s;  /* [hidden x inter], [hidden/128 x inter/128] */
} pwo_expert;

/* experts: array indexed by expert id (entries of unrouted experts may hold NULL pointers).
 * selected/weights: [rows x top_k]. Output [rows x hidden] bf16-rounded f32.
 * Mode A = the reference's f32 CPU control (src/lib.rs:5807-5862): f32 activations, f32 SwiGLU,
 * f32 expert outputs, f32 weighted combine in ascending expert id, bf16 at the end.
 * Mode B = routed_mlp_traced (src/text_endpoint.rs:5290-5381) over fp8_linear. */
/* out_raw (may be NULL) receives the f32 combine before the final bf16 round. */
int pwo_moe_layer_mode_a(const float *x, size_t rows, size_t hidden, size_t inter,
                         const pwo_expert *experts, size_t n_experts, const uint32_t *selected,
                         const float *weights, size_t top_k, float *out, float *out_raw);
int pwo_moe_layer_mode_b(const float *x, size_t rows, size_t hidden, size_t inter,
                         const pwo_expert *experts, size_t n_experts, const uint32_t *selected,
                         const float *weights, size_t top_k, float *out, float *out_raw);
/* One complete expert in mode A (config "one routed expert"): y = bf16(down(swiglu(gate x, up x))). */
int pwo_expert_mode_a(const float *x, size_t rows, size_t hidden, size_t inter,
                      const pwo_expert *expert, float *out_f32, float *out_bf16);

/* ---- QKV tensor-parallel layouts ---------------------------------------------------------------- */
int64_t pwo_full_qkv_source_row(int64_t logical_row);
int64_t pwo_full_qkv_scale_row(int64_t logical_row);
int64_t pwo_swa_qkv_source_row(int64_t logical_row);

#ifdef __cplusplus
}
#endif
#endif
