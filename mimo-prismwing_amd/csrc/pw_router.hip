// Routed-MoE router on the device: logits, PyTorch sigmoid, noaux-tc top-8 and renormalised
// weights, so the routes a layer consumes never leave HBM (route_mlp, src/text_endpoint.rs:
// 4342-4380; Metal router GEMV kernels/block_fp8_gemv.metal:317-356).
//
// Logits use this build's declared summation order: 64 lanes each accumulate x[c] * w[e, c]
// with a fused multiply-add over c = lane, lane + 64, ..., then a halving tree (lane l += lane
// l + offset, offset 32 .. 1). The reference's order belongs to Apple Accelerate's SGEMM, which
// is closed; any fixed order is within the routes' tolerance of it, and this one is restated by
// the oracle so the device routes can be checked bit for bit. Scores are the PyTorch sigmoid on
// the SLEEF expf_u10 restatement; the selection and weights are pytorch_noaux_routes
// (pw_topk.h), shared with the host helpers.
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_topk.h"

namespace pw {

template <typename T>
__device__ __forceinline__ float router_value(const T *p, size_t i);
template <>
__device__ __forceinline__ float router_value<float>(const float *p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float router_value<uint16_t>(const uint16_t *p, size_t i)
{
    return f32_from((uint32_t)p[i] << 16);
}

// One wave per (expert, 8-row chunk): scores[p][e] = sigmoid(logit[p][e]).
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void router_scores_kernel(const TX *__restrict__ x, const TW *__restrict__ w,
                                                            uint32_t rows, uint32_t E, uint32_t K,
                                                            float *__restrict__ scores)
{
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t chunks = (rows + 7) >> 3;
    if (wave_id >= E * chunks)
        return;
    const uint32_t e = wave_id % E, p0 = (wave_id / E) * 8;
    const uint32_t np = rows - p0 < 8 ? rows - p0 : 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        acc[j] = 0.0f;
    for (uint32_t c = lane; c < K; c += 64) {
        const float wv = router_value<TW>(w, (size_t)e * K + c);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (j < np)
                acc[j] = __builtin_fmaf(router_value<TX>(x, (size_t)(p0 + j) * K + c), wv, acc[j]);
    }
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
        float v = acc[j];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            v = v + __shfl_down(v, off, 64);
        if (lane == 0 && j < np)
            scores[(size_t)(p0 + j) * E + e] = sigmoid_pytorch(v);
    }
}

// One thread per row: noaux-tc selection over its `E` scores with an LDS scratch of E entries.
// A row that fails (non-finite score or bias, a broken top-k, invalid weights) raises
// FLAG_ROUTE and gets expert ids E (which the layer schedule rejects) with zero weights.
__global__ void router_select_kernel(const float *__restrict__ scores, const float *__restrict__ bias,
                                     uint32_t rows, uint32_t E, uint32_t *__restrict__ selected,
                                     float *__restrict__ weights, uint32_t *tie_rows, uint32_t *flags)
{
    extern __shared__ TopkEntry scratch_all[];
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= rows)
        return;
    TopkEntry *scratch = scratch_all + (size_t)threadIdx.x * E;
    uint32_t sel[8];
    float wt[8];
    bool tie = false;
    const int st = noaux_route_row(scores + (size_t)p * E, bias, E, scratch, sel, wt, &tie);
    if (st != ROUTE_OK) {
        raise_flag(flags, FLAG_ROUTE);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            sel[k] = E;
            wt[k] = 0.0f;
        }
        tie = false;
    }
    *(uint4 *)(selected + (size_t)p * 8) = make_uint4(sel[0], sel[1], sel[2], sel[3]);
    *(uint4 *)(selected + (size_t)p * 8 + 4) = make_uint4(sel[4], sel[5], sel[6], sel[7]);
    *(float4 *)(weights + (size_t)p * 8) = make_float4(wt[0], wt[1], wt[2], wt[3]);
    *(float4 *)(weights + (size_t)p * 8 + 4) = make_float4(wt[4], wt[5], wt[6], wt[7]);
    if (tie && tie_rows)
        atomicAdd(tie_rows, 1u);
}

// Rows per workgroup of the selection: each thread needs E * 8 bytes of LDS.
static uint32_t select_threads(uint32_t E)
{
    uint32_t t = 16;
    while (t > 1 && (size_t)t * E * sizeof(TopkEntry) > 64 * 1024)
        t >>= 1;
    return t;
}

template <typename TX>
static void launch_scores_x(const TX *x, const void *w, bool w_f32, uint32_t rows, uint32_t E, uint32_t K,
                            float *scores, hipStream_t stream)
{
    const uint32_t waves = E * ((rows + 7) >> 3);
    const dim3 grid((waves + 3) / 4), block(256);
    if (w_f32)
        hipLaunchKernelGGL((router_scores_kernel<TX, float>), grid, block, 0, stream, x, (const float *)w, rows, E,
                           K, scores);
    else
        hipLaunchKernelGGL((router_scores_kernel<TX, uint16_t>), grid, block, 0, stream, x, (const uint16_t *)w,
                           rows, E, K, scores);
}

void launch_router(const void *x, bool x_f32, const void *w, bool w_f32, const float *bias, uint32_t rows,
                   uint32_t E, uint32_t K, float *scores, uint32_t *selected, float *weights, uint32_t *tie_rows,
                   uint32_t *flags, hipStream_t stream)
{
    const int t = timer_begin(K_ROUTER, stream);
    if (x_f32)
        launch_scores_x<float>((const float *)x, w, w_f32, rows, E, K, scores, stream);
    else
        launch_scores_x<uint16_t>((const uint16_t *)x, w, w_f32, rows, E, K, scores, stream);
    const uint32_t threads = select_threads(E);
    hipLaunchKernelGGL(router_select_kernel, dim3((rows + threads - 1) / threads), dim3(threads),
                       (size_t)threads * E * sizeof(TopkEntry), stream, scores, bias, rows, E, selected, weights,
                       tie_rows, flags);
    timer_end(t, stream);
}

}  // namespace pw
