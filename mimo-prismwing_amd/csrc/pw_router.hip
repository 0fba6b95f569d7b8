// Routed-MoE router on the device: logits, PyTorch sigmoid, noaux-tc top-8 and renormalised
// weights, so the routes a layer consumes never leave HBM (route_mlp, src/text_endpoint.rs:
// 4342-4380; Metal router GEMV kernels/block_fp8_gemv.metal:317-356).
//
// Logits use this build's declared summation order: a workgroup of 256 threads takes one expert;
// thread g accumulates x[c] * w[e, c] with a fused multiply-add over the 8-column groups
// c0 = 8g, 8g + 2048, 8g + 4096, ... (columns c0 .. c0 + 7 in order), each wave of 64 partials is
// reduced by a halving tree (lane l += lane l + offset, offset 32 .. 1) into w0..w3, and the logit
// is (w0 + w1) + (w2 + w3). The reference's order belongs to Apple Accelerate's SGEMM, which is
// closed; any fixed order is within the routes' tolerance of it, and this one is restated by the
// oracle so the device routes can be checked bit for bit. Scores are the PyTorch sigmoid on the
// SLEEF expf_u10 restatement; the selection and weights are pytorch_noaux_routes (pw_topk.h), with
// nth_element run on the row held in one wave's registers (pw_select_wave.h: the same result, the
// same partition order).
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_select_wave.h"

namespace pw {

// Eight consecutive values of a row: bf16 (one 16-byte load) or f32 (two), loaded raw and
// widened to f32 by unpack.
template <typename T>
struct Raw8;
template <>
struct Raw8<uint16_t> {
    uint4 q;
    __device__ __forceinline__ void load(const uint16_t *p) { q = load_global16(p); }
    __device__ __forceinline__ void unpack(float *v) const
    {
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = f32_from(u[i] << 16);
            v[2 * i + 1] = f32_from(u[i] & 0xffff0000u);
        }
    }
};
template <>
struct Raw8<float> {
    uint4 q0, q1;
    __device__ __forceinline__ void load(const float *p)
    {
        q0 = load_global16(p);
        q1 = load_global16(p + 4);
    }
    __device__ __forceinline__ void unpack(float *v) const
    {
        const uint32_t u[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = f32_from(u[i]);
    }
};

// v + (the value of lane l + OFF) at lanes l < OFF <= 8 (a row_shl DPP move: both lanes in the
// lane's 16-lane row; the other lanes get values of no use)
template <int OFF>
__device__ __forceinline__ float add_from_lane_above(float v)
{
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + OFF,
                                                                     0xf, 0xf, false));
}

// One workgroup per (expert, chunk of up to 8 rows; NR rows loaded, NR >= the chunk's rows):
// scores[p][e] = sigmoid(logit[p][e]) in the declared order. Every thread reads its 8-column
// groups of the expert row and of the chunk's rows with 16-byte loads (rows past the chunk's last
// reread that row, so every load is in bounds and none waits on a branch: a thread's loads of two
// column groups go out together); the activation rows are shared by all experts' workgroups
// through L2. The halving trees of the NR rows run interleaved, their steps within 16 lanes as
// DPP moves.
template <typename TX, typename TW, int NR>
__global__ __launch_bounds__(256) void router_scores_kernel(const TX *__restrict__ x, const TW *__restrict__ w,
                                                            uint32_t rows, uint32_t E, uint32_t K,
                                                            float *__restrict__ scores)
{
    __shared__ float wave_sum[NR][4];
    const uint32_t g = threadIdx.x, lane = g & 63, wave = g >> 6;
    const uint32_t e = blockIdx.x;
    const uint32_t p0 = blockIdx.y * 8;
    const uint32_t np = rows - p0 < (uint32_t)NR ? rows - p0 : (uint32_t)NR;
    float acc[NR];
    const TX *xr[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        acc[j] = 0.0f;
        xr[j] = x + (size_t)(p0 + ((uint32_t)j < np ? (uint32_t)j : np - 1)) * K;
    }
    const TW *wrow = w + (size_t)e * K;
    // column groups c0 = 8 g + 2048 i in ascending i, two per pass
    for (uint32_t c0 = 8 * g; c0 < K; c0 += 4096) {
        const bool has1 = c0 + 2048 < K;
        const uint32_t c1 = has1 ? c0 + 2048 : c0;
        Raw8<TW> w0, w1;
        Raw8<TX> x0[NR], x1[NR];
        w0.load(wrow + c0);
        w1.load(wrow + c1);
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            x0[j].load(xr[j] + c0);
            x1[j].load(xr[j] + c1);
        }
        // every load above is issued before the first use below
        __builtin_amdgcn_sched_barrier(0);
        float wv[8], xv[8];
        w0.unpack(wv);
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            x0[j].unpack(xv);
#pragma unroll
            for (int c = 0; c < 8; ++c)
                acc[j] = __builtin_fmaf(xv[c], wv[c], acc[j]);
        }
        // the second group's sums are kept only where it exists (computed anyway, so its loads
        // stay with the first group's)
        w1.unpack(wv);
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            x1[j].unpack(xv);
            float t = acc[j];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                t = __builtin_fmaf(xv[c], wv[c], t);
            acc[j] = has1 ? t : acc[j];
        }
    }
    // each wave's halving tree (lane l += lane l + off, off = 32 .. 1), ending in lane 0
#pragma unroll
    for (int j = 0; j < NR; ++j)
        acc[j] = acc[j] + __shfl_down(acc[j], 32, 64);
#pragma unroll
    for (int j = 0; j < NR; ++j)
        acc[j] = acc[j] + __shfl_down(acc[j], 16, 64);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        acc[j] = add_from_lane_above<8>(acc[j]);
        acc[j] = add_from_lane_above<4>(acc[j]);
        acc[j] = add_from_lane_above<2>(acc[j]);
        acc[j] = add_from_lane_above<1>(acc[j]);
    }
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < NR; ++j)
            wave_sum[j][wave] = acc[j];
    }
    __syncthreads();
    if (g < np) {
        const float logit = (wave_sum[g][0] + wave_sum[g][1]) + (wave_sum[g][2] + wave_sum[g][3]);
        scores[(size_t)(p0 + g) * E + e] = sigmoid_pytorch(logit);
    }
}

// One wave per row: the row's corrected scores stay in the wave's registers (position p = 64 c +
// lane in register c), select_route_row runs the top-8 partition on them (pw_select_wave.h), and
// lane 0 writes the row. A row that fails (non-finite score or bias, a broken top-k, invalid
// weights) raises FLAG_ROUTE and gets expert ids E (which the layer schedule rejects) with zero
// weights.
template <int NC>
__global__ __launch_bounds__(64) void router_select_kernel(const float *__restrict__ scores,
                                                           const float *__restrict__ bias, uint32_t rows,
                                                           uint32_t E, uint32_t *__restrict__ selected,
                                                           float *__restrict__ weights, uint32_t *tie_rows,
                                                           uint32_t *flags)
{
    __shared__ TopkEntry lds_pairs[64 * NC];
    const uint32_t p = blockIdx.x;
    if (p >= rows)
        return;
    DeviceWave w;
    uint32_t sel_k;
    float w_k;
    bool tie = false;
    const int st = select_route_row<NC>(w, scores + (size_t)p * E, bias, E, lds_pairs, sel_k, w_k, &tie);
    const uint32_t lane = w.lane();
    if (st != ROUTE_OK) {
        sel_k = E;
        w_k = 0.0f;
        tie = false;
        if (lane == 0)
            raise_flag(flags, FLAG_ROUTE);
    }
    if (lane < 8) {
        selected[(size_t)p * 8 + lane] = sel_k;
        weights[(size_t)p * 8 + lane] = w_k;
    }
    if (lane == 0 && tie && tie_rows)
        atomicAdd(tie_rows, 1u);
}

template <typename TX, typename TW>
static void launch_scores_xw(const TX *x, const TW *w, uint32_t rows, uint32_t E, uint32_t K, float *scores,
                             hipStream_t stream)
{
    const dim3 grid(E, (rows + 7) / 8), block(256);
    if (rows == 1) hipLaunchKernelGGL((router_scores_kernel<TX, TW, 1>), grid, block, 0, stream, x, w, rows, E, K, scores);
    else if (rows == 2) hipLaunchKernelGGL((router_scores_kernel<TX, TW, 2>), grid, block, 0, stream, x, w, rows, E, K, scores);
    else if (rows <= 4) hipLaunchKernelGGL((router_scores_kernel<TX, TW, 4>), grid, block, 0, stream, x, w, rows, E, K, scores);
    else hipLaunchKernelGGL((router_scores_kernel<TX, TW, 8>), grid, block, 0, stream, x, w, rows, E, K, scores);
}

template <typename TX>
static void launch_scores_x(const TX *x, const void *w, bool w_f32, uint32_t rows, uint32_t E, uint32_t K,
                            float *scores, hipStream_t stream)
{
    if (w_f32)
        launch_scores_xw(x, (const float *)w, rows, E, K, scores, stream);
    else
        launch_scores_xw(x, (const uint16_t *)w, rows, E, K, scores, stream);
}

void launch_router_scores(const void *x, bool x_f32, const void *w, bool w_f32, uint32_t rows, uint32_t E,
                          uint32_t K, float *scores, hipStream_t stream)
{
    if (x_f32)
        launch_scores_x<float>((const float *)x, w, w_f32, rows, E, K, scores, stream);
    else
        launch_scores_x<uint16_t>((const uint16_t *)x, w, w_f32, rows, E, K, scores, stream);
}

void launch_router_select(const float *scores, const float *bias, uint32_t rows, uint32_t E, uint32_t *selected,
                          float *weights, uint32_t *tie_rows, uint32_t *flags, hipStream_t stream)
{
#define PW_SELECT(NC)                                                                                         \
    hipLaunchKernelGGL(router_select_kernel<NC>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, selected, \
                       weights, tie_rows, flags)
    if (E <= 64) PW_SELECT(1);
    else if (E <= 128) PW_SELECT(2);
    else if (E <= 256) PW_SELECT(4);
    else if (E <= 512) PW_SELECT(8);
    else PW_SELECT(16);
#undef PW_SELECT
}

void launch_router(const void *x, bool x_f32, const void *w, bool w_f32, const float *bias, uint32_t rows,
                   uint32_t E, uint32_t K, float *scores, uint32_t *selected, float *weights, uint32_t *tie_rows,
                   uint32_t *flags, hipStream_t stream)
{
    const int t = timer_begin(K_ROUTER, stream);
    launch_router_scores(x, x_f32, w, w_f32, rows, E, K, scores, stream);
    launch_router_select(scores, bias, rows, E, selected, weights, tie_rows, flags, stream);
    timer_end(t, stream);
}

}  // namespace pw
