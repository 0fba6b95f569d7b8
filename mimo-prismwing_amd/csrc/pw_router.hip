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
// SLEEF expf_u10 restatement; the selection and weights are pytorch_noaux_routes (pw_topk.h),
// with nth_element's partitions split across a wave (same result, same partition order).
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_topk.h"

namespace pw {

// Eight consecutive values of a row as f32: bf16 (one 16-byte load) or f32 (two).
__device__ __forceinline__ void load8(const uint16_t *p, float *v)
{
    const uint4 q = load_global16(p);
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = f32_from(u[i] << 16);
        v[2 * i + 1] = f32_from(u[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ void load8(const float *p, float *v)
{
    const uint4 q0 = load_global16(p), q1 = load_global16(p + 4);
    const uint32_t u[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = f32_from(u[i]);
}

// One workgroup per (expert, 8-row chunk): scores[p][e] = sigmoid(logit[p][e]) in the declared
// order. Every thread reads its 8-column groups of the expert row and of the chunk's rows with
// 16-byte loads; the activation rows are shared by all experts' workgroups through L2.
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void router_scores_kernel(const TX *__restrict__ x, const TW *__restrict__ w,
                                                            uint32_t rows, uint32_t E, uint32_t K,
                                                            float *__restrict__ scores)
{
    __shared__ float wave_sum[8][4];
    const uint32_t g = threadIdx.x, lane = g & 63, wave = g >> 6;
    const uint32_t e = blockIdx.x;
    const uint32_t p0 = blockIdx.y * 8;
    const uint32_t np = rows - p0 < 8 ? rows - p0 : 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        acc[j] = 0.0f;
    const TW *wrow = w + (size_t)e * K;
    const TX *xrow = x + (size_t)p0 * K;
#pragma unroll 2
    for (uint32_t c0 = 8 * g; c0 < K; c0 += 2048) {
        float wv[8];
        load8(wrow + c0, wv);
        float xv[8][8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (j < np)
                load8(xrow + (size_t)j * K + c0, xv[j]);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (j < np)
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    acc[j] = __builtin_fmaf(xv[j][c], wv[c], acc[j]);
    }
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
        float v = acc[j];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            v = v + __shfl_down(v, off, 64);
        if (lane == 0)
            wave_sum[j][wave] = v;
    }
    __syncthreads();
    if (g < np) {
        const float logit = (wave_sum[g][0] + wave_sum[g][1]) + (wave_sum[g][2] + wave_sum[g][3]);
        scores[(size_t)(p0 + g) * E + e] = sigmoid_pytorch(logit);
    }
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t wave_ballot(bool b) { return __ballot(b); }

// libc++ nth_element(a, a + nth, a + n) run by one whole wave on LDS. The steps that touch a few
// elements (median of three, small ranges, the rare all-not-greater fallback, the pivot fix-up) are
// run by every lane alike on the same LDS words; the Hoare partition is split across the lanes:
// with A the ascending positions in [first + 1, j0] not greater than the pivot and B the descending
// positions in [first, j0 - 1] greater than it, the serial loop swaps A[t] with B[t] exactly while
// A[t] < B[t], stops i at min(A[T], B[T - 1]) (A[0] if T = 0) and moves the pivot from A[r] to B[r]
// when r < T. `apos` and `bpos` hold n positions each.
__device__ void nth_element_wave(TopkEntry *a, uint32_t nth, uint32_t n, uint32_t *apos, uint32_t *bpos,
                                 uint32_t lane)
{
    uint32_t first = 0, last = n;
    for (;;) {
        if (nth == last)
            return;
        if (topk_small(a + first, a + last))
            return;
        const uint32_t len = last - first;
        uint32_t m = first + len / 2;
        const uint32_t lm1 = last - 1;
        unsigned swaps = topk_sort3(a + first, a + m, a + lm1);
        __syncthreads();
        const float pv = a[m].v;
        uint32_t j0 = lm1;
        if (!(a[first].v > pv)) {
            // guard: the highest position in (first, lm1) greater than the pivot
            int32_t q = -1;
            for (int32_t c = (int32_t)lm1 - 1; c > (int32_t)first && q < 0; c -= 64) {
                const int32_t p = c - (int32_t)lane;
                const uint64_t mask = wave_ballot(p > (int32_t)first && a[p].v > pv);
                if (mask)
                    q = c - (int32_t)__builtin_ctzll(mask);
            }
            if (q >= 0) {
                topk_swap(a[first], a[q]);
                ++swaps;
                j0 = (uint32_t)q;
                __syncthreads();
            } else {
                TopkEntry *next;
                const bool done = topk_fallback_partition(a + first, a + nth, a + last, &next);
                __syncthreads();
                if (done)
                    return;
                first = (uint32_t)(next - a);
                continue;
            }
        }
        uint32_t i = first + 1;
        if (i < j0) {
            const uint32_t i0 = i;
            uint32_t na = 0, mrank = 0;
            for (uint32_t c = i0; c <= j0; c += 64) {
                const uint32_t p = c + lane;
                const bool ng = p <= j0 && !(a[p].v > pv);
                const uint64_t mask = wave_ballot(ng);
                if (ng)
                    apos[na + lanes_below(mask)] = p;
                if (m > c) {
                    const uint64_t below_m = m - c >= 64 ? ~0ull : ((1ull << (m - c)) - 1);
                    mrank += (uint32_t)__builtin_popcountll(mask & below_m);
                }
                na += (uint32_t)__builtin_popcountll(mask);
            }
            uint32_t nb = 0;
            for (int32_t c = (int32_t)j0 - 1; c >= (int32_t)first; c -= 64) {
                const int32_t p = c - (int32_t)lane;
                const bool gt = p >= (int32_t)first && a[p].v > pv;
                const uint64_t mask = wave_ballot(gt);
                if (gt)
                    bpos[nb + lanes_below(mask)] = (uint32_t)p;
                nb += (uint32_t)__builtin_popcountll(mask);
            }
            __syncthreads();
            const uint32_t pairs = na < nb ? na : nb;
            uint32_t T = 0;
            for (uint32_t c = 0; c < pairs; c += 64) {
                const uint32_t t = c + lane;
                const uint64_t mask = wave_ballot(t < pairs && apos[t] < bpos[t]);
                T += (uint32_t)__builtin_popcountll(mask);
                if (~mask)
                    break;
            }
            i = T > 0 ? (apos[T] < bpos[T - 1] ? apos[T] : bpos[T - 1]) : apos[0];
            if (m >= i0 && m <= j0 && mrank < T)
                m = bpos[mrank];
            for (uint32_t c = 0; c < T; c += 64) {
                const uint32_t t = c + lane;
                if (t < T) {
                    const uint32_t pa = apos[t], pb = bpos[t];
                    const TopkEntry ea = a[pa], eb = a[pb];
                    a[pa] = eb;
                    a[pb] = ea;
                }
            }
            swaps += T;
            __syncthreads();
        }
        if (i != m && a[m].v > a[i].v) {
            topk_swap(a[i], a[m]);
            ++swaps;
        }
        __syncthreads();
        if (nth == i)
            return;
        if (swaps == 0) {
            // already partitioned: is the side holding nth non-increasing?
            const uint32_t lo = nth < i ? first : i, end = nth < i ? i : last;
            bool sorted = true;
            for (uint32_t c = lo + 1; c < end && sorted; c += 64) {
                const uint32_t k = c + lane;
                sorted = wave_ballot(k < end && a[k].v > a[k - 1].v) == 0;
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

// One wave per row: the lanes stage the row's corrected scores in LDS with coalesced loads, the
// wave runs the top-8 partition, the rejected maximum is a wave reduction, and lane 0 finishes the
// row. A row that fails (non-finite score or bias, a broken top-k, invalid weights) raises
// FLAG_ROUTE and gets expert ids E (which the layer schedule rejects) with zero weights.
__global__ __launch_bounds__(64) void router_select_kernel(const float *__restrict__ scores,
                                                           const float *__restrict__ bias, uint32_t rows,
                                                           uint32_t E, uint32_t *__restrict__ selected,
                                                           float *__restrict__ weights, uint32_t *tie_rows,
                                                           uint32_t *flags)
{
    extern __shared__ uint4 lds_sel[];  // E TopkEntry, E scores, E + E positions
    const uint32_t p = blockIdx.x, lane = threadIdx.x;
    if (p >= rows)
        return;
    TopkEntry *ent = (TopkEntry *)lds_sel;
    float *s_row = (float *)(ent + E);
    uint32_t *apos = (uint32_t *)(s_row + E), *bpos = apos + E;
    bool bad = false;
    for (uint32_t e = lane; e < E; e += 64) {
        const float s = scores[(size_t)p * E + e], b = bias[e];
        bad |= !finite_f32_bits(s) || !finite_f32_bits(b);
        s_row[e] = s;
        ent[e].v = s + b;
        ent[e].i = (int32_t)e;
    }
    const bool any_bad = wave_ballot(bad) != 0;
    __syncthreads();
    uint32_t sel[8];
    float wt[8];
    bool tie = false;
    int st = ROUTE_NONFINITE;
    if (!any_bad) {
        nth_element_wave(ent, 7, E, apos, bpos, lane);
        float rejected = -__builtin_inff();
        for (uint32_t k = 8 + lane; k < E; k += 64)
            rejected = ent[k].v > rejected ? ent[k].v : rejected;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(rejected, off, 64);
            rejected = o > rejected ? o : rejected;
        }
        st = noaux_finish_row(s_row, ent, rejected, sel, wt, &tie);
    }
    if (lane != 0)
        return;
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

template <typename TX>
static void launch_scores_x(const TX *x, const void *w, bool w_f32, uint32_t rows, uint32_t E, uint32_t K,
                            float *scores, hipStream_t stream)
{
    const dim3 grid(E, (rows + 7) / 8), block(256);
    if (w_f32)
        hipLaunchKernelGGL((router_scores_kernel<TX, float>), grid, block, 0, stream, x, (const float *)w, rows, E, K,
                           scores);
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
    hipLaunchKernelGGL(router_select_kernel, dim3(rows), dim3(64), (size_t)E * (sizeof(TopkEntry) + 3 * sizeof(float)),
                       stream, scores, bias, rows, E, selected, weights, tie_rows, flags);
    timer_end(t, stream);
}

}  // namespace pw
