// BF16 wide linear for decode widths (attention o_proj [4096 x 8192], LM head [vocab x 4096]):
// y[p, r] = round_bf16(sum_c bf16(W[r, c]) * x[p, c]) in f32, the reference's
// execute_bf16_linear (src/wide_metal_moe.rs:728-834: bf16_gemm8_shared_weight,
// kernels/block_fp8_gemv.metal:358-397, then bf16_round_in_place :219-232) and its CPU twin
// bf16_linear (src/text_endpoint.rs:3347-3380: decode the bf16 tensor, SGEMM, round).
//
// Work item: (64 or 128 weight rows, one K split of KC = BPW * 128 columns). Four or eight waves
// of 16 rows; every lane issues all of its weight loads at once (16 bytes = 8 bf16 per
// instruction, one row per lane, 64 contiguous bytes of each of 16 rows per instruction), so a
// wave keeps 16 KB in flight at BPW = 4. The activation rows of the K split go straight into LDS
// (direct-to-LDS loads) and are shared by the workgroup's waves. Activations are bf16 planes (f32 inputs arrive as three exact
// planes), so v_mfma_f32_16x16x32_bf16 forms exact products and accumulates in f32; only the f32
// summation order differs from the reference's. Split-K partials go to a buffer and
// bf16_reduce_kernel adds them in split order 0..KS-1 (deterministic), then rounds to bf16.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

// XF32: the activations arrive as f32 rows (a.xf, W <= 16): each thread loads its share of the
// K split's columns before the weights, and once those older loads are in, splits them into the
// three planes in LDS while the weights are still on their way (no separate split launch).
template <int NS, int NT, int BPW, int WAVES, bool XF32 = false>
__global__ __launch_bounds__(64 * WAVES) void bf16_split_kernel(const Bf16Args a)
{
    extern __shared__ uint4 lds_x[];  // [NS * W][KC / 8 + 1] 16-byte units
    constexpr uint32_t KC = BPW * 128, UNITS = KC / 8, STRIDE = UNITS + 1;
    constexpr uint32_t LANES = UNITS < 64 ? UNITS : 64, CPR = UNITS / LANES;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const uint32_t s = blockIdx.x % a.KS, g = blockIdx.x / a.KS;
    const uint32_t K = a.K, R = a.R, W = a.W;
    const uint32_t k0 = s * KC;
    const uint32_t row_base = g * (16 * WAVES) + wave * 16;
    // rows past R (a partial last group) load the last row: in-bounds reads whose outputs are dropped
    const uint32_t row = row_base + r16 < R ? row_base + r16 : R - 1;

    // 0. (XF32) this thread's f32 activation units (8 columns each) of the K split, rows past W
    //    rereading row W - 1
    constexpr uint32_t XU = XF32 ? (16 * UNITS + 64 * WAVES - 1) / (64 * WAVES) : 1;
    float4 xr[XU][2];
    if constexpr (XF32) {
        static_assert(NS == 3 && NT == 1, "f32 rows split into three planes, at most 16 rows");
#pragma unroll
        for (uint32_t i = 0; i < XU; ++i) {
            const uint32_t u = (uint32_t)tid + i * 64 * WAVES, t = u / UNITS, c = u % UNITS;
            const float *src = a.xf + (size_t)(t < W ? t : W - 1) * K + k0 + c * 8;
            xr[i][0] = *(const float4 *)src;
            xr[i][1] = *(const float4 *)(src + 4);
        }
    }

    // 1. every weight byte of this wave's 16 rows and K split, in flight at once
    const uint16_t *wrow = a.w + (size_t)row * K + k0 + q * 8;
    uint4 wv[BPW][4];
#pragma unroll
    for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            wv[j][c] = load_global16(wrow + j * 128 + c * 32);

    // 2. the activation rows of this K split -> LDS [plane][token][KC/8 + 1]: the f32 units split
    //    into their planes (their loads were issued before the weights', so the split waits only
    //    for them), or the bf16 planes copied straight into LDS, fully unrolled and dealt
    //    round-robin to the waves
    if constexpr (XF32) {
#pragma unroll
        for (uint32_t i = 0; i < XU; ++i) {
            const uint32_t u = (uint32_t)tid + i * 64 * WAVES, t = u / UNITS, c = u % UNITS;
            if (t < W) {
                const float v[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                                    xr[i][1].x, xr[i][1].y, xr[i][1].z, xr[i][1].w};
                uint32_t pk[3][4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint16_t h0, m0, l0, h1, m1, l1;
                    split3_bf16(v[2 * e], h0, m0, l0);
                    split3_bf16(v[2 * e + 1], h1, m1, l1);
                    pk[0][e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    pk[1][e] = (uint32_t)m0 | ((uint32_t)m1 << 16);
                    pk[2][e] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                }
#pragma unroll
                for (uint32_t p = 0; p < 3; ++p)
                    lds_x[(p * W + t) * STRIDE + c] = make_uint4(pk[p][0], pk[p][1], pk[p][2], pk[p][3]);
            }
        }
    } else {
#pragma unroll
        for (uint32_t t = 0; t < 16u * NT; ++t) {
            if (t < W) {
#pragma unroll
                for (uint32_t p = 0; p < (uint32_t)NS; ++p)
#pragma unroll
                    for (uint32_t c = 0; c < CPR; ++c)
                        if (((t * NS + p) * CPR + c) % WAVES == (uint32_t)wave && (uint32_t)lane < LANES)
                            lds_load16(a.x + p * a.x_plane + (size_t)t * K + k0 + (c * 64 + lane) * 8,
                                       lds_x + (p * W + t) * STRIDE + c * 64);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // 3. MFMA over the split: 32-column chunks, the lane's k-group q of each
    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
        acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bf16x8 A = bf16x8_from_u4(wv[j][c]);
            const uint32_t unit = j * 16 + c * 4 + q;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t t = nt * 16 + r16;
#pragma unroll
                for (int p = 0; p < NS; ++p) {
                    uint4 xv = make_uint4(0, 0, 0, 0);
                    if (t < W)
                        xv = lds_x[(p * W + t) * STRIDE + unit];
                    acc[nt] = mfma_bf16_16x16x32(A, bf16x8_from_u4(xv), acc[nt]);
                }
            }
        }

    // 4. split partials [KS][W][R]: lane holds rows row_base + 4q + i of token 16 nt + r16
    const uint32_t r4 = row_base + q * 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = nt * 16 + r16;
        if (t >= W)
            continue;
        float *dst = a.partial + ((size_t)s * W + t) * R + r4;
        if (r4 + 3 < R) {
            *(float4 *)dst = make_float4(acc[nt][0], acc[nt][1], acc[nt][2], acc[nt][3]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (r4 + i < R)
                    dst[i] = acc[nt][i];
        }
    }
}

// Split sums in order 0..KS-1, then bf16_round_in_place (a non-finite result raises
// FLAG_ROUND_NONFINITE, the reference's error bit 32). One thread per output.
__global__ __launch_bounds__(256) void bf16_reduce_kernel(const float *__restrict__ partial, uint32_t ks, size_t n,
                                                          float *__restrict__ y32, uint16_t *__restrict__ y16,
                                                          uint32_t round_f32, uint32_t *flags)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    float v;
    if (ks <= 16) {
        float part[16];  // every split's value requested before the first add
#pragma unroll
        for (uint32_t s = 0; s < 16; ++s)
            part[s] = s < ks ? partial[(size_t)s * n + i] : 0.f;
        v = part[0];
#pragma unroll
        for (uint32_t s = 1; s < 16; ++s)
            if (s < ks)
                v += part[s];
    } else {
        v = partial[i];
        for (uint32_t s = 1; s < ks; ++s)
            v += partial[(size_t)s * n + i];
    }
    const float r = round_bf16(v);
    if (!finite_f32(r))
        raise_flag(flags, FLAG_ROUND_NONFINITE);
    if (y32)
        y32[i] = round_f32 ? r : v;
    if (y16)
        y16[i] = (uint16_t)(f32_bits(r) >> 16);
}

int bf16_blocks_per_wave(uint32_t K, int planes, uint32_t W, size_t lds_cap)
{
    const uint32_t blocks = K / 128;
    for (int bpw = 4; bpw > 1; bpw /= 2)
        if (blocks % bpw == 0 && (size_t)planes * W * (bpw * 16 + 1) * 16 <= lds_cap)
            return bpw;
    return 1;
}

template <int NS, int NT, int WAVES, bool XF32 = false>
static void launch_bf16_waves(const Bf16Args &a, int bpw, hipStream_t stream)
{
    const dim3 grid(((a.R + 16 * WAVES - 1) / (16 * WAVES)) * a.KS), block(64 * WAVES);
    const size_t lds = (size_t)NS * a.W * (bpw * 16 + 1) * 16;
    if (bpw == 4)
        hipLaunchKernelGGL((bf16_split_kernel<NS, NT, 4, WAVES, XF32>), grid, block, lds, stream, a);
    else if (bpw == 2)
        hipLaunchKernelGGL((bf16_split_kernel<NS, NT, 2, WAVES, XF32>), grid, block, lds, stream, a);
    else
        hipLaunchKernelGGL((bf16_split_kernel<NS, NT, 1, WAVES, XF32>), grid, block, lds, stream, a);
}

// Projections of many rows (the LM head) take 128 rows per workgroup, so one staged copy of the
// activations feeds twice the weight rows; smaller ones (o_proj) keep 64 rows and twice the
// workgroups.
template <int NS, int NT, bool XF32 = false>
static void launch_bf16_nt(const Bf16Args &a, int bpw, hipStream_t stream)
{
    if (a.R >= 16384)
        launch_bf16_waves<NS, NT, 8, XF32>(a, bpw, stream);
    else
        launch_bf16_waves<NS, NT, 4, XF32>(a, bpw, stream);
}

void launch_bf16_linear(const Bf16Args &a, int planes, int bpw, float *y32, uint16_t *y16, uint32_t round_f32,
                        uint32_t *flags, hipStream_t stream)
{
    const int t = timer_begin(K_BF16_LINEAR, stream);
    if (a.xf) {
        launch_bf16_nt<3, 1, true>(a, bpw, stream);  // the caller keeps a.xf to W <= 16
    } else if (planes == 3) {
        if (a.W > 16) launch_bf16_nt<3, 2>(a, bpw, stream); else launch_bf16_nt<3, 1>(a, bpw, stream);
    } else {
        if (a.W > 16) launch_bf16_nt<1, 2>(a, bpw, stream); else launch_bf16_nt<1, 1>(a, bpw, stream);
    }
    const size_t n = (size_t)a.W * a.R;
    hipLaunchKernelGGL(bf16_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a.partial, a.KS, n,
                       y32, y16, round_f32, flags);
    timer_end(t, stream);
}

}  // namespace pw
