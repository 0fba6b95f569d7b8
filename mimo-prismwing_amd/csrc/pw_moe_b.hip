// Mode B routed-expert projections for the decode MoE layer and the one-expert forward: dynamic
// per-(row, 128-column) e4m3 activations against the block-FP8 weights on the FP8 MFMA, one
// 128-column block per instruction, total += dot * weight_scale * activation_scale per block
// (src/wide_metal_moe.rs:404-421, :1080-1166; Metal block_fp8_gemm{count}_sglang_blockscaled
// and bf16_staged_swiglu, kernels/block_fp8_gemv.metal:139-160, :935-1046).
//
// Work item: (routed expert, 16 weight rows), the whole K in one workgroup of eight waves. Wave w
// takes the 128-column blocks [w * BPW, (w + 1) * BPW); its share of the expert's activation codes
// goes straight from global memory into LDS (global_load_lds, rows padded by one 16-byte unit so
// the 16 token rows of a read fall in distinct banks) and is read only by that wave, so no barrier
// precedes the MFMAs; every weight load of the wave is issued before its first MFMA, and the
// in-order memory counter lets block j's MFMA start as soon as block j's weights arrive. The
// eight split sums meet in LDS and are added in split order 0..7.
//   gate/up: 16 rows of gate and the same 16 rows of up (RM = 16), or, for a lone expert and
//            for one-row experts, 8 + 8 rows stacked into one MFMA operand (RM = 8: twice the
//            workgroups); epilogue bf16_staged_swiglu -> hidden f32 [P][I] (bf16 values).
//   down:    16 rows of down over the re-quantised hidden codes; epilogue bf16_round_in_place of
//            the expert output (src/wide_metal_moe.rs:1236-1251) -> y [P][H], or, for a lone
//            expert, the output rows themselves.
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_route_job.h"

namespace pw {

// Workgroup i runs on XCD i % 8; with G row groups per expert (G a multiple of 8) XCD x takes the
// contiguous groups [x G/8, (x + 1) G/8) of each expert. A lone expert keeps the strided order.
__device__ __forceinline__ uint32_t xcd_group(uint32_t local, uint32_t G, bool single)
{
    return G % 8 == 0 && !single ? (local % 8) * (G / 8) + local / 8 : local;
}

// The codes of this wave's K split [k0, k0 + KC) for the work item's rows -> LDS rows of `stride`
// 16-byte units (row t at lds + t * stride, from column unit kw / 16 of the row, kw being the
// split's column within the workgroup's share of K). Row t of the work item is
// activation row ae.off + t (SLOTS: the down's slot rows) or ae.tok[t] (the gate/up's token rows).
// Fully unrolled over the sixteen possible rows: a loop would make the compiler wait for every
// outstanding load before its first iteration. Returns the activation row of the lane's own row
// (lane r16 < cnt) and sets bad_row when a row was out of range.
template <uint32_t KC, bool SLOTS>
__device__ __forceinline__ uint32_t stage_codes(const uint8_t *codes, uint32_t K, uint32_t k0, uint32_t kw,
                                                const ActiveExpert &ae, uint32_t n_rows, uint4 *lds, uint32_t stride,
                                                int lane, bool &bad_row)
{
    constexpr uint32_t PER = KC / 16, LANES = PER < 64 ? PER : 64, CPR = PER / LANES;
    static_assert(PER % LANES == 0, "whole 64-unit chunks");
    const int r16 = lane & 15;
    uint32_t mine = 0;
#pragma unroll
    for (uint32_t t = 0; t < 16u; ++t) {
        if (t < ae.cnt) {
            uint32_t src = SLOTS ? ae.off + t : (uint32_t)ae.tok[t];
            if (src >= n_rows) {
                bad_row = true;
                src = n_rows - 1;
            }
            mine = (uint32_t)r16 == t ? src : mine;
#pragma unroll
            for (uint32_t c = 0; c < CPR; ++c)
                if ((uint32_t)lane < LANES)
                    lds_load16(codes + (size_t)src * K + k0 + (c * 64 + lane) * 16, lds + t * stride + (kw >> 4) + c * 64);
        }
    }
    return mine;
}

// The activation scales of the lane's row for this wave's blocks (zero for lanes past the rows).
template <int BPW>
__device__ __forceinline__ void act_scales(const float *row_scales, bool ok, float *sa)
{
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const float v = load_g(row_scales + j);
        sa[j] = ok ? v : 0.f;
    }
}

__device__ __forceinline__ i32x8 i32x8_of(const uint4 &a, const uint4 &b)
{
    return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// LDS bytes of a whole-K work item: the staged codes of up to `cap` rows, at least the eight split
// partials of `mats` operands.
static size_t b_lds(uint32_t cap, uint32_t K, int mats)
{
    const size_t stage = (size_t)cap * (K / 16 + 1) * 16, red = (size_t)8 * mats * 64 * 16;
    return stage > red ? stage : red;
}

// JOB: the launch also carries args.job (the route weights, in its first ROUTE_JOB_WGS workgroups).
template <int BPW, int RM, bool JOB>
__global__ __launch_bounds__(512) void moe_b_gateup_fused_kernel(const MoeBArgs args)
{
    constexpr int MATS = RM == 16 ? 2 : 1;  // 16-row MFMA operands per block
    extern __shared__ uint4 lds_x[];         // codes [cnt][K/16 + 1]; then the split partials [8][MATS][64]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // split index, wave-uniform
    const int q = lane >> 4, r16 = lane & 15;
    uint32_t bid = blockIdx.x;
    if constexpr (JOB) {
        if (route_job_prologue(args.job, lds_x, &bid))
            return;  // one of the route-weights workgroups
    }
    const uint32_t G = args.R / RM;
    const uint32_t a = bid / G;
    const uint32_t g = xcd_group(bid % G, G, args.single);
    const ActiveExpert ae = args.single ? args.one : load_entry(args.active, a);
    if (ae.cnt == 0)
        return;
    if (ae.cnt > 16u || ae.cnt > args.cap) {
        if (tid == 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t K = args.K, blocks = K >> 7;
    constexpr uint32_t KC = BPW * 128;
    const uint32_t k0 = wave * KC;
    const uint32_t row0 = g * RM;
    const uint32_t stride = K / 16 + 1;

    // 1. this wave's K split of the expert's token rows (codes) -> LDS; then the activation scales
    bool bad_row = false;
    const uint32_t tok = stage_codes<KC, false>(args.codes, K, k0, k0, ae, args.rows, lds_x, stride, lane, bad_row);
    if (bad_row && tid == 0)
        raise_flag(args.flags, FLAG_SCHEDULE);
    asm volatile("" ::: "memory");  // the copies stay the oldest memory operations
    const bool ok = (uint32_t)r16 < ae.cnt;
    float sa[BPW];
    act_scales<BPW>(args.scales + (size_t)tok * blocks + (k0 >> 7), ok, sa);

    // 2. this wave's weight bytes of gate and up, all in flight at once (lane: row r16, columns
    //    q * 32 .. q * 32 + 31 of each block, the FP8 MFMA's operand layout), then the block scales
    uint4 wv[MATS][BPW][2];
    float sc[MATS][BPW];
    if constexpr (RM == 16) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint8_t *wrow = (m ? ae.ep.up_w : ae.ep.gate_w) + (size_t)(row0 + r16) * K + k0 + q * 32;
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                wv[m][j][0] = load_global16(wrow + j * 128);
                wv[m][j][1] = load_global16(wrow + j * 128 + 16);
            }
        }
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int j = 0; j < BPW; ++j)
                sc[m][j] = load_g((m ? ae.ep.up_s : ae.ep.gate_s) + (row0 >> 7) * blocks + (k0 >> 7) + j);
    } else {
        // operand row r16: gate row row0 + r16 (r16 < 8) or up row row0 + r16 - 8; output rows
        // 4q..4q+3 are gate rows for q < 2 and up rows for q >= 2, so each lane scales by its
        // output rows' matrix
        const uint8_t *wrow = (r16 < 8 ? ae.ep.gate_w : ae.ep.up_w) + (size_t)(row0 + (r16 & 7)) * K + k0 + q * 32;
#pragma unroll
        for (int j = 0; j < BPW; ++j) {
            wv[0][j][0] = load_global16(wrow + j * 128);
            wv[0][j][1] = load_global16(wrow + j * 128 + 16);
        }
#pragma unroll
        for (int j = 0; j < BPW; ++j) {
            const float gs = load_g(ae.ep.gate_s + (row0 >> 7) * blocks + (k0 >> 7) + j);
            const float us = load_g(ae.ep.up_s + (row0 >> 7) * blocks + (k0 >> 7) + j);
            sc[0][j] = q < 2 ? gs : us;
        }
    }

    // the copies are the oldest loads: once all but the weight loads are done they are in LDS
    wait_vmcnt<MATS * BPW * 2>();

    // 3. per block: the code dot products on the FP8 MFMA (exact in f32), then
    //    total += dot * weight_scale * activation_scale
    f32x4 tot[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        tot[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
        if (ok) {
            const uint4 *xp = lds_x + r16 * stride + (k0 >> 4) + j * 8 + q * 2;
            x0 = xp[0];
            x1 = xp[1];
        }
        const i32x8 xb = i32x8_of(x0, x1);
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            const f32x4 p = mfma_fp8_16x16x128(i32x8_of(wv[m][j][0], wv[m][j][1]), xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tot[m][i] = __builtin_fmaf(p[i] * sc[m][j], sa[j], tot[m][i]);
        }
    }

    // 4. the eight split sums meet in LDS (after every wave is done with its codes)
    __syncthreads();
    f32x4 *red = (f32x4 *)lds_x;  // [8 splits][MATS][64 lanes]
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        red[(wave * MATS + m) * 64 + lane] = tot[m];
    __syncthreads();
    if (wave != 0)
        return;
    // lane: rows 4q .. 4q + 3 of the 16, token r16; split sums in order 0..7
    float s[MATS][4];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        f32x4 sum = red[m * 64 + lane];
#pragma unroll
        for (int sp = 1; sp < 8; ++sp) {
            const f32x4 o = red[(sp * MATS + m) * 64 + lane];
            sum[0] += o[0];
            sum[1] += o[1];
            sum[2] += o[2];
            sum[3] += o[3];
        }
        s[m][0] = sum[0]; s[m][1] = sum[1]; s[m][2] = sum[2]; s[m][3] = sum[3];
    }
    float gu[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        gu[0][i] = s[0][i];
        if constexpr (RM == 16)
            gu[1][i] = s[MATS - 1][i];
        else
            gu[1][i] = __shfl(s[0][i], (lane + 32) & 63, 64);  // the up rows of this lane's gate rows
    }
    if (!ok || (RM == 8 && q >= 2))
        return;
    // bf16_staged_swiglu: gate and up rounded to bf16, silu rounded, the product rounded
    bool bad = false;
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float gv = round_bf16(gu[0][i]);
        const float uv = round_bf16(gu[1][i]);
        o[i] = round_bf16(silu_bf16_staged(gv) * uv);
        bad |= !finite_f32(gv) || !finite_f32(uv) || !finite_f32(o[i]);
    }
    *(float4 *)(args.out + (size_t)(ae.off + r16) * args.R + row0 + q * 4) = make_float4(o[0], o[1], o[2], o[3]);
    if (bad)
        raise_flag(args.flags, FLAG_SWIGLU_NONFINITE);
}

template <int BPW>
__global__ __launch_bounds__(512) void moe_b_down_fused_kernel(const MoeBArgs args)
{
    extern __shared__ uint4 lds_x[];  // codes [cnt][8 * KC/16 + 1]; then the split partials [8][64]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    // work item (expert a, 16-row group g, K share s of KS): the KS shares of one row group are
    // consecutive workgroups
    const uint32_t KS = args.KS, G = args.R / 16;
    const uint32_t a = blockIdx.x / (G * KS), rem = blockIdx.x % (G * KS);
    const uint32_t s = rem % KS;
    const uint32_t g = xcd_group(rem / KS, G, args.single);
    const ActiveExpert ae = args.single ? args.one : load_entry(args.active, a);
    if (ae.cnt == 0 || ae.cnt > 16u || ae.cnt > args.cap)
        return;  // the gate/up launch flagged such an entry
    const uint32_t K = args.K, blocks = K >> 7;
    constexpr uint32_t KC = BPW * 128;
    const uint32_t kw = wave * KC;          // this wave's columns within the share
    const uint32_t k0 = s * 8 * KC + kw;    // ... and within the row
    const uint32_t row0 = g * 16;
    const uint32_t stride = 8 * KC / 16 + 1;

    // 1. the expert's slot rows (hidden codes, this wave's K split) -> LDS; the activation scales
    bool bad_row = false;
    const uint32_t slot = stage_codes<KC, true>(args.codes, K, k0, kw, ae, args.rows, lds_x, stride, lane, bad_row);
    asm volatile("" ::: "memory");
    const bool ok = (uint32_t)r16 < ae.cnt;
    float sa[BPW];
    act_scales<BPW>(args.scales + (size_t)slot * blocks + (k0 >> 7), ok, sa);

    // 2. this wave's weight bytes, all in flight, then the block scales
    uint4 wv[BPW][2];
    const uint8_t *wrow = ae.ep.down_w + (size_t)(row0 + r16) * K + k0 + q * 32;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        wv[j][0] = load_global16(wrow + j * 128);
        wv[j][1] = load_global16(wrow + j * 128 + 16);
    }
    float sc[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j)
        sc[j] = load_g(ae.ep.down_s + (row0 >> 7) * blocks + (k0 >> 7) + j);
    wait_vmcnt<BPW * 2>();

    // 3. block partials
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
        if (ok) {
            const uint4 *xp = lds_x + r16 * stride + (kw >> 4) + j * 8 + q * 2;
            x0 = xp[0];
            x1 = xp[1];
        }
        const f32x4 p = mfma_fp8_16x16x128(i32x8_of(wv[j][0], wv[j][1]), i32x8_of(x0, x1), f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i)
            tot[i] = __builtin_fmaf(p[i] * sc[j], sa[j], tot[i]);
    }

    // 4. split sums in order 0..7; one share: the expert output rounded to bf16; KS shares: the
    //    share's sum into partial[s], which the next launch adds in share order and rounds
    __syncthreads();
    f32x4 *red = (f32x4 *)lds_x;
    red[wave * 64 + lane] = tot;
    __syncthreads();
    if (wave != 0 || !ok)
        return;
    f32x4 sum = red[lane];
#pragma unroll
    for (int sp = 1; sp < 8; ++sp) {
        const f32x4 o = red[sp * 64 + lane];
        sum[0] += o[0];
        sum[1] += o[1];
        sum[2] += o[2];
        sum[3] += o[3];
    }
    const size_t at = (size_t)(ae.off + r16) * args.R + row0 + q * 4;
    if (KS > 1) {
        *(float4 *)(args.partial + (size_t)s * args.rows * args.R + at) = make_float4(sum[0], sum[1], sum[2], sum[3]);
        return;
    }
    float r[4];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[i] = round_bf16(sum[i]);
        bad |= !finite_f32(r[i]);
    }
    if (args.out)
        *(float4 *)(args.out + at) = make_float4(r[0], r[1], r[2], r[3]);
    if (args.out_bf16)
        *(uint2 *)(args.out_bf16 + at) = make_uint2((f32_bits(r[0]) >> 16) | (f32_bits(r[1]) & 0xffff0000u),
                                                    (f32_bits(r[2]) >> 16) | (f32_bits(r[3]) & 0xffff0000u));
    if (bad && args.single)
        raise_flag(args.flags, FLAG_ROUND_NONFINITE);
}

// 128-column blocks per wave when a workgroup's eight waves cover K (K a multiple of 1024 with
// K / 1024 a power of two up to 16), or 0.
static int b_bpw(uint32_t K)
{
    if (K % 1024 != 0)
        return 0;
    const uint32_t bpw = K / 1024;
    return bpw == 1 || bpw == 2 || bpw == 4 || bpw == 8 || bpw == 16 ? (int)bpw : 0;
}

template <class Kernel>
static void launch_b(Kernel kernel, uint32_t grid, size_t lds, const MoeBArgs &args, hipStream_t stream)
{
    if (lds > 65536)
        (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), lds, stream, args);
}

// gate/up: one workgroup covers K (BPW <= 4: at most 16 weight loads in flight per lane)
static bool gateup_fits(uint32_t K, uint32_t R, uint32_t cap)
{
    const int bpw = b_bpw(K);
    return bpw != 0 && bpw <= 4 && R % 16 == 0 && cap <= 16 && b_lds(cap, K, 2) <= 160 * 1024;
}

// down: at most four blocks per wave; wider K is cut into KS shares of 4096 columns, whose sums go
// through memory (a lone expert only: its output rounding then runs as one more launch)
static uint32_t down_shares(uint32_t K)
{
    const int bpw = b_bpw(K);
    return bpw <= 4 ? 1u : (uint32_t)bpw / 4;
}

static bool down_fits(uint32_t K, uint32_t R, uint32_t cap, bool single)
{
    const uint32_t ks = down_shares(K);
    return b_bpw(K) != 0 && R % 16 == 0 && cap <= 16 && (ks == 1 || single) && b_lds(cap, K / ks, 1) <= 160 * 1024;
}

bool moe_b_fused_shapes(uint32_t H, uint32_t I, uint32_t cap, bool single)
{
    return gateup_fits(H, I, cap) && down_fits(I, H, cap, single);
}

bool launch_moe_b_gateup_fused(const MoeBArgs &args, uint32_t max_active, hipStream_t stream)
{
    if (!gateup_fits(args.K, args.R, args.cap))
        return false;
    const int bpw = b_bpw(args.K);
    const bool half = args.single || args.cap == 1;
    const size_t lds = b_lds(args.cap, args.K, half ? 1 : 2);
    const uint32_t grid = max_active * (args.R / (half ? 8 : 16)) + (args.job.rows ? ROUTE_JOB_WGS : 0);
#define PW_GU_J(B, J)                                                                                \
    do {                                                                                             \
        if (half) launch_b(moe_b_gateup_fused_kernel<B, 8, J>, grid, lds, args, stream);             \
        else launch_b(moe_b_gateup_fused_kernel<B, 16, J>, grid, lds, args, stream);                 \
    } while (0)
#define PW_GU(B)                                                                                     \
    do {                                                                                             \
        if (args.job.rows) PW_GU_J(B, true); else PW_GU_J(B, false);                                 \
    } while (0)
    if (bpw == 4) PW_GU(4);
    else if (bpw == 2) PW_GU(2);
    else PW_GU(1);
#undef PW_GU
#undef PW_GU_J
    return true;
}

uint32_t launch_moe_b_down_fused(const MoeBArgs &args_in, uint32_t max_active, hipStream_t stream)
{
    if (!down_fits(args_in.K, args_in.R, args_in.cap, args_in.single))
        return 0;
    MoeBArgs args = args_in;
    args.KS = down_shares(args.K);
    const int bpw = b_bpw(args.K) / (int)args.KS;
    const size_t lds = b_lds(args.cap, args.K / args.KS, 1);
    const uint32_t grid = max_active * (args.R / 16) * args.KS;
    switch (bpw) {
    case 4: launch_b(moe_b_down_fused_kernel<4>, grid, lds, args, stream); break;
    case 2: launch_b(moe_b_down_fused_kernel<2>, grid, lds, args, stream); break;
    default: launch_b(moe_b_down_fused_kernel<1>, grid, lds, args, stream); break;
    }
    return args.KS;
}

}  // namespace pw
