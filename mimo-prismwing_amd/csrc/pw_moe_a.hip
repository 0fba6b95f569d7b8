// Mode A routed-expert projections (FP8 weight x bf16 / exact-f32 activation, f32 accumulation)
// for the decode MoE layer: gate+up with SwiGLU, and down.
//
// Reference semantics: the f32 CPU control of the reference's MoE block (src/lib.rs:5807-5862):
// gate = x W_g^T, up = x W_u^T, h = (g / (1 + e^-g)) * u, y = h W_d^T, all f32; kernels
// block_fp8_gemm{1..8}_shared_weight_lut_blocked and swiglu_f32 (kernels/block_fp8_gemv.metal:
// 241-252, 751-933).
//
// Work item: (routed expert, 64 weight rows, one K split of KC columns). A workgroup of four
// waves reads each of its 64 rows x KC bytes exactly once. The expert's routed activation rows for
// the K split go straight from global memory into LDS (global_load_lds, padded rows so the later
// 16-byte reads are conflict-free) and are shared by the four waves; then every lane issues all of
// its weight loads (16 bytes per instruction, one weight row per lane, plain loads), at most eight
// 128-column blocks per lane, so a wave keeps 16 KB in flight on 64 VGPRs and several waves fit
// on each SIMD. e4m3 -> bf16 is exact (v_cvt_scalef32_pk_bf16_fp8); activations are bf16 planes
// (f32 values arrive as three exact planes), so v_mfma_f32_16x16x32_bf16 forms exact products and
// accumulates in f32. The 128x128 block scale multiplies each block partial in registers.
// Split-K partials go to a global buffer; the following kernel sums them in split order 0..KS-1
// (deterministic): moe_a_swiglu_kernel for gate/up (SwiGLU written as three exact bf16 planes for
// the down projection), the combine (or the single-expert output rounding) for down.
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_route_job.h"

namespace pw {

// JOB: the launch also carries args.job in its first ROUTE_JOB_WGS workgroups (the routed decode
// step's down; only that instantiation is compiled with it).
template <int MATS, int NS, int NT, int BPW, bool JOB = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NT == 1 ? 4 : 2))) void moe_a_split_kernel(const SplitArgs args)
{
    extern __shared__ uint4 lds_x[];  // [NS * cnt][KC/8 + 1]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int q = lane >> 4, r16 = lane & 15;
    uint32_t bid = blockIdx.x;
    if constexpr (JOB) {
        if (route_job_prologue(args.job, lds_x, &bid))
            return;  // one of the route-weights workgroups
    }
    const uint32_t G = args.R >> 6;
    const uint32_t s = bid % args.KS;
    const uint32_t g = (bid / args.KS) % G;
    const uint32_t a = bid / (args.KS * G);
    const ActiveExpert ae = args.single ? args.one : load_entry(args.active, a);
    if (ae.cnt == 0)
        return;
    if (ae.cnt > 16u * NT || ae.cnt > args.cap) {
        if (tid == 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t K = args.K;
    constexpr uint32_t KC = BPW * 128;
    const uint32_t k0 = s * KC;
    const uint32_t row_base = g * 64 + wave * 16;  // this wave's 16 rows

    // 1. token rows of routed slots 16..31 (lane t holds slot t's row; slots 0..15 come with the
    //    schedule entry): gate/up gather the token rows, down reads its own slot rows. Issued
    //    first, so the staging below waits only for it.
    uint32_t tok = 0;
    if constexpr (MATS == 2 && NT == 2) {
        if ((uint32_t)lane >= 16 && (uint32_t)lane < ae.cnt)
            tok = args.single ? (uint32_t)lane : load_g(args.placement_pos + ae.off + lane);
    }

    // 2. every weight byte of this wave's rows and K split, in flight at once
    const uint8_t *wbase[MATS];
    const float *sbase[MATS];
    if constexpr (MATS == 2) {
        wbase[0] = ae.ep.gate_w;
        wbase[1] = ae.ep.up_w;
        sbase[0] = ae.ep.gate_s;
        sbase[1] = ae.ep.up_s;
    } else {
        wbase[0] = ae.ep.down_w;
        sbase[0] = ae.ep.down_s;
    }
    uint4 wv[MATS][BPW][2];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        const uint8_t *wrow = wbase[m] + (size_t)(row_base + r16) * K + k0 + q * 16;
#pragma unroll
        for (int j = 0; j < BPW; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wv[m][j][h] = load_global16(wrow + j * 128 + h * 64);
    }
    // block scales of this wave's 16 rows (one 128-row scale block, wave-uniform)
    const uint32_t blocks = K >> 7;
    const uint32_t srow = row_base >> 7;
    float sc[MATS][BPW];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < BPW; ++j)
            sc[m][j] = load_g(sbase[m] + srow * blocks + (k0 >> 7) + j);

    // 3. the routed activation rows of this K split -> LDS [plane][token][KC/8 + 1], one
    //    direct-to-LDS instruction per (plane, token, 64-unit chunk), no registers involved
    constexpr uint32_t PER_ROW = KC / 8;                      // 16-byte units per row
    constexpr uint32_t STRIDE = PER_ROW + 1;                  // padded LDS row
    constexpr uint32_t LANES = PER_ROW < 64 ? PER_ROW : 64;   // active lanes per instruction
    constexpr uint32_t CPR = PER_ROW / LANES;                 // instructions per row
    // Fully unrolled over (token, plane, chunk) -- a loop here would make the compiler wait for
    // every outstanding weight load before its first iteration -- and dealt round-robin to the
    // four waves.
    bool bad_row = false;
#pragma unroll
    for (uint32_t t = 0; t < 16u * NT; ++t) {
        if (t < ae.cnt) {
            uint32_t src = ae.off + t;
            if constexpr (MATS == 2) {
                src = t < 16 ? (uint32_t)ae.tok[t] : __builtin_amdgcn_readlane(tok, t);
                if (src >= args.rows) {
                    bad_row = true;
                    src = args.rows - 1;
                }
            }
#pragma unroll
            for (uint32_t p = 0; p < (uint32_t)NS; ++p)
#pragma unroll
                for (uint32_t c = 0; c < CPR; ++c)
                    if (((t * NS + p) * CPR + c) % 4 == (uint32_t)wave && (uint32_t)lane < LANES)
                        lds_load16(args.x + p * args.x_plane + (size_t)src * K + k0 + (c * 64 + lane) * 8,
                                   lds_x + (p * ae.cnt + t) * STRIDE + c * 64);
        }
    }
    if (bad_row && lane == 0)
        raise_flag(args.flags, FLAG_SCHEDULE);

    // the LDS rows this wave loaded are complete before the barrier publishes them
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // 4. block partials on the MFMA, block scale in registers
    f32x4 tot[MATS][NT];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            tot[m][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        f32x4 acc[MATS][NT];
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                acc[m][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bf16x8 A[MATS][2];
#pragma unroll
            for (int m = 0; m < MATS; ++m) {
                A[m][0] = fp8x8_to_bf16x8(wv[m][j][h].x, wv[m][j][h].y);
                A[m][1] = fp8x8_to_bf16x8(wv[m][j][h].z, wv[m][j][h].w);
            }
            const uint32_t cu = j * 16 + h * 8 + q * 2;  // column in 16-byte units
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t t = nt * 16 + r16;
                const bool ok = t < ae.cnt;
#pragma unroll
                for (int p = 0; p < NS; ++p) {
                    uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                    if (ok) {
                        const uint4 *xp = lds_x + (p * ae.cnt + t) * STRIDE + cu;
                        x0 = xp[0];
                        x1 = xp[1];
                    }
#pragma unroll
                    for (int m = 0; m < MATS; ++m) {
                        acc[m][nt] = mfma_bf16_16x16x32(A[m][0], bf16x8_from_u4(x0), acc[m][nt]);
                        acc[m][nt] = mfma_bf16_16x16x32(A[m][1], bf16x8_from_u4(x1), acc[m][nt]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    tot[m][nt][i] = __builtin_fmaf(sc[m][j], acc[m][nt][i], tot[m][nt][i]);
    }

    // 5. split-K partials: partial[s][m][slot][row]. The splits are summed in split order by the
    //    next kernel (moe_a_swiglu_kernel, or the combine for the down projection): no
    //    cross-workgroup synchronisation, so no device-scope cache maintenance per workgroup.
    const uint32_t P = args.P, R = args.R;
    const uint32_t row4 = row_base + q * 4;
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const uint32_t t = nt * 16 + r16;
            if (t < ae.cnt)
                *(float4 *)(args.partial + (((size_t)s * MATS + m) * P + ae.off + t) * R + row4) =
                    make_float4(tot[m][nt][0], tot[m][nt][1], tot[m][nt][2], tot[m][nt][3]);
        }
}

// Gate/up over the whole K in one workgroup, SwiGLU fused: the decode fast path when the expert's
// routed rows fit LDS (NS * cnt <= 8). Work item: (routed expert, 16 weight rows of gate and of
// up). Eight waves split K (wave w: blocks [w * BPW, (w + 1) * BPW)), each issuing all of its
// weight loads at once (the same per-lane stream as the split kernel); the expert's routed
// activation rows for the whole K go straight into LDS; the eight partial sums meet in LDS and
// are added in split order 0..7 -- the same order and the same arithmetic as the split kernel
// followed by moe_a_swiglu_kernel, so the hidden planes are bit-identical -- and the SwiGLU is
// written as three exact bf16 planes. No split partials go through memory.
// RM = 8 (the one-expert forward): a work item is 8 rows of gate and the same 8 rows of up, stacked
// into one 16-row MFMA operand (lanes 0..7 of a row group read gate rows, 8..15 up rows), so a lone
// expert spreads over twice the workgroups; output rows 0..7 are gate, 8..15 up, and each gate
// lane takes its up values from the lane 32 above. The sums are the same as with RM = 16.
// Route a of a one-token batch as a schedule entry: expert route_ids[a] (ids past the bank take its
// last expert; the down+combine flags them), placement slot a, token row 0.
__device__ __forceinline__ ActiveExpert route_entry(const SplitArgs &args, uint32_t a)
{
    const uint32_t id = load_g(args.route_ids + a);
    ActiveExpert ae{};
    ae.ep = args.bank[id < args.E ? id : args.E - 1];
    ae.off = a;
    ae.cnt = 1;
    ae.tok[0] = 0;
    return ae;
}

// JOB: the launch also carries args.job (the route weights, in its first ROUTE_JOB_WGS workgroups);
// the launches without one are compiled without that code.
template <int NS, int BPW, int RM, bool JOB>
__global__ __launch_bounds__(512) void moe_a_gateup_fused_kernel(const SplitArgs args, uint16_t *__restrict__ hidden)
{
    constexpr int MATS = RM == 16 ? 2 : 1;  // 16-row MFMA operands per block
    extern __shared__ uint4 lds_x[];  // [NS * cnt][K/8 + 1]; then the split partials [8][2][64]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // split index, wave-uniform
    const int q = lane >> 4, r16 = lane & 15;
    // Workgroup i runs on XCD i % 8. XCD x takes the contiguous row groups [x G/8, (x + 1) G/8) of
    // each routed expert (1 MB of gate and 1 MB of up at G = 128), not every eighth 16-row group:
    // the strided form gave each XCD's loads a common set of address bits and ran 4% slower, and
    // up to 7% slower for some physical placements of the bank. A lone expert (the one-expert
    // forward, the dense MLP) keeps the strided order, which measured 1 µs faster there. Which
    // workgroup computes which rows does not change any sum.
    uint32_t bid = blockIdx.x;
    if constexpr (JOB) {
        if (route_job_prologue(args.job, lds_x, &bid))
            return;  // one of the route-weights workgroups
    }
    const uint32_t G = args.R / RM;
    const uint32_t a = bid / G, local = bid % G;
    const uint32_t g = G % 8 == 0 && !args.single ? (local % 8) * (G / 8) + local / 8 : local;
    const ActiveExpert ae = args.single ? args.one : (args.route_ids ? route_entry(args, a) : load_entry(args.active, a));
    if (ae.cnt == 0)
        return;
    if (ae.cnt > 16u || ae.cnt > args.cap) {
        if (tid == 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t K = args.K;
    constexpr uint32_t KC = BPW * 128;
    const uint32_t k0 = wave * KC;
    const uint32_t row0 = g * RM;

    // 1. the routed activation rows, whole K (= 8 * KC), planes -> LDS: wave w copies the 64
    //    16-byte units of its own K split of every row and plane, fully unrolled (one instruction
    //    per row and plane, since KC / 8 = 64 units), and reads nothing else of the stage
    static_assert(KC / 8 == 64, "one 64-lane copy per row and split");
    constexpr uint32_t per_row = 8 * KC / 8, stride = per_row + 1;
    bool bad_row = false;
#pragma unroll
    for (uint32_t t = 0; t < 16u; ++t) {
        if (t < ae.cnt) {
            uint32_t src = ae.tok[t];
            if (src >= args.rows) {
                bad_row = true;
                src = args.rows - 1;
            }
#pragma unroll
            for (uint32_t p = 0; p < (uint32_t)NS; ++p)
                lds_load16(args.x + p * args.x_plane + (size_t)src * K + k0 + lane * 8,
                           lds_x + (p * ae.cnt + t) * stride + wave * 64);
        }
    }
    if (bad_row && tid == 0)
        raise_flag(args.flags, FLAG_SCHEDULE);
    asm volatile("" ::: "memory");  // the copies stay the oldest memory operations

    // 2. this wave's weight bytes of gate and up, all in flight at once
    uint4 wv[MATS][BPW][2];
    const uint32_t blocks = K >> 7;
    float sc[MATS][BPW];
    if constexpr (RM == 16) {
        const uint8_t *wbase[2] = {ae.ep.gate_w, ae.ep.up_w};
        const float *sbase[2] = {ae.ep.gate_s, ae.ep.up_s};
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint8_t *wrow = wbase[m] + (size_t)(row0 + r16) * K + k0 + q * 16;
#pragma unroll
            for (int j = 0; j < BPW; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    wv[m][j][h] = load_global16(wrow + j * 128 + h * 64);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int j = 0; j < BPW; ++j)
                sc[m][j] = load_g(sbase[m] + (row0 >> 7) * blocks + (k0 >> 7) + j);
    } else {
        // operand row r16: gate row row0 + r16 (r16 < 8) or up row row0 + r16 - 8; output rows
        // 4q..4q+3 are gate rows for q < 2 and up rows for q >= 2, so each lane scales by its
        // output rows' matrix
        const uint8_t *wrow = (r16 < 8 ? ae.ep.gate_w : ae.ep.up_w) + (size_t)(row0 + (r16 & 7)) * K + k0 + q * 16;
#pragma unroll
        for (int j = 0; j < BPW; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wv[0][j][h] = load_global16(wrow + j * 128 + h * 64);
        const float *srow = (q < 2 ? ae.ep.gate_s : ae.ep.up_s) + (row0 >> 7) * blocks + (k0 >> 7);
#pragma unroll
        for (int j = 0; j < BPW; ++j)
            sc[0][j] = load_g(srow + j);
    }

    // the copies are the oldest loads: once all but the weight loads are done they are in LDS, and
    // block j's MFMAs then start as soon as its weights arrive, while later blocks are in flight
    wait_vmcnt<MATS * BPW * 2>();

    // 3. block partials on the MFMA, block scale in registers (as moe_a_split_kernel)
    f32x4 tot[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        tot[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool ok = (uint32_t)r16 < ae.cnt;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        f32x4 acc[MATS];
#pragma unroll
        for (int m = 0; m < MATS; ++m)
            acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bf16x8 A[MATS][2];
#pragma unroll
            for (int m = 0; m < MATS; ++m) {
                A[m][0] = fp8x8_to_bf16x8(wv[m][j][h].x, wv[m][j][h].y);
                A[m][1] = fp8x8_to_bf16x8(wv[m][j][h].z, wv[m][j][h].w);
            }
            const uint32_t cu = (k0 >> 3) + j * 16 + h * 8 + q * 2;
#pragma unroll
            for (int p = 0; p < NS; ++p) {
                uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                if (ok) {
                    const uint4 *xp = lds_x + (p * ae.cnt + r16) * stride + cu;
                    x0 = xp[0];
                    x1 = xp[1];
                }
#pragma unroll
                for (int m = 0; m < MATS; ++m) {
                    acc[m] = mfma_bf16_16x16x32(A[m][0], bf16x8_from_u4(x0), acc[m]);
                    acc[m] = mfma_bf16_16x16x32(A[m][1], bf16x8_from_u4(x1), acc[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tot[m][i] = __builtin_fmaf(sc[m][j], acc[m][i], tot[m][i]);
    }

    // 4. the eight split partials meet in LDS (after every wave is done with the activations)
    __syncthreads();
    f32x4 *red = (f32x4 *)lds_x;  // [8 splits][MATS][64 lanes]
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        red[(wave * MATS + m) * 64 + lane] = tot[m];
    __syncthreads();
    if (wave != 0)
        return;
    // lane: rows 4q .. 4q + 3 of the 16, token r16; split sums in order 0..7, then the SwiGLU
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
    float v[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[0][i] = s[0][i];
        if constexpr (RM == 16)
            v[1][i] = s[1][i];
        else
            v[1][i] = __shfl(s[0][i], (lane + 32) & 63, 64);  // the up rows of this lane's gate rows
    }
    if (!ok || (RM == 8 && q >= 2))
        return;
    uint16_t hp[3][4];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float gv = v[0][i];
        const float hv = (gv / (1.0f + expf(-gv))) * v[1][i];
        bad |= !finite_f32(hv);
        split3_bf16(hv, hp[0][i], hp[1][i], hp[2][i]);
    }
    const size_t plane = (size_t)args.P * args.R;
    uint16_t *dst = hidden + (size_t)(ae.off + r16) * args.R + row0 + q * 4;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
        *(uint2 *)(dst + pl * plane) = make_uint2((uint32_t)hp[pl][0] | ((uint32_t)hp[pl][1] << 16),
                                                  (uint32_t)hp[pl][2] | ((uint32_t)hp[pl][3] << 16));
    if (bad)
        raise_flag(args.flags, FLAG_SWIGLU_NONFINITE);
}

// LDS bytes of the fused gate/up stage: NS planes x cnt rows x (K/8 + 1) 16-byte units, at least
// the eight split partials.
static size_t fused_lds(int ns, uint32_t cnt, uint32_t K)
{
    const size_t stage = (size_t)ns * cnt * (K / 8 + 1) * 16, red = (size_t)8 * 2 * 64 * 16;
    return stage > red ? stage : red;
}

bool launch_moe_a_gateup_fused(int ns, const SplitArgs &args, uint32_t max_active, uint16_t *hidden_planes,
                               hipStream_t stream)
{
    // four 128-column blocks per wave and split (the split kernel's gate/up stream), eight splits
    if (args.K != 8 * 4 * 128 || args.R % 16 != 0 || (uint32_t)ns * args.cap > 8)
        return false;
    const size_t lds = fused_lds(ns, args.cap, args.K);
    // a lone expert (the one-expert forward) and one-row experts (a one-token batch) take 8 + 8-row
    // work items: twice the workgroups
    const bool half = args.R % 8 == 0 && (args.single || args.cap == 1);
    const dim3 grid(max_active * (args.R / (half ? 8 : 16)) + (args.job.rows ? ROUTE_JOB_WGS : 0)), block(512);
#define PW_FUSED_J(NS, RM, J)                                                                                \
    do {                                                                                                      \
        if (lds > 65536)                                                                                      \
            (void)hipFuncSetAttribute((const void *)moe_a_gateup_fused_kernel<NS, 4, RM, J>,                  \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                  \
        hipLaunchKernelGGL((moe_a_gateup_fused_kernel<NS, 4, RM, J>), grid, block, lds, stream, args,         \
                           hidden_planes);                                                                    \
    } while (0)
#define PW_FUSED(NS, RM)                                                                                     \
    do {                                                                                                      \
        if (args.job.rows) PW_FUSED_J(NS, RM, true); else PW_FUSED_J(NS, RM, false);                          \
    } while (0)
    if (ns == 3) {
        if (half) PW_FUSED(3, 8); else PW_FUSED(3, 16);
    } else {
        if (half) PW_FUSED(1, 8); else PW_FUSED(1, 16);
    }
#undef PW_FUSED
#undef PW_FUSED_J
    return true;
}

// Down over the whole K in one workgroup for one expert's rows, output rounding fused: the
// one-expert forward's last launch (dense MLP, complete expert). Work item: 16 rows of down.
// Eight waves split K = I (wave w: blocks [w * BPW, (w + 1) * BPW)), each with all of its weight
// loads in flight at once; the expert's three bf16 hidden planes (rows 0..cnt-1) go straight into
// LDS; the eight split sums meet in LDS and are added in split order 0..7, then rounded to bf16 (or
// kept as raw f32) and written as the output rows: no split partials through memory, no rounding
// launch.
template <int BPW>
__global__ __launch_bounds__(512) void moe_a_down_out_kernel(const SplitArgs args, float *__restrict__ out_f32,
                                                             uint16_t *__restrict__ out_bf16, uint32_t raw)
{
    extern __shared__ uint4 lds_x[];  // [3 * cnt][K/8 + 1]; then the split partials [8][64]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // split index, wave-uniform
    const int q = lane >> 4, r16 = lane & 15;
    const ActiveExpert &ae = args.one;
    const uint32_t cnt = ae.cnt;
    if (cnt == 0 || cnt > args.cap) {
        if (tid == 0 && cnt != 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t K = args.K, R = args.R;
    constexpr uint32_t KC = BPW * 128;
    const uint32_t k0 = wave * KC;
    const uint32_t row0 = blockIdx.x * 16;

    // 1. the hidden rows (three planes, whole K) -> LDS: wave w copies its K split of every row and
    //    plane (KC / 8 16-byte units per row, at most 64 lanes per instruction) and reads only that
    constexpr uint32_t PER_SPLIT = KC / 8, LANES = PER_SPLIT < 64 ? PER_SPLIT : 64, CPS = PER_SPLIT / LANES;
    // (unrolled over the eight possible rows: a loop would make the compiler wait for every
    // outstanding weight load before its first iteration)
    const uint32_t stride = K / 8 + 1;
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t)
        if (t < cnt) {
#pragma unroll
            for (uint32_t p = 0; p < 3; ++p)
#pragma unroll
                for (uint32_t c = 0; c < CPS; ++c)
                    if ((uint32_t)lane < LANES)
                        lds_load16(args.x + p * args.x_plane + (size_t)t * K + k0 + (c * 64 + lane) * 8,
                                   lds_x + (p * cnt + t) * stride + (k0 >> 3) + c * 64);
        }
    asm volatile("" ::: "memory");  // the copies stay the oldest memory operations

    // 2. this wave's weight bytes, all in flight at once, and its block scales
    uint4 wv[BPW][2];
    const uint8_t *wrow = ae.ep.down_w + (size_t)(row0 + r16) * K + k0 + q * 16;
#pragma unroll
    for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            wv[j][h] = load_global16(wrow + j * 128 + h * 64);
    const uint32_t blocks = K >> 7;
    float sc[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j)
        sc[j] = load_g(ae.ep.down_s + (row0 >> 7) * blocks + (k0 >> 7) + j);

    // the copies are done once all but the weight loads are; block j's MFMAs start when its weights arrive
    wait_vmcnt<BPW * 2>();

    // 3. block partials on the MFMA, block scale in registers (as moe_a_split_kernel)
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool ok = (uint32_t)r16 < cnt;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bf16x8 A0 = fp8x8_to_bf16x8(wv[j][h].x, wv[j][h].y);
            const bf16x8 A1 = fp8x8_to_bf16x8(wv[j][h].z, wv[j][h].w);
            const uint32_t cu = (k0 >> 3) + j * 16 + h * 8 + q * 2;
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                if (ok) {
                    const uint4 *xp = lds_x + (p * cnt + r16) * stride + cu;
                    x0 = xp[0];
                    x1 = xp[1];
                }
                acc = mfma_bf16_16x16x32(A0, bf16x8_from_u4(x0), acc);
                acc = mfma_bf16_16x16x32(A1, bf16x8_from_u4(x1), acc);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            tot[i] = __builtin_fmaf(sc[j], acc[i], tot[i]);
    }

    // 4. the eight split partials meet in LDS (after every wave is done with the activations),
    //    summed in split order; lane: rows 4q .. 4q + 3 of the 16, row r16 of the output
    __syncthreads();
    f32x4 *red = (f32x4 *)lds_x;  // [8 splits][64 lanes]
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
    bool bad = false;
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[i] = round_bf16(sum[i]);
        bad |= !finite_f32(r[i]);
    }
    const size_t at = (size_t)r16 * R + row0 + q * 4;
    if (out_f32)
        *(float4 *)(out_f32 + at) = raw ? make_float4(sum[0], sum[1], sum[2], sum[3]) : make_float4(r[0], r[1], r[2], r[3]);
    if (out_bf16)
        *(uint2 *)(out_bf16 + at) = make_uint2((f32_bits(r[0]) >> 16) | (f32_bits(r[1]) & 0xffff0000u),
                                               (f32_bits(r[2]) >> 16) | (f32_bits(r[3]) & 0xffff0000u));
    if (bad)
        raise_flag(args.flags, FLAG_ROUND_NONFINITE);
}

bool launch_moe_a_down_out(const SplitArgs &args, float *out_f32, uint16_t *out_bf16, bool raw, hipStream_t stream)
{
    // eight K splits of one or two 128-column blocks each, output rows in whole 16-row tiles,
    // the three hidden planes of up to eight rows within LDS
    const uint32_t K = args.K;
    if (!args.single || (K != 8 * 128 && K != 16 * 128) || args.R % 16 != 0 || args.one.cnt > 8)
        return false;
    const size_t stage = (size_t)3 * args.one.cnt * (K / 8 + 1) * 16, red = (size_t)8 * 64 * 16;
    const size_t lds = stage > red ? stage : red;
    const dim3 grid(args.R >> 4), block(512);
    if (K == 16 * 128) {
        if (lds > 65536)
            (void)hipFuncSetAttribute((const void *)moe_a_down_out_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lds);
        hipLaunchKernelGGL((moe_a_down_out_kernel<2>), grid, block, lds, stream, args, out_f32, out_bf16, raw ? 1u : 0u);
    } else {
        hipLaunchKernelGGL((moe_a_down_out_kernel<1>), grid, block, lds, stream, args, out_f32, out_bf16, raw ? 1u : 0u);
    }
    return true;
}

// Down and combine of a one-token batch in one launch (the decode layer at width 1: eight routed
// experts with one slot each). Work item: 16 output rows. Sixteen waves: wave w takes routed
// expert w / 2 (the schedule's, in ascending id, or route w / 2 of a batch passed as routes) and K
// half w % 2, which is exactly the split-K
// down's work for those rows (KS = 2, eight 128-column blocks per split, the same MFMA sequence and
// block-scale order), so each split sum is the same f32 value. The sums meet in LDS; lanes 0..15
// of wave 0 then form each output row as the combine does: per expert in ascending id, the split
// sums added in split order, times the route weight, added to the row in f32 without fused
// multiply-add, then rounded to bf16. No per-placement outputs go through memory and no combine
// launch follows.
__global__ __launch_bounds__(1024) void moe_a_down_combine1_kernel(const SplitArgs args, const MoePlan *__restrict__ plan,
                                                                   const float *__restrict__ placement_w,
                                                                   float *__restrict__ out_f32,
                                                                   uint16_t *__restrict__ out_bf16, uint32_t raw)
{
    constexpr int BPW = 8;
    constexpr uint32_t KC = BPW * 128, PER_SPLIT = KC / 8, STRIDE = PER_SPLIT + 1;
    extern __shared__ uint4 lds_x[];  // per wave [3][KC/8 + 1]; then the split sums [16 waves][16 rows]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const uint32_t a = (uint32_t)wave >> 1, s = (uint32_t)wave & 1;
    const uint32_t K = args.K;
    const uint32_t row0 = blockIdx.x * 16;
    float *red = (float *)(lds_x + 16 * 3 * STRIDE);  // [16 waves][16 rows]
    uint32_t *rank_slot = (uint32_t *)(red + 16 * 16);  // [8] routes: the slot of each expert rank
    float *rank_w = (float *)(rank_slot + 8);           // [8] routes: the weight of each expert rank
    // routes without a schedule: waves 2a and 2a + 1 take route a itself (its pointer entry is
    // loaded with the routes, so the weights wait on two round trips); lane i < 8 ranks route i by
    // (expert id, route index), so the combine takes the experts in ascending id like the
    // schedule; duplicates, ids past the bank and non-finite weights are rejected
    uint32_t n_active;
    bool rejected;  // routes that fail the schedule's checks: the combine writes zeros, as the schedule's does
    ActiveExpert ae{};
    if (args.route_ids) {
        ae = route_entry(args, a);
        const uint32_t li = (uint32_t)lane & 7;
        const uint32_t id = load_g(args.route_ids + li);
        const float rw = load_g(args.route_w + li);
        uint32_t rank = 0;
        bool dup = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t idj = __shfl(id, j, 64);
            rank += idj < id || (idj == id && (uint32_t)j < li);
            dup |= idj == id && (uint32_t)j != li;
        }
        const bool bad = dup || id >= args.E || !finite_f32(rw);
        rejected = __ballot(lane < 8 && bad) != 0;
        if (wave == 0 && lane < 8) {
            rank_slot[rank] = li;
            rank_w[rank] = rw;
            if (bad)
                raise_flag(args.flags, FLAG_SCHEDULE);
        }
        n_active = 8;
    } else {
        n_active = plan->n_active;
        rejected = plan->rejected != 0;
    }
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    if (a < n_active) {
        if (!args.route_ids)
            ae = load_entry(args.active, a);
        if (ae.cnt != 1 && lane == 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        const uint32_t k0 = s * KC;
        // 1. the expert's hidden row (its one slot) for this K half, three planes -> this wave's own
        //    LDS region; then the block scales; then this wave's weight bytes (16 rows x K half), all
        //    in flight. In that order the in-order memory counter lets the MFMAs of block j start
        //    when block j's weights arrive, while the later blocks are still on their way.
        uint4 *xs = lds_x + wave * 3 * STRIDE;
        const uint32_t slot = ae.off < args.P ? ae.off : 0;
#pragma unroll
        for (uint32_t p = 0; p < 3; ++p)
#pragma unroll
            for (uint32_t c = 0; c < PER_SPLIT / 64; ++c)
                lds_load16(args.x + p * args.x_plane + (size_t)slot * K + k0 + (c * 64 + lane) * 8,
                           xs + p * STRIDE + c * 64);
        asm volatile("" ::: "memory");  // the copies stay the oldest memory operations
        const uint32_t blocks = K >> 7;
        float sc[BPW];
#pragma unroll
        for (int j = 0; j < BPW; ++j)
            sc[j] = load_g(ae.ep.down_s + (row0 >> 7) * blocks + (k0 >> 7) + j);
        uint4 wv[BPW][2];
        const uint8_t *wrow = ae.ep.down_w + (size_t)(row0 + r16) * K + k0 + q * 16;
#pragma unroll
        for (int j = 0; j < BPW; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wv[j][h] = load_global16(wrow + j * 128 + h * 64);
        wait_vmcnt<2 * BPW>();  // every load but the youngest 2 * BPW: this wave's copies (its own region)
        // 2. block partials on the MFMA (token column 0; the other columns multiply zeros)
#pragma unroll
        for (int j = 0; j < BPW; ++j) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bf16x8 A0 = fp8x8_to_bf16x8(wv[j][h].x, wv[j][h].y);
                const bf16x8 A1 = fp8x8_to_bf16x8(wv[j][h].z, wv[j][h].w);
                const uint32_t cu = j * 16 + h * 8 + q * 2;
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                    if (r16 == 0) {
                        x0 = xs[p * STRIDE + cu];
                        x1 = xs[p * STRIDE + cu + 1];
                    }
                    acc = mfma_bf16_16x16x32(A0, bf16x8_from_u4(x0), acc);
                    acc = mfma_bf16_16x16x32(A1, bf16x8_from_u4(x1), acc);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tot[i] = __builtin_fmaf(sc[j], acc[i], tot[i]);
        }
        if (r16 == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[wave * 16 + q * 4 + i] = tot[i];
    }
    __syncthreads();
    if (wave != 0 || lane >= 16)
        return;
    // 4. the combine for output row row0 + lane, with every expert's route weight fetched first (from
    //    LDS with routes; with a schedule, the eight slots and then the eight weights in flight)
    const uint32_t ne = n_active < 8 ? n_active : 8;
    float wt[8];
    if (args.route_ids) {
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e)
            wt[e] = rank_w[e];
    } else {
        uint32_t sl[8];
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e)
            sl[e] = e < ne ? args.active[e].off : 0u;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e)
            wt[e] = placement_w[sl[e] < args.P ? sl[e] : 0];
    }
    float acc = 0.f;
#pragma unroll
    for (uint32_t e = 0; e < 8; ++e) {
        if (e < ne) {
            // the waves of the e-th expert in ascending id: those of its route (with routes) or 2e, 2e + 1
            const uint32_t wa = args.route_ids ? rank_slot[e] : e;
            const float y = red[(2 * wa) * 16 + lane] + red[(2 * wa + 1) * 16 + lane];
            acc = __fadd_rn(acc, __fmul_rn(y, wt[e]));
        }
    }
    acc = rejected ? 0.f : acc;
    const float r = round_bf16(acc);
    const size_t at = row0 + lane;
    if (out_f32)
        out_f32[at] = raw ? acc : r;
    if (out_bf16)
        out_bf16[at] = (uint16_t)(f32_bits(r) >> 16);
    if (!finite_f32(r))
        raise_flag(args.flags, FLAG_ROUND_NONFINITE);
}

bool moe_a_one_token_direct(uint32_t H, uint32_t I)
{
    // the fused gate/up's K (eight splits of four blocks) and the one-token down's (I = 2048)
    return H == 8 * 4 * 128 && I == 2048 && I % 16 == 0 && H % 16 == 0;
}

bool launch_moe_a_down_combine1(const SplitArgs &args, const MoePlan *plan, const float *placement_w, float *out_f32,
                                uint16_t *out_bf16, bool raw, hipStream_t stream)
{
    // the split-K down's plan at I = 2048 (two splits of eight blocks); the caller's batch is one
    // token, so its eight placements are the rows
    if (args.P != 8 || args.rows != 8 || args.K != 2048 || args.R % 16 != 0)
        return false;
    const size_t lds = (size_t)16 * 3 * (1024 / 8 + 1) * 16 + 16 * 16 * 4 + 8 * 4 + 8 * 4;
    (void)hipFuncSetAttribute((const void *)moe_a_down_combine1_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    hipLaunchKernelGGL(moe_a_down_combine1_kernel, dim3(args.R >> 4), dim3(1024), lds, stream, args, plan,
                       placement_w, out_f32, out_bf16, raw ? 1u : 0u);
    return true;
}

// Gate/up split sums (in split order 0..KS-1) -> h = (g / (1 + e^-g)) * u in f32 (swiglu_f32,
// kernels/block_fp8_gemv.metal:241-252; CPU src/lib.rs:5840-5844), written as three exact bf16
// planes for the down projection's MFMA. One thread per (slot, 4 rows). With KS known at compile
// time every partial load is issued before the first add (one memory round trip); KS = 0 is the
// generic loop.
template <int KS>
__global__ __launch_bounds__(256) void moe_a_swiglu_kernel(const float *__restrict__ partial, uint32_t ks_rt,
                                                           uint32_t P, uint32_t R, uint16_t *__restrict__ hidden,
                                                           uint32_t *flags)
{
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t per_slot = R >> 2;
    if (idx >= P * per_slot)
        return;
    const uint32_t slot = idx / per_slot, row4 = (idx - slot * per_slot) * 4;
    float v[2][4];
    if constexpr (KS > 0) {
        float4 part[2][KS];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int sp = 0; sp < KS; ++sp)
                part[m][sp] = *(const float4 *)(partial + (((size_t)sp * 2 + m) * P + slot) * R + row4);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            float4 sum = part[m][0];
#pragma unroll
            for (int sp = 1; sp < KS; ++sp) {
                sum.x += part[m][sp].x;
                sum.y += part[m][sp].y;
                sum.z += part[m][sp].z;
                sum.w += part[m][sp].w;
            }
            v[m][0] = sum.x; v[m][1] = sum.y; v[m][2] = sum.z; v[m][3] = sum.w;
        }
    } else {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            float4 sum = *(const float4 *)(partial + ((size_t)m * P + slot) * R + row4);
            for (uint32_t sp = 1; sp < ks_rt; ++sp) {
                const float4 o = *(const float4 *)(partial + (((size_t)sp * 2 + m) * P + slot) * R + row4);
                sum.x += o.x;
                sum.y += o.y;
                sum.z += o.z;
                sum.w += o.w;
            }
            v[m][0] = sum.x; v[m][1] = sum.y; v[m][2] = sum.z; v[m][3] = sum.w;
        }
    }
    uint16_t hp[3][4];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float gv = v[0][i];
        const float hv = (gv / (1.0f + expf(-gv))) * v[1][i];
        bad |= !finite_f32(hv);
        split3_bf16(hv, hp[0][i], hp[1][i], hp[2][i]);
    }
    const size_t plane = (size_t)P * R;
    uint16_t *dst = hidden + (size_t)slot * R + row4;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
        *(uint2 *)(dst + pl * plane) = make_uint2((uint32_t)hp[pl][0] | ((uint32_t)hp[pl][1] << 16),
                                                  (uint32_t)hp[pl][2] | ((uint32_t)hp[pl][3] << 16));
    if (bad)
        raise_flag(flags, FLAG_SWIGLU_NONFINITE);
}

void launch_moe_a_swiglu(const float *partial, uint32_t ks, uint32_t P, uint32_t I, uint16_t *hidden_planes,
                         uint32_t *flags, hipStream_t stream)
{
    const uint32_t n = P * (I >> 2);
    const dim3 grid((n + 255) / 256), block(256);
#define PW_SWIGLU(KS) hipLaunchKernelGGL((moe_a_swiglu_kernel<KS>), grid, block, 0, stream, partial, ks, P, I, \
                                         hidden_planes, flags)
    switch (ks) {
    case 1: PW_SWIGLU(1); break;
    case 2: PW_SWIGLU(2); break;
    case 4: PW_SWIGLU(4); break;
    case 8: PW_SWIGLU(8); break;
    default: PW_SWIGLU(0); break;
    }
#undef PW_SWIGLU
}

// LDS bytes of a split: NS planes x cnt rows x (KC/8 + 1) 16-byte units.
static size_t split_lds(int ns, uint32_t cnt, uint32_t kc) { return (size_t)ns * cnt * (kc / 8 + 1) * 16; }

SplitPlan plan_split(uint32_t K, int mats, int ns, uint32_t max_cnt)
{
    // widest K split with at most eight 128-column weight blocks per lane (64 VGPRs of weights)
    // whose activation stage fits 64 KB of LDS
    SplitPlan sp{};
    for (uint32_t bpw = 8 / (uint32_t)mats; bpw >= 1; bpw /= 2) {
        const uint32_t kc = bpw * 128;
        if ((K % kc == 0 && split_lds(ns, max_cnt, kc) <= 65536) || bpw == 1) {
            sp.bpw = bpw;
            sp.kc = kc;
            sp.ks = K / kc;
            sp.lds = split_lds(ns, max_cnt, kc);
            return sp;
        }
    }
    return sp;
}

template <int MATS, int NS, int NT>
static void launch_split_nt(const SplitArgs &args, const SplitPlan &sp, uint32_t grid, hipStream_t stream)
{
    switch (sp.bpw) {
    case 8:
        if constexpr (MATS == 1) {
            if (args.job.rows)
                hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 8, true>), dim3(grid + ROUTE_JOB_WGS), dim3(256),
                                   sp.lds, stream, args);
            else
                hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 8>), dim3(grid), dim3(256), sp.lds, stream, args);
            break;
        }
        [[fallthrough]];
    case 4:
        hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 4>), dim3(grid), dim3(256), sp.lds, stream, args);
        break;
    case 2:
        hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 2>), dim3(grid), dim3(256), sp.lds, stream, args);
        break;
    default:
        hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 1>), dim3(grid), dim3(256), sp.lds, stream, args);
        break;
    }
}

void launch_moe_a_split(int mats, int ns, int nt, const SplitArgs &args, const SplitPlan &sp,
                        uint32_t max_active, hipStream_t stream)
{
    const uint32_t grid = max_active * (args.R >> 6) * sp.ks;
    if (mats == 2) {
        if (ns == 3) { if (nt == 2) launch_split_nt<2, 3, 2>(args, sp, grid, stream); else launch_split_nt<2, 3, 1>(args, sp, grid, stream); }
        else { if (nt == 2) launch_split_nt<2, 1, 2>(args, sp, grid, stream); else launch_split_nt<2, 1, 1>(args, sp, grid, stream); }
    } else {
        if (nt == 2) launch_split_nt<1, 3, 2>(args, sp, grid, stream); else launch_split_nt<1, 3, 1>(args, sp, grid, stream);
    }
}

}  // namespace pw
