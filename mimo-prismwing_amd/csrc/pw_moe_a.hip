// Mode A routed-expert projections (FP8 weight x bf16 / exact-f32 activation, f32 accumulation)
// for the decode MoE layer: gate+up with SwiGLU, and down.
//
// Reference semantics: the f32 CPU control of the reference's MoE block (src/lib.rs:5807-5862):
// gate = x W_g^T, up = x W_u^T, h = (g / (1 + e^-g)) * u, y = h W_d^T, all f32; kernels
// block_fp8_gemm{1..8}_shared_weight_lut_blocked and swiglu_f32 (kernels/block_fp8_gemv.metal:
// 241-252, 751-933).
//
// Work item: (routed expert, 64 weight rows, one K split of KC columns). A workgroup of four
// waves reads each of its 64 rows x KC bytes exactly once: every lane issues all of its weight
// loads (16 bytes per instruction, one row per lane, global nontemporal loads) before anything
// else, so each wave keeps up to 32 KB in flight. The expert's routed activation rows for the K
// split are staged once in LDS (padded rows, conflict-free 16-byte reads) and shared by the four
// waves. e4m3 -> bf16 is exact (v_cvt_scalef32_pk_bf16_fp8); activations are bf16 planes (f32
// values arrive as three exact planes), so v_mfma_f32_16x16x32_bf16 forms exact products and
// accumulates in f32. The 128x128 block scale multiplies each block partial in registers.
// Split-K partials go to a global buffer; the last workgroup of a tile to finish (acquire/release
// counter) sums them in split order 0..KS-1 -- deterministic -- and runs the epilogue: SwiGLU
// (written as three exact bf16 planes for the down projection) or the expert output row.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

template <int MATS, int NS, int NT, int BPW>
__global__ __launch_bounds__(256) void moe_a_split_kernel(const SplitArgs args)
{
    extern __shared__ uint4 lds_x[];  // [NS * cnt][KC/8 + 1]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar scale loads
    const int q = lane >> 4, r16 = lane & 15;
    const uint32_t G = args.R >> 6;
    const uint32_t s = blockIdx.x % args.KS;
    const uint32_t g = (blockIdx.x / args.KS) % G;
    const uint32_t a = blockIdx.x / (args.KS * G);
    const ActiveExpert ae = args.active[a];
    if (ae.cnt == 0)
        return;
    if (ae.cnt > 16u * NT) {
        if (tid == 0)
            raise_flag(args.flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t K = args.K, KC = BPW * 128;
    const uint32_t k0 = s * KC;
    const uint32_t row_base = g * 64 + wave * 16;  // this wave's 16 rows
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

    // 0. source rows of the activation units this thread stages (issued before the weights, so
    //    the staging loads below never wait behind the weight stream)
    const uint32_t per_row = KC >> 3, stride = per_row + 1;
    const uint32_t units = NS * ae.cnt * per_row;
    constexpr int UMAX = NS * NT * 16 * BPW * 16 / 256;
    uint32_t srcrow[UMAX];
#pragma unroll
    for (int k = 0; k < UMAX; ++k) {
        const uint32_t u = tid + k * 256;
        uint32_t src = ae.off + (u / per_row) % ae.cnt;
        if (u < units && args.placement_pos) {
            src = args.placement_pos[src];
            src = src < args.rows ? src : args.rows - 1;
        }
        srcrow[k] = src;
    }

    // 1. every weight byte of this wave's rows and K split, in flight at once
    uint4 wv[MATS][BPW][2];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        const uint8_t *wrow = wbase[m] + (size_t)(row_base + r16) * K + k0 + q * 16;
#pragma unroll
        for (int j = 0; j < BPW; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wv[m][j][h] = load_stream16(wrow + j * 128 + h * 64);
    }

    // block scales of this wave's 16 rows (one 128-row scale block), scalar loads
    const uint32_t blocks = K >> 7;
    const uint32_t srow = row_base >> 7;
    float sc[MATS][BPW];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < BPW; ++j)
            sc[m][j] = sbase[m][srow * blocks + (k0 >> 7) + j];

    // 2. stage the routed activation rows of this K split in LDS: [plane][token][KC/8 + 1]
    uint4 xv[UMAX];
#pragma unroll
    for (int k = 0; k < UMAX; ++k) {
        const uint32_t u = tid + k * 256;
        if (u < units) {
            const uint32_t c = u % per_row, p = u / (per_row * ae.cnt);
            xv[k] = load_global16(args.x + p * args.x_plane + (size_t)srcrow[k] * K + k0 + c * 8);
        }
    }
#pragma unroll
    for (int k = 0; k < UMAX; ++k) {
        const uint32_t u = tid + k * 256;
        if (u < units) {
            const uint32_t c = u % per_row, rowi = u / per_row;  // rowi = p * cnt + t
            lds_x[rowi * stride + c] = xv[k];
        }
    }
    __syncthreads();

    // 3. block partials on the MFMA, block scale in registers
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
            const uint32_t cu = j * 16 + h * 8 + q * 2;  // column in uint4 units
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t t = nt * 16 + r16;
                const bool ok = t < ae.cnt;
#pragma unroll
                for (int p = 0; p < NS; ++p) {
                    uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                    if (ok) {
                        const uint4 *xp = lds_x + (p * ae.cnt + t) * stride + cu;
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

    // 4. split-K partials: partial[s][m][slot][row]
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
    __threadfence();
    __syncthreads();
    __shared__ uint32_t s_last;
    if (tid == 0) {
        uint32_t *ctr = args.counters + a * G + g;
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == args.KS - 1;
        if (s_last)
            __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last)
        return;
    __threadfence();

    // 5. epilogue by the last workgroup: sum the splits in order, then SwiGLU or the output row
    bool bad = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = nt * 16 + r16;
        if (t >= ae.cnt)
            continue;
        const uint32_t slot = ae.off + t;
        float v[MATS][4];
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            const uint4 first = load_global16(args.partial + ((size_t)m * P + slot) * R + row4);
            float4 sum = make_float4(f32_from(first.x), f32_from(first.y), f32_from(first.z), f32_from(first.w));
            for (uint32_t sp = 1; sp < args.KS; ++sp) {
                const uint4 o = load_global16(args.partial + (((size_t)sp * MATS + m) * P + slot) * R + row4);
                sum.x += f32_from(o.x);
                sum.y += f32_from(o.y);
                sum.z += f32_from(o.z);
                sum.w += f32_from(o.w);
            }
            v[m][0] = sum.x; v[m][1] = sum.y; v[m][2] = sum.z; v[m][3] = sum.w;
        }
        if constexpr (MATS == 2) {
            uint16_t hp[3][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gv = v[0][i];
                const float hv = (gv / (1.0f + expf(-gv))) * v[1][i];
                bad |= !finite_f32(hv);
                split3_bf16(hv, hp[0][i], hp[1][i], hp[2][i]);
            }
            uint16_t *dst = args.hidden + (size_t)slot * R + row4;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                *(uint2 *)(dst + pl * args.h_plane) =
                    make_uint2((uint32_t)hp[pl][0] | ((uint32_t)hp[pl][1] << 16),
                               (uint32_t)hp[pl][2] | ((uint32_t)hp[pl][3] << 16));
        } else {
            *(float4 *)(args.y + (size_t)slot * R + row4) = make_float4(v[0][0], v[0][1], v[0][2], v[0][3]);
        }
    }
    if (bad)
        raise_flag(args.flags, FLAG_SWIGLU_NONFINITE);
}

// LDS bytes of a split: NS planes x cnt rows x (KC/8 + 1) 16-byte units.
static size_t split_lds(int ns, uint32_t cnt, uint32_t kc) { return (size_t)ns * cnt * (kc / 8 + 1) * 16; }

SplitPlan plan_split(uint32_t K, int ns, uint32_t max_cnt)
{
    // widest K split whose activation stage fits 64 KB of LDS, at most 8 blocks per lane
    SplitPlan sp{};
    for (uint32_t bpw = 8; bpw >= 2; bpw /= 2) {
        const uint32_t kc = bpw * 128;
        if (K % kc == 0 && split_lds(ns, max_cnt, kc) <= 65536) {
            sp.bpw = bpw;
            sp.kc = kc;
            sp.ks = K / kc;
            sp.lds = split_lds(ns, max_cnt, kc);
            return sp;
        }
    }
    sp.bpw = 1;
    sp.kc = 128;
    sp.ks = K / 128;
    sp.lds = split_lds(ns, max_cnt, 128);
    return sp;
}

template <int MATS, int NS, int NT>
static void launch_split_nt(const SplitArgs &args, const SplitPlan &sp, uint32_t grid, hipStream_t stream)
{
    switch (sp.bpw) {
    case 8:
        hipLaunchKernelGGL((moe_a_split_kernel<MATS, NS, NT, 8>), dim3(grid), dim3(256), sp.lds, stream, args);
        break;
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
