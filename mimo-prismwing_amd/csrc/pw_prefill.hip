// Routed-expert prefill in mode B: the MoE layer over many token rows as one grouped block-FP8
// GEMM per projection on the FP8 MFMA. The reference runs its layer-major prefill as 128-row
// slices through WideMetalMoeRuntime::execute (run_layer_major_moe_slice_mode,
// src/text_endpoint.rs:4951-5287; src/wide_metal_moe.rs:852-1314); every placement's result
// depends only on its own token row, so one pass over all rows gives the slices' results.
//
// Per projection (block_fp8_gemm{count}_sglang_blockscaled, kernels/block_fp8_gemv.metal:
// 935-1046; CPU equation src/wide_metal_moe.rs:404-421):
//   y[p, r] = sum over 128-column blocks b, ascending, of
//             (sum_{c in b} dec(W[r, c]) * dec(q[p, c])) * S_w[r/128, b] * a[p, b]
// with e4m3 activation codes q and per-(row, block) scales a from the dynamic quantiser. One
// v_mfma_scale_f32_16x16x128_f8f6f4 (unit E8M0 scales) forms each block's FP8 products; the two
// scales are applied in f32, sequentially over b (the same per-block arithmetic as the decode
// mode B kernels).
//
// Tiles: (64 placement slots of one routed expert = an m-tile) x (64 weight rows = an n-tile). A
// workgroup of four waves (16 weight rows each) walks K in 128-column steps, double-buffered: the
// next step's weight bytes (one weight row per lane) and activation codes load into registers
// while the current step runs on the MFMA; the codes then go to the other LDS buffer (16-byte
// units XOR-swizzled by token so the B-operand reads spread over the LDS banks), and a barrier
// that orders LDS only lets the weight prefetch stay in flight. The m-tile's activation scales
// are staged once, transposed ([block][token]).
// Epilogues: gate/up -> bf16-staged SwiGLU (bf16_staged_swiglu, kernels/block_fp8_gemv.metal:
// 139-160) -> hidden as bf16; down -> bf16 expert output (bf16_round_in_place,
// src/wide_metal_moe.rs:1236-1251). Then the combine sums each token's eight outputs.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

constexpr uint32_t PF_MT = 64;      // placement slots per m-tile
constexpr uint32_t PF_UNITS = 8;    // 16-byte units per 128-byte token row of a step

// Tile table: ceil(count / 64) m-tiles per routed expert, ascending expert order. One workgroup of
// 1024 threads, one thread per schedule entry (banks hold at most 1024 experts).
__global__ __launch_bounds__(1024) void prefill_tiles_kernel(const MoePlan *__restrict__ plan,
                                                             const ActiveExpert *__restrict__ active,
                                                             uint32_t max_active, uint2 *__restrict__ tiles,
                                                             uint32_t max_tiles, uint32_t *__restrict__ n_tiles,
                                                             uint32_t *flags)
{
    __shared__ uint32_t s_scan[48];
    const uint32_t a = threadIdx.x;
    const uint32_t n_active = plan->n_active;
    const uint32_t cnt = (a < max_active && a < n_active) ? active[a].cnt : 0u;
    const uint32_t nt = (cnt + PF_MT - 1) / PF_MT;
    uint32_t total;
    const uint32_t off = block_exclusive_scan(nt, s_scan, &total);
    for (uint32_t i = 0; i < nt; ++i)
        if (off + i < max_tiles)
            tiles[off + i] = make_uint2(a, i * PF_MT);
    if (a == 0) {
        n_tiles[0] = total < max_tiles ? total : max_tiles;
        if (total > max_tiles)
            raise_flag(flags, FLAG_SCHEDULE);
    }
}

struct PrefillArgs {
    const ActiveExpert *active;
    const uint2 *tiles;             // [max_tiles] (schedule entry, first slot of the m-tile)
    const uint32_t *n_tiles;
    const uint32_t *placement_pos;  // gate/up: token row of each placement slot
    const uint8_t *codes;           // activation codes [rows][K] (down: rows = placement slots)
    const float *scales;            // activation scales [rows][K / 128]
    uint32_t K, R, rows, max_tiles;
    uint16_t *out;                  // [P][R] bf16: hidden (gate/up) or expert output (down)
    uint32_t *flags;
};

template <int MATS>
struct PfWeights {
    uint4 v[MATS][2];
};

template <int MATS>
__device__ __forceinline__ void pf_load_weights(PfWeights<MATS> &w, const uint8_t *const *wrow, uint32_t k0)
{
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        w.v[m][0] = load_stream16(wrow[m] + k0);
        w.v[m][1] = load_stream16(wrow[m] + k0 + 16);
    }
}

// Activation codes of one step, two 16-byte loads per lane: tokens [8c, 8c + 8) of the m-tile
// for c = 2 * wave + u; lane i holds global unit (i % 8) ^ (token % 8) of token 8c + i / 8 and
// stores it as LDS unit i % 8 of that token (unit index 64c + i: conflict-free writes).
__device__ __forceinline__ void pf_load_codes(uint4 (&c)[2], const uint8_t *const *src, uint32_t k0)
{
#pragma unroll
    for (int u = 0; u < 2; ++u)
        c[u] = load_global16(src[u] + k0);
}

__device__ __forceinline__ void pf_store_codes(uint4 *buf, const uint4 (&c)[2], int wave, int lane)
{
#pragma unroll
    for (int u = 0; u < 2; ++u)
        buf[(2 * wave + u) * 64 + lane] = c[u];
}

// Workgroup barrier ordering LDS accesses only: outstanding global loads (the next step's
// prefetch) stay in flight across it, which __syncthreads() would wait for.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int MATS>
__device__ __forceinline__ void pf_compute(f32x4 (&tot)[MATS][4], const PfWeights<MATS> &w, const uint4 *buf,
                                           const float *lds_scale, const float *lds_wscale, uint32_t blocks,
                                           uint32_t b, int q, int r16)
{
    float sw[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        sw[m] = lds_wscale[m * blocks + b];
    i32x8 A[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
        A[m] = i32x8{(int)w.v[m][0].x, (int)w.v[m][0].y, (int)w.v[m][0].z, (int)w.v[m][0].w,
                     (int)w.v[m][1].x, (int)w.v[m][1].y, (int)w.v[m][1].z, (int)w.v[m][1].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = 16 * j + r16;
        const float sa = lds_scale[b * PF_MT + t];
        const uint4 c0 = buf[t * PF_UNITS + ((2 * q) ^ (t & 7))];
        const uint4 c1 = buf[t * PF_UNITS + ((2 * q + 1) ^ (t & 7))];
        const i32x8 xb = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            const f32x4 p = mfma_fp8_16x16x128(A[m], xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tot[m][j][i] = __builtin_fmaf(p[i] * sw[m], sa, tot[m][j][i]);
        }
    }
}

template <int MATS>
__global__ __launch_bounds__(256) void prefill_b_kernel(const PrefillArgs args)
{
    __shared__ uint4 lds_codes[2][PF_MT * PF_UNITS];  // two 8 KB steps, swizzled
    extern __shared__ float lds_scale[];              // [K / 128][64] activation, then [MATS][K / 128] weight
    constexpr int MAXB = 64;                          // K <= 8192
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const uint32_t mt = blockIdx.x % args.max_tiles, ntile = blockIdx.x / args.max_tiles;
    if (mt >= args.n_tiles[0])
        return;
    const uint2 tl = args.tiles[mt];
    const ActiveExpert ae = args.active[tl.x];
    const uint32_t m0 = tl.y;
    if (m0 >= ae.cnt)
        return;
    const uint32_t cnt_t = ae.cnt - m0 < PF_MT ? ae.cnt - m0 : PF_MT;
    const uint32_t K = args.K, blocks = K >> 7;
    const uint32_t row_base = ntile * 64 + wave * 16;
    const uint32_t slot0 = ae.off + m0;

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
    const uint8_t *wrow[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        wrow[m] = wbase[m] + (size_t)(row_base + r16) * K + q * 32;
        sbase[m] += (row_base >> 7) * blocks;
    }
    // step 0's weights first: their addresses depend only on the schedule entry
    PfWeights<MATS> w0, w1;
    pf_load_weights<MATS>(w0, wrow, 0);

    // activation row of each slot of the m-tile (lane t: slot t). Slots past the tile's count
    // repeat its last slot: in-bounds loads whose output columns are never stored.
    uint32_t tok = slot0 + ((uint32_t)lane < cnt_t ? (uint32_t)lane : cnt_t - 1);
    if constexpr (MATS == 2)
        tok = load_g(args.placement_pos + tok);
    // weight block scales of the workgroup's 64 rows (one 128-row scale block): [m][b]
    float *lds_wscale = lds_scale + blocks * PF_MT;
    const uint32_t m_of = (uint32_t)tid / blocks;
    float wsc = 0.f;
    if ((uint32_t)tid < MATS * blocks)
        wsc = load_g(sbase[m_of < MATS ? m_of : 0] + (tid - m_of * blocks));
    if constexpr (MATS == 2) {
        if (tok >= args.rows) {
            raise_flag(args.flags, FLAG_SCHEDULE);
            tok = args.rows - 1;
        }
    }
    // activation scales of the m-tile, transposed: lds_scale[b * 64 + t] (lane = token); all
    // loads issued before the first LDS write
    float asc[MAXB / 4];
#pragma unroll
    for (int k = 0; k < MAXB / 4; ++k) {
        const uint32_t b = wave + 4 * k;
        asc[k] = b < blocks ? load_g(args.scales + (size_t)tok * blocks + b) : 0.f;
    }
    // per-lane sources of this wave's two code loads per step
    const uint8_t *csrc[2];
    const uint32_t g = ((uint32_t)lane ^ ((uint32_t)lane >> 3)) & 7;  // global unit of LDS unit lane % 8
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint32_t t = 8 * (2 * wave + u) + (lane >> 3);
        const uint32_t row = __shfl(tok, (int)t, 64);
        csrc[u] = args.codes + (size_t)row * K + g * 16;
    }
    uint4 cr[2];
    pf_load_codes(cr, csrc, 0);
    if ((uint32_t)tid < MATS * blocks)
        lds_wscale[tid] = wsc;
#pragma unroll
    for (int k = 0; k < MAXB / 4; ++k) {
        const uint32_t b = wave + 4 * k;
        if (b < blocks)
            lds_scale[b * PF_MT + lane] = asc[k];
    }

    f32x4 tot[MATS][4];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            tot[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    pf_store_codes(lds_codes[0], cr, wave, lane);
    lds_barrier();
    // Step b computes from (w0 | w1, lds_codes[b & 1]) while step b + 1's weights and codes load;
    // the codes go to the other LDS buffer after the compute, then one barrier. The steady-state
    // loop has no branches, so the scheduling barrier keeps the store (and its wait for the
    // prefetched codes) behind the compute; the last one or two steps are peeled.
    uint32_t b = 0;
    for (; b + 2 < blocks; b += 2) {
        pf_load_codes(cr, csrc, (b + 1) << 7);
        pf_load_weights<MATS>(w1, wrow, (b + 1) << 7);
        pf_compute<MATS>(tot, w0, lds_codes[0], lds_scale, lds_wscale, blocks, b, q, r16);
        __builtin_amdgcn_sched_barrier(0);
        pf_store_codes(lds_codes[1], cr, wave, lane);
        lds_barrier();
        pf_load_codes(cr, csrc, (b + 2) << 7);
        pf_load_weights<MATS>(w0, wrow, (b + 2) << 7);
        pf_compute<MATS>(tot, w1, lds_codes[1], lds_scale, lds_wscale, blocks, b + 1, q, r16);
        __builtin_amdgcn_sched_barrier(0);
        pf_store_codes(lds_codes[0], cr, wave, lane);
        lds_barrier();
    }
    if (b + 1 < blocks) {  // two steps left
        pf_load_codes(cr, csrc, (b + 1) << 7);
        pf_load_weights<MATS>(w1, wrow, (b + 1) << 7);
        pf_compute<MATS>(tot, w0, lds_codes[0], lds_scale, lds_wscale, blocks, b, q, r16);
        __builtin_amdgcn_sched_barrier(0);
        pf_store_codes(lds_codes[1], cr, wave, lane);
        lds_barrier();
        pf_compute<MATS>(tot, w1, lds_codes[1], lds_scale, lds_wscale, blocks, b + 1, q, r16);
    } else {  // one step left
        pf_compute<MATS>(tot, w0, lds_codes[0], lds_scale, lds_wscale, blocks, b, q, r16);
    }

    // epilogue: lane holds rows row_base + 4q + i of tokens 16j + r16
    bool bad = false;
    const uint32_t R = args.R;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = 16 * j + r16;
        if (t >= cnt_t)
            continue;
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (MATS == 2) {
                const float gv = round_bf16(tot[0][j][i]);
                const float uv = round_bf16(tot[1][j][i]);
                const float silu = round_bf16(gv / (1.0f + expf(-gv)));
                const float h = round_bf16(silu * uv);
                bad |= !finite_f32(gv) || !finite_f32(uv) || !finite_f32(h);
                o[i] = (uint16_t)(f32_bits(h) >> 16);
            } else {
                o[i] = (uint16_t)(f32_bits(round_bf16(tot[0][j][i])) >> 16);
            }
        }
        *(uint2 *)(args.out + (size_t)(slot0 + t) * R + row_base + 4 * q) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
    }
    if (bad)
        raise_flag(args.flags, FLAG_SWIGLU_NONFINITE);
}

// route_weighted_scatter_add_f32 + final bf16 round over bf16 expert outputs: each token sums
// its eight placements in ascending expert id, out += y * w in f32 (no fused multiply-add).
__global__ __launch_bounds__(256) void prefill_combine_kernel(
    const uint16_t *__restrict__ y, const float *__restrict__ placement_w, const uint32_t *__restrict__ row_slots,
    uint32_t rows, uint32_t H, float *__restrict__ out_f32, uint16_t *__restrict__ out_bf16, uint32_t raw,
    uint32_t *flags)
{
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;  // four values of one token row
    const uint32_t per_row = H >> 2;
    if (idx >= rows * per_row)
        return;
    const uint32_t row = idx / per_row, c4 = idx - row * per_row;
    const uint32_t P = rows * 8;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t slot = row_slots[row * 8 + j];
        slot = slot < P ? slot : 0;
        const float w = placement_w[slot];
        const uint2 v = *(const uint2 *)(y + (size_t)slot * H + c4 * 4);
        const float f[4] = {f32_from(v.x << 16), f32_from(v.x & 0xffff0000u), f32_from(v.y << 16),
                            f32_from(v.y & 0xffff0000u)};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc[i] = __fadd_rn(acc[i], __fmul_rn(f[i], w));
    }
    bool bad = false;
    const size_t at = (size_t)row * H + c4 * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float r = round_bf16(acc[i]);
        bad |= !finite_f32(r);
        if (out_f32)
            out_f32[at + i] = raw ? acc[i] : r;
        if (out_bf16)
            out_bf16[at + i] = (uint16_t)(f32_bits(r) >> 16);
    }
    if (bad)
        raise_flag(flags, FLAG_ROUND_NONFINITE);
}

uint32_t prefill_max_tiles(uint32_t rows, uint32_t E)
{
    const uint32_t P = rows * 8;
    const uint32_t max_active = E < P ? E : P;
    return max_active + (P + PF_MT - 1) / PF_MT;
}

void launch_moe_prefill(const ExpertPtrs *bank, const MoeBuffers &mb, const PrefillBuffers &pb, const void *x,
                        bool x_f32, uint32_t rows, uint32_t E, uint32_t H, uint32_t I, float *out_f32,
                        uint16_t *out_bf16, bool raw, uint32_t *flags, hipStream_t stream)
{
    const uint32_t P = rows * 8;
    const uint32_t max_active = E < P ? E : P;
    const uint32_t max_tiles = prefill_max_tiles(rows, E);
    launch_quant_group128(x, x_f32, rows, H, mb.xq, mb.xs, flags, stream);
    hipLaunchKernelGGL(prefill_tiles_kernel, dim3(1), dim3(1024), 0, stream, mb.plan, mb.active, max_active,
                       pb.tiles, max_tiles, pb.n_tiles, flags);

    PrefillArgs ga{};
    ga.active = mb.active;
    ga.tiles = pb.tiles;
    ga.n_tiles = pb.n_tiles;
    ga.placement_pos = mb.placement_pos;
    ga.codes = mb.xq;
    ga.scales = mb.xs;
    ga.K = H;
    ga.R = I;
    ga.rows = rows;
    ga.max_tiles = max_tiles;
    ga.out = pb.hidden;
    ga.flags = flags;
    int t = timer_begin(K_PREFILL_GATEUP, stream);
    hipLaunchKernelGGL(prefill_b_kernel<2>, dim3(max_tiles * (I / 64)), dim3(256),
                       (size_t)(H / 128) * (PF_MT + 2) * 4, stream, ga);
    timer_end(t, stream);
    // re-quantise the bf16-staged hidden activations per (placement, 128 group)
    launch_quant_group128(pb.hidden, false, P, I, mb.hq, mb.hs, flags, stream);

    PrefillArgs da = ga;
    da.placement_pos = nullptr;
    da.codes = mb.hq;
    da.scales = mb.hs;
    da.K = I;
    da.R = H;
    da.rows = P;
    da.out = pb.y;
    t = timer_begin(K_PREFILL_DOWN, stream);
    hipLaunchKernelGGL(prefill_b_kernel<1>, dim3(max_tiles * (H / 64)), dim3(256),
                       (size_t)(I / 128) * (PF_MT + 1) * 4, stream, da);
    timer_end(t, stream);

    const uint32_t n4 = rows * (H >> 2);
    t = timer_begin(K_MOE_COMBINE, stream);
    hipLaunchKernelGGL(prefill_combine_kernel, dim3((n4 + 255) / 256), dim3(256), 0, stream, pb.y, mb.placement_w,
                       mb.row_slots, rows, H, out_f32, out_bf16, raw ? 1u : 0u, flags);
    timer_end(t, stream);
}

}  // namespace pw
