// Block-scaled FP8 projections for decode widths (1..32 activation rows) on gfx950.
//
// Mode A (FP8 weight x f32/bf16 activation, f32 accumulation) follows the reference's
// block_fp8_gemv_parallel_lut_blocked / block_fp8_gemm{1..8}_shared_weight_lut_blocked
// (kernels/block_fp8_gemv.metal:665-703, :751-800, :855-933) and its CPU twin mapped_fp8_gemv
// (src/lib.rs:1272-1309). Mode B (dynamic FP8 activation, block-scaled) follows
// block_fp8_gemm{1..32}_sglang_blockscaled (kernels/block_fp8_gemv.metal:935-1046).
//
// Design: a 64-lane wave owns a 16-row output tile. Each lane streams 16 (mode A) or 32 (mode B)
// weight bytes of one row per instruction, so one wave-load covers 16 rows x 64 (128) contiguous
// bytes. Mode A converts e4m3 to bf16 exactly (v_cvt_scalef32_pk_bf16_fp8) and feeds
// v_mfma_f32_16x16x32_bf16 with the activation rows as the 16-wide N operand; f32 activations
// are split once into three bf16 planes (hi + mid + lo == x exactly), so every product is exact
// and only the f32 accumulation order differs from the reference. Mode B feeds
// the e4m3 codes of weights and activations straight into v_mfma_scale_f32_16x16x128_f8f6f4:
// one instruction is one 128-column scale block. The 128x128 block scale (and in mode B the
// per-token activation scale) is applied to the f32 block partial in registers. The waves of a
// workgroup split K and are reduced through LDS in a fixed order, so results are deterministic.
// Decode widths are HBM-bound; MFMA is used because f32 VALU FMA (no packed math) cannot reach
// 8 TB/s x 8 rows x 2 FLOP/B.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

template <int NT>
struct Acc {
    f32x4 v[NT];
};

// ------------------------------------------------------------------------------------ mode A
// Activations arrive as NS bf16 planes [NS][W][K] (NS = 1: bf16 input; NS = 3: an f32 input split
// exactly into hi + mid + lo), so the inner loop does no conversion work on them.
// STAGE: each wave first copies its round's activation columns of the W rows into its own LDS region
// with direct-to-LDS loads (no registers), then issues its weight loads; those copies are the oldest
// loads in the in-order memory counter, so block j's MFMAs start when block j's weights arrive. The
// unstaged form reads the activations from global memory inside the MFMA loop, after every weight
// load of the round, so each round's first MFMA also waits for those reads.
// XF32 (staged, NS = 3, one row): the row arrives as f32 (xf) instead of planes; each lane loads
// its 8-column units of the wave's columns before the weights and, once the weights are issued,
// splits them into the three planes in the wave's LDS region (no separate split launch).
template <int NS, int KSPLIT, int NT, int BPW, bool STAGE, bool XF32 = false>
__global__ __launch_bounds__(64 * KSPLIT) void linear_a_kernel(
    const ProjTile *__restrict__ tiles, uint32_t n_tiles, const uint16_t *__restrict__ x, uint32_t W,
    uint32_t K, float *__restrict__ y_f32, uint16_t *__restrict__ y_bf16, uint32_t N,
    uint32_t round_f32, const float *__restrict__ xf)
{
    static_assert(!XF32 || (STAGE && NS == 3 && NT == 1), "f32 rows are split while staging");
    const size_t plane = (size_t)W * K;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    __shared__ f32x4 red[KSPLIT > 1 ? KSPLIT : 1][NT][64];
    extern __shared__ uint4 lds_xa[];  // STAGE: per wave [NS][W][ROW] 16-byte units
    constexpr uint32_t UNITS = BPW * 16, ROW = UNITS + 1;  // a row's units per round (+1: bank spread)
    uint4 *xs = lds_xa + (size_t)wave * NS * W * ROW;
    const uint32_t blocks = K >> 7;

    for (uint32_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        const ProjTile tile = tiles[t];
        const bool row_ok = (uint32_t)r16 < tile.valid;
        const uint8_t *wrow = tile.w + (size_t)r16 * K + q * 16;
        f32x4 total[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            total[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // K in rounds of KSPLIT * BPW blocks (one round whenever K <= 128 * KSPLIT * BPW): wave w
        // takes blocks [round + w * BPW, round + (w + 1) * BPW), and issues every weight load and
        // block scale of them before its first MFMA
        for (uint32_t round = 0; round < blocks; round += KSPLIT * BPW) {
            const uint32_t b0 = round + (uint32_t)wave * BPW;
            // whole rounds: this wave issues exactly 2 BPW weight loads after its copies
            const bool whole = b0 + BPW <= blocks;
            // the wave's columns [128 b0, 128 (b0 + BPW)) of every activation row (whole blocks
            // only; a partial round copies the blocks it has)
            const uint32_t units = (b0 < blocks ? (blocks - b0 < (uint32_t)BPW ? blocks - b0 : BPW) : 0) * 16;
            constexpr uint32_t XU = XF32 ? (UNITS + 63) / 64 : 1;  // XF32: f32 units per lane
            float4 xr[XU][2];
            if constexpr (XF32) {
                if (units) {
#pragma unroll
                    for (uint32_t i = 0; i < XU; ++i) {
                        const uint32_t u = (uint32_t)lane + 64 * i, uc = u < units ? u : units - 1;
                        const float *src = xf + ((size_t)b0 << 7) + uc * 8;
                        xr[i][0] = *(const float4 *)src;
                        xr[i][1] = *(const float4 *)(src + 4);
                    }
                }
            } else if constexpr (STAGE) {
                for (uint32_t s = 0; s < (uint32_t)NS; ++s)
                    for (uint32_t t = 0; t < W; ++t)
                        for (uint32_t u0 = 0; u0 < units; u0 += 64)
                            if (u0 + (uint32_t)lane < units)
                                lds_load16(x + s * plane + (size_t)t * K + ((size_t)b0 << 7) + (u0 + lane) * 8,
                                           xs + (s * W + t) * ROW + u0);
                asm volatile("" ::: "memory");  // the copies stay the oldest memory operations
            }
            uint4 wv[BPW][2];
            float sc[BPW];
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                const uint32_t b = b0 + j;
                wv[j][0] = make_uint4(0, 0, 0, 0);
                wv[j][1] = wv[j][0];
                sc[j] = 0.f;
                if (b < blocks) {
                    if (row_ok) {
                        wv[j][0] = load_global16(wrow + ((size_t)b << 7));
                        wv[j][1] = load_global16(wrow + ((size_t)b << 7) + 64);
                    }
                    sc[j] = tile.s[b];
                }
            }
            if constexpr (XF32) {
                // the row's units split into the planes of the wave's region (plane p at p * ROW)
                if (units) {
#pragma unroll
                    for (uint32_t i = 0; i < XU; ++i) {
                        const uint32_t u = (uint32_t)lane + 64 * i;
                        if (u < units) {
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
                            for (uint32_t pl = 0; pl < 3; ++pl)
                                xs[pl * ROW + u] = make_uint4(pk[pl][0], pk[pl][1], pk[pl][2], pk[pl][3]);
                        }
                    }
                }
            } else if constexpr (STAGE) {
                // every load but this wave's youngest 2 BPW weight loads: its copies have landed
                if (whole)
                    wait_vmcnt<2 * BPW>();
                else
                    wait_vmcnt<0>();
            }
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                const uint32_t b = b0 + j;
                if (b >= blocks)
                    break;
                f32x4 acc[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t col = (b << 7) + half * 64 + q * 16;
                    const bf16x8 a0 = fp8x8_to_bf16x8(wv[j][half].x, wv[j][half].y);
                    const bf16x8 a1 = fp8x8_to_bf16x8(wv[j][half].z, wv[j][half].w);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const uint32_t token = nt * 16 + r16;
#pragma unroll
                        for (int s = 0; s < NS; ++s) {
                            uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                            if (token < W) {
                                if constexpr (STAGE) {
                                    const uint4 *xp = xs + (s * W + token) * ROW + j * 16 + half * 8 + q * 2;
                                    x0 = xp[0];
                                    x1 = xp[1];
                                } else {
                                    const uint4 *xp = (const uint4 *)(x + s * plane + (size_t)token * K + col);
                                    x0 = xp[0];
                                    x1 = xp[1];
                                }
                            }
                            acc[nt] = mfma_bf16_16x16x32(a0, bf16x8_from_u4(x0), acc[nt]);
                            acc[nt] = mfma_bf16_16x16x32(a1, bf16x8_from_u4(x1), acc[nt]);
                        }
                    }
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        total[nt][i] = __builtin_fmaf(sc[j], acc[nt][i], total[nt][i]);
            }
            if constexpr (STAGE)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next copies
        }

        if constexpr (KSPLIT > 1) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                red[wave][nt][lane] = total[nt];
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    f32x4 s = red[0][nt][lane];
                    for (int w = 1; w < KSPLIT; ++w) {
                        const f32x4 o = red[w][nt][lane];
                        s[0] += o[0]; s[1] += o[1]; s[2] += o[2]; s[3] += o[3];
                    }
                    total[nt] = s;
                }
            }
        }
        if (wave == 0) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t token = nt * 16 + r16;
                if (token >= W)
                    continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t row = q * 4 + i;
                    if (row >= tile.valid)
                        continue;
                    const size_t at = (size_t)token * N + tile.out_row + row;
                    const float v = total[nt][i];
                    if (y_f32)
                        y_f32[at] = round_f32 ? round_bf16(v) : v;
                    if (y_bf16)
                        y_bf16[at] = bf16_bits(v);
                }
            }
        }
        if constexpr (KSPLIT > 1)
            __syncthreads();
    }
}

// Two 16-row tiles per workgroup for the staged form of wider batches (up to 8 activation rows):
// eight waves split K (BPW = 4 blocks each), every wave loads the weights of both tiles for its
// split and reads each activation unit from LDS once for both, so a copied activation row feeds
// twice the weight rows of linear_a_kernel's 16-row workgroups (whose eight-row copies cost L2
// requests equal to the weights' own) and the grid halves. The split partials meet in LDS (over
// the stage, after every wave is done with it) and are added in split order 0..7.
template <int NS>
__global__ __launch_bounds__(512) void linear_a_pair_kernel(
    const ProjTile *__restrict__ tiles, uint32_t n_tiles, const uint16_t *__restrict__ x, uint32_t W,
    uint32_t K, float *__restrict__ y_f32, uint16_t *__restrict__ y_bf16, uint32_t N, uint32_t round_f32)
{
    constexpr int KSPLIT = 8, BPW = 4, RT = 2;  // the epilogue's tile selects assume RT = 2
    const size_t plane = (size_t)W * K;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    extern __shared__ uint4 lds_xa[];  // per wave [NS][W][ROW] 16-byte units; then [KSPLIT][RT][64] f32x4
    constexpr uint32_t UNITS = BPW * 16, ROW = UNITS + 1;
    uint4 *xs = lds_xa + (size_t)wave * NS * W * ROW;
    const uint32_t blocks = K >> 7;

    for (uint32_t pr = blockIdx.x; pr * RT < n_tiles; pr += gridDim.x) {
        ProjTile tile[RT];
        bool live[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t t = pr * RT + r;
            live[r] = t < n_tiles;
            tile[r] = tiles[live[r] ? t : n_tiles - 1];
        }
        f32x4 total[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r)
            total[r] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t round = 0; round < blocks; round += KSPLIT * BPW) {
            const uint32_t b0 = round + (uint32_t)wave * BPW;
            const bool whole = b0 + BPW <= blocks;
            // this wave's columns of every activation row -> its LDS region (as linear_a_kernel)
            const uint32_t units = (b0 < blocks ? (blocks - b0 < (uint32_t)BPW ? blocks - b0 : BPW) : 0) * 16;
            for (uint32_t sp = 0; sp < (uint32_t)NS; ++sp)
                for (uint32_t t = 0; t < W; ++t)
                    for (uint32_t u0 = 0; u0 < units; u0 += 64)
                        if (u0 + (uint32_t)lane < units)
                            lds_load16(x + sp * plane + (size_t)t * K + ((size_t)b0 << 7) + (u0 + lane) * 8,
                                       xs + (sp * W + t) * ROW + u0);
            asm volatile("" ::: "memory");  // the copies stay the oldest memory operations
            uint4 wv[RT][BPW][2];
            float sc[RT][BPW];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const bool row_ok = live[r] && (uint32_t)r16 < tile[r].valid;
                const uint8_t *wrow = tile[r].w + (size_t)r16 * K + q * 16;
#pragma unroll
                for (int j = 0; j < BPW; ++j) {
                    const uint32_t b = b0 + j;
                    wv[r][j][0] = make_uint4(0, 0, 0, 0);
                    wv[r][j][1] = wv[r][j][0];
                    sc[r][j] = 0.f;
                    if (b < blocks) {
                        if (row_ok) {
                            wv[r][j][0] = load_global16(wrow + ((size_t)b << 7));
                            wv[r][j][1] = load_global16(wrow + ((size_t)b << 7) + 64);
                        }
                        sc[r][j] = tile[r].s[b];
                    }
                }
            }
            // every load but this wave's youngest 2 RT BPW weight loads: its copies have landed
            if (whole)
                wait_vmcnt<2 * RT * BPW>();
            else
                wait_vmcnt<0>();
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                const uint32_t b = b0 + j;
                if (b >= blocks)
                    break;
                f32x4 acc[RT];
#pragma unroll
                for (int r = 0; r < RT; ++r)
                    acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    bf16x8 a[RT][2];
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
                        a[r][0] = fp8x8_to_bf16x8(wv[r][j][half].x, wv[r][j][half].y);
                        a[r][1] = fp8x8_to_bf16x8(wv[r][j][half].z, wv[r][j][half].w);
                    }
#pragma unroll
                    for (int sp = 0; sp < NS; ++sp) {
                        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
                        if ((uint32_t)r16 < W) {
                            const uint4 *xp = xs + (sp * W + r16) * ROW + j * 16 + half * 8 + q * 2;
                            x0 = xp[0];
                            x1 = xp[1];
                        }
#pragma unroll
                        for (int r = 0; r < RT; ++r) {
                            acc[r] = mfma_bf16_16x16x32(a[r][0], bf16x8_from_u4(x0), acc[r]);
                            acc[r] = mfma_bf16_16x16x32(a[r][1], bf16x8_from_u4(x1), acc[r]);
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < RT; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        total[r][i] = __builtin_fmaf(sc[r][j], acc[r][i], total[r][i]);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next copies
        }
        // split partials in LDS over the stage (every wave is past its reads), summed in split order
        __syncthreads();
        f32x4 *red = (f32x4 *)lds_xa;
#pragma unroll
        for (int r = 0; r < RT; ++r)
            red[(wave * RT + r) * 64 + lane] = total[r];
        __syncthreads();
        const bool mine = wave == 0 ? live[0] : live[1];  // waves 0 and 1 write tiles 0 and 1
        if (wave < RT && mine) {
            f32x4 sum = red[wave * 64 + lane];
#pragma unroll
            for (int w = 1; w < KSPLIT; ++w) {
                const f32x4 o = red[(w * RT + wave) * 64 + lane];
                sum[0] += o[0];
                sum[1] += o[1];
                sum[2] += o[2];
                sum[3] += o[3];
            }
            const ProjTile tl = wave == 0 ? tile[0] : tile[1];
            if ((uint32_t)r16 < W) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t row = q * 4 + i;
                    if (row >= tl.valid)
                        continue;
                    const size_t at = (size_t)r16 * N + tl.out_row + row;
                    const float v = sum[i];
                    if (y_f32)
                        y_f32[at] = round_f32 ? round_bf16(v) : v;
                    if (y_bf16)
                        y_bf16[at] = bf16_bits(v);
                }
            }
        }
        __syncthreads();  // the partials are read before the next pair's copies overwrite them
    }
}

// ------------------------------------------------------------------------------------ mode B
template <int KSPLIT, int NT, int BPW>
__global__ __launch_bounds__(64 * KSPLIT) void linear_b_kernel(
    const ProjTile *__restrict__ tiles, uint32_t n_tiles, const uint8_t *__restrict__ codes,
    const float *__restrict__ act_scales, uint32_t W, uint32_t K, float *__restrict__ y_f32,
    uint16_t *__restrict__ y_bf16, uint32_t N, uint32_t round_f32)
{
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    __shared__ f32x4 red[KSPLIT > 1 ? KSPLIT : 1][NT][64];
    const uint32_t blocks = K >> 7;

    for (uint32_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        const ProjTile tile = tiles[t];
        const bool row_ok = (uint32_t)r16 < tile.valid;
        const uint8_t *wrow = tile.w + (size_t)r16 * K + q * 32;
        f32x4 total[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            total[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // K in rounds of KSPLIT * BPW blocks, every weight load of a wave's blocks issued first
        // (as in linear_a_kernel)
        for (uint32_t round = 0; round < blocks; round += KSPLIT * BPW) {
            const uint32_t b0 = round + (uint32_t)wave * BPW;
            uint4 wv[BPW][2];
            float sw[BPW];
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                const uint32_t b = b0 + j;
                wv[j][0] = make_uint4(0, 0, 0, 0);
                wv[j][1] = wv[j][0];
                sw[j] = 0.f;
                if (b < blocks) {
                    if (row_ok) {
                        wv[j][0] = load_global16(wrow + ((size_t)b << 7));
                        wv[j][1] = load_global16(wrow + ((size_t)b << 7) + 16);
                    }
                    sw[j] = tile.s[b];
                }
            }
#pragma unroll
            for (int j = 0; j < BPW; ++j) {
                const uint32_t b = b0 + j;
                if (b >= blocks)
                    break;
                const uint32_t col = (b << 7) + q * 32;
                const i32x8 wa = {(int)wv[j][0].x, (int)wv[j][0].y, (int)wv[j][0].z, (int)wv[j][0].w,
                                  (int)wv[j][1].x, (int)wv[j][1].y, (int)wv[j][1].z, (int)wv[j][1].w};
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const uint32_t token = nt * 16 + r16;
                    uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
                    float sa = 0.f;
                    if (token < W) {
                        const uint4 *cp = (const uint4 *)(codes + (size_t)token * K + col);
                        c0 = cp[0];
                        c1 = cp[1];
                        sa = act_scales[(size_t)token * blocks + b];
                    }
                    const i32x8 xb = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w,
                                      (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
                    const f32x4 p = mfma_fp8_16x16x128(wa, xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        total[nt][i] = __builtin_fmaf(p[i] * sw[j], sa, total[nt][i]);
                }
            }
        }
        if constexpr (KSPLIT > 1) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                red[wave][nt][lane] = total[nt];
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    f32x4 s = red[0][nt][lane];
                    for (int w = 1; w < KSPLIT; ++w) {
                        const f32x4 o = red[w][nt][lane];
                        s[0] += o[0]; s[1] += o[1]; s[2] += o[2]; s[3] += o[3];
                    }
                    total[nt] = s;
                }
            }
        }
        if (wave == 0) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t token = nt * 16 + r16;
                if (token >= W)
                    continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t row = q * 4 + i;
                    if (row >= tile.valid)
                        continue;
                    const size_t at = (size_t)token * N + tile.out_row + row;
                    const float v = total[nt][i];
                    if (y_f32)
                        y_f32[at] = round_f32 ? round_bf16(v) : v;
                    if (y_bf16)
                        y_bf16[at] = bf16_bits(v);
                }
            }
        }
        if constexpr (KSPLIT > 1)
            __syncthreads();
    }
}

// ------------------------------------------------------------------ dynamic FP8 quantiser
// dynamic_fp8_quantized_group128 (kernels/block_fp8_gemv.metal:84-137) and its CPU authority
// dynamic_fp8_activations (src/text_endpoint.rs:3008-3051): scale = max(absmax, 1e-10) / 448;
// code = nearest e4m3 of clamp(x/scale). A non-finite input raises FLAG_QUANT_NONFINITE and
// counts as 0 in the group maximum.
// One 128-column group per 16 lanes, 16 groups per 256-thread workgroup (quant_group128_team).
template <typename T>
__global__ __launch_bounds__(256) void quant_group128_kernel(const T *__restrict__ x, uint32_t rows,
                                                             uint32_t K, uint8_t *__restrict__ codes,
                                                             float *__restrict__ scales,
                                                             uint32_t *flags)
{
    const uint32_t group = blockIdx.x * 16 + (threadIdx.x >> 4);
    if (group < rows * (K >> 7))  // whole 16-lane groups leave together
        quant_group128_team<T>(x, group, threadIdx.x & 15, codes, scales, flags);
}

// f32 [n] -> bf16 planes hi [n], mid [n], lo [n] with x == hi + mid + lo.
__global__ __launch_bounds__(256) void split_planes_kernel(const float *__restrict__ x, uint32_t n,
                                                           uint16_t *__restrict__ planes)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    uint16_t h, m, l;
    split3_bf16(x[i], h, m, l);
    planes[i] = h;
    planes[n + i] = m;
    planes[2 * (size_t)n + i] = l;
}

// ------------------------------------------------------------------------------- launchers
static int grid_for(uint32_t n_tiles, uint32_t max_grid)
{
    return (int)(n_tiles < max_grid ? n_tiles : max_grid);
}

void launch_split_planes(const float *x, uint32_t n, uint16_t *planes, hipStream_t stream)
{
    hipLaunchKernelGGL(split_planes_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, n, planes);
}

// K split of a 16-row tile: KSPLIT waves x BPW 128-column blocks per wave, every weight byte of a
// wave requested before its first MFMA. KSPLIT grows until the launch has about eight waves per
// CU (2048 on 256 CUs) and until eight blocks per wave cover K in one round; a wave keeps at least
// one block. At most 16 waves (8 for batches of more than 16 rows, whose two token tiles need more
// than the 128 registers a 1024-thread workgroup leaves).
struct LinearSplit {
    int ks, bpw;
};

static LinearSplit pick_split(uint32_t blocks, uint32_t W, uint32_t n_tiles)
{
    const uint32_t max_ks = W <= 16 ? 16u : 8u;
    uint32_t ks = 1;
    while (ks < max_ks && ((uint64_t)ks * n_tiles < 2048 || ks * 8 < blocks))
        ks *= 2;
    while (ks > 1 && ks / 2 >= blocks)
        ks /= 2;
    uint32_t bpw = 1;
    while (ks * bpw < blocks && bpw < 8)
        bpw *= 2;
    return LinearSplit{(int)ks, (int)bpw};
}

// LDS of the staged form: KSPLIT waves x NS planes x W rows x (16 BPW + 1) 16-byte units.
static size_t staged_lds(int ns, int ksplit, int bpw, uint32_t W)
{
    return (size_t)ksplit * ns * W * (16 * bpw + 1) * 16;
}

// The staged form takes batches of up to 8 rows whose activations fit 80 KB of LDS per workgroup
// (eight rows of a 4096-column projection at four waves: 66 KB, two workgroups per CU).
constexpr size_t LINEAR_STAGE_LDS = 80 * 1024;

template <int NS, int KSPLIT, int BPW>
static void launch_a_split(const ProjTile *tiles, uint32_t n_tiles, const uint16_t *x, uint32_t W, uint32_t K,
                           float *y32, uint16_t *y16, uint32_t N, uint32_t round_f32, hipStream_t stream)
{
    const int grid = grid_for(n_tiles, 65535);
    const size_t lds = staged_lds(NS, KSPLIT, BPW, W);
    if (W <= 8 && lds + sizeof(f32x4) * KSPLIT * 64 <= LINEAR_STAGE_LDS) {
        if (lds > 48 * 1024)
            (void)hipFuncSetAttribute((const void *)linear_a_kernel<NS, KSPLIT, 1, BPW, true>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL((linear_a_kernel<NS, KSPLIT, 1, BPW, true>), dim3(grid), dim3(64 * KSPLIT), lds, stream,
                           tiles, n_tiles, x, W, K, y32, y16, N, round_f32, nullptr);
    }
    else if (KSPLIT == 16 || W <= 16)
        hipLaunchKernelGGL((linear_a_kernel<NS, KSPLIT, 1, BPW, false>), dim3(grid), dim3(64 * KSPLIT), 0, stream,
                           tiles, n_tiles, x, W, K, y32, y16, N, round_f32, nullptr);
    else if constexpr (KSPLIT < 16)
        hipLaunchKernelGGL((linear_a_kernel<NS, KSPLIT, 2, BPW, false>), dim3(grid), dim3(64 * KSPLIT), 0, stream,
                           tiles, n_tiles, x, W, K, y32, y16, N, round_f32, nullptr);
}

template <int NS>
static void launch_a_planes(const ProjTile *tiles, uint32_t n_tiles, const uint16_t *x, uint32_t W, uint32_t K,
                            float *y32, uint16_t *y16, uint32_t N, uint32_t round_f32, hipStream_t stream)
{
    // batches of 4..8 rows over many tiles: two tiles per staged workgroup (linear_a_pair_kernel),
    // when eight splits of four blocks cover K in whole rounds and the stage fits
    const size_t pair_lds = staged_lds(NS, 8, 4, W);
    if (W >= 4 && W <= 8 && n_tiles >= 512 && (K >> 7) % 32 == 0 && pair_lds <= LINEAR_STAGE_LDS &&
        pair_lds >= (size_t)8 * 2 * 64 * 16) {
        if (pair_lds > 48 * 1024)
            (void)hipFuncSetAttribute((const void *)linear_a_pair_kernel<NS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)pair_lds);
        const uint32_t pairs = (n_tiles + 1) / 2;
        hipLaunchKernelGGL((linear_a_pair_kernel<NS>), dim3(grid_for(pairs, 65535)), dim3(512), pair_lds, stream, tiles,
                           n_tiles, x, W, K, y32, y16, N, round_f32);
        return;
    }
    const LinearSplit sp = pick_split(K >> 7, W, n_tiles);
#define PW_A(KS, BPW) launch_a_split<NS, KS, BPW>(tiles, n_tiles, x, W, K, y32, y16, N, round_f32, stream)
#define PW_A_BPW(KS)                                                                                       \
    do {                                                                                                   \
        if (sp.bpw == 8) PW_A(KS, 8); else if (sp.bpw == 4) PW_A(KS, 4); else if (sp.bpw == 2) PW_A(KS, 2); \
        else PW_A(KS, 1);                                                                                  \
    } while (0)
    if (sp.ks == 16) PW_A_BPW(16); else if (sp.ks == 8) PW_A_BPW(8); else if (sp.ks == 4) PW_A_BPW(4);
    else if (sp.ks == 2) PW_A_BPW(2); else PW_A_BPW(1);
#undef PW_A_BPW
#undef PW_A
}

void launch_linear_a(const ProjTile *tiles, uint32_t n_tiles, const uint16_t *x, int planes,
                     uint32_t W, uint32_t K, float *y32, uint16_t *y16, uint32_t N,
                     uint32_t round_f32, hipStream_t stream)
{
    const int t = timer_begin(K_LINEAR_A, stream);
    if (planes == 3)
        launch_a_planes<3>(tiles, n_tiles, x, W, K, y32, y16, N, round_f32, stream);
    else
        launch_a_planes<1>(tiles, n_tiles, x, W, K, y32, y16, N, round_f32, stream);
    timer_end(t, stream);
}

template <int KSPLIT, int BPW>
static void launch_a_xf32(const ProjTile *tiles, uint32_t n_tiles, const float *xf, uint32_t K, float *y32,
                          uint16_t *y16, uint32_t N, uint32_t round_f32, hipStream_t stream)
{
    const size_t lds = staged_lds(3, KSPLIT, BPW, 1);
    if (lds > 48 * 1024)
        (void)hipFuncSetAttribute((const void *)linear_a_kernel<3, KSPLIT, 1, BPW, true, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((linear_a_kernel<3, KSPLIT, 1, BPW, true, true>), dim3(grid_for(n_tiles, 65535)),
                       dim3(64 * KSPLIT), lds, stream, tiles, n_tiles, nullptr, 1u, K, y32, y16, N, round_f32, xf);
}

void launch_linear_a_f32(const ProjTile *tiles, uint32_t n_tiles, const float *xf, uint16_t *scratch, uint32_t W,
                         uint32_t K, float *y32, uint16_t *y16, uint32_t N, uint32_t round_f32,
                         hipStream_t stream)
{
    if (W == 1) {
        // the split the planes would take (one row: never the paired form), staged if it fits
        const LinearSplit sp = pick_split(K >> 7, 1, n_tiles);
        // (sixteen waves of eight blocks never fit the stage, and are not instantiated)
        if (!(sp.ks == 16 && sp.bpw == 8) &&
            staged_lds(3, sp.ks, sp.bpw, 1) + sizeof(f32x4) * sp.ks * 64 <= LINEAR_STAGE_LDS) {
            const int t = timer_begin(K_LINEAR_A, stream);
#define PW_X(KS, BPW) launch_a_xf32<KS, BPW>(tiles, n_tiles, xf, K, y32, y16, N, round_f32, stream)
#define PW_X_BPW(KS)                                                                                       \
    do {                                                                                                   \
        if (sp.bpw == 8) PW_X(KS, 8); else if (sp.bpw == 4) PW_X(KS, 4); else if (sp.bpw == 2) PW_X(KS, 2); \
        else PW_X(KS, 1);                                                                                  \
    } while (0)
            if (sp.ks == 16) {
                if (sp.bpw == 4) PW_X(16, 4); else if (sp.bpw == 2) PW_X(16, 2); else PW_X(16, 1);
            } else if (sp.ks == 8) PW_X_BPW(8); else if (sp.ks == 4) PW_X_BPW(4);
            else if (sp.ks == 2) PW_X_BPW(2); else PW_X_BPW(1);
#undef PW_X_BPW
#undef PW_X
            timer_end(t, stream);
            return;
        }
    }
    launch_split_planes(xf, W * K, scratch, stream);
    launch_linear_a(tiles, n_tiles, scratch, 3, W, K, y32, y16, N, round_f32, stream);
}

template <int KSPLIT, int BPW>
static void launch_b_split(const ProjTile *tiles, uint32_t n_tiles, const uint8_t *codes, const float *scales,
                           uint32_t W, uint32_t K, float *y32, uint16_t *y16, uint32_t N, uint32_t round_f32,
                           hipStream_t stream)
{
    const int grid = grid_for(n_tiles, 65535);
    if constexpr (KSPLIT == 16)
        hipLaunchKernelGGL((linear_b_kernel<KSPLIT, 1, BPW>), dim3(grid), dim3(64 * KSPLIT), 0, stream, tiles,
                           n_tiles, codes, scales, W, K, y32, y16, N, round_f32);
    else if (W <= 16)
        hipLaunchKernelGGL((linear_b_kernel<KSPLIT, 1, BPW>), dim3(grid), dim3(64 * KSPLIT), 0, stream, tiles,
                           n_tiles, codes, scales, W, K, y32, y16, N, round_f32);
    else
        hipLaunchKernelGGL((linear_b_kernel<KSPLIT, 2, BPW>), dim3(grid), dim3(64 * KSPLIT), 0, stream, tiles,
                           n_tiles, codes, scales, W, K, y32, y16, N, round_f32);
}

void launch_linear_b(const ProjTile *tiles, uint32_t n_tiles, const uint8_t *codes,
                     const float *scales, uint32_t W, uint32_t K, float *y32, uint16_t *y16,
                     uint32_t N, uint32_t round_f32, hipStream_t stream)
{
    const LinearSplit sp = pick_split(K >> 7, W, n_tiles);
    const int t = timer_begin(K_LINEAR_B, stream);
#define PW_B(KS, BPW) launch_b_split<KS, BPW>(tiles, n_tiles, codes, scales, W, K, y32, y16, N, round_f32, stream)
#define PW_B_BPW(KS)                                                                                       \
    do {                                                                                                   \
        if (sp.bpw == 8) PW_B(KS, 8); else if (sp.bpw == 4) PW_B(KS, 4); else if (sp.bpw == 2) PW_B(KS, 2); \
        else PW_B(KS, 1);                                                                                  \
    } while (0)
    if (sp.ks == 16) PW_B_BPW(16); else if (sp.ks == 8) PW_B_BPW(8); else if (sp.ks == 4) PW_B_BPW(4);
    else if (sp.ks == 2) PW_B_BPW(2); else PW_B_BPW(1);
#undef PW_B_BPW
#undef PW_B
    timer_end(t, stream);
}

void launch_quant_group128(const void *x, bool x_f32, uint32_t rows, uint32_t K, uint8_t *codes,
                           float *scales, uint32_t *flags, hipStream_t stream)
{
    const uint32_t groups = rows * (K >> 7);
    const int grid = (int)((groups + 15) / 16);
    const int t = timer_begin(K_QUANT, stream);
    if (x_f32)
        hipLaunchKernelGGL(quant_group128_kernel<float>, dim3(grid), dim3(256), 0, stream,
                           (const float *)x, rows, K, codes, scales, flags);
    else
        hipLaunchKernelGGL(quant_group128_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream,
                           (const uint16_t *)x, rows, K, codes, scales, flags);
    timer_end(t, stream);
}

}  // namespace pw
