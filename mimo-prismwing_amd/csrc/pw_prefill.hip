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
// scales are multiplied together and applied in f32, sequentially over b.
//
// Tiles: (128 placement slots of one routed expert = an m-tile) x (256 weight rows = an n-tile);
// 128 slots hold a whole expert's placements at the uniform-routing count (64 on average, 93 at
// most for 2048 tokens), so its weights stream once, and a skewed routing's busiest experts need
// few m-tiles (each of which streams the expert's weights again); 16-token MFMA tiles past the
// m-tile's placements are skipped. Gate and
// up run as one stacked projection (2I output columns per slot), then a SwiGLU + re-quantisation
// kernel, then down. A workgroup walks K in 256-column steps with two kinds of waves, so the two
// streams never wait on each other in the in-order memory counter: eight consumer waves (32 weight
// rows each, two 16-row MFMA groups sharing every code read) load their weight bytes (one row per
// lane) into a register ring (two steps of two 128-column blocks) and run the MFMAs; one producer
// wave copies the m-tile's activation codes (cache hits, shared by the expert's n-tiles) with
// direct-to-LDS loads into a two-step LDS ring (16-byte units XOR-swizzled by token so the
// B-operand reads spread over the LDS banks).
// One LDS-only barrier per step publishes a ring slot and frees the previous one; the weight
// stream stays in flight across it. The m-tile's activation scales (transposed, [block][token])
// and the tile's weight block scales are staged in LDS once.
// Epilogues: every projection rounds to bf16 (bf16_round_in_place, src/wide_metal_moe.rs:
// 1236-1251); bf16_staged_swiglu (kernels/block_fp8_gemv.metal:139-160) runs on the bf16 gate and
// up outputs. The combine then sums each token's eight outputs.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

// Against 96-slot m-tiles, 2048 tokens: uniform routing unchanged (256 m-tiles either way), Zipf
// routing 341 -> 311 m-tiles, layer 1693 -> 1595 us.
constexpr uint32_t PF_MT = PREFILL_MT;            // placement slots per m-tile
// n-tiles per workgroup, where they divide evenly. Consecutive n-tiles share the workgroup's
// set-up and run the weight stream on across n-tiles, but put more m-tiles' activation codes in an
// XCD's L2 at once (32 CUs / (n-tiles per m-tile / PF_NSUB) m-tiles): the down projection's codes
// (128 slots x I bytes) take four, the gate/up projection's (128 token rows x H bytes) one.
constexpr uint32_t PF_NSUB_GATEUP = 1, PF_NSUB_DOWN = 4;
constexpr int PF_TT = (int)PF_MT / 16;            // 16-token MFMA tiles per m-tile
static_assert(PF_MT % 16 == 0 && PF_MT > 64 && PF_MT <= 128, "two 64-slot token lanes cover an m-tile");
constexpr uint32_t PF_UNITS = 8;                  // 16-byte units per 128-byte token row of a step
constexpr int PF_CONS = 8;                        // consumer waves per workgroup, 16 RG weight rows each
constexpr int PF_WAVES = PF_CONS + 1;             // and one producer wave (the codes ring)
// Gate/up workgroups start their K loop at column step (8 n-tile group + expert id % 8) % nsteps
// (and wrap), so the workgroups in flight, which advance through K at about the same rate, read
// different offsets of their weight rows instead of all the same 256 bytes of rows 4 KB apart (with
// every workgroup in step, the gate/up GEMM ran 13% slower for some physical placements of the
// bank; down, with four n-tiles per workgroup, does not need it). The sixteen n-tile groups of an
// m-tile share two start steps, so they read two code steps at a time; the start depends on nothing
// the rest of the batch sets, so a token's results do not either.
constexpr bool PF_ROTATE_GATEUP = true, PF_ROTATE_DOWN = false;
constexpr uint32_t PF_BLK = PF_MT * PF_UNITS;     // 16-byte code units per 128-column block
static_assert(PF_BLK % 64 == 0, "a block's codes are whole 64-lane copies");

// K-step shape: SB 128-column blocks per step, WS weight steps in flight per consumer lane, D code
// steps in the LDS ring. Two-block steps ask for 256 contiguous bytes of every weight row at once
// (more DRAM page hits than 128-byte pieces); one-block steps cover an odd number of blocks.
template <int SB_, int WS_, int D_, int RG_>
struct PfCfg {
    static constexpr int SB = SB_, WS = WS_, D = D_;
    static constexpr int RG = RG_;                         // 16-row groups per consumer wave
    static constexpr uint32_t NROWS = 16 * RG * PF_CONS;   // weight rows per n-tile
    static constexpr uint32_t NSB = (NROWS + 127) / 128;   // 128-row weight scale blocks per n-tile
    // two row groups hold twice the weight registers: one workgroup per CU (three waves per SIMD);
    // one row group fits five waves per SIMD with up to six 16-token tiles, four with more
    static constexpr int WAVES_PER_EU = RG == 1 ? (PF_TT > 6 ? 4 : 5) : 3;
    static constexpr int G = WS > D ? WS : D;              // steps per unrolled group
    static constexpr uint32_t STEP = SB * PF_BLK;          // 16-byte code units per step
    static_assert(G % WS == 0 && G % D == 0, "ring sizes divide the unrolled group");
};
// Both projections run 32-row consumer waves (256-row n-tiles, 165 VGPRs, one workgroup of nine
// waves per CU): every activation code copied into LDS feeds twice the weight rows, and that copy
// traffic (L2 hits) competes with the weight stream. Against 16-row waves at two workgroups per CU,
// 2048 tokens: gate/up 944 -> 827 us, down 505 -> 481 us. Odd block counts take one-block steps
// with 16-row waves (two row groups of a four-step weight ring would not fit in registers).
using PfWide = PfCfg<2, 2, 2, 2>;
using PfNarrow = PfCfg<1, 4, 4, 1>;

// Tile table: ceil(count / 128) m-tiles per routed expert, ascending expert order, each with its
// expert's weights and its slots. One workgroup of 1024 threads, one thread per schedule entry
// (banks hold at most 1024 experts).
__global__ __launch_bounds__(1024) void prefill_tiles_kernel(const MoePlan *__restrict__ plan,
                                                             const ActiveExpert *__restrict__ active,
                                                             const uint32_t *__restrict__ active_expert,
                                                             uint32_t max_active, PfTileDesc *__restrict__ tiles,
                                                             uint32_t max_tiles, uint32_t *__restrict__ n_tiles,
                                                             uint32_t *flags)
{
    __shared__ uint32_t s_scan[48];
    const uint32_t a = threadIdx.x;
    const uint32_t n_active = plan->n_active;
    const bool live = a < max_active && a < n_active;
    const uint32_t cnt = live ? active[a].cnt : 0u;
    const uint32_t nt = (cnt + PF_MT - 1) / PF_MT;
    uint32_t total;
    const uint32_t off = block_exclusive_scan(nt, s_scan, &total);
    if (live) {
        const ActiveExpert ae = active[a];
        for (uint32_t i = 0; i < nt; ++i)
            if (off + i < max_tiles) {
                PfTileDesc td;
                td.ep = ae.ep;
                td.slot0 = ae.off + i * PF_MT;
                td.cnt = cnt - i * PF_MT < PF_MT ? cnt - i * PF_MT : PF_MT;
                td.expert = active_expert[a];
                td.pad = 0;
                tiles[off + i] = td;
            }
    }
    if (a == 0) {
        n_tiles[0] = total < max_tiles ? total : max_tiles;
        if (total > max_tiles)
            raise_flag(flags, FLAG_SCHEDULE);
    }
}

struct PrefillArgs {
    const PfTileDesc *tiles;        // [max_tiles]
    const uint32_t *n_tiles;
    const uint32_t *placement_pos;  // gate/up: token row of each placement slot (down: null)
    const uint8_t *codes;           // activation codes [rows][K] (down: rows = placement slots)
    const float *scales;            // activation scales [rows][K / 128]
    uint32_t K;                     // columns
    uint32_t R;                     // output columns per slot: 2I (gate then up) or H
    uint32_t R1;                    // rows of the first matrix (gate/up: I; down: H)
    uint32_t rows, max_tiles;
    uint32_t n_sub;                 // consecutive n-tiles per workgroup (divides the n-tile count)
    uint16_t *out;                  // [P][R] bf16
    uint32_t *flags;
};

// One K step's weight bytes of this lane: for each of the step's blocks, its row's columns
// [16q, 16q + 16) and [64 + 16q, 80 + 16q) of the 128-column block (q = lane / 16), so each load
// instruction reads 64 contiguous bytes of each of 16 rows and a step asks for SB * 128
// contiguous bytes of every row at once. The MFMA's K order within a block is permuted alike for
// the codes, so the block dot product covers the same 128 products.
template <class C>
struct PfW {
    uint4 v[C::RG][2 * C::SB];
};

// src: the wave's first weight row at the step's first column (wave-uniform); loff: the lane's row
// and column offset (r16 rows, 16 q columns); group g is 16 g rows further (rstride = 16 K bytes)
template <class C>
__device__ __forceinline__ void pf_issue_w(PfW<C> &w, const uint8_t *src, uint32_t loff, size_t rstride)
{
#pragma unroll
    for (int g = 0; g < C::RG; ++g)
#pragma unroll
        for (int h = 0; h < C::SB; ++h) {
            w.v[g][2 * h] = load_global16(src + g * rstride + 128 * h + loff);
            w.v[g][2 * h + 1] = load_global16(src + g * rstride + 128 * h + 64 + loff);
        }
}

// One step: its blocks in ascending order, each block's FP8 products from one MFMA per active
// 16-token tile, then tot += p * (S_w * a) in f32 (the two scales multiplied once per token and
// block, four fused multiply-adds per tile). Each block's weight registers are refilled from next
// (the wave's rows at the step WS ahead, possibly of the workgroup's next n-tile) as soon as its
// MFMAs have read them, half a step earlier than a refill of the whole step. cl0 / cl1: the lane's
// two code units of token r16 in a block (tile j adds 16 tokens = 128 units).
template <class C, int NT>
__device__ __forceinline__ void pf_compute(f32x4 (&tot)[C::RG][NT], PfW<C> &w, const uint4 *slot,
                                           const float *lds_scale, const float *lds_wscale, uint32_t k, int r16,
                                           const uint8_t *next, uint32_t loff, size_t rstride, uint32_t cl0,
                                           uint32_t cl1)
{
#pragma unroll
    for (int h = 0; h < C::SB; ++h) {
        const uint32_t b = k * C::SB + h;
        const float sw = lds_wscale[b];
        const uint4 *buf = slot + h * PF_BLK;
        i32x8 A[C::RG];
#pragma unroll
        for (int g = 0; g < C::RG; ++g)
            A[g] = i32x8{(int)w.v[g][2 * h].x,     (int)w.v[g][2 * h].y,     (int)w.v[g][2 * h].z,
                         (int)w.v[g][2 * h].w,     (int)w.v[g][2 * h + 1].x, (int)w.v[g][2 * h + 1].y,
                         (int)w.v[g][2 * h + 1].z, (int)w.v[g][2 * h + 1].w};
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t t = 16 * j + r16;
            const float sc = sw * lds_scale[b * PF_MT + t];
            const uint4 c0 = buf[cl0 + 128 * j];
            const uint4 c1 = buf[cl1 + 128 * j];
            const i32x8 xb = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w,
                              (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
#pragma unroll
            for (int g = 0; g < C::RG; ++g) {
                const f32x4 p = mfma_fp8_16x16x128(A[g], xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    tot[g][j][i] = __builtin_fmaf(p[i], sc, tot[g][j][i]);
            }
        }
#pragma unroll
        for (int g = 0; g < C::RG; ++g) {
            w.v[g][2 * h] = load_global16(next + g * rstride + 128 * h + loff);
            w.v[g][2 * h + 1] = load_global16(next + g * rstride + 128 * h + 64 + loff);
        }
    }
}

// What the producer and consumer waves of one workgroup share (set up by prefill_b_kernel): one
// m-tile and n_sub consecutive n-tiles, run one after another.
struct PfTile {
    uint4 *ring;               // [D][STEP] code units, swizzled
    const float *lds_scale;    // [blocks][PF_MT] activation scales
    const float *lds_wscale;   // [n_sub * NSB][blocks] weight block scales of the n-tiles' 128-row blocks
    const uint8_t *mat0, *mat1; // output columns [0, R1): rows of mat0 (gate or down), [R1, R): mat1 (up)
    uint16_t *out;             // the wave's first output: slot0 row, column col0 + wave * 16 RG
    uint32_t K, R, R1, nsteps, n_sub;
    uint32_t rot;              // K step order: loop step k reads column step (k + rot) % nsteps
    uint32_t wcol;             // the wave's first output column in the first n-tile
    uint32_t loff;             // the lane's weight offset: r16 rows and 16 q columns
    uint32_t cnt;              // placement slots of the m-tile
    const uint8_t *codes;      // activation codes [rows][K] (the producer's)
    uint32_t *lds_tok;         // [PF_MT] token rows of the m-tile's slots, written by the producer
};

// Column step of loop step k < nsteps (wave-uniform).
__device__ __forceinline__ uint32_t pf_col_step(const PfTile &tl, uint32_t k)
{
    const uint32_t c = k + tl.rot;
    return c >= tl.nsteps ? c - tl.nsteps : c;
}

// Wave-uniform address of the wave's first weight row in n-tile sub: column wcol + sub * NROWS is
// row col - R1 of mat1 when col >= R1, else row col of mat0 (columns past R, of a partial last
// n-tile, read row 0 and are never stored).
template <class C>
__device__ __forceinline__ const uint8_t *pf_wave_rows(const PfTile &tl, uint32_t sub)
{
    const uint32_t col = tl.wcol + sub * C::NROWS;
    const uint32_t row = col >= tl.R ? 0u : (col >= tl.R1 ? col - tl.R1 : col);
    return (col >= tl.R1 && col < tl.R ? tl.mat1 : tl.mat0) + (size_t)row * tl.K;
}

// Waits until at most (C::D - 2) steps of copies (2 nt token groups per block) are outstanding.
template <class C>
__device__ __forceinline__ void pf_wait_copies(uint32_t nt)
{
    if constexpr (C::D == 2) {
        wait_vmcnt<0>();
    } else {
        static_assert((C::D - 2) * 2 * PF_TT * C::SB < 64, "vmcnt has six bits");
        switch (nt) {
        case 1: wait_vmcnt<(C::D - 2) * 2 * 1 * C::SB>(); break;
        case 2: wait_vmcnt<(C::D - 2) * 2 * 2 * C::SB>(); break;
        case 3: wait_vmcnt<(C::D - 2) * 2 * 3 * C::SB>(); break;
        case 4: wait_vmcnt<(C::D - 2) * 2 * 4 * C::SB>(); break;
        case 5: wait_vmcnt<(C::D - 2) * 2 * 5 * C::SB>(); break;
        case 6: wait_vmcnt<(C::D - 2) * 2 * 6 * C::SB>(); break;
        case 7: wait_vmcnt<(C::D - 2) * 2 * 7 * C::SB>(); break;
        default: wait_vmcnt<(C::D - 2) * 2 * PF_TT * C::SB>(); break;
        }
    }
}

// The producer wave: the codes ring over the workgroup's n-tiles (the m-tile's codes again for
// every n-tile), the nt active 16-token tiles' codes of each step. Step k's copy of block h covers
// token groups c = 0 .. 2 nt - 1 of 8 tokens: lane i reads global unit (i % 8) ^ (token % 8) of
// token 8c + i / 8 (its row from the token rows tok, lane t of tok[0] or tok[1]) and lands at LDS
// unit 64c + i (unit i % 8 of that token).
template <class C>
__device__ __forceinline__ void pf_produce(const PfTile &tl, const uint32_t (&tok)[2], uint32_t nt, int lane)
{
    const uint32_t K = tl.K, nsteps = tl.nsteps;
    const uint32_t nc = 2 * nt;
    const uint32_t unit = (((uint32_t)lane ^ ((uint32_t)lane >> 3)) & 7) * 16;
    // global steps k = 0 .. n_sub * nsteps - 1 (column step k % nsteps), indices clamped to the
    // last step
    const uint32_t total = tl.n_sub * nsteps, tlast = total - 1;
    const auto copy_step = [&](uint32_t s) {
        uint4 *slot = tl.ring + (s % C::D) * C::STEP;
        const uint32_t k0 = pf_col_step(tl, (s < tlast ? s : tlast) % nsteps) * (128 * C::SB);
        for (uint32_t c = 0; c < nc; ++c) {
            const uint32_t t = 8 * c + ((uint32_t)lane >> 3);
            const uint32_t row = __shfl(c < 8 ? tok[0] : tok[1], (int)(t & 63), 64);
            const uint8_t *src = tl.codes + (size_t)row * K + unit + k0;
#pragma unroll
            for (int h = 0; h < C::SB; ++h)
                lds_load16(src + 128 * h, slot + h * PF_BLK + c * 64);
        }
    };
    // steps 0 .. C::D - 2 into slots 0 .. C::D - 2
    for (uint32_t s = 0; s + 1 < (uint32_t)C::D; ++s)
        copy_step(s);
    for (uint32_t k = 0; k < total; ++k) {
        // step k's copy (and every older one) is complete; C::D - 2 younger steps stay in flight
        pf_wait_copies<C>(nt);
        lds_barrier();  // publishes slot k % C::D; every consumer is done with step k - 1
        copy_step(k + C::D - 1);
    }
    wait_vmcnt<0>();  // no copy may land in LDS after the workgroup ends
}

// One workgroup's waves over NT active 16-token tiles. The producer wave takes its token rows
// back from LDS (it stored them there itself), so they are not held in registers through the
// consumers' code. The consumer waves run the K loops of the workgroup's n-tiles, the MFMAs and
// each n-tile's bf16 outputs; the last WS steps of an n-tile load the next n-tile's first weight
// steps, so the weight stream runs on across n-tiles.
template <class C, int NT>
__device__ __forceinline__ void pf_body(const PfTile &tl, int wave, int lane)
{
    if (wave >= PF_CONS) {
        asm volatile("" ::: "memory");
        const uint32_t tok[2] = {tl.lds_tok[lane], tl.lds_tok[64 + lane]};
        pf_produce<C>(tl, tok, NT, lane);
        return;
    }
    const uint32_t K = tl.K, nsteps = tl.nsteps, last = nsteps - 1;
    const int q = lane >> 4, r16 = lane & 15;
    const size_t rstride = (size_t)16 * K;
    const uint32_t loff = tl.loff;
    const uint32_t lane_out = (uint32_t)r16 * tl.R + 4 * (uint32_t)q;  // the lane's output offset
    const uint8_t *rows = pf_wave_rows<C>(tl, 0);
    PfW<C> w[C::WS];
#pragma unroll
    for (int i = 0; i < C::WS; ++i)
        pf_issue_w<C>(w[i], rows + pf_col_step(tl, (uint32_t)i < last ? (uint32_t)i : last) * (128 * C::SB), loff,
                      rstride);
    // the lane's code units of token r16 in a block: units q and q + 4, swizzled by token % 8 (the
    // same for token r16 + 16 j); opaque to the compiler, which would otherwise fold the tile
    // offsets into one address register per tile and half instead of immediate offsets
    uint32_t cl0 = (uint32_t)r16 * PF_UNITS + ((uint32_t)q ^ ((uint32_t)r16 & 7u));
    uint32_t cl1 = (uint32_t)r16 * PF_UNITS + (((uint32_t)q + 4u) ^ ((uint32_t)r16 & 7u));
    asm volatile("" : "+v"(cl0), "+v"(cl1));
    // this wave's activation scale copies (issued before the weights) are complete before the
    // first barrier publishes them
    wait_vmcnt<2 * C::SB * C::WS * C::RG>();

    const uint32_t blocks = K >> 7;
    for (uint32_t sub = 0; sub < tl.n_sub; ++sub) {
        // the next n-tile's rows (this one's for the last n-tile: the tail reloads its last step,
        // cache hits, keeping every load unconditional)
        const bool more = sub + 1 < tl.n_sub;
        const uint8_t *nrows = more ? pf_wave_rows<C>(tl, sub + 1) : rows;
        const float *wsc = tl.lds_wscale + ((sub * C::NROWS + (uint32_t)wave * 16 * C::RG) >> 7) * blocks;
        f32x4 tot[C::RG][NT];
#pragma unroll
        for (int g = 0; g < C::RG; ++g)
#pragma unroll
            for (int j = 0; j < NT; ++j)
                tot[g][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        // weights of step kk: this n-tile's, or past its last step the next n-tile's first ones
        const auto next_src = [&](uint32_t k) {
            const uint32_t kk = k + C::WS;
            return kk <= last ? rows + pf_col_step(tl, kk) * (128 * C::SB)
                              : (more ? nrows + pf_col_step(tl, kk - nsteps) * (128 * C::SB)
                                      : rows + pf_col_step(tl, last) * (128 * C::SB));
        };

        // Step k: barrier (slot k % C::D published), compute from weight slot k % C::WS, each
        // block's registers reloaded with step k + C::WS's block right after use. Whole groups of
        // C::G steps run without early exits (static ring indices, one loop state at the loop
        // head); the last steps are peeled (one n-tile per workgroup: the launcher gives several
        // only where the steps are whole groups, so every n-tile starts at ring slot 0).
        const uint32_t nfull = nsteps - nsteps % C::G;
        for (uint32_t b = 0; b < nfull; b += C::G) {
#pragma unroll
            for (int i = 0; i < C::G; ++i) {
                const uint32_t k = b + i;
                lds_barrier();
                pf_compute<C, NT>(tot, w[i % C::WS], tl.ring + (i % C::D) * C::STEP, tl.lds_scale, wsc,
                                  pf_col_step(tl, k), r16, next_src(k), loff, rstride, cl0, cl1);
            }
        }
#pragma unroll
        for (int i = 0; i < C::G - 1; ++i) {
            const uint32_t k = nfull + i;
            if (k >= nsteps)
                break;
            lds_barrier();
            pf_compute<C, NT>(tot, w[i % C::WS], tl.ring + (i % C::D) * C::STEP, tl.lds_scale, wsc,
                              pf_col_step(tl, k), r16, next_src(k), loff, rstride, cl0, cl1);
        }

        // epilogue: lane holds rows 16 g + 4q + i of the wave's 16 RG for tokens 16j + r16 -> bf16,
        // stored at the wave's base (token 16 j, row 16 g) plus the lane's offset
        const uint32_t store_t = tl.wcol + sub * C::NROWS < tl.R ? tl.cnt : 0u;
        // opaque per n-tile, or the compiler hoists every token tile's 64-bit lane address out of
        // the n-tile loop (sixteen registers, spilled)
        uint32_t lo = lane_out;
        asm volatile("" : "+v"(lo));
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t t = 16 * j + r16;
            if (t >= store_t)
                continue;
#pragma unroll
            for (int g = 0; g < C::RG; ++g) {
                uint16_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = (uint16_t)(f32_bits(round_bf16(tot[g][j][i])) >> 16);
                uint16_t *dst = tl.out + sub * C::NROWS + (size_t)(16 * j) * tl.R + 16 * g;
                *(uint2 *)(dst + lo) =
                    make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
            }
        }
        rows = nrows;
    }
}

// One projection workgroup: n_sub consecutive n-tiles of NROWS weight rows (of gate, up or down)
// x one m-tile of placement slots, bf16-rounded outputs (bf16_round_in_place of every projection,
// src/wide_metal_moe.rs:1236-1251). Output columns [0, R1) come from the first matrix (gate, or
// down), the rest from the second (up).
template <class C>
__global__ __launch_bounds__(64 * PF_WAVES) __attribute__((amdgpu_waves_per_eu(C::WAVES_PER_EU))) void prefill_b_kernel(const PrefillArgs args)
{
    extern __shared__ uint4 lds_pf[];
    const uint32_t K = args.K, blocks = K >> 7;
    const uint32_t nsteps = blocks / C::SB;  // the launcher checks blocks % SB
    uint4 *ring = lds_pf;                                   // [D][STEP] code units, swizzled
    float *lds_scale = (float *)(ring + C::D * C::STEP);    // [blocks][PF_MT] activation scales
    uint32_t *lds_tok = (uint32_t *)(lds_scale + blocks * PF_MT);  // [PF_MT] token rows (producer)
    float *lds_wscale = (float *)(lds_tok + PF_MT);       // [n_sub * NSB][blocks] weight block scales
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    // XCD-aware order: workgroups go round-robin to the 8 XCDs (blockIdx % 8), so XCD x takes
    // m-tiles x, x + 8, ... and runs all n-tile groups of one m-tile back to back: the m-tile's
    // activation codes stay in that XCD's L2 while its n-tiles stream their weight rows, and the
    // m-tiles (counted on the device) spread evenly over the XCDs.
    const uint32_t n_sub = args.n_sub;
    const uint32_t n_groups = (args.R + C::NROWS - 1) / C::NROWS / n_sub;  // the launcher checks n_sub
    const uint32_t local = blockIdx.x >> 3;
    const uint32_t mt = (blockIdx.x & 7) + 8 * (local / n_groups), group = local % n_groups;
    // the tile count and the tile's descriptor in one round trip (the descriptor index clamped:
    // the grid holds whole groups of eight m-tiles)
    const uint32_t n_mtiles = args.n_tiles[0];
    const PfTileDesc td = args.tiles[mt < args.max_tiles ? mt : args.max_tiles - 1];
    if (mt >= n_mtiles || td.cnt == 0)
        return;
    const ExpertPtrs &ep = td.ep;
    const uint32_t cnt_t = td.cnt < PF_MT ? td.cnt : PF_MT;
    const uint32_t col0 = group * n_sub * C::NROWS;       // first output column of the workgroup
    const uint32_t slot0 = td.slot0;
    const bool gather = args.placement_pos != nullptr;

    // token rows of the m-tile's slots (lane: slots lane and 64 + lane, the second only below PF_MT;
    // slots past the tile's count repeat its last slot: in-bounds loads whose output columns are
    // never stored)
    uint32_t tok[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t t = 64 * h + (h ? (uint32_t)lane % (PF_MT - 64) : (uint32_t)lane);
        tok[h] = slot0 + (t < cnt_t ? t : cnt_t - 1);
        if (gather)
            tok[h] = load_g(args.placement_pos + tok[h]);
    }
    if (gather) {
        bool bad = false;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bad |= tok[h] >= args.rows;
            tok[h] = tok[h] < args.rows ? tok[h] : args.rows - 1;
        }
        if (bad)
            raise_flag(args.flags, FLAG_SCHEDULE);
    }
    // weight block scales of the n-tiles' 128-row blocks ([n_sub * NSB][blocks]; each 128 output
    // columns come from one 128-row block of one matrix, R1 and R being multiples of 128) and the
    // m-tile's activation scales, transposed (lds_scale[b * PF_MT + t]) with 4-byte direct-to-LDS
    // loads (lane = token; a second instruction covers tokens 64 .. PF_MT - 1), spread over all
    // waves
    for (uint32_t i = tid; i < n_sub * C::NSB * blocks; i += 64 * PF_WAVES) {
        const uint32_t hb = i / blocks, b = i - hb * blocks;
        const uint32_t col = col0 + 128 * hb;
        const uint32_t row = col >= args.R ? 0u : (col >= args.R1 ? col - args.R1 : col);
        const float *sm = gather ? (col >= args.R1 && col < args.R ? ep.up_s : ep.gate_s) : ep.down_s;
        lds_wscale[i] = load_g(sm + (row >> 7) * blocks + b);
    }
    for (uint32_t b = wave; b < blocks; b += PF_WAVES) {
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void *)(args.scales + (size_t)tok[0] * blocks + b),
            (__attribute__((address_space(3))) void *)(lds_scale + b * PF_MT), 4, 0, 0);
        if (lane < (int)PF_MT - 64)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(args.scales + (size_t)tok[1] * blocks + b),
                (__attribute__((address_space(3))) void *)(lds_scale + b * PF_MT + 64), 4, 0, 0);
    }
    if (wave >= PF_CONS) {  // the producer's token rows, read back in its loop
        lds_tok[lane] = tok[0];
        lds_tok[64 + lane] = tok[1];
    }

    // the wave's 16 RG rows (inside one 128-row block) in each n-tile
    const uint32_t wrow0 = wave * 16 * C::RG;
    PfTile tile;
    tile.ring = ring;
    tile.lds_scale = lds_scale;
    tile.lds_wscale = lds_wscale;
    tile.mat0 = gather ? ep.gate_w : ep.down_w;
    tile.mat1 = gather ? ep.up_w : ep.down_w;
    tile.out = args.out + (size_t)slot0 * args.R + col0 + wrow0;
    tile.K = K;
    tile.R = args.R;
    tile.R1 = args.R1;
    tile.nsteps = nsteps;
    tile.n_sub = n_sub;
    // the start step depends on the n-tile group and the expert only, never on where the batch put
    // the m-tile: a token's sums run in the same order whatever else is routed with it
    tile.rot = (gather ? PF_ROTATE_GATEUP : PF_ROTATE_DOWN) ? (8 * group + (td.expert & 7)) % nsteps : 0u;
    tile.wcol = col0 + wrow0;
    tile.loff = (uint32_t)r16 * K + (uint32_t)q * 16;
    tile.cnt = cnt_t;
    tile.codes = args.codes;
    tile.lds_tok = lds_tok;
    // the workgroup's 16-token tiles that hold placements (1..PF_TT); whole tiles past them are skipped
    switch ((cnt_t + 15) >> 4) {
    case 1: pf_body<C, 1>(tile, wave, lane); break;
    case 2: pf_body<C, 2>(tile, wave, lane); break;
    case 3: pf_body<C, 3>(tile, wave, lane); break;
    case 4: pf_body<C, 4>(tile, wave, lane); break;
    case 5: pf_body<C, 5>(tile, wave, lane); break;
    case 6: pf_body<C, (PF_TT > 6 ? 6 : PF_TT)>(tile, wave, lane); break;
    case 7: pf_body<C, (PF_TT > 7 ? 7 : PF_TT)>(tile, wave, lane); break;
    default: pf_body<C, PF_TT>(tile, wave, lane); break;
    }
}

// silu_bf16_staged for all 65,536 bf16 bit patterns: the table entry of bits b is the function's
// value at the bf16 number b, computed by the shared device function once, so a lookup gives the
// same bits as evaluating it in place.
__global__ __launch_bounds__(256) void silu_table_kernel(uint16_t *__restrict__ table)
{
    const uint32_t b = blockIdx.x * 256 + threadIdx.x;  // grid covers exactly 65,536 entries
    table[b] = (uint16_t)(f32_bits(silu_bf16_staged(f32_from(b << 16))) >> 16);
}

void launch_silu_table(uint16_t *table, hipStream_t stream)
{
    hipLaunchKernelGGL(silu_table_kernel, dim3(256), dim3(256), 0, stream, table);
}

// Elementwise bf16_staged_swiglu (kernels/block_fp8_gemv.metal:139-160; CPU
// src/text_endpoint.rs:5336-5343) on f32 arrays: out = round(round(silu(round(g))) * round(u)).
// With a table the silu comes from it (the prefill form), else it is evaluated in place (the
// decode form). One thread per value.
__global__ __launch_bounds__(256) void swiglu_staged_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                            uint32_t n, const uint16_t *__restrict__ silu_table,
                                                            float *__restrict__ out, uint32_t *flags)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n)
        return;
    const float g = round_bf16(gate[i]), u = round_bf16(up[i]);
    const float silu = silu_table ? f32_from((uint32_t)silu_table[f32_bits(g) >> 16] << 16) : silu_bf16_staged(g);
    const float h = round_bf16(silu * u);
    out[i] = h;
    if (!finite_f32(g) || !finite_f32(u) || !finite_f32(h))
        raise_flag(flags, FLAG_SWIGLU_NONFINITE);
}

void launch_swiglu_staged(const float *gate, const float *up, uint32_t n, const uint16_t *silu_table, float *out,
                          uint32_t *flags, hipStream_t stream)
{
    hipLaunchKernelGGL(swiglu_staged_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, gate, up, n, silu_table,
                       out, flags);
}

constexpr int SWQ_GPT = 2;  // 128-column groups per 16-lane team of prefill_swiglu_quant_kernel

// bf16_staged_swiglu (kernels/block_fp8_gemv.metal:139-160; CPU src/text_endpoint.rs:5336-5343)
// on the bf16 gate/up outputs, h = round(round(g / (1 + e^-g)) * u), fused with the dynamic
// per-(slot, 128-column group) re-quantisation of h for the down projection
// (dynamic_fp8_quantized_group128, kernels/block_fp8_gemv.metal:84-137). 16 lanes per group,
// eight consecutive values per lane (16-byte loads of gate and up), SWQ_GPT groups per team;
// gu [P][2I] bf16 (gate columns, then up). The silu factor comes from silu_table (65,536 bf16
// entries indexed by the gate's bits, built by silu_table_kernel), which keeps the exponential
// and the division out of this VALU-bound kernel.
__global__ __launch_bounds__(256) void prefill_swiglu_quant_kernel(const uint16_t *__restrict__ gu, uint32_t P,
                                                                   uint32_t I, uint32_t gpr_shift,
                                                                   const uint16_t *__restrict__ silu_table,
                                                                   uint8_t *__restrict__ codes,
                                                                   float *__restrict__ scales, uint32_t *flags)
{
    // a 16-lane team takes SWQ_GPT consecutive groups, all of their loads issued before the first
    // table gather (the kernel is bound by that chain of latencies, not by its instructions)
    const uint32_t lane16 = threadIdx.x & 15;
    const uint32_t groups_per_row = I >> 7, n_groups = P * groups_per_row;
    const uint32_t group0 = (blockIdx.x * 16 + (threadIdx.x >> 4)) * SWQ_GPT;
    if (group0 >= n_groups)  // whole 16-lane teams leave together
        return;
    uint32_t gw[SWQ_GPT][4], uw[SWQ_GPT][4];
    uint32_t slot[SWQ_GPT], col[SWQ_GPT];
#pragma unroll
    for (int j = 0; j < SWQ_GPT; ++j) {
        const uint32_t group = group0 + j < n_groups ? group0 + j : group0;
        // gpr_shift: log2 of the groups per row where that is a power of two (a shift, not a division)
        slot[j] = gpr_shift < 32 ? group >> gpr_shift : group / groups_per_row;
        col[j] = (group - slot[j] * groups_per_row) * 128 + lane16 * 8;
        const uint16_t *row = gu + (size_t)slot[j] * 2 * I;
        const uint4 g4 = *(const uint4 *)(row + col[j]), u4 = *(const uint4 *)(row + I + col[j]);
        gw[j][0] = g4.x, gw[j][1] = g4.y, gw[j][2] = g4.z, gw[j][3] = g4.w;
        uw[j][0] = u4.x, uw[j][1] = u4.y, uw[j][2] = u4.z, uw[j][3] = u4.w;
    }
    uint32_t sb[SWQ_GPT][8];
#pragma unroll
    for (int j = 0; j < SWQ_GPT; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            sb[j][i] = load_g(silu_table + ((i & 1) ? (gw[j][i >> 1] >> 16) : (gw[j][i >> 1] & 0xffffu)));
    // non-finite gate / up values: a bf16 half whose exponent field is all ones carries into its
    // bit 15 when 0x80 is added to the masked field (two values per word, no carry between them)
    uint32_t nf = 0, emax = 0;
#pragma unroll
    for (int j = 0; j < SWQ_GPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            nf |= ((gw[j][i] & 0x7f807f80u) + 0x00800080u) | ((uw[j][i] & 0x7f807f80u) + 0x00800080u);
#pragma unroll
    for (int j = 0; j < SWQ_GPT; ++j) {
        if (group0 + j >= n_groups)
            break;
        float h[8];
        uint32_t ge = 0;  // the largest exponent field of the lane's h values
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t ub = uw[j][i >> 1];
            const float uv = f32_from((i & 1) ? (ub & 0xffff0000u) : (ub << 16));
            // a non-finite h is flagged and coded 0, so its NaN payload never matters
            h[i] = round_bf16_or_nonfinite(f32_from(sb[j][i] << 16) * uv);
            ge = max(ge, f32_bits(h[i]) & 0x7f800000u);
        }
        emax = max(emax, ge);
        // every h of the wave finite (the usual case, a wave-uniform branch): no per-value selects
        const bool all_finite = __ballot(ge == 0x7f800000u) == 0;
        float m = 0.f;
        if (all_finite) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                m = fmaxf(m, fabsf(h[i]));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                m = fmaxf(m, finite_f32(h[i]) ? fabsf(h[i]) : 0.f);
        }
        m = row16_max(m);  // the group's 16 lanes form one DPP row
        const float scale = scale_of_bf16_max(m);  // m is a bf16 value
        if (lane16 == 0)
            scales[group0 + j] = scale;
        const float rcp = 1.0f / scale;  // h is bf16: one division per group (quant_ratio_bf16)
        float n[8];
        if (all_finite) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                n[i] = quant_ratio_bf16(h[i], scale, rcp);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                n[i] = finite_f32(h[i]) ? quant_ratio_bf16(h[i], scale, rcp) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            n[i] = fminf(fmaxf(n[i], -448.f), 448.f);  // n is finite: the same as the clamp by comparisons
        uint32_t packed[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            packed[i] = encode2_e4m3fn(n[4 * i], n[4 * i + 1]) | (encode2_e4m3fn(n[4 * i + 2], n[4 * i + 3]) << 16);
        *(uint2 *)(codes + (size_t)slot[j] * I + col[j]) = make_uint2(packed[0], packed[1]);
    }
    if ((nf & 0x80008000u) || emax == 0x7f800000u)
        raise_flag(flags, FLAG_SWIGLU_NONFINITE);
}

// route_weighted_scatter_add_f32 + final bf16 round over bf16 expert outputs: each token sums
// its eight placements in ascending expert id, out += y * w in f32 (no fused multiply-add). One
// thread per eight consecutive columns of a token row (16-byte loads of each placement's outputs).
// A rejected batch (the schedule raised FLAG_SCHEDULE) writes zeros.
__global__ __launch_bounds__(256) void prefill_combine_kernel(
    const uint16_t *__restrict__ y, const float *__restrict__ placement_w, const uint32_t *__restrict__ row_slots,
    uint32_t rows, uint32_t H, const MoePlan *__restrict__ plan, float *__restrict__ out_f32,
    uint16_t *__restrict__ out_bf16, uint32_t raw, uint32_t *flags)
{
    const bool rejected = plan->rejected != 0;
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;  // eight values of one token row
    const uint32_t per_row = H >> 3;
    if (idx >= rows * per_row)
        return;
    const uint32_t row = idx / per_row, c8 = idx - row * per_row;
    const uint32_t P = rows * 8;
    const uint4 s0 = *(const uint4 *)(row_slots + (size_t)row * 8), s1 = *(const uint4 *)(row_slots + (size_t)row * 8 + 4);
    uint32_t slot[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float w[8];
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        slot[j] = slot[j] < P ? slot[j] : 0;
        w[j] = placement_w[slot[j]];
        v[j] = *(const uint4 *)(y + (size_t)slot[j] * H + c8 * 8);
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t u[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(f32_from(u[i] << 16), w[j]));
            acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(f32_from(u[i] & 0xffff0000u), w[j]));
        }
    }
    bool bad = false;
    const size_t at = (size_t)row * H + c8 * 8;
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        acc[i] = rejected ? 0.f : acc[i];
        r[i] = round_bf16(acc[i]);
        bad |= !finite_f32(r[i]);
    }
    if (out_f32) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            o[i] = raw ? acc[i] : r[i];
        *(float4 *)(out_f32 + at) = make_float4(o[0], o[1], o[2], o[3]);
        *(float4 *)(out_f32 + at + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (out_bf16) {
        uint32_t pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            pk[i] = (f32_bits(r[2 * i]) >> 16) | (f32_bits(r[2 * i + 1]) & 0xffff0000u);
        *(uint4 *)(out_bf16 + at) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
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

// n-tiles per workgroup: nsub where it divides the n-tile count, every n-tile is whole and the K
// steps are whole unrolled groups (each n-tile's loop then starts at ring slot 0), else one
template <class C>
static void launch_prefill_cfg(PrefillArgs a, uint32_t nsub, hipStream_t stream)
{
    const uint32_t blocks = a.K / 128, n_ntiles = (a.R + C::NROWS - 1) / C::NROWS;
    a.n_sub = (n_ntiles % nsub == 0 && a.R % C::NROWS == 0 && (blocks / C::SB) % C::G == 0) ? nsub : 1;
    const size_t lds = (size_t)C::D * C::STEP * 16 + (size_t)blocks * (PF_MT + a.n_sub * C::NSB) * 4 + PF_MT * 4;
    if (lds > 65536)  // wide K: up to 160 KB of LDS per workgroup on gfx950
        (void)hipFuncSetAttribute((const void *)prefill_b_kernel<C>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
    const uint32_t grid = 8 * ((a.max_tiles + 7) / 8) * (n_ntiles / a.n_sub);
    hipLaunchKernelGGL((prefill_b_kernel<C>), dim3(grid), dim3(64 * PF_WAVES), lds, stream, a);
}

static void launch_prefill_projection(const PrefillArgs &a, uint32_t nsub, hipStream_t stream)
{
    if ((a.K / 128) % PfWide::SB == 0)
        launch_prefill_cfg<PfWide>(a, nsub, stream);
    else
        launch_prefill_cfg<PfNarrow>(a, nsub, stream);
}

void launch_moe_prefill(const ExpertPtrs *bank, const MoeBuffers &mb, const PrefillBuffers &pb, const void *x,
                        bool x_f32, uint32_t rows, uint32_t E, uint32_t H, uint32_t I, float *out_f32,
                        uint16_t *out_bf16, bool raw, uint32_t *flags, hipStream_t stream, bool scheduled_long)
{
    (void)bank;
    const uint32_t P = rows * 8;
    const uint32_t max_active = E < P ? E : P;
    const uint32_t max_tiles = prefill_max_tiles(rows, E);
    if (!scheduled_long) {
        launch_quant_group128(x, x_f32, rows, H, mb.xq, mb.xs, flags, stream);
        hipLaunchKernelGGL(prefill_tiles_kernel, dim3(1), dim3(1024), 0, stream, mb.plan, mb.active,
                           mb.active_expert, max_active, pb.tiles, max_tiles, pb.n_tiles, flags);
    }

    // gate and up as one stacked projection of 2I output columns per slot
    PrefillArgs ga{};
    ga.tiles = pb.tiles;
    ga.n_tiles = pb.n_tiles;
    ga.placement_pos = mb.placement_pos;
    ga.codes = mb.xq;
    ga.scales = mb.xs;
    ga.K = H;
    ga.R = 2 * I;
    ga.R1 = I;
    ga.rows = rows;
    ga.max_tiles = max_tiles;
    ga.out = pb.hidden;
    ga.flags = flags;
    int t = timer_begin(K_PREFILL_GATEUP, stream);
    launch_prefill_projection(ga, PF_NSUB_GATEUP, stream);
    timer_end(t, stream);
    // bf16-staged SwiGLU + re-quantisation of the hidden per (placement, 128 group)
    const uint32_t groups = P * (I >> 7);
    t = timer_begin(K_MOE_SWIGLU, stream);
    const uint32_t gpr = I >> 7;
    const uint32_t gpr_shift = (gpr & (gpr - 1)) == 0 ? (uint32_t)__builtin_ctz(gpr) : 32u;
    hipLaunchKernelGGL(prefill_swiglu_quant_kernel, dim3((groups + 16 * SWQ_GPT - 1) / (16 * SWQ_GPT)), dim3(256), 0,
                       stream, pb.hidden, P, I, gpr_shift, pb.silu, mb.hq, mb.hs, flags);
    timer_end(t, stream);

    PrefillArgs da = ga;
    da.placement_pos = nullptr;
    da.codes = mb.hq;
    da.scales = mb.hs;
    da.K = I;
    da.R = H;
    da.R1 = H;
    da.rows = P;
    da.out = pb.y;
    t = timer_begin(K_PREFILL_DOWN, stream);
    launch_prefill_projection(da, PF_NSUB_DOWN, stream);
    timer_end(t, stream);

    const uint32_t n8 = rows * (H >> 3);
    t = timer_begin(K_MOE_COMBINE, stream);
    hipLaunchKernelGGL(prefill_combine_kernel, dim3((n8 + 255) / 256), dim3(256), 0, stream, pb.y, mb.placement_w,
                       mb.row_slots, rows, H, mb.plan, out_f32, out_bf16, raw ? 1u : 0u, flags);
    timer_end(t, stream);
}

}  // namespace pw
