// Routed-MoE decode layer on gfx950: schedule, fused gate/up + SwiGLU, down projection and the
// router-weighted combine.
//
// Reference path: WideMetalMoeRuntime::execute_configured (src/wide_metal_moe.rs:852-1314) runs,
// per routed expert in ascending id, quantise -> gate -> up -> SwiGLU -> quantise -> down ->
// round -> scatter-add, then one final bf16 round. Its CPU authorities are routed_mlp_traced
// (src/text_endpoint.rs:5290-5381, mode B) and the f32 CPU control of src/lib.rs:5807-5862
// (mode A).
//
// Here one launch covers every routed expert of the layer. The schedule is built on the device
// from the route buffers (ids + weights per token), in the reference's BTreeMap order: experts
// ascending, positions ascending inside an expert. A tile is (active expert, 16 weight rows); its
// workgroup reads those weight rows exactly once for all of that expert's routed token rows
// (1..32), which is the reference's "one weight read amortised over all routed tokens". Gate and
// up rows of the same intermediate index share a tile, so SwiGLU happens in registers on the MFMA
// accumulators. The down projection writes one f32 row per placement, and the combine sums each
// token's eight placements in ascending expert id (the reference's order) before the bf16 round.
#include "pw_device.h"
#include "pw_launch.h"
#include "pw_route_job.h"
#include "pw_select_wave.h"

namespace pw {

// ------------------------------------------------------------------------------- schedule
// One workgroup (1024 threads, E <= 1024 experts). LDS holds a bit per (expert, token row): the
// rank of a placement inside its expert is the number of set bits below its row, so placements
// land in ascending row order without sorting (the reference's BTreeMap<expert, [(position,
// weight)]>, src/text_endpoint.rs:4767-4775). Counts and offsets come from block-wide scans; a
// per-(expert, 32-row word) prefix of the counts (when it fits in LDS) makes each rank O(1).
// Token rows are handled one per thread: their eight ids and weights are read once.
struct RouteRow {
    uint32_t e[8];
    float w[8];
};

__device__ __forceinline__ RouteRow load_route_row(const uint32_t *ids, const float *weights, uint32_t p)
{
    const uint4 i0 = *(const uint4 *)(ids + (size_t)p * 8), i1 = *(const uint4 *)(ids + (size_t)p * 8 + 4);
    const float4 w0 = *(const float4 *)(weights + (size_t)p * 8), w1 = *(const float4 *)(weights + (size_t)p * 8 + 4);
    return RouteRow{{i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w}, {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w}};
}

// Sets row p's bit in the mask word of each of its experts; true when a route is invalid (an id
// out of range, a non-finite weight, the same expert twice in one token's routes).
__device__ __forceinline__ bool mark_route_row(const RouteRow &rr, uint32_t p, uint32_t E, uint32_t words,
                                               uint32_t *mask)
{
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t e = rr.e[j];
        if (e >= E || !finite_f32(rr.w[j])) {
            bad = true;
            continue;
        }
        const uint32_t old = atomicOr(&mask[e * words + (p >> 5)], 1u << (p & 31));
        bad |= (old & (1u << (p & 31))) != 0;
    }
    return bad;
}

// Row p's placements: slot = expert offset + rank of p among the expert's rows.
__device__ __forceinline__ void place_route_row(const RouteRow &rr, uint32_t p, uint32_t E, uint32_t words,
                                                uint32_t P, uint32_t with_prefix, const uint32_t *mask,
                                                const uint16_t *pref, const uint32_t *offset,
                                                uint32_t *placement_pos, float *placement_w, uint32_t *row_slots)
{
    const uint32_t wd = p >> 5, below = (1u << (p & 31)) - 1u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t ei = rr.e[j];
        if (ei >= E || !finite_f32(rr.w[j]))
            continue;
        uint32_t rank = __popc(mask[ei * words + wd] & below);
        if (with_prefix) {
            rank += pref[ei * words + wd];
        } else {
            for (uint32_t w = 0; w < wd; ++w)
                rank += __popc(mask[ei * words + w]);
        }
        const uint32_t slot = offset[ei] + rank;
        if (slot >= P)
            continue;  // only when the routes were rejected
        placement_pos[slot] = p;
        placement_w[slot] = rr.w[j];
        // position of this placement among its token's eight, ordered by expert id
        uint32_t before = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            before += rr.e[k] < ei ? 1u : 0u;
        row_slots[(size_t)p * 8 + (before & 7)] = slot;
    }
}

__global__ __launch_bounds__(1024) void moe_schedule_kernel(
    const ExpertPtrs *__restrict__ bank, const uint32_t *__restrict__ ids,
    const float *__restrict__ weights, uint32_t rows, uint32_t E, uint32_t max_active, uint32_t with_prefix,
    MoePlan *plan, uint32_t *__restrict__ active_expert, uint32_t *__restrict__ active_offset,
    ActiveExpert *__restrict__ active, uint32_t *__restrict__ placement_pos, float *__restrict__ placement_w,
    uint32_t *__restrict__ row_slots, uint32_t *flags)
{
    extern __shared__ uint32_t lds[];
    const uint32_t words = (rows + 31) >> 5;
    uint32_t *mask = lds;                              // [E][words]
    uint32_t *offset = mask + E * words;               // [E]
    uint16_t *pref = (uint16_t *)(offset + E);         // [E][words] set bits in earlier words
    __shared__ uint32_t s_bad, s_max, s_scan[48];
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t P = rows * 8;
    // the loads every later phase waits on go out first: this thread's token row (kept in
    // registers when every row has its own thread) and its expert's weight pointers
    const bool one_pass = rows <= nthr;
    RouteRow mine{};
    if (one_pass && tid < rows)
        mine = load_route_row(ids, weights, tid);
    // this thread's expert's ExpertPtrs (48 bytes) in three native vectors (a struct or array copy
    // held across the barriers below would be kept in scratch memory)
    u32x4 ep0 = {0u, 0u, 0u, 0u}, ep1 = ep0, ep2 = ep0;
    if (tid < E) {
        const u32x4 *src = (const u32x4 *)(bank + tid);
        ep0 = src[0];
        ep1 = src[1];
        ep2 = src[2];
    }
    if (tid == 0) {
        s_bad = 0;
        s_max = 0;
    }
    for (uint32_t i = tid; i < E * words; i += nthr)
        mask[i] = 0;
    __syncthreads();
    bool bad = false;
    if (one_pass) {
        if (tid < rows)
            bad = mark_route_row(mine, tid, E, words, mask);
    } else {
        for (uint32_t p = tid; p < rows; p += nthr)
            bad |= mark_route_row(load_route_row(ids, weights, p), p, E, words, mask);
    }
    if (bad)
        atomicOr(&s_bad, 1u);
    __syncthreads();
    // thread e: expert e's count, its slot offset and its index among the routed experts
    const uint32_t e = tid;
    uint32_t c = 0;
    if (e < E)
        for (uint32_t w = 0; w < words; ++w) {
            if (with_prefix)
                pref[e * words + w] = (uint16_t)c;
            c += __popc(mask[e * words + w]);
        }
    uint32_t total, n_active;
    const uint32_t off = block_exclusive_scan(c, s_scan, &total);
    const uint32_t act = block_exclusive_scan(c ? 1u : 0u, s_scan, &n_active);
    if (e < E) {
        offset[e] = off;
        if (c) {
            active_expert[act] = e;
            active_offset[act] = off;
            // token rows of the first 16 slots, ascending, packed two per word (static indices
            // only: a dynamically indexed register array would move to scratch memory)
            uint32_t tw[8] = {};
            uint32_t w = 0, bits = mask[e * words];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                while (!bits && w + 1 < words)
                    bits = mask[e * words + ++w];
                const uint32_t t = bits ? w * 32 + __builtin_ctz(bits) : 0u;
                tw[k >> 1] |= t << (16 * (k & 1));
                bits &= bits - 1;
            }
            if (act < max_active) {
                // ActiveExpert: ExpertPtrs, off, cnt, tok[16], pad[2] as six 16-byte stores
                u32x4 *dst = (u32x4 *)(active + act);
                dst[0] = ep0;
                dst[1] = ep1;
                dst[2] = ep2;
                dst[3] = u32x4{off, c, tw[0], tw[1]};
                dst[4] = u32x4{tw[2], tw[3], tw[4], tw[5]};
                dst[5] = u32x4{tw[6], tw[7], 0u, 0u};
            }
            atomicMax(&s_max, c);
        }
    }
    if (tid == 0)
        active_offset[n_active] = total;
    // entries past the last routed expert: cnt = 0, the projection workgroups exit at once
    for (uint32_t a = n_active + tid; a < max_active; a += nthr) {
        uint4 *dst = (uint4 *)(active + a);
#pragma unroll
        for (int i = 0; i < 6; ++i)
            dst[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    // every consumer index starts valid even when the route buffers are rejected
    if (s_bad || total != P)
        for (uint32_t i = tid; i < P; i += nthr) {
            placement_pos[i] = 0;
            placement_w[i] = 0.f;
            row_slots[i] = 0;
        }
    __syncthreads();
    if (one_pass) {
        if (tid < rows)
            place_route_row(mine, tid, E, words, P, with_prefix, mask, pref, offset, placement_pos, placement_w,
                            row_slots);
    } else {
        for (uint32_t p = tid; p < rows; p += nthr)
            place_route_row(load_route_row(ids, weights, p), p, E, words, P, with_prefix, mask, pref, offset,
                            placement_pos, placement_w, row_slots);
    }
    if (tid == 0) {
        plan->n_active = n_active;
        plan->n_placements = total;
        plan->max_count = s_max;
        plan->rejected = (s_bad || total != P) ? 1u : 0u;
        if (s_bad || total != P)
            raise_flag(flags, FLAG_SCHEDULE);
    }
}

// ------------------------------------------------------------------ long-batch schedule
// The same schedule for prefill-sized batches in three short launches over many workgroups (one
// workgroup would hold E x rows bits in LDS and do every step on one CU):
//   moe_sched_mark_kernel: one wave per 64 token rows checks its routes (as mark_route_row) and
//     writes the (expert, 32-row word) bitmap words and their popcounts;
//   moe_sched_plan_kernel: one workgroup forms each expert's count and per-word prefix counts,
//     the slot offsets and routed-expert tables (block scans in ascending expert id), the largest
//     count and the plan; its other workgroups, when given a QuantJob, quantise the activation
//     rows (64 groups of 128 columns each) on the CUs the one plan workgroup leaves idle;
//   moe_sched_place_kernel: one thread per token row writes its eight placements at
//     offset[e] + prefix[e][word] + (bits below the row in its word) -- ascending rows per
//     expert, as in moe_schedule_kernel -- and the token row of each of an expert's first 16
//     slots into its ActiveExpert entry.
// Rejected routes (an id >= E, a non-finite weight, an expert named twice by one token, or any
// count mismatch) raise FLAG_SCHEDULE and leave every placement table zero.
constexpr uint32_t SCHED_WG_MAX_ROWS = 128;  // longer batches take the three-launch schedule
constexpr uint32_t SCHED_MAX_WORDS = 128;     // 4096 rows

struct SchedScratch {
    uint32_t *mask;  // [E][W] row bits per (expert, 32-row word)
    uint8_t *cnt;    // [E][Wp] popcounts (Wp = W rounded up to 16)
    uint16_t *pref;  // [E][Wp] exclusive per-word prefix of the counts
    uint32_t *offs;  // [E] first slot of each expert
    uint32_t *acts;  // [E] index among the routed experts (~0 when not routed)
    uint32_t *badw;  // [ceil(rows / 64)] rejected routes per wave of rows
};

static inline size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

static SchedScratch sched_carve(void *base, uint32_t rows, uint32_t E, size_t *bytes)
{
    const size_t W = (rows + 31) / 32, Wp = (W + 15) & ~(size_t)15, nwg = (rows + 63) / 64;
    SchedScratch ss{};
    size_t at = 0;
    char *b = (char *)base;
    ss.mask = (uint32_t *)(b + at);
    at += align16(E * W * 4);
    ss.cnt = (uint8_t *)(b + at);
    at += align16(E * Wp);
    ss.pref = (uint16_t *)(b + at);
    at += align16(E * Wp * 2);
    ss.offs = (uint32_t *)(b + at);
    at += align16((size_t)E * 4);
    ss.acts = (uint32_t *)(b + at);
    at += align16((size_t)E * 4);
    ss.badw = (uint32_t *)(b + at);
    at += align16(nwg * 4);
    if (bytes)
        *bytes = at;
    return ss;
}

size_t moe_sched_scratch_bytes(uint32_t rows, uint32_t E)
{
    if (rows <= SCHED_WG_MAX_ROWS)
        return 0;
    size_t bytes = 0;
    (void)sched_carve(nullptr, rows, E, &bytes);
    return bytes;
}

__global__ __launch_bounds__(64) void moe_sched_mark_kernel(const uint32_t *__restrict__ ids,
                                                            const float *__restrict__ weights, uint32_t rows,
                                                            uint32_t E, SchedScratch ss)
{
    extern __shared__ uint32_t lmask[];  // [E][2]: the bitmap words of this wave's 64 rows
    const uint32_t lane = threadIdx.x, p = blockIdx.x * 64 + lane;
    const uint32_t W = (rows + 31) >> 5, Wp = (W + 15) & ~15u;
    const bool has = p < rows;
    RouteRow rr{};
    if (has)
        rr = load_route_row(ids, weights, p);
    for (uint32_t i = lane; i < 2 * E; i += 64)
        lmask[i] = 0u;
    __syncthreads();
    const bool bad = has && mark_route_row(rr, lane, E, 2, lmask);
    __syncthreads();
    const uint32_t w0 = blockIdx.x * 2;
    for (uint32_t i = lane; i < 2 * E; i += 64) {
        const uint32_t e = i >> 1, w = w0 + (i & 1);
        if (w < W) {
            const uint32_t m = lmask[i];
            ss.mask[(size_t)e * W + w] = m;
            ss.cnt[(size_t)e * Wp + w] = (uint8_t)__popc(m);
        }
    }
    const bool any = __ballot(bad) != 0;
    if (lane == 0)
        ss.badw[blockIdx.x] = any ? 1u : 0u;
}

// With a tile table (tt.tiles non-null), also the prefill's m-tiles: ceil(count / PREFILL_MT) per
// routed expert in ascending expert order, each with the expert's weights and its slots (none
// when the routes are rejected).
__global__ __launch_bounds__(1024) void moe_sched_plan_kernel(
    const ExpertPtrs *__restrict__ bank, uint32_t rows, uint32_t E, uint32_t max_active, SchedScratch ss,
    MoePlan *plan, uint32_t *__restrict__ active_expert, uint32_t *__restrict__ active_offset,
    ActiveExpert *__restrict__ active, uint32_t *__restrict__ placement_pos, float *__restrict__ placement_w,
    uint32_t *__restrict__ row_slots, uint32_t *flags, PfTileTable tt, QuantJob qj)
{
    if (blockIdx.x > 0) {
        const uint32_t group = (blockIdx.x - 1) * 64 + (threadIdx.x >> 4);
        if (group < qj.rows * (qj.K >> 7)) {  // whole 16-lane groups leave together
            if (qj.f32)
                quant_group128_team((const float *)qj.x, group, threadIdx.x & 15, qj.codes, qj.scales, flags);
            else
                quant_group128_team((const uint16_t *)qj.x, group, threadIdx.x & 15, qj.codes, qj.scales, flags);
        }
        return;
    }
    __shared__ uint32_t s_scan[48], s_bad, s_max;
    const uint32_t tid = threadIdx.x, e = tid;
    const uint32_t W = (rows + 31) >> 5, Wp = (W + 15) & ~15u, nwg = (rows + 63) >> 6;
    const uint32_t P = rows * 8;
    // the loads every later step waits on go out first: this expert's weight pointers and all of
    // its per-word counts (W <= 128: at most eight 16-byte loads)
    u32x4 ep0 = {0u, 0u, 0u, 0u}, ep1 = ep0, ep2 = ep0;
    uint4 cv[SCHED_MAX_WORDS / 16];
    if (e < E) {
        const u32x4 *src = (const u32x4 *)(bank + e);
        ep0 = src[0];
        ep1 = src[1];
        ep2 = src[2];
        const uint4 *crow = (const uint4 *)(ss.cnt + (size_t)e * Wp);
#pragma unroll
        for (uint32_t g = 0; g < SCHED_MAX_WORDS / 16; ++g)
            cv[g] = g * 16 < W ? crow[g] : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid == 0) {
        s_bad = 0;
        s_max = 0;
    }
    __syncthreads();
    for (uint32_t i = tid; i < nwg; i += blockDim.x)
        if (ss.badw[i])
            atomicOr(&s_bad, 1u);
    // expert e's count and the exclusive prefix of its per-word counts (words past W count 0)
    uint32_t c = 0;
    if (e < E) {
        uint4 *prow = (uint4 *)(ss.pref + (size_t)e * Wp);
#pragma unroll
        for (uint32_t g = 0; g < SCHED_MAX_WORDS / 16; ++g) {
            const uint32_t b[4] = {cv[g].x, cv[g].y, cv[g].z, cv[g].w};
            uint32_t pr[8];
#pragma unroll
            for (uint32_t k = 0; k < 16; ++k) {
                const uint32_t n = g * 16 + k < W ? (b[k >> 2] >> (8 * (k & 3))) & 0xffu : 0u;
                if (k & 1)
                    pr[k >> 1] |= c << 16;
                else
                    pr[k >> 1] = c;
                c += n;
            }
            if (g * 16 < W) {
                prow[2 * g] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
                prow[2 * g + 1] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
            }
        }
    }
    uint32_t total, n_active;
    const uint32_t off = block_exclusive_scan(c, s_scan, &total);
    const uint32_t act = block_exclusive_scan(c ? 1u : 0u, s_scan, &n_active);
    if (e < E) {
        ss.offs[e] = off;
        ss.acts[e] = c ? act : 0xffffffffu;
        if (c) {
            active_expert[act] = e;
            active_offset[act] = off;
            if (act < max_active) {
                // ExpertPtrs, off, cnt, then tok[16] (the place kernel fills it) and the pad
                u32x4 *dst = (u32x4 *)(active + act);
                dst[0] = ep0;
                dst[1] = ep1;
                dst[2] = ep2;
                dst[3] = u32x4{off, c, 0u, 0u};
                dst[4] = u32x4{0u, 0u, 0u, 0u};
                dst[5] = u32x4{0u, 0u, 0u, 0u};
            }
            atomicMax(&s_max, c);
        }
    }
    if (tid == 0)
        active_offset[n_active] = total;
    for (uint32_t a = n_active + tid; a < max_active; a += blockDim.x) {
        uint4 *dst = (uint4 *)(active + a);
#pragma unroll
        for (int i = 0; i < 6; ++i)
            dst[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    const bool rejected = s_bad != 0 || total != P;
    if (tt.tiles) {
        const uint32_t live = e < E && c && act < max_active ? c : 0u;
        const uint32_t nt = (live + PREFILL_MT - 1) / PREFILL_MT;
        uint32_t n_tiles;
        const uint32_t first = block_exclusive_scan(nt, s_scan, &n_tiles);
        for (uint32_t i = 0; i < nt; ++i)
            if (first + i < tt.max_tiles) {
                u32x4 *dst = (u32x4 *)(tt.tiles + first + i);
                dst[0] = ep0;
                dst[1] = ep1;
                dst[2] = ep2;
                dst[3] = u32x4{off + i * PREFILL_MT, live - i * PREFILL_MT < PREFILL_MT ? live - i * PREFILL_MT
                                                                                       : PREFILL_MT, e, 0u};
            }
        if (tid == 0) {
            tt.n_tiles[0] = rejected ? 0u : (n_tiles < tt.max_tiles ? n_tiles : tt.max_tiles);
            if (n_tiles > tt.max_tiles)
                raise_flag(flags, FLAG_SCHEDULE);
        }
    }
    if (rejected)
        for (uint32_t i = tid; i < P; i += blockDim.x) {
            placement_pos[i] = 0;
            placement_w[i] = 0.f;
            row_slots[i] = 0;
        }
    if (tid == 0) {
        plan->n_active = n_active;
        plan->n_placements = total;
        plan->max_count = s_max;
        plan->rejected = rejected ? 1u : 0u;
        if (rejected)
            raise_flag(flags, FLAG_SCHEDULE);
    }
}

__global__ __launch_bounds__(64) void moe_sched_place_kernel(
    const uint32_t *__restrict__ ids, const float *__restrict__ weights, uint32_t rows, uint32_t E,
    uint32_t max_active, SchedScratch ss, const MoePlan *__restrict__ plan, ActiveExpert *__restrict__ active,
    uint32_t *__restrict__ placement_pos, float *__restrict__ placement_w, uint32_t *__restrict__ row_slots)
{
    const uint32_t p = blockIdx.x * 64 + threadIdx.x;
    if (p >= rows || plan->rejected)
        return;  // rejected: the plan kernel left the tables zero
    const uint32_t W = (rows + 31) >> 5, Wp = (W + 15) & ~15u, P = rows * 8;
    const RouteRow rr = load_route_row(ids, weights, p);
    const uint32_t wd = p >> 5, below = (1u << (p & 31)) - 1u;
    // every table load of the eight placements first (accepted routes: every id < E)
    uint32_t m[8], pr[8], off[8], ac[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t e = rr.e[j] < E ? rr.e[j] : 0u;
        m[j] = ss.mask[(size_t)e * W + wd];
        pr[j] = ss.pref[(size_t)e * Wp + wd];
        off[j] = ss.offs[e];
        ac[j] = ss.acts[e];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t ei = rr.e[j];
        const uint32_t rank = pr[j] + __popc(m[j] & below);
        const uint32_t slot = off[j] + rank;
        if (ei >= E || slot >= P)
            continue;
        placement_pos[slot] = p;
        placement_w[slot] = rr.w[j];
        // position of this placement among its token's eight, ordered by expert id
        uint32_t before = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            before += rr.e[k] < ei ? 1u : 0u;
        row_slots[(size_t)p * 8 + (before & 7)] = slot;
        if (rank < 16 && ac[j] < max_active)
            active[ac[j]].tok[rank] = (uint16_t)p;
    }
}

// Per-expert slot ranges from the routed-expert tables: expert e's placements are
// [off[e], off[e + 1]) and off[E] is the placement count. One thread per entry: the first routed
// expert with id >= e, by binary search over active_expert[0, U) (ascending ids).
__global__ __launch_bounds__(256) void expert_offsets_kernel(const MoePlan *__restrict__ plan,
                                                             const uint32_t *__restrict__ active_expert,
                                                             const uint32_t *__restrict__ active_offset, uint32_t E,
                                                             uint32_t *__restrict__ off)
{
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e > E)
        return;
    const uint32_t U = plan->n_active < E ? plan->n_active : E;
    uint32_t lo = 0, hi = U;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (active_expert[mid] < e)
            lo = mid + 1;
        else
            hi = mid;
    }
    off[e] = active_offset[lo];
}

void launch_expert_offsets(const MoeBuffers &mb, uint32_t E, uint32_t *expert_offsets, hipStream_t stream)
{
    hipLaunchKernelGGL(expert_offsets_kernel, dim3((E + 1 + 255) / 256), dim3(256), 0, stream, mb.plan,
                       mb.active_expert, mb.active_offset, E, expert_offsets);
}

// Rows per projection entry when the one-wave schedule cuts experts into pieces.
constexpr uint32_t PIECE_ROWS = 4;

// The schedule of a decode batch runs in one wave (moe_schedule_wave_kernel) under these bounds.
static bool wave_schedule(uint32_t rows, uint32_t E, uint32_t max_active)
{
    return rows <= 8 && E <= 1024 && max_active <= 64;
}

// ------------------------------------------------------------------ decode-batch schedule
// The same schedule for a decode batch (rows <= 8, so at most 64 placements: one per lane) in one
// wave, with no workgroup barriers: a bitmap of the routed expert ids in LDS ranks each placement's
// expert among the routed ones (ascending id, the BTreeMap order), and every per-expert table is
// then filled lane-parallel (lane a: the a-th routed expert). Route rejection follows
// moe_schedule_kernel: an id >= E, a non-finite weight or a token naming one expert twice raises
// FLAG_SCHEDULE and leaves the placement tables zeroed.
// LDS of the one-wave schedule besides the bank's pointer table.
struct alignas(16) SchedWaveLds {
    uint32_t bitmap[32];      // routed expert ids (E <= 1024)
    uint32_t expert_of[64];   // by rank
    uint32_t route[64];       // lane p's expert id where its route is valid, else NO_ROUTE
    uint32_t rows_of[1024];   // bit r: token row r routes to the expert (valid routes only)
    uint16_t tok_of[64 * 16]; // token rows of each expert's first 16 placements
};
constexpr uint32_t NO_ROUTE = 0xffffffffu;

// Orders the LDS accesses of one wave's lanes (its LDS operations complete in order; this waits for
// them and keeps the compiler from moving memory accesses across).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// The one-wave schedule on lane a's route (id, w) (lanes a < rows * 8; the rest pass zeros), with
// the bank's pointer table already in lds_bank (E x 48 bytes) and visible to this wave. Only this
// wave touches `lds`, so it needs no workgroup barrier (the routed-layer entry that selects the
// routes runs it after its other waves have left).
//
// Lane p = 8 r + k holds route k of token row r. Its slot (lower expert ids first, then lower token
// rows) is the placements of the experts ranked below its own plus the earlier token rows routed to
// its expert: the set bits below r of rows_of[id] (a token row names an expert at most once among
// its valid routes).
__device__ __forceinline__ void schedule_wave_body(
    uint32_t id, float w, uint32_t rows, uint32_t E, uint32_t max_active, const u32x4 *lds_bank, SchedWaveLds &lds,
    MoePlan *plan, uint32_t *__restrict__ active_expert, uint32_t *__restrict__ active_offset,
    ActiveExpert *__restrict__ active, uint32_t *__restrict__ placement_pos, float *__restrict__ placement_w,
    uint32_t *__restrict__ row_slots, ActiveExpert *__restrict__ pieces, uint32_t max_pieces, uint32_t *flags)
{
    uint32_t *bitmap = lds.bitmap, *expert_of = lds.expert_of, *rows_of = lds.rows_of;
    uint16_t *tok_of = lds.tok_of;
    const int lane = threadIdx.x & 63;
    const uint32_t P = rows * 8;
    const uint32_t nw = (E + 31) >> 5;
    const uint32_t r = (uint32_t)lane >> 3, k = (uint32_t)lane & 7;
    if ((uint32_t)lane < nw)
        bitmap[lane] = 0u;
    u32x4 *tz = (u32x4 *)tok_of + 2 * lane;
    tz[0] = u32x4{0u, 0u, 0u, 0u};
    tz[1] = u32x4{0u, 0u, 0u, 0u};
    bool ok = (uint32_t)lane < P && id < E && finite_f32(w);
    lds.route[lane] = ok ? id : NO_ROUTE;
    if (id < E)
        rows_of[id] = 0u;
    wave_lds_sync();
    // the token row's eight routes; a token naming one expert twice: the later slot is rejected
    const u32x4 g0 = ((const u32x4 *)lds.route)[2 * r], g1 = ((const u32x4 *)lds.route)[2 * r + 1];
    const uint32_t grp[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    bool dup = false;
    uint32_t before = 0;  // the token row's valid routes to lower expert ids
#pragma unroll
    for (uint32_t m = 0; m < 8; ++m) {
        dup |= m < k && grp[m] == id;
        before += grp[m] < id ? 1u : 0u;
    }
    ok &= !dup;
    const bool bad = __ballot((uint32_t)lane < P && !ok) != 0;
    if (ok) {
        atomicOr(&bitmap[id >> 5], 1u << (id & 31));
        atomicOr(&rows_of[id], 1u << r);
    }
    wave_lds_sync();
    // rank of this lane's expert: routed ids below it
    const uint32_t word = (uint32_t)lane < nw ? bitmap[lane] : 0u;
    const uint32_t wc = __popc(word);
    const uint32_t wincl = wave_inclusive_scan(wc);
    const uint32_t U = __builtin_amdgcn_readlane(wincl, 63);
    const int src = ok ? (int)(id >> 5) : 0;
    const uint32_t wsel = __shfl(word, src, 64), esel = __shfl(wincl - wc, src, 64);
    const uint32_t rank = ok ? esel + __popc(wsel & ((1u << (id & 31)) - 1u)) : 0u;
    const uint32_t mine = ok ? rows_of[id] : 0u;
    if (ok)
        expert_of[rank] = id;
    wave_lds_sync();
    // lane a: the a-th routed expert
    const uint32_t a = (uint32_t)lane;
    const uint32_t e_a = a < U ? expert_of[a] : 0u;
    const uint32_t c_a = a < U ? __popc(rows_of[e_a]) : 0u;
    const uint32_t incl = wave_inclusive_scan(c_a);
    const uint32_t off_a = incl - c_a, total = __builtin_amdgcn_readlane(incl, 63);
    // this placement's index inside its expert -> token row table, and its slot
    const uint32_t t = __popc(mine & ((1u << r) - 1u));
    const uint32_t slot = (uint32_t)__shfl((int)off_a, (int)rank, 64) + t;
    if (ok && t < 16)
        tok_of[rank * 16 + t] = (uint16_t)r;
    wave_lds_sync();
    u32x4 ep0 = {0u, 0u, 0u, 0u}, ep1 = ep0, ep2 = ep0;
    if (a < U && a < max_active) {
        ep0 = lds_bank[e_a * 3];
        ep1 = lds_bank[e_a * 3 + 1];
        ep2 = lds_bank[e_a * 3 + 2];
    }
    if (a < max_active) {
        uint32_t tw[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            tw[k] = a < U ? (uint32_t)tok_of[a * 16 + 2 * k] | ((uint32_t)tok_of[a * 16 + 2 * k + 1] << 16) : 0u;
        u32x4 *dst = (u32x4 *)(active + a);
        dst[0] = ep0;
        dst[1] = ep1;
        dst[2] = ep2;
        dst[3] = u32x4{a < U ? off_a : 0u, c_a, tw[0], tw[1]};
        dst[4] = u32x4{tw[2], tw[3], tw[4], tw[5]};
        dst[5] = u32x4{tw[6], tw[7], 0u, 0u};
    }
    if (a < U) {
        active_expert[a] = e_a;
        active_offset[a] = off_a;
    }
    if (lane == 0)
        active_offset[U] = total;
    // the projections' entries: each routed expert's slots in pieces of at most PIECE_ROWS, so
    // their LDS stages are sized for that many rows (see launch_a_moe); a piece carries its slots'
    // token rows (slots 0..15 of an expert: PIECE_ROWS * pieces <= 16 here)
    const uint32_t np = (c_a + PIECE_ROWS - 1) / PIECE_ROWS;  // 0 past the routed experts
    const uint32_t pincl = wave_inclusive_scan(np);
    const uint32_t pbase = pincl - np, npieces = __builtin_amdgcn_readlane(pincl, 63);
    for (uint32_t i = 0; i < np; ++i) {
        if (pbase + i < max_pieces) {
            const uint32_t left = c_a - i * PIECE_ROWS;
            const uint32_t pc = left < PIECE_ROWS ? left : PIECE_ROWS;
            const uint16_t *tk = tok_of + a * 16 + i * PIECE_ROWS;
            u32x4 *dst = (u32x4 *)(pieces + pbase + i);
            dst[0] = ep0;
            dst[1] = ep1;
            dst[2] = ep2;
            dst[3] = u32x4{off_a + i * PIECE_ROWS, pc, (uint32_t)tk[0] | ((uint32_t)tk[1] << 16),
                           (uint32_t)tk[2] | ((uint32_t)tk[3] << 16)};
            dst[4] = u32x4{0u, 0u, 0u, 0u};
            dst[5] = u32x4{0u, 0u, 0u, 0u};
        }
    }
    for (uint32_t d = npieces + (uint32_t)lane; d < max_pieces; d += 64) {
        u32x4 *dst = (u32x4 *)(pieces + d);
#pragma unroll
        for (int i = 0; i < 6; ++i)
            dst[i] = u32x4{0u, 0u, 0u, 0u};
    }
    if ((uint32_t)lane < P) {
        if (bad) {
            placement_pos[lane] = 0;
            placement_w[lane] = 0.f;
            row_slots[lane] = 0;
        } else {
            placement_pos[slot] = (uint32_t)lane >> 3;
            placement_w[slot] = w;
            row_slots[(size_t)(lane >> 3) * 8 + (before & 7)] = slot;
        }
    }
    const uint32_t mx = wave_max_u32(c_a);
    if (lane == 0) {
        plan->n_active = U;
        plan->n_placements = total;
        plan->max_count = mx;
        plan->rejected = bad ? 1u : 0u;
        if (bad)
            raise_flag(flags, FLAG_SCHEDULE);
    }
}


__global__ __launch_bounds__(64) void moe_schedule_wave_kernel(
    const ExpertPtrs *__restrict__ bank, const uint32_t *__restrict__ ids, const float *__restrict__ weights,
    uint32_t rows, uint32_t E, uint32_t max_active, MoePlan *plan, uint32_t *__restrict__ active_expert,
    uint32_t *__restrict__ active_offset, ActiveExpert *__restrict__ active, uint32_t *__restrict__ placement_pos,
    float *__restrict__ placement_w, uint32_t *__restrict__ row_slots, ActiveExpert *__restrict__ pieces,
    uint32_t max_pieces, uint32_t *flags, const QuantJob qj)
{
    extern __shared__ u32x4 lds_bank[];  // the bank's ExpertPtrs table, E x 48 bytes
    __shared__ SchedWaveLds sl;
    const int lane = threadIdx.x;
    if (blockIdx.x > 0) {
        // workgroups 1.. quantise the activation rows of qj (four 128-column groups each) while
        // workgroup 0 schedules
        const uint32_t group = (blockIdx.x - 1) * 4 + ((uint32_t)lane >> 4);
        if (group < qj.rows * (qj.K >> 7)) {
            if (qj.f32)
                quant_group128_team<float>((const float *)qj.x, group, lane & 15, qj.codes, qj.scales, flags);
            else
                quant_group128_team<uint16_t>((const uint16_t *)qj.x, group, lane & 15, qj.codes, qj.scales, flags);
        }
        return;
    }
    const uint32_t P = rows * 8;
    // the routes and the whole pointer table go out together (one memory round trip in all)
    uint32_t id = 0;
    float w = 0.f;
    if ((uint32_t)lane < P) {
        id = ids[lane];
        w = weights[lane];
    }
    const uint32_t units = E * 3;  // 16-byte units of the table
    for (uint32_t u0 = 0; u0 < units; u0 += 64)
        if (u0 + (uint32_t)lane < units)
            lds_load16((const u32x4 *)bank + u0 + lane, lds_bank + u0);
    __builtin_amdgcn_s_waitcnt(0);  // the table copy has landed in LDS (and the routes are in)
    schedule_wave_body(id, w, rows, E, max_active, lds_bank, sl, plan, active_expert, active_offset, active,
                       placement_pos, placement_w, row_slots, pieces, max_pieces, flags);
}

// Row p's eight experts into ids[0..7] by one wave: fast_top8_set (ascending ids), or where that
// cannot decide, select_route_row (its order; ids E when the row's routing fails).
template <int NC>
__device__ __forceinline__ void row_expert_set(const float *scores_row, const float *bias, uint32_t E, TopkEntry *pairs,
                                               uint32_t *ids)
{
    DeviceWave w;
    if (fast_top8_set<NC>(w, scores_row, bias, E, ids))
        return;
    uint32_t sel_k;
    float w_k;
    bool tie = false;
    const int st = select_route_row<NC>(w, scores_row, bias, E, pairs, sel_k, w_k, &tie);
    if (w.lane() < 8)
        ids[w.lane()] = st == ROUTE_OK ? sel_k : E;
}

// The expert sets alone (a one-token batch's direct layer reads them as its routes): one wave per
// row, row_expert_set into set_ids [rows][8].
template <int NC>
__global__ __launch_bounds__(64) void route_set_kernel(const float *__restrict__ scores, const float *__restrict__ bias,
                                                       uint32_t rows, uint32_t E, uint32_t *__restrict__ set_ids)
{
    __shared__ TopkEntry pairs[64 * NC];
    if (blockIdx.x < rows)
        row_expert_set<NC>(scores + (size_t)blockIdx.x * E, bias, E, pairs, set_ids + (size_t)blockIdx.x * 8);
}

void launch_route_set(const float *scores, const float *bias, uint32_t rows, uint32_t E, uint32_t *set_ids,
                      hipStream_t stream)
{
    if (E <= 64) hipLaunchKernelGGL(route_set_kernel<1>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, set_ids);
    else if (E <= 128) hipLaunchKernelGGL(route_set_kernel<2>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, set_ids);
    else if (E <= 256) hipLaunchKernelGGL(route_set_kernel<4>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, set_ids);
    else if (E <= 512) hipLaunchKernelGGL(route_set_kernel<8>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, set_ids);
    else hipLaunchKernelGGL(route_set_kernel<16>, dim3(rows), dim3(64), 0, stream, scores, bias, rows, E, set_ids);
}

// A decode batch's expert sets and its schedule in one launch, the route weights left to
// route_weights_kernel. Wave r < rows finds row r's eight experts with fast_top8_set (the set
// select_route_row selects, found without the partition when the row's boundary is not tied);
// a row with a tied boundary or a non-finite value runs select_route_row itself (failing rows get
// ids E, which the schedule rejects). Wave 0 then builds the schedule from the sets with weights
// 0 in place of the route weights, and writes the sets to set_ids for the weights kernel's
// check. With a QuantJob, workgroups 1.. quantise its activation rows (mode B) meanwhile.
template <int NC>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void route_set_schedule_kernel(
    const float *__restrict__ scores, const float *__restrict__ bias, const ExpertPtrs *__restrict__ bank,
    uint32_t rows, uint32_t E, uint32_t max_active, uint32_t *__restrict__ set_ids, MoePlan *plan,
    uint32_t *__restrict__ active_expert, uint32_t *__restrict__ active_offset, ActiveExpert *__restrict__ active,
    uint32_t *__restrict__ placement_pos, float *__restrict__ placement_w, uint32_t *__restrict__ row_slots,
    ActiveExpert *__restrict__ pieces, uint32_t max_pieces, uint32_t *flags, const QuantJob qj)
{
    extern __shared__ u32x4 lds_bank[];  // the bank's ExpertPtrs table, E x 48 bytes
    __shared__ TopkEntry pairs[8][64 * NC];
    __shared__ uint32_t r_id[64];
    __shared__ SchedWaveLds sl;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (blockIdx.x > 0) {
        // 32 128-column groups per workgroup (16 lanes each)
        const uint32_t group = (blockIdx.x - 1) * 32 + (threadIdx.x >> 4);
        if (group < qj.rows * (qj.K >> 7)) {
            if (qj.f32)
                quant_group128_team<float>((const float *)qj.x, group, lane & 15, qj.codes, qj.scales, flags);
            else
                quant_group128_team<uint16_t>((const uint16_t *)qj.x, group, lane & 15, qj.codes, qj.scales, flags);
        }
        return;
    }
    const uint32_t units = E * 3;  // 16-byte units of the table
    for (uint32_t u0 = wave * 64; u0 < units; u0 += 512)
        if (u0 + lane < units)
            lds_load16((const u32x4 *)bank + u0 + lane, lds_bank + u0);
    if (wave < rows)
        row_expert_set<NC>(scores + (size_t)wave * E, bias, E, pairs[wave], r_id + wave * 8);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the table copy has landed in LDS
    __syncthreads();
    if (wave != 0)
        return;
    const uint32_t P = rows * 8;
    const uint32_t id = lane < P ? r_id[lane] : 0u;
    if (lane < P)
        set_ids[lane] = id;
    schedule_wave_body(id, 0.0f, rows, E, max_active, lds_bank, sl, plan, active_expert, active_offset, active,
                       placement_pos, placement_w, row_slots, pieces, max_pieces, flags);
}

bool launch_route_set_schedule(const float *scores, const float *bias, const ExpertPtrs *bank, uint32_t rows,
                               uint32_t E, uint32_t max_active, uint32_t *set_ids, const MoeBuffers &mb,
                               uint32_t *flags, hipStream_t stream, const QuantJob *quant)
{
    if (rows < 1 || rows > 8 || E < 9 || E > 256 || max_active > 64)
        return false;
    const size_t table = (size_t)E * sizeof(ExpertPtrs);  // <= 12 KB
    const QuantJob qj = quant ? *quant : QuantJob{};
    const uint32_t quant_wgs = (qj.rows * (qj.K >> 7) + 31) / 32;
    const int t = timer_begin(K_ROUTE_SCHEDULE, stream);
#define PW_RSS(NC)                                                                                                 \
    hipLaunchKernelGGL(route_set_schedule_kernel<NC>, dim3(1 + quant_wgs), dim3(512), table, stream, scores, bias,  \
                       bank, rows, E, max_active, set_ids, mb.plan, mb.active_expert, mb.active_offset, mb.active,  \
                       mb.placement_pos, mb.placement_w, mb.row_slots, mb.pieces, rows * 8, flags, qj)
    if (E <= 64) PW_RSS(1);
    else if (E <= 128) PW_RSS(2);
    else PW_RSS(4);
#undef PW_RSS
    timer_end(t, stream);
    return true;
}

// The route weights of a batch scheduled by route_set_schedule_kernel as a launch of its own (when
// no expert launch of the layer carries them): one wave per row (route_weights_row).
template <int NC>
__global__ __launch_bounds__(64) void route_weights_kernel(const RouteJob job)
{
    __shared__ TopkEntry lds_pairs[64 * NC];
    if (blockIdx.x < job.rows)
        route_weights_row<NC>(job, blockIdx.x, lds_pairs);
}

void launch_route_weights(const RouteJob &job, hipStream_t stream)
{
    if (job.E <= 64) hipLaunchKernelGGL(route_weights_kernel<1>, dim3(job.rows), dim3(64), 0, stream, job);
    else if (job.E <= 128) hipLaunchKernelGGL(route_weights_kernel<2>, dim3(job.rows), dim3(64), 0, stream, job);
    else hipLaunchKernelGGL(route_weights_kernel<4>, dim3(job.rows), dim3(64), 0, stream, job);
}

// --------------------------------------------------------------- shared tile preamble
struct ExpertTile {
    ExpertPtrs ep;
    uint32_t off;    // first placement slot of this expert
    uint32_t cnt;    // placements of this expert
    bool live;
};

__device__ __forceinline__ ExpertTile expert_tile(const MoePlan *plan, const uint32_t *active_expert,
                                                  const uint32_t *active_offset, const ExpertPtrs *bank,
                                                  uint32_t a)
{
    ExpertTile t;
    t.live = a < plan->n_active;
    if (!t.live)
        return t;
    const uint32_t e = active_expert[a];
    t.off = active_offset[a];
    t.cnt = active_offset[a + 1] - t.off;
    t.ep = bank[e];
    return t;
}

// Deterministic cross-wave sum (wave order 0..KSPLIT-1) of NT x f32x4 per lane, result in wave 0.
template <int KSPLIT, int NT>
__device__ __forceinline__ void reduce_waves(f32x4 (*red)[NT][64], f32x4 *v, int wave, int lane)
{
    if constexpr (KSPLIT > 1) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            red[wave][nt][lane] = v[nt];
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                f32x4 s = red[0][nt][lane];
                for (int w = 1; w < KSPLIT; ++w) {
                    const f32x4 o = red[w][nt][lane];
                    s[0] += o[0]; s[1] += o[1]; s[2] += o[2]; s[3] += o[3];
                }
                v[nt] = s;
            }
        }
    }
}

// ------------------------------------------------------------- mode B, gate/up + SwiGLU
// block_fp8_gemm{count}_sglang_blockscaled gate and up, then bf16_staged_swiglu
// (kernels/block_fp8_gemv.metal:139-160, :935-1046; fused twin :1048-1186).
template <int KSPLIT, int NT>
__global__ __launch_bounds__(64 * KSPLIT) void moe_b_gateup_kernel(
    const ExpertPtrs *__restrict__ bank, const MoePlan *__restrict__ plan,
    const uint32_t *__restrict__ active_expert, const uint32_t *__restrict__ active_offset,
    const uint32_t *__restrict__ placement_pos, const uint8_t *__restrict__ xq,
    const float *__restrict__ xs, uint32_t rows, uint32_t H, uint32_t I, float *__restrict__ hidden,
    uint32_t *flags)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    __shared__ f32x4 red_g[KSPLIT][NT][64];
    __shared__ f32x4 red_u[KSPLIT][NT][64];
    const uint32_t tiles_per_expert = I >> 4;
    // XCD x (workgroup i runs on XCD i % 8) takes a contiguous eighth of each expert's row tiles
    const uint32_t a = blockIdx.x / tiles_per_expert, lt = blockIdx.x % tiles_per_expert;
    const uint32_t rt = tiles_per_expert % 8 == 0 ? (lt % 8) * (tiles_per_expert / 8) + lt / 8 : lt;
    const ExpertTile et = expert_tile(plan, active_expert, active_offset, bank, a);
    if (!et.live)
        return;
    if (et.cnt > 16u * NT) {
        if (threadIdx.x == 0)
            raise_flag(flags, FLAG_SCHEDULE);
        return;
    }
    const uint32_t row0 = rt << 4;
    const uint32_t blocks = H >> 7;
    const uint8_t *grow = et.ep.gate_w + (size_t)(row0 + r16) * H;
    const uint8_t *urow = et.ep.up_w + (size_t)(row0 + r16) * H;
    const float *gs = et.ep.gate_s + (row0 >> 7) * blocks;
    const float *us = et.ep.up_s + (row0 >> 7) * blocks;
    uint32_t pos[NT];
    bool tok_ok[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = nt * 16 + r16;
        tok_ok[nt] = t < et.cnt;
        pos[nt] = tok_ok[nt] ? placement_pos[et.off + t] : 0;
        pos[nt] = pos[nt] < rows ? pos[nt] : rows - 1;
    }
    f32x4 tg[NT], tu[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        tg[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        tu[nt] = tg[nt];
    }
    const uint32_t b_begin = wave * blocks / KSPLIT, b_end = (wave + 1) * blocks / KSPLIT;
    for (uint32_t b = b_begin; b < b_end; ++b) {
        const uint32_t col = (b << 7) + q * 32;
        const uint4 g0 = load_global16(grow + col);
        const uint4 g1 = load_global16(grow + col + 16);
        const uint4 u0 = load_global16(urow + col);
        const uint4 u1 = load_global16(urow + col + 16);
        const i32x8 ga = {(int)g0.x, (int)g0.y, (int)g0.z, (int)g0.w, (int)g1.x, (int)g1.y, (int)g1.z, (int)g1.w};
        const i32x8 ua = {(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
        const float sg = gs[b], su = us[b];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
            float sa = 0.f;
            if (tok_ok[nt]) {
                const uint4 *cp = (const uint4 *)(xq + (size_t)pos[nt] * H + col);
                c0 = cp[0];
                c1 = cp[1];
                sa = xs[(size_t)pos[nt] * blocks + b];
            }
            const i32x8 xb = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
            const f32x4 pg = mfma_fp8_16x16x128(ga, xb, f32x4{0.f, 0.f, 0.f, 0.f});
            const f32x4 pu = mfma_fp8_16x16x128(ua, xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                tg[nt][i] = __builtin_fmaf(pg[i] * sg, sa, tg[nt][i]);
                tu[nt][i] = __builtin_fmaf(pu[i] * su, sa, tu[nt][i]);
            }
        }
    }
    reduce_waves<KSPLIT, NT>(red_g, tg, wave, lane);
    reduce_waves<KSPLIT, NT>(red_u, tu, wave, lane);
    if (wave != 0)
        return;
    bool bad = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        if (!tok_ok[nt])
            continue;
        const uint32_t t = nt * 16 + r16;
        float4 out;
        float *o = (float *)&out;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float g = round_bf16(tg[nt][i]);
            const float u = round_bf16(tu[nt][i]);
            o[i] = round_bf16(silu_bf16_staged(g) * u);
            bad |= !finite_f32(g) || !finite_f32(u) || !finite_f32(o[i]);
        }
        *(float4 *)(hidden + (size_t)(et.off + t) * I + row0 + q * 4) = out;
    }
    if (bad)
        raise_flag(flags, FLAG_SWIGLU_NONFINITE);
}

// ------------------------------------------------------------------ mode B, down projection
template <int KSPLIT, int NT>
__global__ __launch_bounds__(64 * KSPLIT) void moe_b_down_kernel(
    const ExpertPtrs *__restrict__ bank, const MoePlan *__restrict__ plan,
    const uint32_t *__restrict__ active_expert, const uint32_t *__restrict__ active_offset,
    const uint8_t *__restrict__ hq, const float *__restrict__ hs, uint32_t H, uint32_t I,
    float *__restrict__ y, uint32_t *flags)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    __shared__ f32x4 red[KSPLIT][NT][64];
    const uint32_t tiles_per_expert = H >> 4;
    const uint32_t a = blockIdx.x / tiles_per_expert, rt = blockIdx.x % tiles_per_expert;
    const ExpertTile et = expert_tile(plan, active_expert, active_offset, bank, a);
    if (!et.live || et.cnt > 16u * NT)
        return;
    const uint32_t row0 = rt << 4;
    const uint32_t blocks = I >> 7;
    const uint8_t *drow = et.ep.down_w + (size_t)(row0 + r16) * I;
    const float *ds = et.ep.down_s + (row0 >> 7) * blocks;
    uint32_t slot[NT];
    bool tok_ok[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = nt * 16 + r16;
        tok_ok[nt] = t < et.cnt;
        slot[nt] = et.off + (tok_ok[nt] ? t : 0);
    }
    f32x4 tot[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
        tot[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t b_begin = wave * blocks / KSPLIT, b_end = (wave + 1) * blocks / KSPLIT;
    for (uint32_t b = b_begin; b < b_end; ++b) {
        const uint32_t col = (b << 7) + q * 32;
        const uint4 d0 = load_global16(drow + col);
        const uint4 d1 = load_global16(drow + col + 16);
        const i32x8 da = {(int)d0.x, (int)d0.y, (int)d0.z, (int)d0.w, (int)d1.x, (int)d1.y, (int)d1.z, (int)d1.w};
        const float sd = ds[b];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
            float sa = 0.f;
            if (tok_ok[nt]) {
                const uint4 *cp = (const uint4 *)(hq + (size_t)slot[nt] * I + col);
                c0 = cp[0];
                c1 = cp[1];
                sa = hs[(size_t)slot[nt] * blocks + b];
            }
            const i32x8 xb = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
            const f32x4 p = mfma_fp8_16x16x128(da, xb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tot[nt][i] = __builtin_fmaf(p[i] * sd, sa, tot[nt][i]);
        }
    }
    reduce_waves<KSPLIT, NT>(red, tot, wave, lane);
    if (wave != 0)
        return;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        if (!tok_ok[nt])
            continue;
        // bf16_round_in_place of the expert output (src/wide_metal_moe.rs:1236-1251)
        *(float4 *)(y + (size_t)slot[nt] * H + row0 + q * 4) =
            make_float4(round_bf16(tot[nt][0]), round_bf16(tot[nt][1]), round_bf16(tot[nt][2]),
                        round_bf16(tot[nt][3]));
    }
}

// ------------------------------------------------------------------------------- combine
// route_weighted_scatter_add_f32 + the final bf16_round_in_place (kernels/block_fp8_gemv.metal:
// 299-315, src/wide_metal_moe.rs:1252-1286); CPU twin src/text_endpoint.rs:5365-5373. Each token
// sums its eight placements in ascending expert id, out += y * w in f32 (no fused multiply-add),
// then rounds to bf16.
// Sum of `ks` split-K partials of 4 consecutive values, in split order (ks = 1: plain load).
__device__ __forceinline__ float4 split_sum4(const float *p, uint32_t ks, size_t stride)
{
    float4 v = *(const float4 *)p;
    for (uint32_t s = 1; s < ks; ++s) {
        const float4 o = *(const float4 *)(p + s * stride);
        v.x += o.x;
        v.y += o.y;
        v.z += o.z;
        v.w += o.w;
    }
    return v;
}

template <int KS>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float *__restrict__ y, uint32_t ks_rt, size_t split_stride, const float *__restrict__ placement_w,
    const uint32_t *__restrict__ row_slots, uint32_t rows, uint32_t H, const MoePlan *__restrict__ plan,
    float *__restrict__ out_f32, uint16_t *__restrict__ out_bf16, uint32_t raw, uint32_t *flags)
{
    // a rejected batch (the schedule raised FLAG_SCHEDULE) writes zeros, whatever its expert outputs hold
    const bool rejected = plan->rejected != 0;
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;  // one float4 of one token row
    const uint32_t per_row = H >> 2;
    if (idx >= rows * per_row)
        return;
    const uint32_t row = idx / per_row, c4 = idx % per_row;
    const uint4 s0 = *(const uint4 *)(row_slots + row * 8), s1 = *(const uint4 *)(row_slots + row * 8 + 4);
    uint32_t slot[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        slot[j] = slot[j] < rows * 8 ? slot[j] : 0;
        w[j] = placement_w[slot[j]];
    }
    float4 v[8];
    if constexpr (KS > 0) {
        // every split partial of the eight slots in flight at once, summed in split order
        float4 part[8][KS];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int s = 0; s < KS; ++s)
                part[j][s] = *(const float4 *)(y + (size_t)s * split_stride + (size_t)slot[j] * H + c4 * 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = part[j][0];
#pragma unroll
            for (int s = 1; s < KS; ++s) {
                v[j].x += part[j][s].x;
                v[j].y += part[j][s].y;
                v[j].z += part[j][s].z;
                v[j].w += part[j][s].w;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[j] = split_sum4(y + (size_t)slot[j] * H + c4 * 4, ks_rt, split_stride);
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        acc[0] = __fadd_rn(acc[0], __fmul_rn(v[j].x, w[j]));
        acc[1] = __fadd_rn(acc[1], __fmul_rn(v[j].y, w[j]));
        acc[2] = __fadd_rn(acc[2], __fmul_rn(v[j].z, w[j]));
        acc[3] = __fadd_rn(acc[3], __fmul_rn(v[j].w, w[j]));
    }
    bool bad = false;
    const size_t at = (size_t)row * H + c4 * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc[i] = rejected ? 0.f : acc[i];
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

// ------------------------------------------------------------------- single-expert plan
// One expert applied to rows 0..rows-1 (the reference's complete-expert measurement,
// src/lib.rs:4008-6590 "L3" harness): the plan has one active expert whose placements are the
// rows themselves, so the same gate/up and down kernels run unchanged.
__global__ void moe_single_plan_kernel(const ExpertPtrs *bank, uint32_t expert, uint32_t rows,
                                       MoePlan *plan, uint32_t *active_expert,
                                       uint32_t *active_offset, ActiveExpert *active,
                                       uint32_t *placement_pos, float *placement_w)
{
    const uint32_t i = threadIdx.x;
    if (i == 0) {
        plan->n_active = 1;
        plan->n_placements = rows;
        plan->max_count = rows;
        plan->rejected = 0u;
        active_expert[0] = expert;
        active_offset[0] = 0;
        active_offset[1] = rows;
        ActiveExpert ae{};
        ae.ep = bank[expert];
        ae.off = 0;
        ae.cnt = rows;
        for (uint32_t k = 0; k < 16; ++k)
            ae.tok[k] = (uint16_t)k;
        active[0] = ae;
    }
    if (i < rows) {
        placement_pos[i] = i;
        placement_w[i] = 1.0f;
    }
}

// y [rows x H] f32 -> output (bf16-rounded f32 or bf16 bits).
__global__ __launch_bounds__(256) void round_output_kernel(const float *__restrict__ y, uint32_t ks,
                                                           size_t split_stride, uint32_t n,
                                                           float *__restrict__ out_f32,
                                                           uint16_t *__restrict__ out_bf16,
                                                           uint32_t raw, uint32_t *flags)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    float v = y[i];
    for (uint32_t s = 1; s < ks; ++s)
        v += y[s * split_stride + i];
    const float r = round_bf16(v);
    if (!finite_f32(r))
        raise_flag(flags, FLAG_ROUND_NONFINITE);
    if (out_f32)
        out_f32[i] = raw ? v : r;
    if (out_bf16)
        out_bf16[i] = (uint16_t)(f32_bits(r) >> 16);
}

// ------------------------------------------------------------------------------- launchers
bool launch_moe_schedule(const ExpertPtrs *bank, const uint32_t *ids, const float *weights,
                         uint32_t rows, uint32_t E, uint32_t max_active, const MoeBuffers &mb,
                         uint32_t *flags, hipStream_t stream, const PfTileTable *tiles, const QuantJob *quant,
                         bool *quantised)
{
    bool long_batch = false;
    if (quantised)
        *quantised = false;
    const uint32_t words = (rows + 31) >> 5;
    size_t lds = (size_t)(E * words + E) * sizeof(uint32_t);
    const size_t with_prefix_lds = lds + (size_t)E * words * sizeof(uint16_t);
    const uint32_t with_prefix = words > 1 && with_prefix_lds <= 160 * 1024;
    if (with_prefix)
        lds = with_prefix_lds;
    if (lds > 65536)  // long prefill batches: up to 160 KB of LDS per workgroup on gfx950
        (void)hipFuncSetAttribute((const void *)moe_schedule_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
    const int t = timer_begin(K_MOE_SCHEDULE, stream);
    if (wave_schedule(rows, E, max_active)) {
        const size_t table = (size_t)E * sizeof(ExpertPtrs);
        if (table > 32768)
            (void)hipFuncSetAttribute((const void *)moe_schedule_wave_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)table);
        // with `quant` and somewhere to report it, the activation rows are quantised in the same launch
        const QuantJob qj = quant && quantised ? *quant : QuantJob{};
        const uint32_t quant_wgs = (qj.rows * (qj.K >> 7) + 3) / 4;
        hipLaunchKernelGGL(moe_schedule_wave_kernel, dim3(1 + quant_wgs), dim3(64), table, stream, bank, ids, weights,
                           rows, E, max_active, mb.plan, mb.active_expert, mb.active_offset, mb.active,
                           mb.placement_pos, mb.placement_w, mb.row_slots, mb.pieces, rows * 8, flags, qj);
        if (quant_wgs)
            *quantised = true;
    }
    else if (rows <= SCHED_WG_MAX_ROWS)
        hipLaunchKernelGGL(moe_schedule_kernel, dim3(1), dim3(1024), lds, stream, bank, ids, weights, rows,
                           E, max_active, with_prefix, mb.plan, mb.active_expert, mb.active_offset, mb.active,
                           mb.placement_pos, mb.placement_w, mb.row_slots, flags);
    else {
        // rows <= 4096 (SCHED_MAX_WORDS words) and E <= 1024 (one plan thread per expert)
        const SchedScratch ss = sched_carve(mb.sched, rows, E, nullptr);
        const uint32_t nwg = (rows + 63) / 64;
        hipLaunchKernelGGL(moe_sched_mark_kernel, dim3(nwg), dim3(64), (size_t)E * 8, stream, ids, weights, rows, E,
                           ss);
        const PfTileTable tt = tiles ? *tiles : PfTileTable{nullptr, nullptr, 0};
        const QuantJob qj = quant ? *quant : QuantJob{};
        const uint32_t quant_wgs = (qj.rows * (qj.K >> 7) + 63) / 64;
        hipLaunchKernelGGL(moe_sched_plan_kernel, dim3(1 + quant_wgs), dim3(1024), 0, stream, bank, rows, E,
                           max_active, ss, mb.plan, mb.active_expert, mb.active_offset, mb.active,
                           mb.placement_pos, mb.placement_w, mb.row_slots, flags, tt, qj);
        long_batch = true;
        if (quantised && quant)
            *quantised = true;
        hipLaunchKernelGGL(moe_sched_place_kernel, dim3(nwg), dim3(64), 0, stream, ids, weights, rows, E, max_active,
                           ss, mb.plan, mb.active, mb.placement_pos, mb.placement_w, mb.row_slots);
    }
    timer_end(t, stream);
    return long_batch;
}

// Mode A: gate/up (+SwiGLU) then down, both as split-K expert projections (pw_moe_a.hip).
// Where the one-expert forward's rounded output goes when its down projection writes it directly.
struct DirectOut {
    float *f32;
    uint16_t *bf16;
    bool raw;
};

static ExpertOut launch_a_moe(const MoeBuffers &mb, const void *x, bool x_f32, uint32_t rows,
                              uint32_t placements, uint32_t max_active, uint32_t max_count, uint32_t H,
                              uint32_t I, uint32_t *flags, hipStream_t stream, const ActiveExpert *one = nullptr,
                              const DirectOut *direct = nullptr, const ExpertPtrs *bank = nullptr,
                              const OneTokenRoutes *routes = nullptr, const RouteJob *job = nullptr,
                              bool *job_done = nullptr)
{
    const int nt = max_count > 16 ? 2 : 1;
    const uint32_t cnt = max_count < 16u * nt ? max_count : 16u * nt;
    const uint16_t *xp = (const uint16_t *)x;
    if (x_f32) {
        launch_split_planes((const float *)x, rows * H, mb.x_planes, stream);
        xp = mb.x_planes;
    }
    SplitArgs ga{};
    ga.active = mb.active;
    ga.placement_pos = mb.placement_pos;
    ga.x = xp;
    ga.x_plane = (size_t)rows * H;
    ga.K = H;
    ga.R = I;
    ga.rows = rows;
    ga.P = placements;
    ga.partial = mb.partial;
    ga.flags = flags;
    ga.cap = cnt;
    if (one) {
        ga.single = 1;
        ga.one = *one;
    }
    if (routes) {  // the fused gate/up and the one-token down+combine read the routes themselves
        ga.bank = bank;
        ga.route_ids = routes->ids;
        ga.route_w = routes->w;
        ga.E = routes->E;
    }
    const SplitPlan gp = plan_split(H, 2, x_f32 ? 3 : 1, cnt);
    ga.KS = gp.ks;
    int t = timer_begin(K_MOE_GATEUP, stream);
    // the one-wave schedule also cut every routed expert's slots into entries of at most
    // PIECE_ROWS rows (with their token rows): a decode batch gives most experts one to three
    // rows, and LDS stages sized for four rows let more workgroups share a CU (an expert with more
    // rows reads its weights once per piece; every slot's arithmetic is unchanged)
    const bool pieces = !one && cnt > PIECE_ROWS && wave_schedule(rows, mb.experts, max_active);
    SplitArgs gp_args = ga;
    if (pieces && !x_f32) {
        gp_args.active = mb.pieces;
        gp_args.cap = PIECE_ROWS;
    }
    // the route weights (job) ride in extra workgroups of a launch that runs anyway: the split-K
    // down's (about 1 us there against about 4 us in the gate/up launch, whose workgroups are
    // longer), or the fused gate/up's where the down is the one-token down+combine
    const bool job_in_down = job && !direct;
    if (job && !job_in_down)
        gp_args.job = *job;
    const bool fused = nt == 1 && launch_moe_a_gateup_fused(x_f32 ? 3 : 1, gp_args, pieces && !x_f32 ? placements
                                                            : max_active, mb.hidden_planes, stream);
    if (!fused)
        launch_moe_a_split(2, x_f32 ? 3 : 1, nt, ga, gp, max_active, stream);
    timer_end(t, stream);
    if (!fused) {
        t = timer_begin(K_MOE_SWIGLU, stream);
        launch_moe_a_swiglu(mb.partial, gp.ks, placements, I, mb.hidden_planes, flags, stream);
        timer_end(t, stream);
    }
    if (job && !job_in_down) {
        if (!fused)  // the split gate/up cannot carry the route weights: before the down, on their own
            launch_route_weights(*job, stream);
        *job_done = true;
    }

    SplitArgs da = ga;
    da.placement_pos = nullptr;
    da.x = mb.hidden_planes;
    da.x_plane = (size_t)placements * I;
    da.K = I;
    da.R = H;
    da.rows = placements;
    // down in pieces: a four-row LDS stage (25 KB at hidden 4096) leaves the kernel's 98 VGPRs
    // (four waves per SIMD) to set its occupancy, four workgroups per CU instead of three at eight
    // rows
    if (pieces) {
        da.active = mb.pieces;
        da.cap = PIECE_ROWS;
    }
    t = timer_begin(K_MOE_DOWN, stream);
    // one expert: the whole-K down writes the rounded output rows itself; a one-token batch: down
    // and combine in one launch
    if (direct && (one ? launch_moe_a_down_out(da, direct->f32, direct->bf16, direct->raw, stream)
                       : launch_moe_a_down_combine1(da, mb.plan, mb.placement_w, direct->f32, direct->bf16,
                                                    direct->raw, stream))) {
        timer_end(t, stream);
        return ExpertOut{nullptr, 0, 0};
    }
    const SplitPlan dp = plan_split(I, 1, 3, pieces ? PIECE_ROWS : cnt);
    da.KS = dp.ks;
    if (job_in_down && dp.bpw == 8 && (pieces || nt == 1)) {  // the instantiation compiled with a job
        da.job = *job;
        *job_done = true;
    }
    launch_moe_a_split(1, 3, pieces ? 1 : nt, da, dp, pieces ? placements : max_active, stream);
    if (job_in_down && !*job_done) {  // another down shape: the weights on their own, before the combine
        launch_route_weights(*job, stream);
        *job_done = true;
    }
    timer_end(t, stream);
    return ExpertOut{mb.partial, dp.ks, (size_t)placements * H};
}

// Mode B gate/up, hidden re-quantisation and down as whole-K workgroups (pw_moe_b.hip), after the
// activations were quantised into mb.xq / mb.xs: from the schedule's entries, or for the one expert
// `one` on token rows 0..rows-1. The down writes each expert output rounded to bf16 into y (a lone
// expert: the output rows, y_bf16 too). False, with nothing launched, when the shapes do not fit.
static bool launch_b_fused(const ExpertPtrs *bank, const MoeBuffers &mb, const ActiveExpert *one, uint32_t rows,
                           uint32_t placements,
                           uint32_t max_active, uint32_t max_count, uint32_t H, uint32_t I, float *y,
                           uint16_t *y_bf16, uint32_t *flags, hipStream_t stream, const RouteJob *job = nullptr,
                           bool *job_done = nullptr)
{
    if (!moe_b_fused_shapes(H, I, max_count, one != nullptr))  // both launches take the shapes, or neither runs
        return false;
    MoeBArgs ga{};
    ga.active = mb.active;
    ga.codes = mb.xq;
    ga.scales = mb.xs;
    ga.K = H;
    ga.R = I;
    ga.rows = rows;
    ga.cap = max_count;
    if (one) {
        ga.single = 1;
        ga.one = *one;
    }
    ga.out = mb.hidden;
    ga.flags = flags;
    MoeBArgs da = ga;
    if (job) {  // the gate/up launch carries the route weights (in extra workgroups)
        ga.job = *job;
        *job_done = true;
    }
    da.codes = mb.hq;
    da.scales = mb.hs;
    da.K = I;
    da.R = H;
    da.rows = placements;
    da.out = y;
    da.out_bf16 = y_bf16;
    da.partial = mb.y;  // a lone expert's share sums: [KS][rows][H] within y's [8 rows][H]
    int t = timer_begin(K_MOE_GATEUP, stream);
    (void)launch_moe_b_gateup_fused(ga, max_active, stream);
    timer_end(t, stream);
    // re-quantise the bf16-staged hidden activations per (placement, 128 group)
    launch_quant_group128(mb.hidden, true, placements, I, mb.hq, mb.hs, flags, stream);
    t = timer_begin(K_MOE_DOWN, stream);
    // a lone expert: whole-K down workgroups that write the output rows; routed experts: the
    // split-K down (16 rows per workgroup, four waves of four blocks each), which measured faster
    // there than whole-K workgroups of 16 rows (81 against 98 us at width 8)
    uint32_t ks = 1;
    if (one)
        ks = launch_moe_b_down_fused(da, max_active, stream);
    else
        hipLaunchKernelGGL((moe_b_down_kernel<4, 1>), dim3(max_active * (H >> 4)), dim3(256), 0, stream, bank, mb.plan,
                           mb.active_expert, mb.active_offset, mb.hq, mb.hs, H, I, mb.y, flags);
    timer_end(t, stream);
    if (ks > 1) {
        // the share sums added in share order and rounded (mode B's output is the rounded expert
        // output, also as F32_RAW)
        const uint32_t n = rows * H;
        hipLaunchKernelGGL(round_output_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, mb.y, ks, (size_t)n, n,
                           y, y_bf16, 0u, flags);
    }
    return true;
}

template <int KS, int NT>
static void launch_b_moe(const ExpertPtrs *bank, const MoeBuffers &mb, uint32_t rows, uint32_t placements,
                         uint32_t max_active, uint32_t H, uint32_t I, uint32_t *flags, hipStream_t stream)
{
    const dim3 g1(max_active * (I >> 4)), g2(max_active * (H >> 4)), blk(64 * KS);
    int t = timer_begin(K_MOE_GATEUP, stream);
    hipLaunchKernelGGL((moe_b_gateup_kernel<KS, NT>), g1, blk, 0, stream, bank, mb.plan,
                       mb.active_expert, mb.active_offset, mb.placement_pos, mb.xq, mb.xs, rows, H, I,
                       mb.hidden, flags);
    timer_end(t, stream);
    // re-quantise the bf16-staged hidden activations per (placement, 128 group)
    launch_quant_group128(mb.hidden, true, placements, I, mb.hq, mb.hs, flags, stream);
    t = timer_begin(K_MOE_DOWN, stream);
    hipLaunchKernelGGL((moe_b_down_kernel<KS, NT>), g2, blk, 0, stream, bank, mb.plan,
                       mb.active_expert, mb.active_offset, mb.hq, mb.hs, H, I, mb.y, flags);
    timer_end(t, stream);
}

static ExpertOut launch_experts(uint32_t mode, const ExpertPtrs *bank, const MoeBuffers &mb, const void *x,
                                bool x_f32, uint32_t rows, uint32_t placements, uint32_t max_active,
                                uint32_t max_count, uint32_t H, uint32_t I, uint32_t *flags, hipStream_t stream,
                                const DirectOut *direct = nullptr, const OneTokenRoutes *routes = nullptr,
                                bool x_quantised = false, const RouteJob *job = nullptr, bool *job_done = nullptr)
{
    const bool wide = max_count > 16;
    if (mode == 0)
        return launch_a_moe(mb, x, x_f32, rows, placements, max_active, max_count, H, I, flags, stream, nullptr,
                            direct, bank, routes, job, job_done);
    if (!x_quantised)
        launch_quant_group128(x, x_f32, rows, H, mb.xq, mb.xs, flags, stream);
    if (!wide && launch_b_fused(bank, mb, nullptr, rows, placements, max_active, max_count, H, I, mb.y, nullptr, flags,
                                stream, job, job_done))
        return ExpertOut{mb.y, 1, 0};
    if (wide) launch_b_moe<4, 2>(bank, mb, rows, placements, max_active, H, I, flags, stream);
    else launch_b_moe<4, 1>(bank, mb, rows, placements, max_active, H, I, flags, stream);
    return ExpertOut{mb.y, 1, 0};
}

void launch_moe_layer(uint32_t mode, const ExpertPtrs *bank, const MoeBuffers &mb, const void *x,
                      bool x_f32, uint32_t rows, uint32_t max_active, uint32_t max_count, uint32_t H,
                      uint32_t I, float *out_f32, uint16_t *out_bf16, bool raw, uint32_t *flags,
                      hipStream_t stream, const OneTokenRoutes *routes, bool x_quantised, const RouteJob *job)
{
    const DirectOut direct{out_f32, out_bf16, raw};
    // the route weights (job) must be in place before a kernel reads them: the mode A experts carry
    // them in their split-K down launch (or, for the one-token down+combine, in the gate/up launch),
    // the mode B ones in their whole-K gate/up launch, else they run before the combine
    bool job_done = false;
    const ExpertOut eo = launch_experts(mode, bank, mb, x, x_f32, rows, rows * 8, routes ? 8 : max_active,
                                        routes ? 1 : max_count, H, I, flags, stream, rows == 1 ? &direct : nullptr,
                                        routes, x_quantised, job, &job_done);
    if (job && !job_done)  // no expert launch carried the route weights
        launch_route_weights(*job, stream);
    if (!eo.y)
        return;  // the one-token down wrote the combined output
    const uint32_t n4 = rows * (H >> 2);
    // a short batch (up to 256 workgroups of 256) spreads its gather over twice the CUs with
    // 128-thread workgroups: 8 tokens of 4096 columns take 64 of them
    const uint32_t cb = n4 <= 65536u ? 128u : 256u;
    const int t = timer_begin(K_MOE_COMBINE, stream);
#define PW_COMBINE(KS)                                                                                         \
    hipLaunchKernelGGL((moe_combine_kernel<KS>), dim3((n4 + cb - 1) / cb), dim3(cb), 0, stream, eo.y, eo.ks, \
                       eo.stride, mb.placement_w, mb.row_slots, rows, H, mb.plan, out_f32, out_bf16, raw ? 1u : 0u, \
                       flags)
    switch (eo.ks) {
    case 1: PW_COMBINE(1); break;
    case 2: PW_COMBINE(2); break;
    case 4: PW_COMBINE(4); break;
    default: PW_COMBINE(0); break;
    }
#undef PW_COMBINE
    timer_end(t, stream);
}

void launch_expert_forward(uint32_t mode, const ExpertPtrs *bank, const ExpertPtrs &ep, uint32_t expert,
                           const MoeBuffers &mb, const void *x, bool x_f32, uint32_t rows, uint32_t H, uint32_t I,
                           float *out_f32, uint16_t *out_bf16, bool raw, uint32_t *flags, hipStream_t stream)
{
    ExpertOut eo{};
    if (mode == 0) {
        // mode A takes the expert's schedule entry by value: no plan kernel
        ActiveExpert one{};
        one.ep = ep;
        one.off = 0;
        one.cnt = rows;
        for (uint32_t k = 0; k < 16; ++k)
            one.tok[k] = (uint16_t)k;
        const DirectOut direct{out_f32, out_bf16, raw};
        eo = launch_a_moe(mb, x, x_f32, rows, rows, 1, rows, H, I, flags, stream, &one, &direct);
        if (!eo.y)
            return;  // the down projection wrote the output
    } else {
        // mode B: the whole-K kernels take the expert's entry by value and the down writes the
        // output rows (the expert output rounded to bf16, which is also the F32_RAW result)
        if (rows <= 16) {
            ActiveExpert one{};
            one.ep = ep;
            one.off = 0;
            one.cnt = rows;
            for (uint32_t k = 0; k < 16; ++k)
                one.tok[k] = (uint16_t)k;
            launch_quant_group128(x, x_f32, rows, H, mb.xq, mb.xs, flags, stream);
            if (launch_b_fused(bank, mb, &one, rows, rows, 1, rows, H, I, out_f32, out_bf16, flags, stream))
                return;
        }
        hipLaunchKernelGGL(moe_single_plan_kernel, dim3(1), dim3(256), 0, stream, bank, expert, rows, mb.plan,
                           mb.active_expert, mb.active_offset, mb.active, mb.placement_pos, mb.placement_w);
        eo = launch_experts(mode, bank, mb, x, x_f32, rows, rows, 1, rows, H, I, flags, stream);
    }
    const uint32_t n = rows * H;
    hipLaunchKernelGGL(round_output_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, eo.y, eo.ks, eo.stride,
                       n, out_f32, out_bf16, raw ? 1u : 0u, flags);
}

}  // namespace pw
