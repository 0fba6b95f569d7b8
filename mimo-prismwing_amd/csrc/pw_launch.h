// Host-side launchers of the gfx950 kernels (internal to the library; the public surface is the
// C ABI in include/pwfp8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pw_device.h"

namespace pw {

// Kernels whose launches can be timed with HIP events (benchmark diagnostics).
enum KernelId : uint32_t {
    K_LINEAR_A = 0,
    K_LINEAR_B,
    K_QUANT,
    K_MOE_SCHEDULE,
    K_MOE_GATEUP,
    K_MOE_SWIGLU,
    K_MOE_DOWN,
    K_MOE_COMBINE,
    K_PREFILL_GATEUP,
    K_PREFILL_DOWN,
    K_ROUTER,
    K_BF16_LINEAR,
    K_ROUTE_SCHEDULE,
    K_COUNT
};

// Optional event recorder: when enabled, each timed launch records a start and a stop event on
// the stream it is launched on. Summaries synchronise and sum hipEventElapsedTime per kernel.
struct KernelTimer {
    bool enabled = false;
    uint32_t capacity = 0, used = 0;
    hipEvent_t *events = nullptr;  // [2 * capacity]
    uint32_t *ids = nullptr;       // [capacity]
    int begin(uint32_t id, hipStream_t s)
    {
        if (!enabled || used >= capacity)
            return -1;
        const int slot = (int)used++;
        ids[slot] = id;
        (void)hipEventRecord(events[2 * slot], s);
        return slot;
    }
    void end(int slot, hipStream_t s)
    {
        if (slot >= 0)
            (void)hipEventRecord(events[2 * slot + 1], s);
    }
};

// Per-layer device scratch of the routed-MoE launch, sized for `max_rows` token rows.
struct MoeBuffers {
    MoePlan *plan;
    uint32_t *active_expert;   // [E]
    uint32_t *active_offset;   // [E + 1]
    uint32_t *placement_pos;   // [rows * 8]
    float *placement_w;        // [rows * 8]
    uint32_t *row_slots;       // [rows * 8]
    float *hidden;             // [rows * 8 * I]      mode B bf16-staged SwiGLU output
    uint16_t *hidden_planes;   // [3][rows * 8][I]    mode A SwiGLU output as exact bf16 planes
    uint16_t *x_planes;        // [3][rows][H]        mode A f32 activations as bf16 planes
    float *y;                  // [rows * 8 * H]
    ActiveExpert *active;      // [E]   per routed expert: weights, placement slots
    ActiveExpert *pieces;      // [rows * 8] decode batches (<= 8 rows): the routed experts' slots
                               // in pieces of at most four rows, for the projections
    float *partial;            // split-K partial sums of the mode A projections
    uint8_t *xq;               // [rows * H]      mode B activation codes
    float *xs;                 // [rows * H/128]  mode B activation scales
    uint8_t *hq;               // [rows * 8 * I]
    float *hs;                 // [rows * 8 * I/128]
    void *sched;               // [moe_sched_scratch_bytes] long-batch schedule tables
    uint32_t max_rows;
    uint32_t experts;
};

// The route weights of a batch scheduled from its expert sets alone (launch_route_set_schedule):
// per row, select_route_row gives the routes in the reference's order and their weights, which go
// to the route outputs and to the placements (route_weights_row, pw_route_job.h). The decode
// layer runs it in eight extra workgroups of a launch whose other workgroups stream the experts'
// weights (the mode A split-K down, the mode A one-token gate/up, the mode B gate/up); rows = 0:
// no job.
struct RouteJob {
    const float *scores, *bias;  // router scores [rows][E], bias [E]
    uint32_t rows, E;
    const uint32_t *set_ids;     // [rows][8] the schedule's expert sets
    uint32_t *route_ids;         // [rows][8] out
    float *route_w;              // [rows][8] out
    uint32_t *tie_rows;          // optional tie count
    MoePlan *plan;
    const uint32_t *row_slots;   // null: no schedule (a one-token direct layer)
    float *placement_w;          // the schedule's placement weights, or [rows][8] in set order
    uint32_t *flags;
};
constexpr uint32_t ROUTE_JOB_WGS = 8;  // workgroups a launch adds for a job (one per row)

// Arguments of the split-K mode A expert projection (pw_moe_a.hip).
struct SplitArgs {
    const ActiveExpert *active;
    const uint32_t *placement_pos;  // gate/up: token row per placement slot; down: null (rows = slots)
    const uint16_t *x;              // activation planes [NS][rows][K]
    size_t x_plane;
    uint32_t K, R, KS, rows, P;     // columns, weight rows, K splits, activation rows, placements
    uint32_t cap;                   // routed rows per expert the LDS stage holds
    float *partial;                 // [KS][MATS][P][R]
    uint32_t *flags;
    uint32_t single;                // 1: one expert on rows 0..rows-1, its entry is `one` (no schedule)
    ActiveExpert one;
    // One token's routes with no schedule (route_ids non-null): work item a is the token's route a,
    // expert route_ids[a] of the bank's E, on placement slot a (see moe_a_one_token_direct)
    const ExpertPtrs *bank;
    const uint32_t *route_ids;
    const float *route_w;
    uint32_t E;
    RouteJob job;  // fused gate/up only: run in ROUTE_JOB_WGS extra workgroups
};

// Where a launch left the per-placement expert outputs: `ks` split-K partial sums of [P][H] f32,
// `stride` floats apart, summed in split order by the consumer (ks = 1: plain outputs).
struct ExpertOut {
    const float *y;
    uint32_t ks;
    size_t stride;
};

struct SplitPlan {
    uint32_t bpw, kc, ks;
    size_t lds;
};

// K split of a mode A expert projection (`mats` weight matrices sharing the activations) with K
// columns, NS activation planes and up to max_cnt routed rows per expert.
SplitPlan plan_split(uint32_t K, int mats, int ns, uint32_t max_cnt);
void launch_moe_a_split(int mats, int ns, int nt, const SplitArgs &args, const SplitPlan &sp,
                        uint32_t max_active, hipStream_t stream);
// gate/up split sums -> SwiGLU -> hidden as three bf16 planes [3][P][I]
// BF16 wide linear (pw_bf16.hip): w bf16 [R][K] (K a multiple of 128), x bf16 planes [NS][W][K],
// split-K partials [KS][W][R] f32 summed in split order by the reduce kernel.
struct Bf16Args {
    const uint16_t *w;
    const uint16_t *x;
    const float *xf;  // f32 activations [W][K], W <= 16, split into the three planes while staging (x unused)
    size_t x_plane;
    uint32_t K, R, W, KS;
    float *partial;
};
// 128-column blocks per wave for K (the K split is 128 * that); at most `lds_cap` bytes of LDS
// for NS planes of W activation rows.
int bf16_blocks_per_wave(uint32_t K, int planes, uint32_t W, size_t lds_cap);
void launch_bf16_linear(const Bf16Args &a, int planes, int bpw, float *y32, uint16_t *y16, uint32_t round_f32,
                        uint32_t *flags, hipStream_t stream);

// Gate/up with the SwiGLU fused and no split partials (pw_moe_a.hip), when the routed rows fit the
// LDS stage; returns false (nothing launched) otherwise.
// The one-expert forward's whole-K down projection with the output rounding fused (K = I of 1024
// or 2048, at most eight rows); false when the shape does not fit it.
bool launch_moe_a_down_out(const SplitArgs &args, float *out_f32, uint16_t *out_bf16, bool raw, hipStream_t stream);
// Down and combine of a one-token decode batch in one launch (mode A, I = 2048, eight routed
// experts; args are the down projection's, whose rows are the eight placement slots): the same
// arithmetic as the split-K down followed by the combine; false when the batch does not fit it.
// Only for batches of one token. With args.route_ids (no schedule) it ranks the token's eight
// routes by expert id for the combine and checks them as the schedule would (ids inside the bank,
// no expert twice, finite weights; FLAG_SCHEDULE otherwise); plan and placement_w are then unused.
bool launch_moe_a_down_combine1(const SplitArgs &args, const MoePlan *plan, const float *placement_w, float *out_f32,
                                uint16_t *out_bf16, bool raw, hipStream_t stream);
// Whether a one-token mode A layer of hidden H and intermediate I runs as the fused gate/up and the
// one-token down+combine (both reading the token's routes directly, no schedule launch).
bool moe_a_one_token_direct(uint32_t H, uint32_t I);
bool launch_moe_a_gateup_fused(int ns, const SplitArgs &args, uint32_t max_active, uint16_t *hidden_planes,
                               hipStream_t stream);
void launch_moe_a_swiglu(const float *partial, uint32_t ks, uint32_t P, uint32_t I, uint16_t *hidden_planes,
                         uint32_t *flags, hipStream_t stream);

// Mode B whole-K projections of routed experts (pw_moe_b.hip): e4m3 activation codes with per
// (row, 128-column) scales against the block-FP8 weights. Gate/up reads token rows ae.tok[t] of
// the codes and writes the bf16-staged SwiGLU to hidden [slots][R]; down reads slot rows
// ae.off + t and writes each expert output rounded to bf16 at its slot row.
struct MoeBArgs {
    const ActiveExpert *active;  // schedule entries (unused when single)
    const uint8_t *codes;        // activation codes [rows][K]
    const float *scales;         // activation scales [rows][K/128]
    uint32_t K, R, rows, cap;    // columns, weight rows, activation rows, routed rows per expert at most
    uint32_t single;             // 1: one expert, entry `one` (no schedule)
    ActiveExpert one;
    float *out;                  // gate/up: hidden; down: expert outputs (single: the output rows)
    uint16_t *out_bf16;          // down, single: bf16 output rows (or null)
    uint32_t KS;                 // down: K shares (set by the launcher)
    float *partial;              // down with KS > 1: share sums [KS][rows][R]
    uint32_t *flags;
    RouteJob job;                // gate/up only: run in ROUTE_JOB_WGS extra workgroups
};
// Whether both launches below take hidden H, intermediate I and `cap` rows per expert: K a
// multiple of 1024 with K/1024 a power of two (gate/up: up to 4; down: up to 16, more than 4
// only for a lone expert), R a multiple of 16, at most 16 rows per expert whose codes fit LDS.
bool moe_b_fused_shapes(uint32_t H, uint32_t I, uint32_t cap, bool single);
bool launch_moe_b_gateup_fused(const MoeBArgs &args, uint32_t max_active, hipStream_t stream);
// Returns the K shares it launched with (0: nothing launched). One share: the rounded expert outputs
// are in args.out / args.out_bf16. KS > 1 (a lone expert): the share sums are in args.partial,
// args.rows * R floats apart, for the output rounding to add in share order.
uint32_t launch_moe_b_down_fused(const MoeBArgs &args, uint32_t max_active, hipStream_t stream);

// The runtime points this at its timer for the duration of one ABI call (calls on a runtime are
// serialised by the caller, and each thread has its own pointer).
extern thread_local KernelTimer *tl_timer;
inline int timer_begin(uint32_t id, hipStream_t s) { return tl_timer ? tl_timer->begin(id, s) : -1; }
inline void timer_end(int slot, hipStream_t s)
{
    if (tl_timer)
        tl_timer->end(slot, s);
}

// x: `planes` bf16 planes [planes][W][K] (1: bf16 activations, 3: f32 split by launch_split_planes)
void launch_linear_a(const ProjTile *tiles, uint32_t n_tiles, const uint16_t *x, int planes,
                     uint32_t W, uint32_t K, float *y32, uint16_t *y16, uint32_t N,
                     uint32_t round_f32, hipStream_t stream);
void launch_split_planes(const float *x, uint32_t n, uint16_t *planes, hipStream_t stream);
// Mode A on f32 activation rows [W][K]: one row is split into its planes inside the projection's
// staging; more rows (or a split whose stage would not fit) go through launch_split_planes into
// `scratch` ([3][W][K] bf16) first.
void launch_linear_a_f32(const ProjTile *tiles, uint32_t n_tiles, const float *xf, uint16_t *scratch, uint32_t W,
                         uint32_t K, float *y32, uint16_t *y16, uint32_t N, uint32_t round_f32,
                         hipStream_t stream);
void launch_linear_b(const ProjTile *tiles, uint32_t n_tiles, const uint8_t *codes,
                     const float *scales, uint32_t W, uint32_t K, float *y32, uint16_t *y16,
                     uint32_t N, uint32_t round_f32, hipStream_t stream);
void launch_quant_group128(const void *x, bool x_f32, uint32_t rows, uint32_t K, uint8_t *codes,
                           float *scales, uint32_t *flags, hipStream_t stream);

// One m-tile of the prefill's grouped GEMM (up to PREFILL_MT placement slots of one routed
// expert, in ascending expert order): the expert's weights and the tile's slots, so a GEMM
// workgroup finds its operands in one load.
constexpr uint32_t PREFILL_MT = 128;
struct PfTileDesc {
    ExpertPtrs ep;
    uint32_t slot0;   // first placement slot
    uint32_t cnt;     // placement slots of the tile
    uint32_t expert;  // the routed expert's id (sets the tile's K order, so it never depends on the batch)
    uint32_t pad;
};
static_assert(sizeof(PfTileDesc) == 64, "a tile descriptor is one 64-byte scalar load");
struct PfTileTable {
    PfTileDesc *tiles;  // [max_tiles]
    uint32_t *n_tiles;  // [1]
    uint32_t max_tiles;
};

// Bytes of MoeBuffers::sched the schedule of `rows` token rows over E experts needs (0 for the
// batches scheduled in one workgroup).
size_t moe_sched_scratch_bytes(uint32_t rows, uint32_t E);
// Activation rows [rows][K] (f32 or bf16) for the dynamic FP8 quantiser: codes [rows][K] e4m3 and
// scales [rows][K / 128].
struct QuantJob {
    const void *x;
    uint32_t f32, rows, K;
    uint8_t *codes;
    float *scales;
};
// Returns true when the batch took the long-batch schedule, which also writes the prefill's
// m-tile table when given tiles and quantises `quant` when given (in the same launch as its plan);
// false: the caller launches both itself. With `quantised` non-null, a decode batch's one-wave
// schedule also quantises `quant` (in other workgroups of its launch); *quantised tells whether
// `quant` was done by either path.
bool launch_moe_schedule(const ExpertPtrs *bank, const uint32_t *ids, const float *weights,
                         uint32_t rows, uint32_t E, uint32_t max_active, const MoeBuffers &mb,
                         uint32_t *flags, hipStream_t stream, const PfTileTable *tiles = nullptr,
                         const QuantJob *quant = nullptr, bool *quantised = nullptr);
// expert_offsets [E + 1]: expert e's placement slots are [off[e], off[e + 1]) (after a schedule).
void launch_expert_offsets(const MoeBuffers &mb, uint32_t E, uint32_t *expert_offsets, hipStream_t stream);
// One token's routes for a mode A layer launched without a schedule (moe_a_one_token_direct).
struct OneTokenRoutes {
    const uint32_t *ids;  // [8]
    const float *w;       // [8]
    uint32_t E;           // experts in the bank
};
// routes: a one-token mode A batch that moe_a_one_token_direct accepts, with no schedule launched
// before (mb's schedule tables are not read).
void launch_moe_layer(uint32_t mode, const ExpertPtrs *bank, const MoeBuffers &mb, const void *x,
                      bool x_f32, uint32_t rows, uint32_t max_active, uint32_t max_count, uint32_t H,
                      uint32_t I, float *out_f32, uint16_t *out_bf16, bool raw, uint32_t *flags,
                      hipStream_t stream, const OneTokenRoutes *routes = nullptr, bool x_quantised = false,
                      const RouteJob *job = nullptr);

// Device router (pw_router.hip): x [rows][K] (f32 or bf16) and router weights [E][K] (f32 or bf16)
// -> scores [rows][E], selected / weights [rows][8]; tie_rows (optional) counts boundary ties.
void launch_router(const void *x, bool x_f32, const void *w, bool w_f32, const float *bias, uint32_t rows,
                   uint32_t E, uint32_t K, float *scores, uint32_t *selected, float *weights, uint32_t *tie_rows,
                   uint32_t *flags, hipStream_t stream);
// Its scores kernel alone (scores [rows][E]) and its selection alone (from scores).
void launch_router_scores(const void *x, bool x_f32, const void *w, bool w_f32, uint32_t rows, uint32_t E,
                          uint32_t K, float *scores, hipStream_t stream);
void launch_router_select(const float *scores, const float *bias, uint32_t rows, uint32_t E, uint32_t *selected,
                          float *weights, uint32_t *tie_rows, uint32_t *flags, hipStream_t stream);
// A decode batch's expert sets (fast_top8_set, select_route_row where a boundary is tied) and its
// schedule in one launch, with zero placement weights and the sets in set_ids [rows][8]; with
// `quant`, the launch also quantises those activation rows. False (nothing launched) outside
// rows 1..8, 9..256 experts, 64 routed experts. A RouteJob then writes the routes, their weights
// and the placement weights before the combine: inside one of the layer's expert launches
// (launch_moe_layer's job) or as launch_route_weights.
bool launch_route_set_schedule(const float *scores, const float *bias, const ExpertPtrs *bank, uint32_t rows,
                               uint32_t E, uint32_t max_active, uint32_t *set_ids, const MoeBuffers &mb,
                               uint32_t *flags, hipStream_t stream, const QuantJob *quant = nullptr);
void launch_route_weights(const RouteJob &job, hipStream_t stream);
// The expert sets alone (row_expert_set: one wave per row) into set_ids [rows][8], rows <= 8.
void launch_route_set(const float *scores, const float *bias, uint32_t rows, uint32_t E, uint32_t *set_ids,
                      hipStream_t stream);

// Routed-MoE prefill (mode B grouped block-FP8 GEMM, pw_prefill.hip) after launch_moe_schedule.
struct PrefillBuffers {
    PfTileDesc *tiles;  // [prefill_max_tiles]
    uint32_t *n_tiles;  // [1]
    uint16_t *hidden;   // [rows * 8][2I] bf16 gate and up outputs
    uint16_t *y;        // [rows * 8][H] bf16 expert outputs
    const uint16_t *silu;  // [65536] bf16-staged silu of every bf16 gate, from launch_silu_table
};
void launch_silu_table(uint16_t *table, hipStream_t stream);
// Elementwise bf16-staged SwiGLU of f32 gate/up [n]; silu_table null: silu evaluated in place.
void launch_swiglu_staged(const float *gate, const float *up, uint32_t n, const uint16_t *silu_table, float *out,
                          uint32_t *flags, hipStream_t stream);
uint32_t prefill_max_tiles(uint32_t rows, uint32_t E);
// scheduled_long: launch_moe_schedule returned true for this batch, given pb's tile table and the
// QuantJob of x into mb.xq / mb.xs (the m-tile table and the activation codes are in place).
void launch_moe_prefill(const ExpertPtrs *bank, const MoeBuffers &mb, const PrefillBuffers &pb, const void *x,
                        bool x_f32, uint32_t rows, uint32_t E, uint32_t H, uint32_t I, float *out_f32,
                        uint16_t *out_bf16, bool raw, uint32_t *flags, hipStream_t stream, bool scheduled_long);

void launch_expert_forward(uint32_t mode, const ExpertPtrs *bank, const ExpertPtrs &ep, uint32_t expert,
                           const MoeBuffers &mb,
                           const void *x, bool x_f32, uint32_t rows, uint32_t H, uint32_t I,
                           float *out_f32, uint16_t *out_bf16, bool raw, uint32_t *flags, hipStream_t stream);

// Seeded synthetic data for benchmarks and tests (counter-based, reproducible on one device).
void launch_synth_fp8(uint8_t *w, const float *scales, uint64_t rows, uint64_t cols, uint64_t seed,
                      hipStream_t stream);
void launch_synth_scales(float *s, uint64_t count, uint64_t seed, float log2_lo, float log2_hi,
                         hipStream_t stream);
void launch_synth_normal_bf16(uint16_t *x, uint64_t count, uint64_t seed, float stddev,
                              hipStream_t stream);

}  // namespace pw
