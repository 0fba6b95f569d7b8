/*
 * pwfp8 — MI355X (gfx950) block-scaled FP8 projection and routed-MoE expert path, C ABI.
 *
 * Drop-in replacement for the reference's WideMetalMoeRuntime (x3haloed/mimo-prismwing,
 * src/wide_metal_moe.rs:113-1315) and the CPU routing helpers that feed it. Plain C types only:
 * pointers, sizes, status codes; no exceptions cross the boundary; every call returns an int
 * status (0 = ok, negative = distinct error class) and sets a thread-local message readable with
 * pw_last_error().
 *
 * Numerical modes (the two the reference keeps apart):
 *   PW_MODE_A  FP8 weight x f32/bf16 activation, f32 accumulation (block_fp8_gemv/gemm{1..8}
 *              _shared_weight_lut_blocked, kernels/block_fp8_gemv.metal:665-933; CPU
 *              mapped_fp8_gemv src/lib.rs:1272-1309 and the CPU control src/lib.rs:5807-5862).
 *   PW_MODE_B  dynamic per-(row, 128-column) FP8 activation, block-scaled products, bf16 staged
 *              (block_fp8_gemm{1..32}_sglang_blockscaled, kernels/block_fp8_gemv.metal:935-1046;
 *              CPU fp8_linear src/text_endpoint.rs:3053-3108).
 *
 * Threading: one runtime per device, calls on one runtime are serialised by the caller (the
 * reference's &self + one command queue). Host-memory calls are synchronous like the reference;
 * the *_device calls are asynchronous on the HIP stream given (NULL = the runtime's stream, a
 * blocking stream, so it is ordered with work on the HIP null stream). Calls share the runtime's
 * scratch buffers, so the runtime orders each call's GPU work after the previous call's: a call
 * on another stream than the previous call makes its stream wait for the previous call's work
 * first (nothing is waited for while calls keep to one stream). A caller's stream is not used
 * after the call returns. To overlap work, use one runtime per stream.
 */
#ifndef PWFP8_H
#define PWFP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PW_ABI_VERSION 1

/* ---- status codes -------------------------------------------------------------------------- */
enum {
    PW_OK = 0,
    PW_ERR_ARGUMENT = -1,  /* null pointer, zero or out-of-range size, unknown enum */
    PW_ERR_LAYOUT = -2,    /* weight / scale-grid shape mismatch ("layout mismatch") */
    PW_ERR_NONFINITE = -3, /* non-finite input, scale, route weight, or 0x7f/0xff weight code */
    PW_ERR_SCHEDULE = -4,  /* placements != rows*8, count 0 or > 32, position >= rows, ... */
    PW_ERR_DEVICE = -5,    /* HIP runtime failure */
    PW_ERR_GPU_FLAGS = -6, /* a kernel raised its error bitmask (see stats gpu_flags) */
    PW_ERR_NOMEM = -7,
    PW_ERR_OUTPUT = -8     /* non-finite output */
};

enum { PW_MODE_A = 0, PW_MODE_B = 1 };
/* Activation / output element types. F32 outputs hold bf16-rounded values (the reference's
 * Vec<f32> of bf16 values); F32_RAW (outputs only) is the f32 result before that final round. */
enum { PW_DTYPE_F32 = 0, PW_DTYPE_BF16 = 1, PW_DTYPE_F32_RAW = 2 };
/* Projection layouts: plain row-major, or the checkpoint's four concatenated tensor-parallel QKV
 * shards that the reference deinterleaves on one device (src/text_endpoint.rs:3174-3242,
 * kernels/block_fp8_gemv.metal:259-297). */
enum { PW_LAYOUT_PLAIN = 0, PW_LAYOUT_FULL_QKV_TP4 = 1, PW_LAYOUT_SWA_QKV_TP4 = 2 };
/* Runtime flags: compile_with_fused_gate_up (src/wide_metal_moe.rs:169-171). Gate and up always
 * share one pass here; the flag is kept so callers of both constructors port unchanged. */
enum { PW_RUNTIME_FUSED_GATE_UP = 1 };

/* GPU error bitmask (bits 1..128 keep the reference's Metal error-word meanings). */
#define PW_FLAG_LANES 1u
#define PW_FLAG_QUANT_NONFINITE 2u
#define PW_FLAG_SWIGLU_NONFINITE 4u
#define PW_FLAG_REDUCE_NONFINITE 16u
#define PW_FLAG_ROUND_NONFINITE 32u
#define PW_FLAG_FUSED_SWIGLU_NONFINITE 128u
#define PW_FLAG_SCHEDULE 256u
#define PW_FLAG_OUTPUT_NONFINITE 512u
#define PW_FLAG_ROUTE 1024u /* device router: a row's scores, bias or selection were invalid */

typedef struct pw_runtime pw_runtime;
typedef struct pw_projection pw_projection;
typedef struct pw_expert_bank pw_expert_bank;
typedef struct pw_safetensors pw_safetensors;

/* WideSourceRegion (src/wide_metal_moe.rs:38-78): a tensor inside a larger (e.g. mmapped,
 * page-rounded) host region. */
typedef struct {
    const void *bytes;
    size_t region_bytes;
    size_t tensor_offset;
    size_t tensor_bytes;
} pw_region;

/* WideProjectionBinding (src/wide_metal_moe.rs:80-86). */
typedef struct {
    pw_region weight;      /* F8_E4M3 [rows x columns] */
    pw_region scale;       /* F32 [ceil(rows/128) x columns/128]; [108 x 32] / [116 x 32] for TP4 */
    uint32_t rows;
    uint32_t columns;
    uint32_t layout;       /* PW_LAYOUT_* */
    uint32_t copy_weight;  /* the reference's copy flag; weights are always made HBM-resident */
} pw_projection_desc;

/* One tensor of a concatenated projection (e.g. separate q, k, v), each with its own scale grid
 * ceil(rows/128) x columns/128; a partial trailing 128-row block is allowed. */
typedef struct {
    pw_region weight;
    pw_region scale;
    uint32_t rows;
} pw_segment_desc;

/* WideExpertBinding (src/wide_metal_moe.rs:88-95). */
typedef struct {
    uint32_t expert;
    uint32_t count;                /* placements routed to this expert, 1..32 */
    const uint32_t *positions;     /* [count] token rows, ascending */
    const float *route_weights;    /* [count] */
    const pw_projection *gate;     /* [intermediate x hidden] */
    const pw_projection *up;       /* [intermediate x hidden] */
    const pw_projection *down;     /* [hidden x intermediate] */
} pw_expert_binding;

/* WideLinearExecution (src/wide_metal_moe.rs:106-111). */
typedef struct {
    double wall_ms;
    uint64_t mapped_source_bytes;
    uint64_t resident_source_bytes;
    uint32_t gpu_flags;
} pw_linear_stats;

/* WideMoeExecution (src/wide_metal_moe.rs:97-104). */
typedef struct {
    double wall_ms;
    uint32_t unique_experts;
    uint32_t expert_rows;
    uint64_t mapped_source_bytes;
    uint64_t resident_source_bytes;
    uint32_t gpu_flags;
} pw_moe_stats;

/* ---- runtime ------------------------------------------------------------------------------ */
/* Message of the last failing call on this thread ("" if none). */
const char *pw_last_error(void);
int pw_abi_version(void);
/* WideMetalMoeRuntime::compile / compile_with_fused_gate_up (src/wide_metal_moe.rs:164-239):
 * selects the device, creates the runtime's stream and device error word. */
int pw_runtime_create(int device, uint32_t flags, pw_runtime **out);
void pw_runtime_destroy(pw_runtime *rt);
/* The runtime's HIP stream (hipStream_t) for callers that enqueue device work around it. */
void *pw_runtime_stream(pw_runtime *rt);
/* Synchronise the device (all streams), return and clear the device error bitmask. */
int pw_runtime_take_flags(pw_runtime *rt, uint32_t *flags);

/* Per-kernel HIP-event timing for benchmarks (the reference records GPUStartTime/GPUEndTime per
 * command buffer, src/staged_metal_expert.rs:1763-1771): when enabled, every timed launch records
 * a start and a stop event on the stream it runs on, up to max_launches (0 disables). Kernel
 * names: linear_a, linear_b, quant, moe_schedule, moe_gateup, moe_swiglu, moe_down, moe_combine,
 * prefill_gateup, prefill_down, router, bf16_linear, route_schedule (the expert-set and schedule
 * launch of pw_moe_layer_routed_device). */
int pw_runtime_enable_timing(pw_runtime *rt, uint32_t max_launches);
/* Synchronise the device; report the recorded launches of `kernel` and their summed duration. */
int pw_runtime_timing_summary(pw_runtime *rt, const char *kernel, uint32_t *launches,
                              double *total_ms);
/* Synchronise and forget the recorded launches (the events are kept). */
int pw_runtime_timing_reset(pw_runtime *rt);

/* ---- weight binding ----------------------------------------------------------------------- */
/* Copies a checkpoint-bound FP8 weight view and its scale grid into HBM once (the reference binds
 * no-copy Metal buffers per call, src/wide_metal_moe.rs:259-272, :871-910). Validates like
 * validate_fp8_views_internal (src/lib.rs:1217-1270): nonzero rows/columns, columns % 128 == 0,
 * scale grid size, finite scales; with scan_codes also rejects 0x7f/0xff weight codes. */
int pw_projection_bind(pw_runtime *rt, const pw_projection_desc *desc, int scan_codes,
                       pw_projection **out);
/* Concatenation of separately stored tensors sharing `columns`, output rows in segment order
 * (attention q/k/v with nonuniform scale grids and partial trailing blocks). */
int pw_projection_bind_segments(pw_runtime *rt, const pw_segment_desc *segments, uint32_t count,
                                uint32_t columns, int scan_codes, pw_projection **out);
/* No-copy binding of weights already resident in device memory (layout PW_LAYOUT_PLAIN). */
int pw_projection_bind_device(pw_runtime *rt, const void *weight, const float *scale, uint32_t rows,
                              uint32_t columns, pw_projection **out);
void pw_projection_release(pw_projection *proj);
int pw_projection_shape(const pw_projection *proj, uint32_t *rows, uint32_t *columns);

/* ---- projections --------------------------------------------------------------------------- */
/* WideMetalMoeRuntime::execute_fp8_linear (src/wide_metal_moe.rs:241-385): input f32
 * [rows x columns] (rows 1..32), output [rows x proj_rows] bf16-rounded f32. mode B reproduces
 * the reference call; mode A is the FP8-weight / f32-activation projection. Synchronous. */
int pw_fp8_linear(pw_runtime *rt, uint32_t mode, const float *input, uint32_t rows,
                  const pw_projection *proj, float *output, pw_linear_stats *stats);
/* Device-resident form: input [rows x columns] of input_dtype, output [rows x proj_rows] of
 * output_dtype (f32 output holds bf16-rounded values when round_output != 0), enqueued on stream.
 * Mode B needs the runtime's scratch for the activation codes; rows <= 32. */
int pw_fp8_linear_device(pw_runtime *rt, uint32_t mode, const void *input, uint32_t input_dtype,
                         uint32_t rows, const pw_projection *proj, void *output,
                         uint32_t output_dtype, uint32_t round_output, void *stream);

/* ---- BF16 wide linear ---------------------------------------------------------------------- */
/* Binds a checkpoint BF16 weight view [rows x columns] (o_proj, LM head) and copies it into HBM once
 * (the reference maps the region no-copy per call in execute_bf16_linear,
 * src/wide_metal_moe.rs:728-760, and checks tensor_bytes == rows * columns * 2: a mismatch is
 * PW_ERR_LAYOUT "wide BF16 linear layout mismatch"). columns % 128 == 0. The handle is released
 * with pw_projection_release and reports its shape through pw_projection_shape. */
int pw_bf16_bind(pw_runtime *rt, const pw_region *weight, uint32_t rows, uint32_t columns, pw_projection **out);
/* No-copy binding of BF16 weights already resident in device memory (16-byte aligned). */
int pw_bf16_bind_device(pw_runtime *rt, const void *weight, uint32_t rows, uint32_t columns,
                        pw_projection **out);
/* WideMetalMoeRuntime::execute_bf16_linear (src/wide_metal_moe.rs:728-834; CPU twin bf16_linear,
 * src/text_endpoint.rs:3347-3380): input f32 [rows x columns] (rows 1..32; the reference allows
 * 1..8), output f32 [rows x proj_rows] = round_bf16(sum_c bf16(W[r, c]) * x[p, c]) with f32
 * accumulation. Non-finite input -> PW_ERR_NONFINITE; a non-finite output raises the reference's
 * error bit 32 (PW_FLAG_ROUND_NONFINITE) -> PW_ERR_GPU_FLAGS. Synchronous. */
int pw_bf16_linear(pw_runtime *rt, const float *input, uint32_t rows, const pw_projection *proj, float *output,
                   pw_linear_stats *stats);
/* Device-resident form (input 16-byte aligned, input_dtype F32 or BF16; output_dtype as for
 * pw_fp8_linear_device), enqueued on stream. */
int pw_bf16_linear_device(pw_runtime *rt, const void *input, uint32_t input_dtype, uint32_t rows,
                          const pw_projection *proj, void *output, uint32_t output_dtype, uint32_t round_output,
                          void *stream);

/* Dynamic per-(row, 128-column group) FP8 activation quantiser on device rows
 * (dynamic_fp8_quantized_group128, kernels/block_fp8_gemv.metal:84-137; CPU authority
 * dynamic_fp8_activations, src/text_endpoint.rs:3008-3051): scale = max(absmax, 1e-10)/448,
 * code = nearest e4m3fn of clamp(x/scale, +-448), ties to the even code. codes [rows x cols],
 * scales [rows x cols/128]; x and codes 16-byte aligned. Non-finite inputs raise
 * PW_FLAG_QUANT_NONFINITE. */
int pw_quantize_fp8_group128_device(pw_runtime *rt, const void *x, uint32_t x_dtype, uint32_t rows,
                                    uint32_t cols, uint8_t *codes, float *scales, void *stream);

/* bf16_staged_swiglu (kernels/block_fp8_gemv.metal:139-160, the reference's own elementwise pass
 * between the gate/up and down projections; CPU src/text_endpoint.rs:5336-5343) on device f32
 * arrays: out[i] = round(round(silu(round(gate[i]))) * round(up[i])) with silu(g) = g / (1 + e^-g)
 * and round = bf16 round-to-nearest-even. form 0 evaluates the silu in place, as the decode
 * kernels do; form 1 looks it up in the runtime's 65,536-entry table, as the prefill kernels do
 * (the first such call on a runtime builds the table on the runtime's stream and waits for it).
 * Non-finite gate, up or output values raise PW_FLAG_SWIGLU_NONFINITE. Asynchronous on stream. */
int pw_swiglu_staged_device(pw_runtime *rt, const float *gate, const float *up, uint32_t count, float *out,
                            uint32_t form, void *stream);

/* ---- checkpoint files ------------------------------------------------------------------------ */
/* One tensor of a safetensors file: dtype string ("F8_E4M3", "F32", "BF16", ...), shape, and a
 * region over its bytes inside the read-only file mapping (valid until pw_safetensors_close). */
typedef struct {
    char dtype[16];
    uint32_t rank;
    uint64_t shape[8];
    pw_region region;
} pw_tensor_info;

/* MappedSafetensors::open (src/lib.rs:783-905): maps the file read-only and parses its header:
 * 8-byte little-endian length (nonzero, <= 256 MiB, a multiple of 8, inside the file), a JSON object
 * of {dtype, shape, data_offsets} per tensor plus an optional __metadata__ object; rejects unknown
 * dtypes, empty or zero shapes, sizes that disagree with shape x dtype, payloads past the file,
 * overlapping payloads, duplicate names and files without tensors (PW_ERR_LAYOUT). */
int pw_safetensors_open(const char *path, pw_safetensors **out);
void pw_safetensors_close(pw_safetensors *st);
uint32_t pw_safetensors_count(const pw_safetensors *st);
/* MappedSafetensors::tensor (src/lib.rs:907-930): PW_ERR_ARGUMENT "tensor is absent" if missing. */
int pw_safetensors_tensor(const pw_safetensors *st, const char *name, pw_tensor_info *info);
/* A layer's routed experts from checkpoint files into one HBM allocation the bank owns: for each
 * expert e < n_experts, model.layers.{layer}.mlp.experts.{e}.{gate,up,down}_proj.weight and
 * ..._scale_inv (the names of src/text_endpoint.rs:4785-4845), looked up across the files in order,
 * validated like validate_fp8_views_internal (src/lib.rs:1217-1270: F8_E4M3 rank two of shape
 * [intermediate x hidden] / [hidden x intermediate], F32 scale grids [rows/128 x cols/128], finite
 * scales, and with scan_codes no 0x7f/0xff code), then copied once. */
int pw_expert_bank_from_safetensors(pw_runtime *rt, const pw_safetensors *const *files, uint32_t n_files,
                                    uint32_t layer, uint32_t n_experts, uint32_t hidden, uint32_t intermediate,
                                    int scan_codes, pw_expert_bank **out);

/* ---- routed MoE ---------------------------------------------------------------------------- */
/* WideMetalMoeRuntime::execute / execute_fused_gate_up (src/wide_metal_moe.rs:836-1314): input
 * f32 [rows x hidden] (rows 1..128), one binding per routed expert (any order; placements must
 * cover rows*8 exactly, count 1..32 each), output f32 [rows x hidden] bf16-rounded. */
int pw_moe_execute(pw_runtime *rt, uint32_t mode, uint32_t fused_gate_up, const float *input,
                   uint32_t rows, const pw_expert_binding *experts, uint32_t n_experts,
                   float *output, pw_moe_stats *stats);

/* A layer's routed experts resident in HBM, indexed by expert id (the device analogue of the
 * reference binding each expert's checkpoint regions per call, src/text_endpoint.rs:4790-4841).
 * All experts share shapes gate/up [intermediate x hidden], down [hidden x intermediate]. */
int pw_expert_bank_create(pw_runtime *rt, uint32_t n_experts, const pw_projection *const *gate,
                          const pw_projection *const *up, const pw_projection *const *down,
                          pw_expert_bank **out);
void pw_expert_bank_release(pw_expert_bank *bank);
int pw_expert_bank_shape(const pw_expert_bank *bank, uint32_t *n_experts, uint32_t *hidden,
                         uint32_t *intermediate);

/* One routed-MoE layer with inputs already in device memory: x [rows x hidden] (x_dtype, 16-byte
 * aligned), route_ids / route_weights [rows x 8] (the reference's RoutingTrace selected/weights,
 * src/text_endpoint.rs:4342-4380; 16-byte aligned), output [rows x hidden] (out_dtype,
 * bf16-rounded). The schedule is built on the device in the reference's BTreeMap order (a
 * one-token mode A layer at hidden 4096, intermediate 2048 ranks its eight routes inside its
 * kernels instead: the same order, the same rejections). Invalid routes raise PW_FLAG_SCHEDULE.
 * rows <= 32. Asynchronous on stream; kernel error bits accumulate in the runtime's error word. */
int pw_moe_layer_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                        uint32_t x_dtype, uint32_t rows, const uint32_t *route_ids,
                        const float *route_weights, void *output, uint32_t out_dtype, void *stream);

/* A decode step's routing and its routed layer in one call on device buffers: route_mlp
 * (src/text_endpoint.rs:4342-4380, as pw_route_device runs it over the bank's experts: router_weight
 * [n_experts x hidden] f32 or bf16, bias [n_experts]) followed by the routed layer on those routes
 * (as pw_moe_layer_device), the composition routed_mlp_traced (src/text_endpoint.rs:5290-5381) makes.
 * The routes are also written to route_ids / route_weights [rows x 8] (16-byte aligned), the
 * reference's RoutingTrace. For decode batches of up to 8 rows over banks of up to 256 experts the
 * layer's schedule is built from each row's expert set (found without the top-k partition where the
 * row's top-8 boundary is not tied), and the routes' order and weights (the partition) run in extra
 * workgroups of one of the layer's expert launches, beside the expert weight stream. The same
 * routes and the same output bytes as pw_route_device then pw_moe_layer_device. A row whose routing fails raises
 * PW_FLAG_ROUTE, and the batch is rejected like invalid routes (PW_FLAG_SCHEDULE, zero output).
 * rows 1..32; hidden a multiple of 8; x and router_weight 16-byte aligned. Asynchronous on stream. */
int pw_moe_layer_routed_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                               uint32_t x_dtype, uint32_t rows, const void *router_weight, uint32_t w_dtype,
                               const float *bias, uint32_t *route_ids, float *route_weights, void *output,
                               uint32_t out_dtype, void *stream);

/* No counterpart in the reference: pw_moe_layer_device for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as pw_moe_layer_device, for decode batches of 1..8 rows over
 * banks of at most 256 experts, hidden <= 4096 and intermediate <= 2048 (larger requests fail with
 * PW_ERR_ARGUMENT). Its scratch (schedule tables, activation planes, split-K partials, expert
 * outputs; 12 MiB) is a static device array that each GPU holds until the process ends, looked up
 * once per device by pw_runtime_create; the call allocates nothing. Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU race: calls through one runtime are ordered
 * like its other calls, but two runtimes (or threads) on one device must not run it concurrently.
 * Asynchronous on stream. */
int pw_moe_layer_device_noalloc(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                                uint32_t x_dtype, uint32_t rows, const uint32_t *route_ids,
                                const float *route_weights, void *output, uint32_t out_dtype, void *stream);

/* Routed-MoE prefill over many token rows (rows 1..4096, e.g. 2048 tokens -> 16 384 placements)
 * with inputs in device memory, in mode B: the reference's layer-major prefill runs 128-row
 * slices through WideMetalMoeRuntime::execute (run_layer_major_moe_slice_mode,
 * src/text_endpoint.rs:4951-5287; src/wide_metal_moe.rs:852-1314), here one grouped block-FP8
 * GEMM per projection on the FP8 MFMA (any number of placements per expert). x [rows x hidden]
 * (x_dtype), route_ids / route_weights [rows x 8], output [rows x hidden] (out_dtype,
 * bf16-rounded); x, the routes and the output 16-byte aligned. Asynchronous on stream; kernel error bits accumulate
 * in the runtime's word. The first call on a runtime also builds a 128 KB silu table on the
 * runtime's stream and waits for that stream once. */
int pw_moe_prefill_device(pw_runtime *rt, const pw_expert_bank *bank, const void *x, uint32_t x_dtype,
                          uint32_t rows, const uint32_t *route_ids, const float *route_weights, void *output,
                          uint32_t out_dtype, void *stream);

/* The device routed schedule on its own, for callers that keep the reference's expert placement
 * counts: route_ids / route_weights [rows x 8] (device, 16-byte aligned, rows 1..4096) over the
 * bank's experts -> the reference's BTreeMap<expert, [(position, weight)]>
 * (src/text_endpoint.rs:4767-4775) as device tables: expert_offsets [n_experts + 1] (expert e's
 * placement slots are [offsets[e], offsets[e + 1]), so its placement count is the difference),
 * positions / weights [rows x 8] (token row and router weight of each slot: experts ascending,
 * token rows ascending within an expert) and row_slots [rows x 8] (each token's eight slots in
 * ascending expert id, the combine order of src/text_endpoint.rs:5365-5373). Rejected routes
 * (the checks of WideMetalMoeRuntime::execute, src/wide_metal_moe.rs:858-938) raise
 * PW_FLAG_SCHEDULE. The same schedule the layer entry points build. Asynchronous on stream. */
int pw_moe_schedule_device(pw_runtime *rt, const pw_expert_bank *bank, const uint32_t *route_ids,
                           const float *route_weights, uint32_t rows, uint32_t *expert_offsets,
                           uint32_t *positions, float *weights, uint32_t *row_slots, void *stream);

/* One complete expert (gate/up -> SwiGLU -> down, no routing, no combine) on device rows
 * x [rows x hidden] (16-byte aligned) -> output [rows x hidden] bf16-rounded: the reference's complete-expert
 * measurement (direct-checkpoint L3 expert, src/lib.rs:4008-6590; mode A widths 1..8 via
 * block_fp8_gemm{w}_shared_weight_lut_blocked). rows <= 32. Asynchronous on stream. */
int pw_expert_forward_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t expert,
                             uint32_t mode, const void *x, uint32_t x_dtype, uint32_t rows,
                             void *output, uint32_t out_dtype, void *stream);

/* ---- routing on the device ------------------------------------------------------------------ */
/* route_mlp (src/text_endpoint.rs:4342-4380) on device buffers: logits = x [rows x hidden] .
 * router_weight [experts x hidden]^T (f32 or bf16 each), scores = PyTorch sigmoid (SLEEF
 * expf_u10), corrected = scores + bias, top 8 in libc++ nth_element order, weights renormalised
 * (pytorch_noaux_routes, :4394-4473). Writes route_ids / route_weights [rows x 8] (16-byte
 * aligned; the pw_moe_layer_device / pw_moe_prefill_device inputs), scores [rows x experts] when
 * not NULL, and adds the number of boundary-tie rows to *tie_rows (a device counter) when not
 * NULL. hidden is a multiple of 8 (at most 65536); x and router_weight are 16-byte aligned.
 * Logits sum in a fixed order: 256 partial sums of fused multiply-adds, partial g over the 8-column
 * groups starting at 8g, 8g + 2048, ..., each 64 of them reduced by a halving tree, the four wave
 * sums added as (w0 + w1) + (w2 + w3). An invalid row raises PW_FLAG_ROUTE and gets expert ids =
 * experts (the layer schedule rejects them). rows 1..4096, experts 9..1024. Asynchronous on
 * stream. */
int pw_route_device(pw_runtime *rt, const void *x, uint32_t x_dtype, uint32_t rows, uint32_t hidden,
                    const void *router_weight, uint32_t w_dtype, uint32_t experts, const float *bias,
                    uint32_t *route_ids, float *route_weights, float *scores, uint32_t *tie_rows, void *stream);

/* ---- routing on the host (src/text_endpoint.rs:4342-4473, src/pytorch_topk.cpp:8-30) -------- */
/* pw_pytorch_topk_unsorted_f32 (src/pytorch_topk.cpp:7-30, declared by its caller at
 * src/text_endpoint.rs:2466-2474): the indices of the top_k largest values, in the partition order
 * of libc++'s std::nth_element(first, first + top_k - 1, last) over (value, index) pairs compared
 * greater-by-value. Returns 0; -1 when values or selected is NULL, top_k == 0 or top_k >= count;
 * -2 when the pair buffer cannot be allocated. The reference's own symbol name and signature, so
 * its extern "C" block links unchanged. */
int pw_pytorch_topk_unsorted_f32(const float *values, size_t count, size_t top_k, uint32_t *selected);
/* The same function under this library's pw_ prefix (identical arguments, results and codes). */
int pw_topk_unsorted_f32(const float *values, size_t count, size_t top_k, uint32_t *selected);
/* pytorch_noaux_routes: scores [rows x experts] (sigmoid outputs), bias [experts] ->
 * selected / weights [rows x 8]; *tie_rows counts boundary ties. */
int pw_noaux_routes(const float *scores, const float *bias, uint32_t rows, uint32_t experts,
                    uint32_t *selected, float *weights, uint64_t *tie_rows);
/* route_mlp from logits: PyTorch SLEEF sigmoid, bias, top-8, renormalised weights. */
int pw_route_from_logits(const float *logits, const float *bias, uint32_t rows, uint32_t experts,
                         float *scores, uint32_t *selected, float *weights, uint64_t *tie_rows);

/* ---- layout maps (src/text_endpoint.rs:3174-3242) ------------------------------------------ */
int64_t pw_full_qkv_source_row(int64_t logical_row);
int64_t pw_full_qkv_scale_row(int64_t logical_row);
int64_t pw_swa_qkv_source_row(int64_t logical_row);

/* ---- seeded synthetic data on the device (benchmarks and tests) ---------------------------- */
/* scales[i] = 2^(log2_lo + (log2_hi - log2_lo) u_i), u_i uniform from (seed, i). */
int pw_synth_scales(pw_runtime *rt, float *scales, uint64_t count, uint64_t seed, float log2_lo,
                    float log2_hi);
/* w[r, c] = e4m3(clamp(z / scales[r/128, c/128], +-448)), z ~ N(0,1) from (seed, r*cols + c). */
int pw_synth_fp8(pw_runtime *rt, uint8_t *w, const float *scales, uint64_t rows, uint64_t cols,
                 uint64_t seed);
/* x[i] = bf16(z_i * stddev), z ~ N(0,1) from (seed, i); count even. */
int pw_synth_normal_bf16(pw_runtime *rt, uint16_t *x, uint64_t count, uint64_t seed, float stddev);

#ifdef __cplusplus
}
#endif
#endif /* PWFP8_H */
