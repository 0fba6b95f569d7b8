// C-ABI runtime for the gfx950 block-FP8 projection and routed-MoE path (include/pwfp8.h).
//
// Mirrors WideMetalMoeRuntime (src/wide_metal_moe.rs:113-1315): same call surface, same
// fail-closed validation, same outputs (bf16-rounded f32). What differs is the memory model:
// weights are bound once into HBM (pw_projection / pw_expert_bank) instead of wrapping mmapped
// pages per call, and device-resident entry points let a caller keep activations and routes in
// HBM across calls.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/pwfp8.h"
#include "pw_launch.h"
#include "pw_internal.h"
#include "pw_topk.h"
#include "pw_numerics.h"

using pw::ExpertPtrs;
using pw::MoeBuffers;
using pw::ProjTile;

namespace pw {
thread_local KernelTimer *tl_timer = nullptr;
}

namespace {

const char *const kKernelNames[pw::K_COUNT] = {
    "linear_a", "linear_b", "quant", "moe_schedule", "moe_gateup", "moe_swiglu", "moe_down",
    "moe_combine", "prefill_gateup", "prefill_down", "router", "bf16_linear", "route_schedule"};

thread_local std::string g_error;

}  // namespace

int pw::fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

using pw::fail;

namespace {

#define PW_HIP(call)                                                                            \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            return fail(PW_ERR_DEVICE, "%s failed: %s", #call, hipGetErrorString(e_));          \
    } while (0)

double now_ms()
{
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

bool finite(float v) { return std::isfinite(v); }

struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    ~DevBuf() { release(); }
    void release()
    {
        if (p)
            (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    hipError_t ensure(size_t need)
    {
        if (need <= bytes)
            return hipSuccess;
        release();
        hipError_t e = hipMalloc(&p, need);
        if (e == hipSuccess)
            bytes = need;
        return e;
    }
};

}  // namespace

struct pw_runtime {
    int device = 0;
    uint32_t flags = 0;
    hipStream_t stream = nullptr;
    uint32_t *d_flags = nullptr;
    // scratch: host-call staging and mode-B activation codes
    DevBuf in, out, codes, scales, route_ids, route_w, bank_table;
    // routed-MoE per-layer scratch
    DevBuf moe_plan, moe_active_expert, moe_active_offset, moe_pos, moe_w, moe_slots, moe_hidden,
        moe_hidden_planes, moe_x_planes, moe_y, moe_xq, moe_xs, moe_hq, moe_hs, lin_planes,
        moe_active, moe_pieces, moe_partial, moe_sched, pf_tiles, pf_silu, router_scores, bf16_partial;
    MoeBuffers mb{};
    pw::KernelTimer timer;
    bool silu_ready = false;  // pf_silu holds the complete silu table
    // Calls share the scratch above, so each call is ordered after the previous one: the stream
    // the last call enqueued on, and an event recorded at the end of that call when it was not the
    // runtime's own stream (the runtime never touches a caller's stream after the call returns).
    hipStream_t last_stream = nullptr;
    hipEvent_t order_event = nullptr;
    DevBuf set_ids, set_w;  // the routed layer's expert sets [rows][8] (and their weights, one-token layer)
};

namespace {

// Orders one call's work after the previous call's (they share the runtime's scratch): on entry,
// a stream other than the previous call's waits for the previous call's work; on exit, work
// enqueued on a caller's stream is marked with the runtime's event. No cost while every call uses
// the same stream.
// A call enqueued on a stream under HIP graph capture is left out of this ordering: it neither
// waits on an event recorded outside the capture (a cross-boundary dependency the capture
// rejects) nor records the runtime's event into the graph, and the calls after it are ordered
// against the eager work before it. The caller orders the capture, and every replay of the
// graph, against the runtime's other calls (they share its scratch).
struct StreamOrder {
    pw_runtime *rt;
    hipStream_t s;
    hipError_t err = hipSuccess;
    bool captured = false;
    StreamOrder(pw_runtime *r, hipStream_t stream) : rt(r), s(stream)
    {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        err = hipStreamIsCapturing(s, &status);
        if (err != hipSuccess)
            return;
        captured = status != hipStreamCaptureStatusNone;
        if (!captured && rt->last_stream && rt->last_stream != s) {
            if (rt->last_stream == rt->stream)
                err = hipEventRecord(rt->order_event, rt->stream);
            if (err == hipSuccess)
                err = hipStreamWaitEvent(s, rt->order_event, 0);
        }
    }
    ~StreamOrder()
    {
        if (err != hipSuccess || captured)
            return;
        if (s != rt->stream)
            (void)hipEventRecord(rt->order_event, s);
        rt->last_stream = s;
    }
};

// Points the launchers at the runtime's event timer for the duration of one ABI call.
struct TimerScope {
    explicit TimerScope(pw_runtime *rt) { pw::tl_timer = rt && rt->timer.enabled ? &rt->timer : nullptr; }
    ~TimerScope() { pw::tl_timer = nullptr; }
};

void free_timer(pw::KernelTimer &t)
{
    if (t.events) {
        for (uint32_t i = 0; i < 2 * t.capacity; ++i)
            (void)hipEventDestroy(t.events[i]);
        delete[] t.events;
    }
    delete[] t.ids;
    t = pw::KernelTimer{};
}

}  // namespace

struct pw_projection {
    pw_runtime *rt = nullptr;
    bool bf16 = false;          // BF16 weights [rows][columns] (no scales, no tile table)
    uint8_t *w = nullptr;       // device weight base
    float *s = nullptr;         // device scale base
    bool owns = false;
    uint32_t rows = 0, columns = 0;
    ProjTile *tiles = nullptr;  // device tile table
    uint32_t n_tiles = 0;
    uint64_t weight_bytes = 0, scale_bytes = 0;
};

struct pw_expert_bank {
    pw_runtime *rt = nullptr;
    ExpertPtrs *table = nullptr;  // device [E]
    std::vector<ExpertPtrs> host_table;  // the same pointers, for launches that take one expert by value
    uint32_t n_experts = 0, hidden = 0, intermediate = 0;
    void *owned = nullptr;        // weights and scales the bank owns (checkpoint banks)
    uint64_t owned_bytes = 0;
};

namespace {

hipError_t set_device(pw_runtime *rt) { return hipSetDevice(rt->device); }

// 16-row tiles of one segment: rows [src_row, src_row + rows) of a weight with `columns`
// columns, scale rows scale_base + r/128, output rows out_row + r.
void add_segment_tiles(std::vector<ProjTile> &tiles, const uint8_t *w, const float *s,
                       uint32_t columns, uint64_t src_row, uint32_t rows, uint64_t scale_base,
                       uint32_t out_row)
{
    const uint32_t scale_cols = columns / 128;
    for (uint32_t r = 0; r < rows; r += 16) {
        ProjTile t;
        t.w = w + (src_row + r) * (uint64_t)columns;
        t.s = s + (scale_base + r / 128) * scale_cols;
        t.out_row = out_row + r;
        t.valid = std::min<uint32_t>(16, rows - r);
        tiles.push_back(t);
    }
}

int upload_tiles(pw_projection *p, const std::vector<ProjTile> &tiles)
{
    PW_HIP(hipMalloc(&p->tiles, tiles.size() * sizeof(ProjTile)));
    PW_HIP(hipMemcpy(p->tiles, tiles.data(), tiles.size() * sizeof(ProjTile), hipMemcpyHostToDevice));
    p->n_tiles = (uint32_t)tiles.size();
    return PW_OK;
}

const uint8_t *region_tensor(const pw_region &r) { return (const uint8_t *)r.bytes + r.tensor_offset; }

int check_region(const pw_region &r, size_t expect, const char *what)
{
    if (!r.bytes)
        return fail(PW_ERR_ARGUMENT, "%s region is null", what);
    if (r.tensor_offset + r.tensor_bytes > r.region_bytes && r.region_bytes != 0)
        return fail(PW_ERR_LAYOUT, "%s tensor overruns its region", what);
    if (r.tensor_bytes != expect)
        return fail(PW_ERR_LAYOUT, "%s is %zu bytes, expected %zu (layout mismatch)", what,
                    r.tensor_bytes, expect);
    return PW_OK;
}

int check_weight_codes(const uint8_t *w, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        if (w[i] == 0x7f || w[i] == 0xff)
            return fail(PW_ERR_NONFINITE, "non-finite FP8 weight at byte offset %zu", i);
    return PW_OK;
}

int check_scales(const float *s, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        if (!finite(s[i]))
            return fail(PW_ERR_NONFINITE, "FP8 scale %zu is non-finite", i);
    return PW_OK;
}

bool all_bf16_exact(const float *x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        if (pw::f32_bits(x[i]) & 0xffffu)
            return false;
    return true;
}

// Upload a host f32 activation block, as bf16 when every value is a bf16 value (exact), else
// as f32 (the kernels then split it into bf16 hi + lo).
int stage_input(pw_runtime *rt, const float *x, size_t n, bool &is_f32)
{
    is_f32 = !all_bf16_exact(x, n);
    if (is_f32) {
        PW_HIP(rt->in.ensure(n * 4));
        PW_HIP(hipMemcpyAsync(rt->in.p, x, n * 4, hipMemcpyHostToDevice, rt->stream));
    } else {
        std::vector<uint16_t> h(n);
        for (size_t i = 0; i < n; ++i)
            h[i] = (uint16_t)(pw::f32_bits(x[i]) >> 16);
        PW_HIP(rt->in.ensure(n * 2));
        PW_HIP(hipMemcpyAsync(rt->in.p, h.data(), n * 2, hipMemcpyHostToDevice, rt->stream));
        PW_HIP(hipStreamSynchronize(rt->stream));  // h is released on return
    }
    return PW_OK;
}

int reset_flags(pw_runtime *rt)
{
    PW_HIP(hipMemsetAsync(rt->d_flags, 0, sizeof(uint32_t), rt->stream));
    return PW_OK;
}

// A synchronous host call owns the error word for its duration (like the reference's per-call
// error buffer): it is cleared before the call's kernels and read and cleared after them.
int read_flags(pw_runtime *rt, uint32_t &flags)
{
    PW_HIP(hipMemcpyAsync(&flags, rt->d_flags, sizeof(uint32_t), hipMemcpyDeviceToHost, rt->stream));
    PW_HIP(hipMemsetAsync(rt->d_flags, 0, sizeof(uint32_t), rt->stream));
    PW_HIP(hipStreamSynchronize(rt->stream));
    return PW_OK;
}

#define PW_TRY(expr)                 \
    do {                             \
        int s_ = (expr);             \
        if (s_ != PW_OK)             \
            return s_;               \
    } while (0)

// The device schedule's tables for `rows` token rows over E experts.
int ensure_sched(pw_runtime *rt, uint32_t rows, uint32_t E)
{
    const size_t P = (size_t)rows * 8;
    PW_HIP(rt->moe_plan.ensure(sizeof(pw::MoePlan)));
    PW_HIP(rt->moe_active_expert.ensure((E + 1) * 4));
    PW_HIP(rt->moe_active_offset.ensure((E + 1) * 4));
    PW_HIP(rt->moe_pos.ensure(P * 4));
    PW_HIP(rt->moe_w.ensure(P * 4));
    PW_HIP(rt->moe_slots.ensure(P * 4));
    PW_HIP(rt->moe_active.ensure((size_t)(E + 1) * sizeof(pw::ActiveExpert)));
    PW_HIP(rt->moe_pieces.ensure((P + 1) * sizeof(pw::ActiveExpert)));
    if (const size_t sched = pw::moe_sched_scratch_bytes(rows, E))
        PW_HIP(rt->moe_sched.ensure(sched));
    MoeBuffers &mb = rt->mb;
    mb.plan = (pw::MoePlan *)rt->moe_plan.p;
    mb.active_expert = (uint32_t *)rt->moe_active_expert.p;
    mb.active_offset = (uint32_t *)rt->moe_active_offset.p;
    mb.placement_pos = (uint32_t *)rt->moe_pos.p;
    mb.placement_w = (float *)rt->moe_w.p;
    mb.row_slots = (uint32_t *)rt->moe_slots.p;
    mb.active = (pw::ActiveExpert *)rt->moe_active.p;
    mb.pieces = (pw::ActiveExpert *)rt->moe_pieces.p;
    mb.sched = rt->moe_sched.p;
    return PW_OK;
}

// Routed-MoE scratch for `rows` token rows. mode_a_split: also the mode A buffers (activation
// and hidden bf16 planes, split-K partial sums), which the decode paths (rows <= 128) use.
int ensure_moe(pw_runtime *rt, uint32_t rows, uint32_t E, uint32_t H, uint32_t I, bool mode_a_split = true)
{
    const size_t P = (size_t)rows * 8;
    const int st = ensure_sched(rt, rows, E);
    if (st != PW_OK)
        return st;
    PW_HIP(rt->moe_hidden.ensure(P * I * 4));
    if (mode_a_split) {
        PW_HIP(rt->moe_hidden_planes.ensure(3 * P * I * 2));
        PW_HIP(rt->moe_x_planes.ensure(3 * (size_t)rows * H * 2));
    }
    PW_HIP(rt->moe_y.ensure(P * H * 4));
    PW_HIP(rt->moe_xq.ensure((size_t)rows * H));
    PW_HIP(rt->moe_xs.ensure((size_t)rows * (H / 128) * 4));
    PW_HIP(rt->moe_hq.ensure(P * I));
    PW_HIP(rt->moe_hs.ensure(P * (I / 128) * 4));
    // split-K partials of the mode A projections, sized for the widest split the launch can pick
    const uint32_t cnt = std::min<uint32_t>(rows, 32);
    const size_t ks_gu = std::max(pw::plan_split(H, 2, 1, cnt).ks, pw::plan_split(H, 2, 3, cnt).ks);
    const size_t ks_d = pw::plan_split(I, 1, 3, cnt).ks;
    if (mode_a_split)
        PW_HIP(rt->moe_partial.ensure(std::max(ks_gu * 2 * P * I, ks_d * P * H) * 4));
    MoeBuffers &mb = rt->mb;
    mb.partial = (float *)rt->moe_partial.p;
    mb.hidden = (float *)rt->moe_hidden.p;
    mb.hidden_planes = (uint16_t *)rt->moe_hidden_planes.p;
    mb.x_planes = (uint16_t *)rt->moe_x_planes.p;
    mb.y = (float *)rt->moe_y.p;
    mb.xq = (uint8_t *)rt->moe_xq.p;
    mb.xs = (float *)rt->moe_xs.p;
    mb.hq = (uint8_t *)rt->moe_hq.p;
    mb.hs = (float *)rt->moe_hs.p;
    mb.max_rows = rows;
    mb.experts = E;
    return PW_OK;
}

// The 65,536-entry silu table of the bf16-staged SwiGLU, built once per runtime on the runtime's
// stream and complete (the host waits for it) before any call reads it; a failed build leaves it
// marked unbuilt, so the next call builds it again.
int ensure_silu_table(pw_runtime *rt)
{
    if (rt->silu_ready)
        return PW_OK;
    PW_HIP(rt->pf_silu.ensure(65536 * sizeof(uint16_t)));
    pw::launch_silu_table((uint16_t *)rt->pf_silu.p, rt->stream);
    PW_HIP(hipGetLastError());
    PW_HIP(hipStreamSynchronize(rt->stream));
    rt->silu_ready = true;
    return PW_OK;
}

// The libc++ nth_element top-k and the noaux route row are shared with the device router
// (pw_topk.h).

}  // namespace

// ---- scratch of the entry point that allocates nothing (pw_moe_layer_device_noalloc) ---------
// A decode batch (rows <= 8) over a bank of at most 256 experts, hidden <= 4096 and intermediate
// <= 2048 needs about 10.8 MB of schedule tables, activation planes, split-K partials and expert
// outputs; the array holds 12 MiB. Each GPU the library runs on holds its own copy until the process
// ends. Every call on a GPU shares that GPU's copy (its contents stay from the last call; every
// table the kernels read is written by the same call's schedule first, so nothing needs clearing),
// and calls that overlap on one GPU race.
namespace {
constexpr uint32_t NOALLOC_MAX_ROWS = 8, NOALLOC_MAX_EXPERTS = 256, NOALLOC_MAX_HIDDEN = 4096,
                   NOALLOC_MAX_INTER = 2048;
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)12 << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

void *g_scratch_ptr[NOALLOC_MAX_DEVICES];  // device address of `scratch` on each device
std::mutex g_scratch_mutex;

// With `device` current: look up this device's address of the scratch array once.
int noalloc_scratch_init(int device)
{
    if (device < 0 || device >= NOALLOC_MAX_DEVICES)
        return PW_OK;  // the no-alloc entry point refuses such a device
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device])
        return PW_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(PW_ERR_DEVICE, "scratch array address on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
    return PW_OK;
}

// The routed-MoE buffers of `rows` token rows over E experts carved out of one block at `base`, with
// the sizes ensure_moe allocates (mode A split buffers included); returns the bytes used. base may
// be null to size the block.
size_t carve_moe(char *base, uint32_t rows, uint32_t E, uint32_t H, uint32_t I, MoeBuffers &mb)
{
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += (bytes + 255) & ~(size_t)255;
        return p;
    };
    const size_t P = (size_t)rows * 8;
    const uint32_t cnt = std::min<uint32_t>(rows, 32);
    const size_t ks_gu = std::max(pw::plan_split(H, 2, 1, cnt).ks, pw::plan_split(H, 2, 3, cnt).ks);
    const size_t ks_d = pw::plan_split(I, 1, 3, cnt).ks;
    mb = MoeBuffers{};
    mb.plan = (pw::MoePlan *)take(sizeof(pw::MoePlan));
    mb.active_expert = (uint32_t *)take((E + 1) * 4);
    mb.active_offset = (uint32_t *)take((E + 1) * 4);
    mb.placement_pos = (uint32_t *)take(P * 4);
    mb.placement_w = (float *)take(P * 4);
    mb.row_slots = (uint32_t *)take(P * 4);
    mb.active = (pw::ActiveExpert *)take((size_t)(E + 1) * sizeof(pw::ActiveExpert));
    mb.pieces = (pw::ActiveExpert *)take((P + 1) * sizeof(pw::ActiveExpert));
    mb.hidden = (float *)take(P * I * 4);
    mb.hidden_planes = (uint16_t *)take(3 * P * I * 2);
    mb.x_planes = (uint16_t *)take(3 * (size_t)rows * H * 2);
    mb.y = (float *)take(P * H * 4);
    mb.xq = (uint8_t *)take((size_t)rows * H);
    mb.xs = (float *)take((size_t)rows * (H / 128) * 4);
    mb.hq = (uint8_t *)take(P * I);
    mb.hs = (float *)take(P * (I / 128) * 4);
    mb.partial = (float *)take(std::max(ks_gu * 2 * P * I, ks_d * P * H) * 4);
    mb.sched = nullptr;  // decode batches are scheduled by one wave, without these tables
    mb.max_rows = rows;
    mb.experts = E;
    return off;
}

}  // namespace

// ===================================================================================== C ABI
extern "C" {

const char *pw_last_error(void) { return g_error.c_str(); }

int pw_abi_version(void) { return PW_ABI_VERSION; }

int pw_runtime_create(int device, uint32_t flags, pw_runtime **out)
{
    if (!out)
        return fail(PW_ERR_ARGUMENT, "null output handle");
    *out = nullptr;
    int count = 0;
    PW_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return fail(PW_ERR_ARGUMENT, "device %d out of range (%d devices)", device, count);
    hipDeviceProp_t prop;
    PW_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PW_ERR_DEVICE, "device %d is %s; this library is built for gfx950", device,
                    prop.gcnArchName);
    pw_runtime *rt = new pw_runtime;
    rt->device = device;
    rt->flags = flags;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess)
        // a blocking stream: work the caller enqueued on the null stream (e.g. a framework's default
        // stream) is ordered before the runtime's launches, and vice versa
        e = hipStreamCreateWithFlags(&rt->stream, hipStreamDefault);
    if (e == hipSuccess)
        e = hipEventCreateWithFlags(&rt->order_event, hipEventDisableTiming);
    if (e == hipSuccess)
        e = hipMalloc((void **)&rt->d_flags, sizeof(uint32_t));
    if (e == hipSuccess)
        e = hipMemset(rt->d_flags, 0, sizeof(uint32_t));
    if (e != hipSuccess) {
        pw_runtime_destroy(rt);
        return fail(PW_ERR_DEVICE, "runtime setup failed: %s", hipGetErrorString(e));
    }
    const int st = noalloc_scratch_init(device);
    if (st != PW_OK) {
        pw_runtime_destroy(rt);
        return st;
    }
    *out = rt;
    return PW_OK;
}

void pw_runtime_destroy(pw_runtime *rt)
{
    if (!rt)
        return;
    (void)hipSetDevice(rt->device);
    if (rt->stream)
        (void)hipStreamSynchronize(rt->stream);
    if (rt->d_flags)
        (void)hipFree(rt->d_flags);
    free_timer(rt->timer);
    if (rt->order_event)
        (void)hipEventDestroy(rt->order_event);
    if (rt->stream)
        (void)hipStreamDestroy(rt->stream);
    delete rt;
}

int pw_runtime_enable_timing(pw_runtime *rt, uint32_t max_launches)
{
    if (!rt)
        return fail(PW_ERR_ARGUMENT, "null runtime");
    PW_HIP(set_device(rt));
    PW_HIP(hipDeviceSynchronize());
    free_timer(rt->timer);
    if (max_launches == 0)
        return PW_OK;
    pw::KernelTimer &t = rt->timer;
    t.events = new hipEvent_t[2 * max_launches]();
    t.ids = new uint32_t[max_launches]();
    for (uint32_t i = 0; i < 2 * max_launches; ++i) {
        hipError_t e = hipEventCreate(&t.events[i]);
        if (e != hipSuccess) {
            t.capacity = i / 2;
            free_timer(t);
            return fail(PW_ERR_DEVICE, "hipEventCreate failed: %s", hipGetErrorString(e));
        }
    }
    t.capacity = max_launches;
    t.used = 0;
    t.enabled = true;
    return PW_OK;
}

int pw_runtime_timing_summary(pw_runtime *rt, const char *kernel, uint32_t *launches, double *total_ms)
{
    if (!rt || !kernel || !launches || !total_ms)
        return fail(PW_ERR_ARGUMENT, "null argument");
    uint32_t id = pw::K_COUNT;
    for (uint32_t k = 0; k < pw::K_COUNT; ++k)
        if (std::strcmp(kernel, kKernelNames[k]) == 0)
            id = k;
    if (id == pw::K_COUNT)
        return fail(PW_ERR_ARGUMENT, "unknown kernel name '%s'", kernel);
    PW_HIP(set_device(rt));
    PW_HIP(hipDeviceSynchronize());
    *launches = 0;
    *total_ms = 0.0;
    const pw::KernelTimer &t = rt->timer;
    for (uint32_t i = 0; i < t.used; ++i) {
        if (t.ids[i] != id)
            continue;
        float ms = 0.f;
        PW_HIP(hipEventElapsedTime(&ms, t.events[2 * i], t.events[2 * i + 1]));
        *launches += 1;
        *total_ms += ms;
    }
    return PW_OK;
}

int pw_runtime_timing_reset(pw_runtime *rt)
{
    if (!rt)
        return fail(PW_ERR_ARGUMENT, "null runtime");
    PW_HIP(set_device(rt));
    PW_HIP(hipDeviceSynchronize());
    rt->timer.used = 0;
    return PW_OK;
}

void *pw_runtime_stream(pw_runtime *rt) { return rt ? (void *)rt->stream : nullptr; }

int pw_runtime_take_flags(pw_runtime *rt, uint32_t *flags)
{
    if (!rt || !flags)
        return fail(PW_ERR_ARGUMENT, "null argument");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    // device-resident calls may have run on a caller's stream: wait for all of them
    PW_HIP(hipDeviceSynchronize());
    rt->last_stream = nullptr;  // nothing of an earlier call is pending
    PW_TRY(read_flags(rt, *flags));
    PW_TRY(reset_flags(rt));
    PW_HIP(hipStreamSynchronize(rt->stream));
    return PW_OK;
}

// ------------------------------------------------------------------------------ projections
int pw_projection_bind(pw_runtime *rt, const pw_projection_desc *d, int scan_codes,
                       pw_projection **out)
{
    if (!rt || !d || !out)
        return fail(PW_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    const uint32_t rows = d->rows, cols = d->columns;
    if (rows == 0 || cols == 0 || cols % 128 != 0)
        return fail(PW_ERR_LAYOUT, "FP8 projection dimensions must be nonzero, columns a multiple of 128");
    size_t scale_rows;
    if (d->layout == PW_LAYOUT_PLAIN) {
        scale_rows = (rows + 127) / 128;
    } else if (d->layout == PW_LAYOUT_FULL_QKV_TP4) {
        if (rows != 13568 || cols != 4096)
            return fail(PW_ERR_LAYOUT, "wide full-QKV layout mismatch");
        scale_rows = 108;
    } else if (d->layout == PW_LAYOUT_SWA_QKV_TP4) {
        if (rows != 14848 || cols != 4096)
            return fail(PW_ERR_LAYOUT, "wide SWA-QKV layout mismatch");
        scale_rows = 116;
    } else {
        return fail(PW_ERR_ARGUMENT, "unknown layout %u", d->layout);
    }
    const size_t wbytes = (size_t)rows * cols, sbytes = scale_rows * (cols / 128) * 4;
    PW_TRY(check_region(d->weight, wbytes, "weight"));
    PW_TRY(check_region(d->scale, sbytes, "scale"));
    const uint8_t *hw = region_tensor(d->weight);
    const float *hs = (const float *)region_tensor(d->scale);
    PW_TRY(check_scales(hs, sbytes / 4));
    if (scan_codes)
        PW_TRY(check_weight_codes(hw, wbytes));
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw_projection *p = new pw_projection;
    p->rt = rt;
    p->rows = rows;
    p->columns = cols;
    p->owns = true;
    p->weight_bytes = wbytes;
    p->scale_bytes = sbytes;
    hipError_t e = hipMalloc(&p->w, wbytes);
    if (e == hipSuccess)
        e = hipMalloc(&p->s, sbytes);
    if (e == hipSuccess)
        e = hipMemcpy(p->w, hw, wbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(p->s, hs, sbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        pw_projection_release(p);
        return fail(PW_ERR_DEVICE, "weight upload failed: %s", hipGetErrorString(e));
    }
    std::vector<ProjTile> tiles;
    if (d->layout == PW_LAYOUT_PLAIN) {
        add_segment_tiles(tiles, p->w, p->s, cols, 0, rows, 0, 0);
    } else if (d->layout == PW_LAYOUT_FULL_QKV_TP4) {
        // shards of [Q 3072 | K 192 | V 128], 27 scale rows each (24 Q, 2 K incl. a 64-row
        // partial block, 1 V); outputs deinterleaved as all Q, all K, all V
        for (uint32_t s = 0; s < 4; ++s) {
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3392ull, 3072, s * 27ull, s * 3072);
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3392ull + 3072, 192, s * 27ull + 24, 12288 + s * 192);
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3392ull + 3264, 128, s * 27ull + 26, 13056 + s * 128);
        }
    } else {
        // shards of [Q 3072 | K 384 | V 256], uniform scale rows source_row / 128
        for (uint32_t s = 0; s < 4; ++s) {
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3712ull, 3072, s * 29ull, s * 3072);
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3712ull + 3072, 384, s * 29ull + 24, 12288 + s * 384);
            add_segment_tiles(tiles, p->w, p->s, cols, s * 3712ull + 3456, 256, s * 29ull + 27, 13824 + s * 256);
        }
    }
    int st = upload_tiles(p, tiles);
    if (st != PW_OK) {
        pw_projection_release(p);
        return st;
    }
    *out = p;
    return PW_OK;
}

int pw_projection_bind_segments(pw_runtime *rt, const pw_segment_desc *segs, uint32_t count,
                                uint32_t columns, int scan_codes, pw_projection **out)
{
    if (!rt || !segs || !out || count == 0)
        return fail(PW_ERR_ARGUMENT, "null argument or empty segment list");
    *out = nullptr;
    if (columns == 0 || columns % 128 != 0)
        return fail(PW_ERR_LAYOUT, "columns must be a nonzero multiple of 128");
    size_t total_rows = 0, wbytes = 0, sbytes = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (segs[i].rows == 0)
            return fail(PW_ERR_LAYOUT, "segment %u has no rows", i);
        const size_t w = (size_t)segs[i].rows * columns;
        const size_t s = (size_t)((segs[i].rows + 127) / 128) * (columns / 128) * 4;
        PW_TRY(check_region(segs[i].weight, w, "segment weight"));
        PW_TRY(check_region(segs[i].scale, s, "segment scale"));
        PW_TRY(check_scales((const float *)region_tensor(segs[i].scale), s / 4));
        if (scan_codes)
            PW_TRY(check_weight_codes(region_tensor(segs[i].weight), w));
        total_rows += segs[i].rows;
        wbytes += w;
        sbytes += s;
    }
    if (total_rows > 0xffffffffull)
        return fail(PW_ERR_LAYOUT, "too many rows");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw_projection *p = new pw_projection;
    p->rt = rt;
    p->rows = (uint32_t)total_rows;
    p->columns = columns;
    p->owns = true;
    p->weight_bytes = wbytes;
    p->scale_bytes = sbytes;
    hipError_t e = hipMalloc(&p->w, wbytes);
    if (e == hipSuccess)
        e = hipMalloc(&p->s, sbytes);
    std::vector<ProjTile> tiles;
    size_t woff = 0, soff = 0;
    uint32_t out_row = 0;
    for (uint32_t i = 0; i < count && e == hipSuccess; ++i) {
        const size_t w = (size_t)segs[i].rows * columns;
        const size_t srows = (segs[i].rows + 127) / 128;
        const size_t s = srows * (columns / 128) * 4;
        e = hipMemcpy(p->w + woff, region_tensor(segs[i].weight), w, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy((uint8_t *)p->s + soff, region_tensor(segs[i].scale), s, hipMemcpyHostToDevice);
        add_segment_tiles(tiles, p->w + woff, (const float *)((const uint8_t *)p->s + soff), columns,
                          0, segs[i].rows, 0, out_row);
        woff += w;
        soff += s;
        out_row += segs[i].rows;
    }
    if (e != hipSuccess) {
        pw_projection_release(p);
        return fail(PW_ERR_DEVICE, "segment upload failed: %s", hipGetErrorString(e));
    }
    int st = upload_tiles(p, tiles);
    if (st != PW_OK) {
        pw_projection_release(p);
        return st;
    }
    *out = p;
    return PW_OK;
}

int pw_projection_bind_device(pw_runtime *rt, const void *weight, const float *scale, uint32_t rows,
                              uint32_t columns, pw_projection **out)
{
    if (!rt || !weight || !scale || !out)
        return fail(PW_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    if (rows == 0 || columns == 0 || columns % 128 != 0)
        return fail(PW_ERR_LAYOUT, "FP8 projection dimensions must be nonzero, columns a multiple of 128");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw_projection *p = new pw_projection;
    p->rt = rt;
    p->w = (uint8_t *)weight;
    p->s = (float *)scale;
    p->owns = false;
    p->rows = rows;
    p->columns = columns;
    p->weight_bytes = (uint64_t)rows * columns;
    p->scale_bytes = (uint64_t)((rows + 127) / 128) * (columns / 128) * 4;
    std::vector<ProjTile> tiles;
    add_segment_tiles(tiles, p->w, p->s, columns, 0, rows, 0, 0);
    int st = upload_tiles(p, tiles);
    if (st != PW_OK) {
        pw_projection_release(p);
        return st;
    }
    *out = p;
    return PW_OK;
}

void pw_projection_release(pw_projection *p)
{
    if (!p)
        return;
    if (p->rt)
        (void)hipSetDevice(p->rt->device);
    if (p->owns) {
        if (p->w)
            (void)hipFree(p->w);
        if (p->s)
            (void)hipFree(p->s);
    }
    if (p->tiles)
        (void)hipFree(p->tiles);
    delete p;
}

int pw_projection_shape(const pw_projection *p, uint32_t *rows, uint32_t *columns)
{
    if (!p)
        return fail(PW_ERR_ARGUMENT, "null projection");
    if (rows)
        *rows = p->rows;
    if (columns)
        *columns = p->columns;
    return PW_OK;
}

static int enqueue_linear(pw_runtime *rt, uint32_t mode, const void *x, bool x_f32, uint32_t rows,
                          const pw_projection *p, float *y32, uint16_t *y16, uint32_t round_f32,
                          hipStream_t stream)
{
    if (mode == PW_MODE_A) {
        if (x_f32) {
            const size_t n = (size_t)rows * p->columns;
            PW_HIP(rt->lin_planes.ensure(3 * n * 2));
            pw::launch_linear_a_f32(p->tiles, p->n_tiles, (const float *)x, (uint16_t *)rt->lin_planes.p, rows,
                                    p->columns, y32, y16, p->rows, round_f32, stream);
        } else {
            pw::launch_linear_a(p->tiles, p->n_tiles, (const uint16_t *)x, 1, rows, p->columns, y32, y16,
                                p->rows, round_f32, stream);
        }
    } else if (mode == PW_MODE_B) {
        PW_HIP(rt->codes.ensure((size_t)rows * p->columns));
        PW_HIP(rt->scales.ensure((size_t)rows * (p->columns / 128) * 4));
        pw::launch_quant_group128(x, x_f32, rows, p->columns, (uint8_t *)rt->codes.p,
                                  (float *)rt->scales.p, rt->d_flags, stream);
        pw::launch_linear_b(p->tiles, p->n_tiles, (const uint8_t *)rt->codes.p,
                            (const float *)rt->scales.p, rows, p->columns, y32, y16, p->rows,
                            round_f32, stream);
    } else {
        return fail(PW_ERR_ARGUMENT, "unknown mode %u", mode);
    }
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_fp8_linear(pw_runtime *rt, uint32_t mode, const float *input, uint32_t rows,
                  const pw_projection *p, float *output, pw_linear_stats *stats)
{
    const double t0 = now_ms();
    if (!rt || !input || !p || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (p->bf16)
        return fail(PW_ERR_ARGUMENT, "a BF16 projection runs through pw_bf16_linear");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "wide row count must be between one and 32");
    const size_t n_in = (size_t)rows * p->columns, n_out = (size_t)rows * p->rows;
    for (size_t i = 0; i < n_in; ++i)
        if (!finite(input[i]))
            return fail(PW_ERR_NONFINITE, "wide FP8 linear input is non-finite");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    StreamOrder order(rt, rt->stream);
    PW_HIP(order.err);
    PW_TRY(reset_flags(rt));
    bool x_f32;
    PW_TRY(stage_input(rt, input, n_in, x_f32));
    PW_HIP(rt->out.ensure(n_out * 4));
    PW_TRY(enqueue_linear(rt, mode, rt->in.p, x_f32, rows, p, (float *)rt->out.p, nullptr, 1, rt->stream));
    PW_HIP(hipMemcpyAsync(output, rt->out.p, n_out * 4, hipMemcpyDeviceToHost, rt->stream));
    uint32_t flags = 0;
    PW_TRY(read_flags(rt, flags));
    if (stats) {
        stats->wall_ms = now_ms() - t0;
        stats->mapped_source_bytes = 0;
        stats->resident_source_bytes = p->weight_bytes + p->scale_bytes;
        stats->gpu_flags = flags;
    }
    if (flags)
        return fail(PW_ERR_GPU_FLAGS, "wide FP8 linear kernels set error flags %u", flags);
    for (size_t i = 0; i < n_out; ++i)
        if (!finite(output[i]))
            return fail(PW_ERR_OUTPUT, "wide FP8 linear produced non-finite output");
    return PW_OK;
}

int pw_fp8_linear_device(pw_runtime *rt, uint32_t mode, const void *input, uint32_t input_dtype,
                         uint32_t rows, const pw_projection *p, void *output, uint32_t output_dtype,
                         uint32_t round_output, void *stream)
{
    if (!rt || !input || !p || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (p->bf16)
        return fail(PW_ERR_ARGUMENT, "a BF16 projection runs through pw_bf16_linear_device");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "wide row count must be between one and 32");
    if (input_dtype > PW_DTYPE_BF16 || output_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown dtype");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    float *y32 = output_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr;
    uint16_t *y16 = output_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr;
    const uint32_t round_f32 = output_dtype == PW_DTYPE_F32 && round_output ? 1u : 0u;
    return enqueue_linear(rt, mode, input, input_dtype == PW_DTYPE_F32, rows, p, y32, y16, round_f32, s);
}

// ---- BF16 wide linear ------------------------------------------------------------------------
static int bf16_bind_common(pw_runtime *rt, uint32_t rows, uint32_t columns, pw_projection **out)
{
    if (!rt || !out)
        return fail(PW_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    if (rows == 0 || columns == 0 || columns % 128 != 0)
        return fail(PW_ERR_LAYOUT, "BF16 linear dimensions must be nonzero, columns a multiple of 128");
    return PW_OK;
}

int pw_bf16_bind(pw_runtime *rt, const pw_region *weight, uint32_t rows, uint32_t columns, pw_projection **out)
{
    PW_TRY(bf16_bind_common(rt, rows, columns, out));
    if (!weight || !weight->bytes)
        return fail(PW_ERR_ARGUMENT, "null weight region");
    const size_t bytes = (size_t)rows * columns * 2;
    if (weight->tensor_bytes != bytes || weight->tensor_offset + bytes > weight->region_bytes)
        return fail(PW_ERR_LAYOUT, "wide BF16 linear layout mismatch");
    PW_HIP(set_device(rt));
    pw_projection *p = new pw_projection;
    p->rt = rt;
    p->bf16 = true;
    p->owns = true;
    p->rows = rows;
    p->columns = columns;
    p->weight_bytes = bytes;
    hipError_t e = hipMalloc(&p->w, bytes);
    if (e == hipSuccess)
        e = hipMemcpy(p->w, (const uint8_t *)weight->bytes + weight->tensor_offset, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        pw_projection_release(p);
        return fail(PW_ERR_DEVICE, "BF16 weight upload: %s", hipGetErrorString(e));
    }
    *out = p;
    return PW_OK;
}

int pw_bf16_bind_device(pw_runtime *rt, const void *weight, uint32_t rows, uint32_t columns, pw_projection **out)
{
    PW_TRY(bf16_bind_common(rt, rows, columns, out));
    if (!weight)
        return fail(PW_ERR_ARGUMENT, "null weight");
    if ((uintptr_t)weight & 15)
        return fail(PW_ERR_ARGUMENT, "BF16 weights must be 16-byte aligned");
    pw_projection *p = new pw_projection;
    p->rt = rt;
    p->bf16 = true;
    p->w = (uint8_t *)weight;
    p->rows = rows;
    p->columns = columns;
    p->weight_bytes = (uint64_t)rows * columns * 2;
    *out = p;
    return PW_OK;
}

static int enqueue_bf16_linear(pw_runtime *rt, const void *x, bool x_f32, uint32_t rows, const pw_projection *p,
                               float *y32, uint16_t *y16, uint32_t round_f32, hipStream_t stream)
{
    const int planes = x_f32 ? 3 : 1;
    const uint16_t *xp = (const uint16_t *)x;
    // f32 rows: up to 16 are split into their planes inside the projection's staging; more go
    // through a split launch first
    const bool split_inside = x_f32 && rows <= 16;
    if (x_f32 && !split_inside) {
        const size_t n = (size_t)rows * p->columns;
        PW_HIP(rt->lin_planes.ensure(3 * n * 2));
        pw::launch_split_planes((const float *)x, (uint32_t)n, (uint16_t *)rt->lin_planes.p, stream);
        xp = (const uint16_t *)rt->lin_planes.p;
    }
    const int bpw = pw::bf16_blocks_per_wave(p->columns, planes, rows, 65536);
    pw::Bf16Args a{};
    a.w = (const uint16_t *)p->w;
    a.x = xp;
    a.xf = split_inside ? (const float *)x : nullptr;
    a.x_plane = (size_t)rows * p->columns;
    a.K = p->columns;
    a.R = p->rows;
    a.W = rows;
    a.KS = p->columns / (128u * bpw);
    PW_HIP(rt->bf16_partial.ensure((size_t)a.KS * rows * p->rows * 4));
    a.partial = (float *)rt->bf16_partial.p;
    pw::launch_bf16_linear(a, planes, bpw, y32, y16, round_f32, rt->d_flags, stream);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_bf16_linear(pw_runtime *rt, const float *input, uint32_t rows, const pw_projection *p, float *output,
                   pw_linear_stats *stats)
{
    const double t0 = now_ms();
    if (!rt || !input || !p || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (!p->bf16)
        return fail(PW_ERR_ARGUMENT, "not a BF16 projection");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "wide row count must be between one and 32");
    const size_t n_in = (size_t)rows * p->columns, n_out = (size_t)rows * p->rows;
    for (size_t i = 0; i < n_in; ++i)
        if (!finite(input[i]))
            return fail(PW_ERR_NONFINITE, "wide BF16 linear layout mismatch (non-finite input)");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    StreamOrder order(rt, rt->stream);
    PW_HIP(order.err);
    PW_TRY(reset_flags(rt));
    bool x_f32;
    PW_TRY(stage_input(rt, input, n_in, x_f32));
    PW_HIP(rt->out.ensure(n_out * 4));
    PW_TRY(enqueue_bf16_linear(rt, rt->in.p, x_f32, rows, p, (float *)rt->out.p, nullptr, 1, rt->stream));
    PW_HIP(hipMemcpyAsync(output, rt->out.p, n_out * 4, hipMemcpyDeviceToHost, rt->stream));
    uint32_t flags = 0;
    PW_TRY(read_flags(rt, flags));
    if (stats) {
        stats->wall_ms = now_ms() - t0;
        stats->mapped_source_bytes = 0;
        stats->resident_source_bytes = p->weight_bytes;
        stats->gpu_flags = flags;
    }
    if (flags)
        return fail(PW_ERR_GPU_FLAGS, "wide BF16 linear Metal transaction failed (flags %u)", flags);
    return PW_OK;
}

int pw_bf16_linear_device(pw_runtime *rt, const void *input, uint32_t input_dtype, uint32_t rows,
                          const pw_projection *p, void *output, uint32_t output_dtype, uint32_t round_output,
                          void *stream)
{
    if (!rt || !input || !p || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (!p->bf16)
        return fail(PW_ERR_ARGUMENT, "not a BF16 projection");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "wide row count must be between one and 32");
    if (input_dtype > PW_DTYPE_BF16 || output_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown dtype");
    if ((uintptr_t)input & 15)
        return fail(PW_ERR_ARGUMENT, "input must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    float *y32 = output_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr;
    uint16_t *y16 = output_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr;
    const uint32_t round_f32 = output_dtype == PW_DTYPE_F32 && round_output ? 1u : 0u;
    return enqueue_bf16_linear(rt, input, input_dtype == PW_DTYPE_F32, rows, p, y32, y16, round_f32, s);
}

int pw_quantize_fp8_group128_device(pw_runtime *rt, const void *x, uint32_t x_dtype, uint32_t rows,
                                    uint32_t cols, uint8_t *codes, float *scales, void *stream)
{
    if (!rt || !x || !codes || !scales || rows == 0)
        return fail(PW_ERR_ARGUMENT, "null argument or zero rows");
    if (cols == 0 || cols % 128 != 0)
        return fail(PW_ERR_LAYOUT, "dynamic FP8 activation shape mismatch");
    if (x_dtype > PW_DTYPE_BF16)
        return fail(PW_ERR_ARGUMENT, "unknown dtype");
    if (((uintptr_t)x | (uintptr_t)codes) & 15)
        return fail(PW_ERR_ARGUMENT, "activations and codes must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    pw::launch_quant_group128(x, x_dtype == PW_DTYPE_F32, rows, cols, codes, scales, rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_swiglu_staged_device(pw_runtime *rt, const float *gate, const float *up, uint32_t count, float *out,
                            uint32_t form, void *stream)
{
    if (!rt || !gate || !up || !out || count == 0)
        return fail(PW_ERR_ARGUMENT, "null argument or zero count");
    if (form > 1)
        return fail(PW_ERR_ARGUMENT, "unknown staged SwiGLU form %u", form);
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    if (form == 1)
        PW_TRY(ensure_silu_table(rt));
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    pw::launch_swiglu_staged(gate, up, count, form == 1 ? (const uint16_t *)rt->pf_silu.p : nullptr, out,
                             rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

// ------------------------------------------------------------------------------- routed MoE
static int check_expert_projection(const pw_projection *p, uint32_t rows, uint32_t cols)
{
    return p && p->rows == rows && p->columns == cols && rows % 128 == 0 && cols % 128 == 0;
}

int pw_moe_execute(pw_runtime *rt, uint32_t mode, uint32_t fused_gate_up, const float *input,
                   uint32_t rows, const pw_expert_binding *experts, uint32_t n_experts,
                   float *output, pw_moe_stats *stats)
{
    (void)fused_gate_up;  // gate and up always share one pass
    const double t0 = now_ms();
    if (!rt || !input || !experts || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (mode > PW_MODE_B)
        return fail(PW_ERR_ARGUMENT, "unknown mode %u", mode);
    if (rows < 1 || rows > 128)
        return fail(PW_ERR_ARGUMENT, "wide row count must be between one and 128");
    if (n_experts == 0 || !experts[0].gate || !experts[0].down)
        return fail(PW_ERR_SCHEDULE, "wide MoE input or schedule mismatch");
    const uint32_t H = experts[0].gate->columns, I = experts[0].gate->rows;
    const size_t n_in = (size_t)rows * H;
    for (size_t i = 0; i < n_in; ++i)
        if (!finite(input[i]))
            return fail(PW_ERR_NONFINITE, "wide MoE input or schedule mismatch");
    // validation of src/wide_metal_moe.rs:858-938
    size_t total = 0;
    uint32_t max_count = 0;
    std::vector<uint32_t> ids((size_t)rows * 8), fill(rows, 0);
    std::vector<float> ws((size_t)rows * 8);
    std::vector<ExpertPtrs> table(n_experts);
    std::vector<uint32_t> seen;
    uint64_t resident = 0;
    for (uint32_t k = 0; k < n_experts; ++k) {
        const pw_expert_binding &b = experts[k];
        if (b.count == 0 || b.count > 32 || !b.positions || !b.route_weights ||
            !check_expert_projection(b.gate, I, H) || !check_expert_projection(b.up, I, H) ||
            !check_expert_projection(b.down, H, I))
            return fail(PW_ERR_SCHEDULE, "wide MoE expert %u identity mismatch", b.expert);
        for (uint32_t j = 0; j < b.count; ++j) {
            const uint32_t pos = b.positions[j];
            if (pos >= rows || !finite(b.route_weights[j]))
                return fail(PW_ERR_SCHEDULE, "wide MoE expert %u identity mismatch", b.expert);
            if (fill[pos] >= 8)
                return fail(PW_ERR_SCHEDULE, "wide MoE input or schedule mismatch");
            ids[(size_t)pos * 8 + fill[pos]] = k;
            ws[(size_t)pos * 8 + fill[pos]] = b.route_weights[j];
            fill[pos]++;
        }
        total += b.count;
        max_count = std::max(max_count, b.count);
        table[k] = ExpertPtrs{b.gate->w, b.gate->s, b.up->w, b.up->s, b.down->w, b.down->s};
        if (std::find(seen.begin(), seen.end(), b.expert) == seen.end()) {
            seen.push_back(b.expert);
            resident += b.gate->weight_bytes + b.gate->scale_bytes + b.up->weight_bytes +
                        b.up->scale_bytes + b.down->weight_bytes + b.down->scale_bytes;
        }
    }
    if (total != (size_t)rows * 8)
        return fail(PW_ERR_SCHEDULE, "wide MoE input or schedule mismatch");
    // a position routed twice to the same binding would be summed twice by the reference; the
    // device schedule rejects it, so refuse it here with the same error class
    for (uint32_t p = 0; p < rows; ++p)
        for (int a = 0; a < 8; ++a)
            for (int b2 = a + 1; b2 < 8; ++b2)
                if (ids[(size_t)p * 8 + a] == ids[(size_t)p * 8 + b2])
                    return fail(PW_ERR_SCHEDULE, "position %u routed twice to one expert binding", p);
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    StreamOrder order(rt, rt->stream);
    PW_HIP(order.err);
    PW_TRY(reset_flags(rt));
    bool x_f32;
    PW_TRY(stage_input(rt, input, n_in, x_f32));
    PW_HIP(rt->route_ids.ensure(ids.size() * 4));
    PW_HIP(rt->route_w.ensure(ws.size() * 4));
    PW_HIP(rt->bank_table.ensure(table.size() * sizeof(ExpertPtrs)));
    PW_HIP(hipMemcpyAsync(rt->route_ids.p, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, rt->stream));
    PW_HIP(hipMemcpyAsync(rt->route_w.p, ws.data(), ws.size() * 4, hipMemcpyHostToDevice, rt->stream));
    PW_HIP(hipMemcpyAsync(rt->bank_table.p, table.data(), table.size() * sizeof(ExpertPtrs),
                          hipMemcpyHostToDevice, rt->stream));
    PW_TRY(ensure_moe(rt, rows, n_experts, H, I));
    PW_HIP(rt->out.ensure(n_in * 4));
    const pw::QuantJob qj{rt->in.p, x_f32 ? 1u : 0u, rows, H, rt->mb.xq, rt->mb.xs};
    bool quantised = false;
    pw::launch_moe_schedule((const ExpertPtrs *)rt->bank_table.p, (const uint32_t *)rt->route_ids.p,
                            (const float *)rt->route_w.p, rows, n_experts,
                            std::min<uint32_t>(n_experts, rows * 8), rt->mb, rt->d_flags, rt->stream, nullptr,
                            mode == PW_MODE_B ? &qj : nullptr, mode == PW_MODE_B ? &quantised : nullptr);
    pw::launch_moe_layer(mode, (const ExpertPtrs *)rt->bank_table.p, rt->mb, rt->in.p, x_f32, rows,
                         std::min<uint32_t>(n_experts, rows * 8), max_count, H, I,
                         (float *)rt->out.p, nullptr, false, rt->d_flags, rt->stream, nullptr, quantised);
    PW_HIP(hipGetLastError());
    PW_HIP(hipMemcpyAsync(output, rt->out.p, n_in * 4, hipMemcpyDeviceToHost, rt->stream));
    uint32_t flags = 0;
    PW_TRY(read_flags(rt, flags));  // also completes the stream (ids/ws/table stay valid until here)
    if (stats) {
        stats->wall_ms = now_ms() - t0;
        stats->unique_experts = (uint32_t)seen.size();
        stats->expert_rows = (uint32_t)total;
        stats->mapped_source_bytes = 0;
        stats->resident_source_bytes = resident;
        stats->gpu_flags = flags;
    }
    if (flags)
        return fail(PW_ERR_GPU_FLAGS, "wide MoE semantic kernels set error flags %u", flags);
    for (size_t i = 0; i < n_in; ++i)
        if (!finite(output[i]))
            return fail(PW_ERR_OUTPUT, "wide MoE produced non-finite output");
    return PW_OK;
}

int pw_expert_bank_create(pw_runtime *rt, uint32_t n_experts, const pw_projection *const *gate,
                          const pw_projection *const *up, const pw_projection *const *down,
                          pw_expert_bank **out)
{
    if (!rt || !gate || !up || !down || !out || n_experts == 0)
        return fail(PW_ERR_ARGUMENT, "null argument or empty bank");
    if (n_experts > 1024)  // the device schedule gives one thread to each expert
        return fail(PW_ERR_ARGUMENT, "a bank holds at most 1024 experts (got %u)", n_experts);
    *out = nullptr;
    if (!gate[0])
        return fail(PW_ERR_LAYOUT, "expert 0 has no gate projection");
    const uint32_t I = gate[0]->rows, H = gate[0]->columns;
    std::vector<ExpertPtrs> table(n_experts);
    for (uint32_t e = 0; e < n_experts; ++e) {
        if (!check_expert_projection(gate[e], I, H) || !check_expert_projection(up[e], I, H) ||
            !check_expert_projection(down[e], H, I))
            return fail(PW_ERR_LAYOUT, "expert %u projection shape mismatch", e);
        table[e] = ExpertPtrs{gate[e]->w, gate[e]->s, up[e]->w, up[e]->s, down[e]->w, down[e]->s};
    }
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw_expert_bank *b = new pw_expert_bank;
    b->rt = rt;
    b->n_experts = n_experts;
    b->hidden = H;
    b->intermediate = I;
    b->host_table = table;
    hipError_t e = hipMalloc(&b->table, table.size() * sizeof(ExpertPtrs));
    if (e == hipSuccess)
        e = hipMemcpy(b->table, table.data(), table.size() * sizeof(ExpertPtrs), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        pw_expert_bank_release(b);
        return fail(PW_ERR_DEVICE, "bank upload failed: %s", hipGetErrorString(e));
    }
    *out = b;
    return PW_OK;
}

void pw_expert_bank_release(pw_expert_bank *b)
{
    if (!b)
        return;
    if (b->rt)
        (void)hipSetDevice(b->rt->device);
    if (b->table)
        (void)hipFree(b->table);
    if (b->owned)
        (void)hipFree(b->owned);
    delete b;
}

}  // extern "C"

int pw::set_device_of(pw_runtime *rt)
{
    const hipError_t e = hipSetDevice(rt->device);
    return e == hipSuccess ? PW_OK : fail(PW_ERR_DEVICE, "hipSetDevice: %s", hipGetErrorString(e));
}

int pw::make_owned_bank(pw_runtime *rt, const std::vector<ExpertPtrs> &table, uint32_t hidden, uint32_t intermediate,
                        void *owned, uint64_t owned_bytes, pw_expert_bank **out)
{
    pw_expert_bank *b = new pw_expert_bank;
    b->rt = rt;
    b->n_experts = (uint32_t)table.size();
    b->hidden = hidden;
    b->intermediate = intermediate;
    b->owned = owned;
    b->owned_bytes = owned_bytes;
    b->host_table = table;
    hipError_t e = hipMalloc(&b->table, table.size() * sizeof(ExpertPtrs));
    if (e == hipSuccess)
        e = hipMemcpy(b->table, table.data(), table.size() * sizeof(ExpertPtrs), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        pw_expert_bank_release(b);
        return fail(PW_ERR_DEVICE, "bank upload failed: %s", hipGetErrorString(e));
    }
    *out = b;
    return PW_OK;
}

extern "C" {

int pw_expert_bank_shape(const pw_expert_bank *b, uint32_t *n, uint32_t *h, uint32_t *i)
{
    if (!b)
        return fail(PW_ERR_ARGUMENT, "null bank");
    if (n) *n = b->n_experts;
    if (h) *h = b->hidden;
    if (i) *i = b->intermediate;
    return PW_OK;
}

// A routed layer of `rows` token rows from device route arrays [rows][8]: the schedule, then the
// experts and the combine; a one-token mode A layer of the shape the fused kernels take reads its
// eight routes in those kernels, with no schedule launch.
static void launch_routed_layer(const MoeBuffers &mb, const pw_expert_bank *bank, uint32_t mode, const void *x,
                                bool x_f32, uint32_t rows, const uint32_t *route_ids, const float *route_weights,
                                uint32_t max_active, void *output, uint32_t out_dtype, uint32_t *flags,
                                hipStream_t s)
{
    const uint32_t E = bank->n_experts, H = bank->hidden, I = bank->intermediate;
    float *out_f32 = out_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr;
    uint16_t *out_bf16 = out_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr;
    const bool raw = out_dtype == PW_DTYPE_F32_RAW;
    if (mode == PW_MODE_A && rows == 1 && pw::moe_a_one_token_direct(H, I)) {
        const pw::OneTokenRoutes routes{route_ids, route_weights, E};
        pw::launch_moe_layer(mode, bank->table, mb, x, x_f32, rows, max_active, rows, H, I, out_f32, out_bf16, raw,
                             flags, s, &routes);
        return;
    }
    // mode B: a decode batch's schedule launch also quantises the activations
    const pw::QuantJob qj{x, x_f32 ? 1u : 0u, rows, H, mb.xq, mb.xs};
    bool quantised = false;
    pw::launch_moe_schedule(bank->table, route_ids, route_weights, rows, E, max_active, mb, flags, s, nullptr,
                            mode == PW_MODE_B ? &qj : nullptr, mode == PW_MODE_B ? &quantised : nullptr);
    pw::launch_moe_layer(mode, bank->table, mb, x, x_f32, rows, max_active, rows, H, I, out_f32, out_bf16, raw, flags,
                         s, nullptr, quantised);
}

int pw_moe_layer_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                        uint32_t x_dtype, uint32_t rows, const uint32_t *route_ids,
                        const float *route_weights, void *output, uint32_t out_dtype, void *stream)
{
    if (!rt || !bank || !x || !route_ids || !route_weights || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if ((uintptr_t)x & 15)
        return fail(PW_ERR_ARGUMENT, "activations must be 16-byte aligned");
    if (mode > PW_MODE_B || x_dtype > PW_DTYPE_BF16 || out_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown mode or dtype");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "device MoE row count must be between one and 32");
    if (((uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "route buffers must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    PW_TRY(ensure_moe(rt, rows, bank->n_experts, bank->hidden, bank->intermediate));
    launch_routed_layer(rt->mb, bank, mode, x, x_dtype == PW_DTYPE_F32, rows, route_ids, route_weights,
                        std::min<uint32_t>(bank->n_experts, rows * 8), output, out_dtype, rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_moe_layer_routed_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                               uint32_t x_dtype, uint32_t rows, const void *router_weight, uint32_t w_dtype,
                               const float *bias, uint32_t *route_ids, float *route_weights, void *output,
                               uint32_t out_dtype, void *stream)
{
    if (!rt || !bank || !x || !router_weight || !bias || !route_ids || !route_weights || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (mode > PW_MODE_B || x_dtype > PW_DTYPE_BF16 || w_dtype > PW_DTYPE_BF16 || out_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown mode or dtype");
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "device MoE row count must be between one and 32");
    const uint32_t E = bank->n_experts, H = bank->hidden, I = bank->intermediate;
    if (E <= 8 || E > 1024 || H % 8 || H > 65536)
        return fail(PW_ERR_ARGUMENT, "the router needs 9..1024 experts and a hidden size that is a multiple of 8 "
                                     "(at most 65536)");
    if (((uintptr_t)x | (uintptr_t)router_weight | (uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "activations, router weights and route buffers must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    PW_TRY(ensure_moe(rt, rows, E, H, I));
    PW_HIP(rt->router_scores.ensure((size_t)rows * E * 4));
    float *scores = (float *)rt->router_scores.p;
    const bool x_f32 = x_dtype == PW_DTYPE_F32;
    const uint32_t max_active = std::min<uint32_t>(E, rows * 8);
    const int t = pw::timer_begin(pw::K_ROUTER, s);
    pw::launch_router_scores(x, x_f32, router_weight, w_dtype == PW_DTYPE_F32, rows, E, H, scores, s);
    pw::timer_end(t, s);
    const bool direct = mode == PW_MODE_A && rows == 1 && pw::moe_a_one_token_direct(H, I);
    PW_HIP(rt->set_ids.ensure((size_t)rows * 8 * 4));
    // mode B: the schedule launch also quantises the activations
    const pw::QuantJob qj{x, x_f32 ? 1u : 0u, rows, H, rt->mb.xq, rt->mb.xs};
    if (!direct && pw::launch_route_set_schedule(scores, bias, bank->table, rows, E, max_active,
                                                 (uint32_t *)rt->set_ids.p, rt->mb, rt->d_flags, s,
                                                 mode == PW_MODE_B ? &qj : nullptr)) {
        // the expert sets are scheduled; the routes' order and weights (a serial partition per row)
        // run in extra workgroups of an expert launch (mode A: the down, mode B: the gate/up) while
        // its others stream the experts' weights (or in a launch of their own before the combine)
        pw::RouteJob job{};
        job.scores = scores;
        job.bias = bias;
        job.rows = rows;
        job.E = E;
        job.set_ids = (const uint32_t *)rt->set_ids.p;
        job.route_ids = route_ids;
        job.route_w = route_weights;
        job.plan = rt->mb.plan;
        job.row_slots = rt->mb.row_slots;
        job.placement_w = rt->mb.placement_w;
        job.flags = rt->d_flags;
        pw::launch_moe_layer(mode, bank->table, rt->mb, x, x_f32, rows, max_active, rows, H, I,
                             out_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr,
                             out_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr, out_dtype == PW_DTYPE_F32_RAW,
                             rt->d_flags, s, nullptr, mode == PW_MODE_B, &job);
    } else if (direct && E <= 256) {
        // one token: the expert set is the direct layer's routes; the routes' order and weights
        // (the partition) run in extra workgroups of its gate/up launch and give the weights in the
        // set's order before its down+combine launch
        PW_HIP(rt->set_w.ensure(8 * 4));
        pw::launch_route_set(scores, bias, 1, E, (uint32_t *)rt->set_ids.p, s);
        pw::RouteJob job{};
        job.scores = scores;
        job.bias = bias;
        job.rows = 1;
        job.E = E;
        job.set_ids = (const uint32_t *)rt->set_ids.p;
        job.route_ids = route_ids;
        job.route_w = route_weights;
        job.plan = rt->mb.plan;
        job.row_slots = nullptr;
        job.placement_w = (float *)rt->set_w.p;
        job.flags = rt->d_flags;
        const pw::OneTokenRoutes routes{(const uint32_t *)rt->set_ids.p, (const float *)rt->set_w.p, E};
        pw::launch_moe_layer(mode, bank->table, rt->mb, x, x_f32, rows, max_active, rows, H, I,
                             out_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr,
                             out_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr, out_dtype == PW_DTYPE_F32_RAW,
                             rt->d_flags, s, &routes, false, &job);
    } else {
        pw::launch_router_select(scores, bias, rows, E, route_ids, route_weights, nullptr, rt->d_flags, s);
        launch_routed_layer(rt->mb, bank, mode, x, x_f32, rows, route_ids, route_weights, max_active, output,
                            out_dtype, rt->d_flags, s);
    }
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_moe_layer_device_noalloc(pw_runtime *rt, const pw_expert_bank *bank, uint32_t mode, const void *x,
                                uint32_t x_dtype, uint32_t rows, const uint32_t *route_ids,
                                const float *route_weights, void *output, uint32_t out_dtype, void *stream)
{
    if (!rt || !bank || !x || !route_ids || !route_weights || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if ((uintptr_t)x & 15)
        return fail(PW_ERR_ARGUMENT, "activations must be 16-byte aligned");
    if (mode > PW_MODE_B || x_dtype > PW_DTYPE_BF16 || out_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown mode or dtype");
    if (((uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "route buffers must be 16-byte aligned");
    const uint32_t E = bank->n_experts, H = bank->hidden, I = bank->intermediate;
    if (rows < 1 || rows > NOALLOC_MAX_ROWS)
        return fail(PW_ERR_ARGUMENT, "the no-alloc MoE layer takes 1 to %u token rows (got %u)", NOALLOC_MAX_ROWS,
                    rows);
    if (E > NOALLOC_MAX_EXPERTS || H > NOALLOC_MAX_HIDDEN || I > NOALLOC_MAX_INTER)
        return fail(PW_ERR_ARGUMENT,
                    "the no-alloc MoE layer takes banks of at most %u experts, hidden %u, intermediate %u "
                    "(got %u, %u, %u)", NOALLOC_MAX_EXPERTS, NOALLOC_MAX_HIDDEN, NOALLOC_MAX_INTER, E, H, I);
    MoeBuffers mb{};
    const size_t need = carve_moe(nullptr, rows, E, H, I, mb);
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(PW_ERR_ARGUMENT, "the no-alloc MoE layer needs %zu bytes of scratch, its array holds %zu", need,
                    NOALLOC_SCRATCH_BYTES);
    if (rt->device >= NOALLOC_MAX_DEVICES || !g_scratch_ptr[rt->device])
        return fail(PW_ERR_DEVICE, "no scratch array address for device %d", rt->device);
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    carve_moe((char *)g_scratch_ptr[rt->device], rows, E, H, I, mb);
    launch_routed_layer(mb, bank, mode, x, x_dtype == PW_DTYPE_F32, rows, route_ids, route_weights,
                        std::min<uint32_t>(E, rows * 8), output, out_dtype, rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_moe_prefill_device(pw_runtime *rt, const pw_expert_bank *bank, const void *x, uint32_t x_dtype,
                          uint32_t rows, const uint32_t *route_ids, const float *route_weights, void *output,
                          uint32_t out_dtype, void *stream)
{
    if (!rt || !bank || !x || !route_ids || !route_weights || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (((uintptr_t)x | (uintptr_t)output) & 15)
        return fail(PW_ERR_ARGUMENT, "activations and output must be 16-byte aligned");
    if (x_dtype > PW_DTYPE_BF16 || out_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown dtype");
    if (rows < 1 || rows > 4096)
        return fail(PW_ERR_ARGUMENT, "prefill row count must be between one and 4096");
    if (((uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "route buffers must be 16-byte aligned");
    const uint32_t E = bank->n_experts, H = bank->hidden, I = bank->intermediate;
    if (H % 128 || I % 128)
        return fail(PW_ERR_LAYOUT, "prefill needs hidden and intermediate sizes in multiples of 128");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    PW_TRY(ensure_moe(rt, rows, E, H, I, false));
    const uint32_t max_tiles = pw::prefill_max_tiles(rows, E);
    PW_HIP(rt->pf_tiles.ensure((size_t)max_tiles * sizeof(pw::PfTileDesc) + 16));
    pw::PrefillBuffers pb{};
    pb.tiles = (pw::PfTileDesc *)rt->pf_tiles.p;
    pb.n_tiles = (uint32_t *)((char *)rt->pf_tiles.p + (size_t)max_tiles * sizeof(pw::PfTileDesc));
    pb.hidden = (uint16_t *)rt->moe_hidden.p;  // [P][I] f32 scratch holds the bf16 hidden
    pb.y = (uint16_t *)rt->moe_y.p;            // [P][H] f32 scratch holds the bf16 outputs
    PW_TRY(ensure_silu_table(rt));
    pb.silu = (const uint16_t *)rt->pf_silu.p;
    const uint32_t P = rows * 8;
    const pw::PfTileTable tt{pb.tiles, pb.n_tiles, max_tiles};
    const pw::QuantJob qj{x, x_dtype == PW_DTYPE_F32 ? 1u : 0u, rows, H, rt->mb.xq, rt->mb.xs};
    const bool scheduled_long = pw::launch_moe_schedule(bank->table, route_ids, route_weights, rows, E,
                                                        std::min<uint32_t>(E, P), rt->mb, rt->d_flags, s, &tt, &qj);
    pw::launch_moe_prefill(bank->table, rt->mb, pb, x, x_dtype == PW_DTYPE_F32, rows, E, H, I,
                           out_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr,
                           out_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr,
                           out_dtype == PW_DTYPE_F32_RAW, rt->d_flags, s, scheduled_long);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_moe_schedule_device(pw_runtime *rt, const pw_expert_bank *bank, const uint32_t *route_ids,
                           const float *route_weights, uint32_t rows, uint32_t *expert_offsets,
                           uint32_t *positions, float *weights, uint32_t *row_slots, void *stream)
{
    if (!rt || !bank || !route_ids || !route_weights || !expert_offsets || !positions || !weights || !row_slots)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (rows < 1 || rows > 4096)
        return fail(PW_ERR_ARGUMENT, "schedule row count must be between one and 4096");
    if (((uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "route buffers must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    const uint32_t E = bank->n_experts;
    PW_TRY(ensure_sched(rt, rows, E));
    const size_t P = (size_t)rows * 8;
    pw::launch_moe_schedule(bank->table, route_ids, route_weights, rows, E, std::min<uint32_t>(E, (uint32_t)P),
                            rt->mb, rt->d_flags, s);
    pw::launch_expert_offsets(rt->mb, E, expert_offsets, s);
    PW_HIP(hipMemcpyAsync(positions, rt->mb.placement_pos, P * 4, hipMemcpyDeviceToDevice, s));
    PW_HIP(hipMemcpyAsync(weights, rt->mb.placement_w, P * 4, hipMemcpyDeviceToDevice, s));
    PW_HIP(hipMemcpyAsync(row_slots, rt->mb.row_slots, P * 4, hipMemcpyDeviceToDevice, s));
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_route_device(pw_runtime *rt, const void *x, uint32_t x_dtype, uint32_t rows, uint32_t hidden,
                    const void *router_weight, uint32_t w_dtype, uint32_t experts, const float *bias,
                    uint32_t *route_ids, float *route_weights, float *scores, uint32_t *tie_rows, void *stream)
{
    if (!rt || !x || !router_weight || !bias || !route_ids || !route_weights)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if (x_dtype > PW_DTYPE_BF16 || w_dtype > PW_DTYPE_BF16)
        return fail(PW_ERR_ARGUMENT, "unknown dtype");
    if (rows < 1 || rows > 4096 || hidden == 0 || experts <= 8 || experts > 1024)
        return fail(PW_ERR_ARGUMENT, "router needs 1..4096 rows, a hidden size and 9..1024 experts");
    // rows are read as 8-column groups with 16-byte loads
    if (hidden % 8 || hidden > 65536 || (((uintptr_t)x | (uintptr_t)router_weight) & 15))
        return fail(PW_ERR_ARGUMENT, "router hidden size must be a multiple of 8 (at most 65536) with 16-byte "
                                     "aligned activations and router weights");
    if (((uintptr_t)route_ids | (uintptr_t)route_weights) & 15)
        return fail(PW_ERR_ARGUMENT, "route buffers must be 16-byte aligned");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    float *sc = scores;
    if (!sc) {
        PW_HIP(rt->router_scores.ensure((size_t)rows * experts * 4));
        sc = (float *)rt->router_scores.p;
    }
    pw::launch_router(x, x_dtype == PW_DTYPE_F32, router_weight, w_dtype == PW_DTYPE_F32, bias, rows, experts, hidden,
                      sc, route_ids, route_weights, tie_rows, rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

int pw_expert_forward_device(pw_runtime *rt, const pw_expert_bank *bank, uint32_t expert,
                             uint32_t mode, const void *x, uint32_t x_dtype, uint32_t rows,
                             void *output, uint32_t out_dtype, void *stream)
{
    if (!rt || !bank || !x || !output)
        return fail(PW_ERR_ARGUMENT, "null argument");
    if ((uintptr_t)x & 15)
        return fail(PW_ERR_ARGUMENT, "activations must be 16-byte aligned");
    if (mode > PW_MODE_B || x_dtype > PW_DTYPE_BF16 || out_dtype > PW_DTYPE_F32_RAW)
        return fail(PW_ERR_ARGUMENT, "unknown mode or dtype");
    if (expert >= bank->n_experts)
        return fail(PW_ERR_ARGUMENT, "expert %u outside the bank of %u", expert, bank->n_experts);
    if (rows < 1 || rows > 32)
        return fail(PW_ERR_ARGUMENT, "expert row count must be between one and 32");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    hipStream_t s = stream ? (hipStream_t)stream : rt->stream;
    StreamOrder order(rt, s);
    PW_HIP(order.err);
    PW_TRY(ensure_moe(rt, rows, bank->n_experts, bank->hidden, bank->intermediate));
    pw::launch_expert_forward(mode, bank->table, bank->host_table[expert], expert, rt->mb, x, x_dtype == PW_DTYPE_F32,
                              rows,
                              bank->hidden, bank->intermediate,
                              out_dtype != PW_DTYPE_BF16 ? (float *)output : nullptr,
                              out_dtype == PW_DTYPE_BF16 ? (uint16_t *)output : nullptr,
                              out_dtype == PW_DTYPE_F32_RAW, rt->d_flags, s);
    PW_HIP(hipGetLastError());
    return PW_OK;
}

// ----------------------------------------------------------------------------- host routing
extern "C++" {
namespace {

// nth_element over (value, index) pairs with Idx-wide indices; the first top_k indices in
// partition order, truncated to 32 bits as the reference's static_cast<uint32_t> does.
template <class Idx>
void topk_unsorted(const float *values, size_t count, size_t top_k, uint32_t *selected)
{
    std::vector<pw::TopkEntryT<Idx>> q(count);
    for (size_t i = 0; i < count; ++i)
        q[i] = pw::TopkEntryT<Idx>{values[i], (Idx)i};
    pw::nth_element_libcxx(q.data(), q.data() + top_k - 1, q.data() + count);
    for (size_t i = 0; i < top_k; ++i)
        selected[i] = (uint32_t)q[i].i;
}

}  // namespace
}

int pw_pytorch_topk_unsorted_f32(const float *values, size_t count, size_t top_k, uint32_t *selected)
{
    if (!values || !selected || top_k == 0 || top_k >= count)
        return -1;
    try {
        if (count <= (size_t)INT32_MAX)
            topk_unsorted<int32_t>(values, count, top_k, selected);
        else
            topk_unsorted<int64_t>(values, count, top_k, selected);
    } catch (...) {
        return -2;
    }
    return 0;
}

int pw_topk_unsorted_f32(const float *values, size_t count, size_t top_k, uint32_t *selected)
{
    return pw_pytorch_topk_unsorted_f32(values, count, top_k, selected);
}

int pw_noaux_routes(const float *scores, const float *bias, uint32_t rows, uint32_t experts,
                    uint32_t *selected, float *weights, uint64_t *tie_rows)
{
    constexpr uint32_t K = 8;
    if (!scores || !bias || !selected || !weights || experts <= K)
        return fail(PW_ERR_ARGUMENT, "invalid PyTorch noaux-tc inputs");
    for (size_t i = 0; i < (size_t)rows * experts; ++i)
        if (!finite(scores[i]))
            return fail(PW_ERR_NONFINITE, "invalid PyTorch noaux-tc inputs");
    for (uint32_t e = 0; e < experts; ++e)
        if (!finite(bias[e]))
            return fail(PW_ERR_NONFINITE, "invalid PyTorch noaux-tc inputs");
    std::vector<pw::TopkEntry> scratch(experts);
    uint64_t ties = 0;
    for (uint32_t p = 0; p < rows; ++p) {
        bool tie = false;
        const int st = pw::noaux_route_row(scores + (size_t)p * experts, bias, experts, scratch.data(),
                                           selected + (size_t)p * K, weights + (size_t)p * K, &tie);
        if (st == pw::ROUTE_NONFINITE)
            return fail(PW_ERR_NONFINITE, "invalid PyTorch noaux-tc inputs");
        if (st == pw::ROUTE_TOPK)
            return fail(PW_ERR_SCHEDULE, "PyTorch top-k failed at position %u", p);
        if (st == pw::ROUTE_WEIGHTS)
            return fail(PW_ERR_NONFINITE, "PyTorch route weights invalid at position %u", p);
        ties += tie ? 1 : 0;
    }
    if (tie_rows)
        *tie_rows = ties;
    return PW_OK;
}

int pw_route_from_logits(const float *logits, const float *bias, uint32_t rows, uint32_t experts,
                         float *scores, uint32_t *selected, float *weights, uint64_t *tie_rows)
{
    if (!logits || !scores)
        return fail(PW_ERR_ARGUMENT, "null argument");
    for (size_t i = 0; i < (size_t)rows * experts; ++i)
        scores[i] = pw::sigmoid_pytorch(logits[i]);
    return pw_noaux_routes(scores, bias, rows, experts, selected, weights, tie_rows);
}

// ------------------------------------------------------------------------------ layout maps
int64_t pw_full_qkv_source_row(int64_t r)
{
    constexpr int64_t QS = 3072, SHARD = 3392, Q = 4 * QS, KR = 4 * 192, VR = 4 * 128;
    if (r < 0)
        return -1;
    if (r < Q)
        return (r / QS) * SHARD + r % QS;
    if (r < Q + KR)
        return ((r - Q) / 192) * SHARD + QS + (r - Q) % 192;
    if (r < Q + KR + VR)
        return ((r - Q - KR) / 128) * SHARD + QS + 192 + (r - Q - KR) % 128;
    return -1;
}

int64_t pw_full_qkv_scale_row(int64_t r)
{
    const int64_t src = pw_full_qkv_source_row(r);
    if (src < 0)
        return -1;
    const int64_t shard = src / 3392, local = src % 3392;
    const int64_t ls = local < 3072 ? local / 128 : (local < 3264 ? 24 + (local - 3072) / 128 : 26);
    return shard * 27 + ls;
}

int64_t pw_swa_qkv_source_row(int64_t r)
{
    constexpr int64_t QS = 3072, KS = 384, VS = 256, SHARD = QS + KS + VS;
    if (r < 0)
        return -1;
    if (r < 4 * QS)
        return r / QS * SHARD + r % QS;
    if (r < 4 * (QS + KS))
        return (r - 4 * QS) / KS * SHARD + QS + (r - 4 * QS) % KS;
    if (r < 4 * SHARD)
        return (r - 4 * (QS + KS)) / VS * SHARD + QS + KS + (r - 4 * (QS + KS)) % VS;
    return -1;
}

// ------------------------------------------------------------------------------- synthetic
int pw_synth_scales(pw_runtime *rt, float *scales, uint64_t count, uint64_t seed, float lo, float hi)
{
    if (!rt || !scales || count == 0)
        return fail(PW_ERR_ARGUMENT, "null argument");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw::launch_synth_scales(scales, count, seed, lo, hi, rt->stream);
    PW_HIP(hipGetLastError());
    PW_HIP(hipStreamSynchronize(rt->stream));
    return PW_OK;
}

int pw_synth_fp8(pw_runtime *rt, uint8_t *w, const float *scales, uint64_t rows, uint64_t cols,
                 uint64_t seed)
{
    if (!rt || !w || !scales || rows == 0 || cols == 0 || cols % 128 != 0)
        return fail(PW_ERR_ARGUMENT, "bad synthetic FP8 arguments");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw::launch_synth_fp8(w, scales, rows, cols, seed, rt->stream);
    PW_HIP(hipGetLastError());
    PW_HIP(hipStreamSynchronize(rt->stream));
    return PW_OK;
}

int pw_synth_normal_bf16(pw_runtime *rt, uint16_t *x, uint64_t count, uint64_t seed, float stddev)
{
    if (!rt || !x || count == 0 || count % 2 != 0)
        return fail(PW_ERR_ARGUMENT, "bad synthetic bf16 arguments");
    PW_HIP(set_device(rt));
    TimerScope timer_scope(rt);
    pw::launch_synth_normal_bf16(x, count, seed, stddev, rt->stream);
    PW_HIP(hipGetLastError());
    PW_HIP(hipStreamSynchronize(rt->stream));
    return PW_OK;
}

}  // extern "C"
