#!/usr/bin/env python3
"""Benchmark of the MI355X block-FP8 routed-MoE decode layer (one GPU).

Workload (one step): a width-8 routed-MoE decode layer -- 8 token rows, hidden 4096, top-8 of 256
experts of intermediate 2048, block-FP8 e4m3 weights with 128x128 f32 scales, mode A (FP8 weight x
bf16 activation, f32 accumulation) -- with activations, routes and the 6.4 GB expert bank already
resident in HBM. Routes come from the reference's router numerics (bf16 router weight N(0, 0.02^2),
sigmoid + correction bias U(-0.01, 0.01), top-8, renormalised). Steps cycle over several token
batches so consecutive steps read different expert sets.

value = algorithmic HBM bytes per step (unique routed experts' weights and scales + activations,
routes and outputs) / measured step time.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mimo-prismwing_amd"))

METRIC = "MoE layer µs + HBM GB/s (% of 8 TB/s) at width 1/8; prefill FP8 MFMA TFLOP/s"
HBM_PEAK_GBS = 8000.0
EXPERT_WEIGHT_BYTES = 3 * 2048 * 4096          # gate + up + down e4m3
EXPERT_SCALE_BYTES = (16 * 32 + 16 * 32 + 32 * 16) * 4


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_batches(P, WL, n_batches, rows, zipf):
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    batches = []
    for b in range(n_batches):
        x = WL.activations(rows, WL.SEED_BASE + 100 + b)
        sel, w, _ = WL.route_host(x, rw, bias)
        batches.append((x, sel, w))
    return batches


def upload(torch, WL, batches):
    dev = []
    for x, sel, w in batches:
        dev.append((torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda(),
                    torch.from_numpy(sel.astype(np.int32)).cuda(),
                    torch.from_numpy(w).cuda()))
    return dev


def placement_histogram(sel, experts=256):
    """{placements per routed expert: number of experts} over a batch's routes."""
    counts = np.bincount(np.asarray(sel).reshape(-1), minlength=experts)
    vals, freq = np.unique(counts[counts > 0], return_counts=True)
    return {int(v): int(f) for v, f in zip(vals, freq)}


def step_bytes(sel, rows, hidden=4096):
    u = int(np.unique(sel).size)
    return u, u * (EXPERT_WEIGHT_BYTES + EXPERT_SCALE_BYTES) + rows * hidden * 2 * 2 + rows * 8 * 8


def gateup_bytes(sel, rows, hidden=4096, inter=2048):
    """Gate/up kernel: routed experts' gate and up weights and scales, the bf16 activations, and the
    SwiGLU output written as three bf16 planes per placement."""
    u = int(np.unique(sel).size)
    return u * (2 * inter * hidden + 2 * 16 * 32 * 4) + rows * hidden * 2 + rows * 8 * inter * 2 * 3


SETTLE_S = 0.3


def percentile(ordered, fraction):
    """The reference's wall-time percentile (src/lib.rs:1754-1761): the sorted sample at index
    round((n - 1) * fraction)."""
    return ordered[int(round((len(ordered) - 1) * fraction))]


def timed_steps(torch, stream, run, steps):
    """Mean step time (ms) of `steps` back-to-back steps bracketed by one event pair, then the same
    steps again with an event between consecutive steps: their p10 / median / p90 in µs, the
    reference's summary of a timing sample. Both passes queue behind the caller's warm-up work."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        run(i)
    end.record(stream)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    marks[0].record(stream)
    for i in range(steps):
        run(i)
        marks[i + 1].record(stream)
    torch.cuda.synchronize()
    per = sorted(1000.0 * marks[i].elapsed_time(marks[i + 1]) for i in range(steps))
    spread = {"p10_us": round(percentile(per, 0.10), 2), "median_us": round(percentile(per, 0.50), 2),
              "p90_us": round(percentile(per, 0.90), 2), "samples": steps}
    return start.elapsed_time(end) / steps, spread


def settle(torch, run, seconds=SETTLE_S):
    """Runs the workload untimed for `seconds` of wall time. The GPU lowers its clocks while it idles
    (host-side set-up between legs): 20 layer steps timed right after such a pause measured 285-287
    µs per step against 249.5 µs after 200 ms of the same steps."""
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(16):
            run(i)
            i += 1
        torch.cuda.synchronize()


def time_layer(torch, rt, bank, P, dev_batches, rows, steps, warmup, mode, settle_first=True):
    # launches and events on the runtime's own stream (torch's default stream is the null stream,
    # handle 0, which the library would map to its own stream and the events would not see)
    stream = torch.cuda.ExternalStream(rt.stream)
    out = torch.empty((rows, 4096), dtype=torch.int16, device="cuda")
    nb = len(dev_batches)

    def run(i):
        xt, ids, wts = dev_batches[i % nb]
        rt.moe_layer_device(bank.bank, xt, rows, ids, wts, out, mode=mode, out_dtype=P.DTYPE_BF16,
                            stream=stream.cuda_stream)

    if settle_first:
        settle(torch, run)
    for i in range(warmup):
        run(i)
    # the start event queues behind the warm-up steps: the timed steps start on a busy GPU, with
    # no drained queue or idle gap in front of them
    ms, spread = timed_steps(torch, stream, run, steps)
    flags = rt.take_flags()
    if flags:
        raise RuntimeError(f"kernels raised error flags {flags}")
    return ms, spread


def kernel_times(torch, rt, bank, P, dev_batches, rows, steps, mode):
    """Per-kernel durations from HIP events recorded on the launch stream inside the library."""
    time_layer(torch, rt, bank, P, dev_batches, rows, 2, 0, mode)  # settles the clocks
    rt.enable_timing(steps * 16)  # two passes of up to eight launches per step
    time_layer(torch, rt, bank, P, dev_batches, rows, steps, 0, mode, settle_first=False)
    res = {}
    for k in ("moe_schedule", "quant", "moe_gateup", "moe_swiglu", "moe_down", "moe_combine"):
        n, ms = rt.timing(k)
        if n:
            res[k] = {"launches": n, "avg_us": 1000.0 * ms / n}
    rt.enable_timing(0)
    return res


PREFILL_ROWS = 2048
EXPERT_MACS = 3 * 2048 * 4096                  # multiply-adds per placement (gate, up, down)
FP8_PEAK_TFLOPS = 5000.0                       # MI355X dense FP8 MFMA


def prefill_leg(torch, rt, bank, P, WL, zipf, steps=20, warmup=3):
    """Routed-MoE prefill over 2048 tokens (16 384 placements, mode B grouped FP8 GEMM)."""
    rows = PREFILL_ROWS
    x = WL.activations(rows, WL.SEED_BASE + 4)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    sel, w, _ = WL.route_host(x, rw, bias)
    xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
    ids = torch.from_numpy(sel.astype(np.int32)).cuda()
    wts = torch.from_numpy(w).cuda()
    out = torch.empty((rows, 4096), dtype=torch.int16, device="cuda")
    stream = torch.cuda.ExternalStream(rt.stream)

    def run(i=0):
        rt.moe_prefill_device(bank.bank, xt, rows, ids, wts, out, out_dtype=P.DTYPE_BF16, stream=stream.cuda_stream)

    settle(torch, run)
    for _ in range(warmup):
        run()
    ms, spread = timed_steps(torch, stream, run, steps)
    if rt.take_flags():
        raise RuntimeError("prefill kernels raised error flags")
    rt.enable_timing(steps * 8)
    for _ in range(steps):
        run()
    kt = {}  # average µs per launch (moe_swiglu: the SwiGLU + re-quantisation of the hidden)
    for k in ("moe_schedule", "quant", "prefill_gateup", "moe_swiglu", "prefill_down", "moe_combine"):
        n, tot = rt.timing(k)
        if n:
            kt[k] = round(1000.0 * tot / n, 2)
    rt.enable_timing(0)
    u = int(np.unique(sel).size)
    flops = 2.0 * rows * 8 * EXPERT_MACS
    wbytes = u * (EXPERT_WEIGHT_BYTES + EXPERT_SCALE_BYTES)
    tflops = flops / (ms * 1e-3) / 1e12
    counts = np.bincount(sel.reshape(-1), minlength=256)
    return {"layer_us": round(ms * 1000, 2), "spread_us": spread, "TFLOP/s": round(tflops, 1),
            "fp8_peak_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
            "weight_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1), "unique_experts": u,
            "max_count": int(counts.max()), "m_tiles_128": int(np.sum((counts + 127) // 128)),
            "top_counts": sorted(counts.tolist(), reverse=True)[:8],
            "count_quartiles": [int(v) for v in np.percentile(counts, [0, 25, 50, 75, 100])], "kernels_us": kt}


def _time_calls(torch, rt, run, n_calls, warmup=3):
    """(µs per call, spread) of `run(i)` over n_calls back-to-back calls on the runtime's stream."""
    stream = torch.cuda.ExternalStream(rt.stream)
    settle(torch, lambda i: run(i, stream.cuda_stream), 0.1)
    for i in range(warmup):
        run(i, stream.cuda_stream)
    ms, spread = timed_steps(torch, stream, lambda i: run(i, stream.cuda_stream), n_calls)
    if rt.take_flags():
        raise RuntimeError("kernels raised error flags")
    return 1000.0 * ms, spread


def _bf16_x(torch, WL, rows, hidden, seed):
    return torch.from_numpy(WL.bf16_bits_np(WL.activations(rows, seed, hidden=hidden)).view(np.int16)).cuda()


def projection_legs(torch, rt, bank, P, WL, calls=200, small_only=False):
    """Configs 0, 1 and 3 (one projection, one complete expert, separate q/k/v segments), mode A,
    bf16 in and out. HBM-cold: calls rotate over distinct weights well beyond the 256 MB MALL;
    MALL-warm: one weight copy reused. small_only: configs 0, 1 (widths 1 and 8) and 3 (k 768)
    only, for a kernel trace of the small calls."""
    out = {}
    # config 0: W [2048 x 4096] e4m3 + S [16 x 32], x [1 x 4096] -> y [1 x 2048]
    copies, n, k = 64, 2048, 4096
    w = torch.empty((copies * n, k), dtype=torch.uint8, device="cuda")
    s = torch.empty((copies * n // 128, k // 128), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    rt.synth_scales(s, s.numel(), WL.SEED_BASE + 500)
    rt.synth_fp8(w, s, copies * n, k, WL.SEED_BASE + 501)
    projs = [rt.bind_projection_device(w[i * n:(i + 1) * n], s[i * n // 128:(i + 1) * n // 128], n, k)
             for i in range(copies)]
    x = _bf16_x(torch, WL, 1, k, WL.SEED_BASE + 502)
    y = torch.empty((1, n), dtype=torch.int16, device="cuda")
    alg = n * k + (n // 128) * (k // 128) * 4 + k * 2 + n * 2
    for label, pick in (("hbm_cold", lambda i: projs[i % copies]), ("mall_warm", lambda i: projs[0])):
        us, sp = _time_calls(torch, rt, lambda i, st: rt.fp8_linear_device(pick(i), x, 1, y, mode=P.MODE_A,
                                                                         out_dtype=P.DTYPE_BF16, stream=st), calls)
        out.setdefault("config0_w1", {})[label] = {"us": round(us, 2), "GB/s": round(alg / (us * 1e-6) / 1e9, 1),
                                                   "spread_us": sp}
    out["config0_w1"]["algorithmic_bytes"] = alg
    del projs, w, s
    # config 1: one complete expert (gate/up [2 x 2048 x 4096], down [4096 x 2048]) at widths 1..8
    for width in ((1, 8) if small_only else (1, 2, 4, 8)):
        x = _bf16_x(torch, WL, width, 4096, WL.SEED_BASE + 510 + width)
        y = torch.empty((width, 4096), dtype=torch.int16, device="cuda")
        alg = EXPERT_WEIGHT_BYTES + EXPERT_SCALE_BYTES + width * 4096 * 2 * 2
        rec = {"algorithmic_bytes": alg}
        for label, pick in (("hbm_cold", lambda i: i % 256), ("mall_warm", lambda i: 0)):
            us, sp = _time_calls(torch, rt, lambda i, st: rt.expert_forward_device(
                bank.bank, pick(i), x, width, y, mode=P.MODE_A, out_dtype=P.DTYPE_BF16, stream=st), calls)
            rec[label] = {"us": round(us, 2), "GB/s": round(alg / (us * 1e-6) / 1e9, 1), "spread_us": sp}
        out[f"config1_w{width}"] = rec
    # config 3: separate q [12288], k [768 or 1000], v [512] x 4096 with their own scale grids
    for k_rows in ((768,) if small_only else (768, 1000)):
        seg_rows = (12288, k_rows, 512)
        copies = 10
        hosts = []
        for c in range(copies):
            segs = []
            for j, r in enumerate(seg_rows):
                ws = torch.empty((r, 4096), dtype=torch.uint8, device="cuda")
                ss = torch.empty(((r + 127) // 128, 32), dtype=torch.float32, device="cuda")
                seed = WL.SEED_BASE + 600 + 10 * c + j
                rt.synth_scales(ss, ss.numel(), seed)
                rt.synth_fp8(ws, ss, r, 4096, seed + 5)
                segs.append((ws.cpu().numpy(), ss.cpu().numpy()))
            hosts.append(segs)
        projs = [rt.bind_segments(segs, scan_codes=False) for segs in hosts]
        total = sum(seg_rows)
        for width in (1, 8):
            x = _bf16_x(torch, WL, width, 4096, WL.SEED_BASE + 620 + width)
            y = torch.empty((width, total), dtype=torch.int16, device="cuda")
            alg = total * 4096 + sum((r + 127) // 128 for r in seg_rows) * 32 * 4 + width * (4096 + total) * 2
            rec = {"algorithmic_bytes": alg}
            for label, pick in (("hbm_cold", lambda i: projs[i % copies]), ("mall_warm", lambda i: projs[0])):
                us, sp = _time_calls(torch, rt, lambda i, st: rt.fp8_linear_device(
                    pick(i), x, width, y, mode=P.MODE_A, out_dtype=P.DTYPE_BF16, stream=st), calls)
                rec[label] = {"us": round(us, 2), "GB/s": round(alg / (us * 1e-6) / 1e9, 1), "spread_us": sp}
            out[f"config3_k{k_rows}_w{width}"] = rec
        del projs, hosts
    if small_only:
        return out
    # BF16 wide linear: attention o_proj [4096 x 8192] (64 MB), widths 1 and 8, f32 in, bf16-rounded f32 out
    copies, n, k = 10, 4096, 8192
    wb = torch.randn((copies, n, k), dtype=torch.bfloat16, device="cuda").view(torch.int16)
    bprojs = [rt.bind_bf16_device(wb[i], n, k) for i in range(copies)]
    for width in (1, 8):
        x = torch.randn((width, k), dtype=torch.float32, device="cuda")
        y = torch.empty((width, n), dtype=torch.float32, device="cuda")
        alg = n * k * 2 + width * k * 4 + width * n * 4
        rec = {"algorithmic_bytes": alg}
        for label, pick in (("hbm_cold", lambda i: bprojs[i % copies]), ("mall_warm", lambda i: bprojs[0])):
            us, sp = _time_calls(torch, rt, lambda i, st: rt.bf16_linear_device(pick(i), x, width, y, stream=st),
                                 calls)
            rec[label] = {"us": round(us, 2), "GB/s": round(alg / (us * 1e-6) / 1e9, 1), "spread_us": sp}
        out[f"bf16_o_proj_w{width}"] = rec
    del bprojs, wb
    # the LM head through the same wide linear (src/text_endpoint.rs:5673-5705): [152576 x 4096]
    # bf16, 1.25 GB (beyond the MALL, so every call streams it from HBM), widths 1 and 8
    n, k = 152576, 4096
    wl = (torch.randn((n, k), device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
    lproj = rt.bind_bf16_device(wl, n, k)
    for width in (1, 8):
        x = torch.randn((width, k), dtype=torch.float32, device="cuda")
        y = torch.empty((width, n), dtype=torch.float32, device="cuda")
        alg = n * k * 2 + width * k * 4 + width * n * 4
        us, sp = _time_calls(torch, rt, lambda i, st: rt.bf16_linear_device(lproj, x, width, y, stream=st),
                             max(calls // 4, 20))
        out[f"bf16_lm_head_w{width}"] = {"algorithmic_bytes": alg, "us": round(us, 2),
                                         "GB/s": round(alg / (us * 1e-6) / 1e9, 1), "spread_us": sp}
    del lproj, wl
    out.update(dense_mlp_legs(torch, rt, P, WL, (P.MODE_A, P.MODE_B), calls))
    return out


def dense_mlp_legs(torch, rt, P, WL, modes, calls=200, widths=(1, 8)):
    """The dense layer-0 FP8 MLP (gate/up [16384 x 4096], down [4096 x 16384]) as one-expert banks,
    three copies, through pw_expert_forward_device in each of `modes`, bf16 in and out."""
    out = {}
    dh, di, copies = 4096, 16384, 3
    keep, banks = [], []
    for c in range(copies):
        projs = []
        for j, (rows_, cols_) in enumerate(((di, dh), (di, dh), (dh, di))):
            w = torch.empty((rows_, cols_), dtype=torch.uint8, device="cuda")
            sc = torch.empty((rows_ // 128, cols_ // 128), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            rt.synth_scales(sc, sc.numel(), WL.SEED_BASE + 700 + 10 * c + 2 * j)
            rt.synth_fp8(w, sc, rows_, cols_, WL.SEED_BASE + 701 + 10 * c + 2 * j)
            keep += [w, sc]
            projs.append(rt.bind_projection_device(w, sc, rows_, cols_))
        banks.append(rt.expert_bank([projs[0]], [projs[1]], [projs[2]]))
        keep.append(projs)
    weight_bytes = 3 * dh * di + 3 * (dh // 128) * (di // 128) * 4
    for mode in modes:
        tag = "a" if mode == P.MODE_A else "b"
        for width in widths:
            x = _bf16_x(torch, WL, width, dh, WL.SEED_BASE + 720 + width)
            y = torch.empty((width, dh), dtype=torch.int16, device="cuda")
            alg = weight_bytes + width * dh * 2 * 2
            rec = {"algorithmic_bytes": alg}
            for label, pick in (("hbm_cold", lambda i: banks[i % copies]), ("mall_warm", lambda i: banks[0])):
                us, sp = _time_calls(torch, rt, lambda i, st: rt.expert_forward_device(
                    pick(i), 0, x, width, y, mode=mode, out_dtype=P.DTYPE_BF16, stream=st), calls // 2)
                rec[label] = {"us": round(us, 2), "GB/s": round(alg / (us * 1e-6) / 1e9, 1), "spread_us": sp}
            out[f"dense_mlp_mode_{tag}_w{width}"] = rec
    del banks, keep
    return out


def layer_with_router(torch, rt, bank, P, WL, rows=8, steps=200, warmup=20, two_calls=False):
    """One decode step including its routing, per step: the device router (logits, sigmoid + bias,
    top-8, weights) on the batch's activations, then the width-8 layer on those routes -- as one
    pw_moe_layer_routed_device call (the route selection and the layer's schedule in one launch), or
    with two_calls as pw_route_device then pw_moe_layer_device."""
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    wt = torch.from_numpy(WL.bf16_bits_np(rw).view(np.int16)).cuda()
    bt = torch.from_numpy(bias).cuda()
    xs = [_bf16_x(torch, WL, rows, 4096, WL.SEED_BASE + 100 + b) for b in range(8)]
    ids = torch.empty((rows, 8), dtype=torch.int32, device="cuda")
    wts = torch.empty((rows, 8), dtype=torch.float32, device="cuda")
    out = torch.empty((rows, 4096), dtype=torch.int16, device="cuda")

    def run(i, st):
        x = xs[i % len(xs)]
        if two_calls:
            rt.route_device(x, rows, 4096, wt, 256, bt, ids, wts, stream=st)
            rt.moe_layer_device(bank.bank, x, rows, ids, wts, out, mode=P.MODE_A, out_dtype=P.DTYPE_BF16,
                                stream=st)
        else:
            rt.moe_layer_routed_device(bank.bank, x, rows, wt, bt, ids, wts, out, mode=P.MODE_A,
                                       out_dtype=P.DTYPE_BF16, stream=st)

    us, sp = _time_calls(torch, rt, run, steps, warmup)
    return {"us": round(us, 2), "spread_us": sp, "rows": rows,
            "calls": "pw_route_device + pw_moe_layer_device" if two_calls else "pw_moe_layer_routed_device"}


def router_leg(torch, rt, P, WL, rows=8, calls=200):
    """On-device router (logits, sigmoid, top-8, weights) for one decode batch: x [8 x 4096] bf16,
    router weights [256 x 4096] bf16."""
    x = _bf16_x(torch, WL, rows, 4096, WL.SEED_BASE + 700)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    wt = torch.from_numpy(WL.bf16_bits_np(rw).view(np.int16)).cuda()
    bt = torch.from_numpy(bias).cuda()
    ids = torch.empty((rows, 8), dtype=torch.int32, device="cuda")
    wts = torch.empty((rows, 8), dtype=torch.float32, device="cuda")
    us, sp = _time_calls(torch, rt, lambda i, st: rt.route_device(x, rows, 4096, wt, 256, bt, ids, wts, stream=st),
                         calls)
    return {"us": round(us, 2), "spread_us": sp, "rows": rows}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "moe_decode_w8_gateup_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the gate/up kernel on this workload, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE passes (scaled by the copy-kernel calibration); None if the
    summary is absent."""
    import re
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    return int(m.group(1)) if m else None


def _cpu_threads():
    """Worker threads for the all-cores legs: the process's affinity mask, at most 16 (the host
    share of one GPU)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return max(1, min(16, affinity)), affinity


def cpu_baseline(WL, bank, batch, scalar_budget_s=12.0, blas_budget_s=3.0):
    """CPU legs on a bounded sample of the same layer (the routed experts of one width-8 batch):

    - value: the reference's own CPU path restated (src/lib.rs:5807-5862, oracle.moe_layer_blas):
      f32-dequantised weights (made before timing, as the reference makes them when it loads the
      layer) and f32 SGEMMs per expert, experts dealt over all worker threads (one BLAS thread
      each), combined in ascending expert id; whole layers repeated for ~blas_budget_s;
    - the scalar C oracle (mode A): on one thread over the experts in ascending id until
      ~scalar_budget_s, and the same per-expert arithmetic over all routed experts on all worker
      threads.
    GB/s counts the same algorithmic bytes as the GPU value (e4m3 weights and scales, activations)."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    x, sel, w = batch
    used = sorted(set(sel.reshape(-1).tolist()))
    threads, affinity = _cpu_threads()
    hosts = {e: bank.expert_host(e) for e in used}
    rows_of = {e: np.nonzero(sel == e)[0] for e in used}

    # scalar oracle, one thread, then the same experts over all threads
    done, t_one = [], 0.0
    for e in used:
        t0 = time.perf_counter()
        O.expert_mode_a(x[rows_of[e]], hosts[e])
        t_one += time.perf_counter() - t0
        done.append(e)
        if t_one >= scalar_budget_s:
            break
    def expert_bytes(experts):
        return sum(EXPERT_WEIGHT_BYTES + EXPERT_SCALE_BYTES + x[rows_of[e]].nbytes for e in experts)
    with ThreadPoolExecutor(threads) as pool:
        t0 = time.perf_counter()
        list(pool.map(lambda e: O.expert_mode_a(x[rows_of[e]], hosts[e]), used))
        t_all = time.perf_counter() - t0

        # the reference's CPU BLAS path over the whole layer
        def deq(e):
            gw, gs, uw, us, dw, ds = hosts[e]
            return e, (O.decode_fp8_matrix_f32(gw, gs), O.decode_fp8_matrix_f32(uw, us),
                       O.decode_fp8_matrix_f32(dw, ds))
        dequantised = dict(pool.map(deq, used))
        layer_bytes = step_bytes(sel, x.shape[0])[1]
        with threadpool_limits(1, "blas"):
            O.moe_layer_blas(x, dequantised, sel, w, pool=pool)  # untimed first pass
            reps, t0 = 0, time.perf_counter()
            while reps < 2 or time.perf_counter() - t0 < blas_budget_s:
                O.moe_layer_blas(x, dequantised, sel, w, pool=pool)
                reps += 1
            t_blas = (time.perf_counter() - t0) / reps
            # the reference's mode-B CPU path (routed_mlp_traced with fp8_linear) on the same experts
            O.moe_layer_blas_mode_b(x, dequantised, sel, w, pool=pool)
            reps_b, t0 = 0, time.perf_counter()
            while reps_b < 2 or time.perf_counter() - t0 < blas_budget_s:
                O.moe_layer_blas_mode_b(x, dequantised, sel, w, pool=pool)
                reps_b += 1
            t_blas_b = (time.perf_counter() - t0) / reps_b
    return {"value": round(layer_bytes / t_blas / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "layer_ms": round(t_blas * 1e3, 2),
            "sample": f"the reference's CPU BLAS layer (f32-dequantised weights, f32 SGEMM per expert, "
                      f"oracle.moe_layer_blas) over all {len(used)} routed experts of one width-8 batch, "
                      f"{reps} layers timed on {threads} threads (OpenBLAS, one thread per expert)",
            "hardware_concurrency": os.cpu_count(), "affinity_cpus": affinity,
            "mode_b": {"value": round(layer_bytes / t_blas_b / 1e9, 3), "unit": "GB/s",
                       "layer_ms": round(t_blas_b * 1e3, 2), "cores": threads, "kind": "port",
                       "sample": f"the reference's mode-B CPU layer (routed_mlp_traced: dynamic FP8 activations, "
                                 f"f32 SGEMM against the dequantised weights, bf16 rounding, staged SwiGLU; "
                                 f"oracle.moe_layer_blas_mode_b) over the same {len(used)} experts, {reps_b} "
                                 f"layers on {threads} threads"},
            "scalar_oracle": {"one_thread": {"GB/s": round(expert_bytes(done) / t_one / 1e9, 4),
                                             "experts": len(done), "s": round(t_one, 2)},
                              "all_threads": {"GB/s": round(expert_bytes(used) / t_all / 1e9, 4),
                                              "experts": len(used), "s": round(t_all, 2), "threads": threads}}}


def cpu_prefill_baseline(WL, bank, sample_experts=32, budget_s=4.0):
    """The reference's mode-B CPU path (routed_mlp_traced over fp8_linear, src/text_endpoint.rs:
    5290-5381, :3053-3108; oracle.expert_blas_mode_b) on a bounded sample of the 2048-token prefill:
    the `sample_experts` lowest-id routed experts with all of their placements, f32-dequantised
    before timing, experts dealt over the worker threads (one BLAS thread each). TFLOP/s counts the
    sample's placements at 2 x 3 x 2048 x 4096 flops each, as the GPU prefill's figure does."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    x = WL.activations(PREFILL_ROWS, WL.SEED_BASE + 4)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    sel, _, _ = WL.route_host(x, rw, bias)
    used = sorted(set(sel.reshape(-1).tolist()))[:sample_experts]
    rows_of = {e: np.nonzero(np.any(sel == e, axis=1))[0] for e in used}
    placements = sum(r.size for r in rows_of.values())
    threads, affinity = _cpu_threads()
    with ThreadPoolExecutor(threads) as pool:
        def deq(e):
            gw, gs, uw, us, dw, ds = bank.expert_host(e)
            return e, (O.decode_fp8_matrix_f32(gw, gs), O.decode_fp8_matrix_f32(uw, us),
                       O.decode_fp8_matrix_f32(dw, ds))
        dequantised = dict(pool.map(deq, used))
        run = lambda e: O.expert_blas_mode_b(x[rows_of[e]], *dequantised[e])
        with threadpool_limits(1, "blas"):
            list(pool.map(run, used))  # untimed first pass
            reps, t0 = 0, time.perf_counter()
            while reps < 2 or time.perf_counter() - t0 < budget_s:
                list(pool.map(run, used))
                reps += 1
            t = (time.perf_counter() - t0) / reps
    flops = 2.0 * placements * EXPERT_MACS
    all_placements = PREFILL_ROWS * 8
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample_ms": round(t * 1e3, 2), "layer_ms_estimate": round(t * 1e3 * all_placements / placements, 1),
            "sample": f"the reference's mode-B CPU path (routed_mlp_traced over fp8_linear: dynamic FP8 "
                      f"activations, f32 SGEMM against f32-dequantised weights, bf16 rounding, staged SwiGLU; "
                      f"oracle.expert_blas_mode_b) on the {len(used)} lowest-id routed experts of the 2048-token "
                      f"batch ({placements} of {all_placements} placements), {reps} passes on {threads} threads "
                      f"(OpenBLAS, one thread per expert); layer_ms_estimate scales the sample time by the "
                      f"placement count",
            "hardware_concurrency": os.cpu_count(), "affinity_cpus": affinity}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batches", type=int, default=8, help="token batches cycled over the steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the 2048-token prefill leg and print its line (for profiling)")
    ap.add_argument("--router-only", action="store_true",
                    help="run only the on-device router leg and print its line (for profiling)")
    ap.add_argument("--router-layer-only", action="store_true",
                    help="run only the decode steps with their routing (widths 8 and 1) and print their line")
    ap.add_argument("--routing", choices=("uniform", "zipf"), default="uniform",
                    help="routing of the headline decode leg and of --prefill-only (zipf: for profiling)")
    ap.add_argument("--small-calls-only", action="store_true",
                    help="run only configs 0, 1 and 3 and the one-token layer and print their line (for profiling)")
    ap.add_argument("--mode-b-only", action="store_true",
                    help="run only the mode-B decode layer (width 8, with per-kernel times) and the dense MLP "
                         "in mode B, and print their line (for profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 1 GiB device copy (reference kernel for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported (the expert path "
              "shards by experts across GPUs, which this build does not implement)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": src.numel() * 4,
                          "bytes_written": dst.numel() * 4, "launches": 5}), flush=True)
        return
    import prismwing_amd as P
    from prismwing_amd import workloads as WL

    rt = P.WideMoeRuntime.compile(0)
    if args.router_only:
        print(json.dumps({"workload": "on-device router, 8 token rows, 256 experts, hidden 4096, bf16",
                          **router_leg(torch, rt, P, WL, calls=args.steps)}), flush=True)
        rt.close()
        return
    log("synthesising the 256-expert bank (6.4 GB) on the device")
    bank = WL.synth_bank(rt, 256, seed=WL.SEED_BASE + 2)
    if args.router_layer_only:
        res = {"router_w8": router_leg(torch, rt, P, WL, calls=args.steps),
               "layer_plus_router_w8": layer_with_router(torch, rt, bank, P, WL, steps=args.steps),
               "layer_plus_router_w8_two_calls": layer_with_router(torch, rt, bank, P, WL, steps=args.steps,
                                                                   two_calls=True),
               "layer_plus_router_w1": layer_with_router(torch, rt, bank, P, WL, rows=1, steps=args.steps)}
        print(json.dumps({"workload": "decode steps with their routing, 256 experts, hidden 4096, mode A", **res}),
              flush=True)
        rt.close()
        return
    if args.prefill_only:
        res = prefill_leg(torch, rt, bank, P, WL, zipf=args.routing == "zipf")
        print(json.dumps({"workload": "routed-MoE prefill, 2048 tokens, top-8 of 256 experts, mode B, "
                                      f"{args.routing} routing", **res}), flush=True)
        rt.close()
        return
    if args.small_calls_only:
        b1 = build_batches(P, WL, args.batches, 1, zipf=False)
        ms1, _ = time_layer(torch, rt, bank, P, upload(torch, WL, b1), 1, args.steps, args.warmup, P.MODE_A)
        res = {"w1_layer_us": round(ms1 * 1000, 2), **projection_legs(torch, rt, bank, P, WL, small_only=True)}
        print(json.dumps({"workload": "small calls: configs 0, 1, 3 and the one-token routed layer, mode A", **res}),
              flush=True)
        rt.close()
        return
    if args.mode_b_only:
        bb = build_batches(P, WL, args.batches, 8, zipf=False)
        bd = upload(torch, WL, bb)
        bms, bspread = time_layer(torch, rt, bank, P, bd, 8, args.steps, args.warmup, P.MODE_B)
        kt = kernel_times(torch, rt, bank, P, bd, 8, max(20, args.steps // 4), P.MODE_B)
        b1 = upload(torch, WL, build_batches(P, WL, args.batches, 1, zipf=False))
        ms1, spread1 = time_layer(torch, rt, bank, P, b1, 1, args.steps, args.warmup, P.MODE_B)
        res = {"mode_b_w8": {"layer_us": round(bms * 1000, 2), "spread_us": bspread,
                             "kernels_us": {k: round(v["avg_us"], 2) for k, v in kt.items()}},
               "mode_b_w1": {"layer_us": round(ms1 * 1000, 2), "spread_us": spread1},
               **dense_mlp_legs(torch, rt, P, WL, (P.MODE_B,), calls=args.steps)}
        print(json.dumps({"workload": "mode-B decode layer (widths 8 and 1) and dense MLP, 256 experts, "
                                      "hidden 4096", **res}), flush=True)
        rt.close()
        return
    rows = 8
    batches = build_batches(P, WL, args.batches, rows, zipf=args.routing == "zipf")
    dev_batches = upload(torch, WL, batches)
    sizes = [step_bytes(sel, rows) for _, sel, _ in batches]
    avg_u = float(np.mean([u for u, _ in sizes]))
    avg_bytes = float(np.mean([b for _, b in sizes]))

    log(f"timing {args.steps} steps after {args.warmup} warm-up (avg {avg_u:.2f} unique experts/step)")
    ms, spread = time_layer(torch, rt, bank, P, dev_batches, rows, args.steps, args.warmup, P.MODE_A)
    value = avg_bytes / (ms * 1e-3) / 1e9
    log(f"mode A width 8: {ms * 1000:.1f} us/layer, {value:.0f} GB/s")

    kt = kernel_times(torch, rt, bank, P, dev_batches, rows, max(20, args.steps // 4), P.MODE_A)
    gu = kt["moe_gateup"]
    gu_bytes = float(np.mean([gateup_bytes(sel, rows) for _, sel, _ in batches]))
    achieved = gu_bytes / (gu["avg_us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                "kernel": "moe_a_gateup_fused_kernel (gate+up, SwiGLU fused)", "bytes_per_launch": int(gu_bytes),
                "avg_us": round(gu["avg_us"], 2)}

    extras = {"kernels_us": {k: round(v["avg_us"], 2) for k, v in kt.items()},
              "layer_us": round(ms * 1000, 2), "spread_us": spread, "tokens_per_s": round(rows / (ms * 1e-3), 1),
              "hbm_frac": round(value / HBM_PEAK_GBS, 4), "avg_unique_experts": avg_u,
              "placement_histogram": placement_histogram(np.concatenate([s for _, s, _ in batches]))}
    if not args.no_extras:
        zb = build_batches(P, WL, args.batches, rows, zipf=True)
        zd = upload(torch, WL, zb)
        zs = [step_bytes(sel, rows) for _, sel, _ in zb]
        zms, zspread = time_layer(torch, rt, bank, P, zd, rows, args.steps, args.warmup, P.MODE_A)
        extras["zipf_w8"] = {"layer_us": round(zms * 1000, 2), "spread_us": zspread,
                             "avg_unique_experts": float(np.mean([u for u, _ in zs])),
                             "GB/s": round(float(np.mean([b for _, b in zs])) / (zms * 1e-3) / 1e9, 1),
                             "zipf_s": WL.ZIPF_S, "zipf_kappa": WL.ZIPF_KAPPA,
                             "placement_histogram": placement_histogram(np.concatenate([s for _, s, _ in zb]))}
        bms, bspread = time_layer(torch, rt, bank, P, dev_batches, rows, args.steps, args.warmup, P.MODE_B)
        extras["mode_b_w8"] = {"layer_us": round(bms * 1000, 2), "spread_us": bspread,
                               "GB/s": round(avg_bytes / (bms * 1e-3) / 1e9, 1)}
        b1 = build_batches(P, WL, args.batches, 1, zipf=False)
        d1 = upload(torch, WL, b1)
        s1 = [step_bytes(sel, 1) for _, sel, _ in b1]
        ms1, spread1 = time_layer(torch, rt, bank, P, d1, 1, args.steps, args.warmup, P.MODE_A)
        kt1 = kernel_times(torch, rt, bank, P, d1, 1, max(20, args.steps // 4), P.MODE_A)
        extras["w1"] = {"layer_us": round(ms1 * 1000, 2), "spread_us": spread1,
                        "GB/s": round(float(np.mean([b for _, b in s1])) / (ms1 * 1e-3) / 1e9, 1),
                        "kernels_us": {k: round(v["avg_us"], 2) for k, v in kt1.items()}}
        for zipf in (False, True):
            extras["prefill_t2048" + ("_zipf" if zipf else "")] = prefill_leg(torch, rt, bank, P, WL, zipf)
        extras["router_w8"] = router_leg(torch, rt, P, WL)
        extras["layer_plus_router_w8"] = layer_with_router(torch, rt, bank, P, WL)
        extras["layer_plus_router_w8_two_calls"] = layer_with_router(torch, rt, bank, P, WL, two_calls=True)
        extras["layer_plus_router_w1"] = layer_with_router(torch, rt, bank, P, WL, rows=1)
        extras.update(projection_legs(torch, rt, bank, P, WL))
        for k, v in extras.items():
            if isinstance(v, dict) and k != "kernels_us":
                log(f"{k}: {v}")

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on a bounded sample")
        cpu = cpu_baseline(WL, bank, batches[0])
        log(f"cpu baseline {cpu['value']:.3f} GB/s, {cpu['layer_ms']} ms per layer ({cpu['sample']}); "
            f"scalar oracle {cpu['scalar_oracle']}")
        if "mode_b_w8" in extras:
            extras["mode_b_w8"]["cpu_baseline"] = cpu["mode_b"]
        if "prefill_t2048" in extras:
            log("timing the mode-B CPU path on a sample of the 2048-token prefill")
            extras["prefill_t2048"]["cpu_baseline"] = cpu_prefill_baseline(WL, bank)
            log(f"prefill cpu baseline {extras['prefill_t2048']['cpu_baseline']}")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 x bf16 (f32 acc)",
        "data": "synthetic (seeded; weights, scales, activations, router)",
        "config": {"workload": "routed-MoE decode layer, 8 token rows, top-8 of 256 experts, hidden 4096, "
                               f"intermediate 2048, block-FP8 128x128, mode A, {args.routing} routing",
                   "rows": rows, "experts": 256, "top_k": 8, "hidden": 4096, "intermediate": 2048,
                   "routing": "routes computed before the timed steps and resident in HBM; the device router is "
                              "timed alone (extras.router_w8) and with the layer (extras.layer_plus_router_w8)"},
        "roofline": roofline, "cpu_baseline": cpu, "extras": extras,
    }
    print(json.dumps(line), flush=True)
    rt.close()


if __name__ == "__main__":
    main()
