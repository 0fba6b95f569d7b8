"""Host mirror of WideMetalMoeRuntime (src/wide_metal_moe.rs:113-1315) over the C ABI.

Host-memory calls (``execute_fp8_linear``, ``execute``) take and return numpy f32 arrays like the
reference takes and returns ``&[f32]`` / ``Vec<f32>``. Device-memory calls take torch tensors (or
raw device addresses) and enqueue on the runtime's HIP stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Iterable, Optional, Sequence

import numpy as np

from . import _abi
from ._abi import (DTYPE_BF16, DTYPE_F32, LAYOUT_FULL_QKV_TP4, LAYOUT_PLAIN, LAYOUT_SWA_QKV_TP4,
                   MODE_A, MODE_B, check, lib)


def _ptr(t) -> int:
    """Device address of a torch tensor, or an int address as given."""
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return int(t.data_ptr())


def _region(arr: np.ndarray) -> _abi.Region:
    return _abi.Region(arr.ctypes.data, arr.nbytes, 0, arr.nbytes)


@dataclass
class WideLinearExecution:
    output: np.ndarray
    wall_ms: float
    mapped_source_bytes: int
    resident_source_bytes: int


@dataclass
class WideMoeExecution:
    output: np.ndarray
    wall_ms: float
    unique_experts: int
    expert_rows: int
    mapped_source_bytes: int
    resident_source_bytes: int


class Projection:
    """An FP8 weight and its 128x128 f32 scale grid bound into HBM."""

    def __init__(self, handle: int, rows: int, columns: int, layout: int = LAYOUT_PLAIN):
        self.handle = handle
        self.rows = rows
        self.columns = columns
        self.layout = layout

    def release(self):
        if self.handle:
            lib().pw_projection_release(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


@dataclass
class WideExpertBinding:
    """WideExpertBinding (src/wide_metal_moe.rs:88-95)."""
    expert: int
    positions: Sequence[int]
    route_weights: Sequence[float]
    gate: Projection
    up: Projection
    down: Projection


class ExpertBank:
    def __init__(self, handle: int, n_experts: int, hidden: int, intermediate: int, keep=None):
        self.handle = handle
        self.n_experts = n_experts
        self.hidden = hidden
        self.intermediate = intermediate
        self._keep = keep

    def release(self):
        if self.handle:
            lib().pw_expert_bank_release(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Safetensors:
    """A safetensors file mapped read-only with its header parsed (MappedSafetensors, src/lib.rs:783-972)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().pw_safetensors_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value
        self.path = str(path)

    def __len__(self) -> int:
        return int(lib().pw_safetensors_count(self.handle))

    def tensor(self, name: str):
        """(dtype, shape, bytes) of one tensor; the bytes are a copy of the mapped payload."""
        info = _abi.TensorInfo()
        check(lib().pw_safetensors_tensor(self.handle, name.encode(), ctypes.byref(info)))
        shape = tuple(int(info.shape[i]) for i in range(info.rank))
        data = ctypes.string_at(info.region.bytes, info.region.tensor_bytes)
        return info.dtype.decode(), shape, data

    def close(self):
        if self.handle:
            lib().pw_safetensors_close(self.handle)
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WideMoeRuntime:
    """One runtime per device; calls are serialised by the caller like the reference's &self."""

    def __init__(self, device: int = 0, fused_gate_up: bool = False):
        h = ctypes.c_void_p()
        check(lib().pw_runtime_create(device, _abi.RUNTIME_FUSED_GATE_UP if fused_gate_up else 0,
                                      ctypes.byref(h)))
        self.handle = h.value
        self.device = device
        self.fused_gate_up = fused_gate_up

    # WideMetalMoeRuntime::compile / compile_with_fused_gate_up (src/wide_metal_moe.rs:164-171)
    @classmethod
    def compile(cls, device: int = 0) -> "WideMoeRuntime":
        return cls(device, False)

    @classmethod
    def compile_with_fused_gate_up(cls, device: int = 0) -> "WideMoeRuntime":
        return cls(device, True)

    def close(self):
        if self.handle:
            lib().pw_runtime_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        return lib().pw_runtime_stream(self.handle) or 0

    def enable_timing(self, max_launches: int):
        check(lib().pw_runtime_enable_timing(self.handle, max_launches))

    def timing(self, kernel: str):
        """(launches, total_ms) recorded with HIP events for `kernel` since the last reset."""
        n = ctypes.c_uint32(0)
        ms = ctypes.c_double(0.0)
        check(lib().pw_runtime_timing_summary(self.handle, kernel.encode(), ctypes.byref(n), ctypes.byref(ms)))
        return n.value, ms.value

    def reset_timing(self):
        check(lib().pw_runtime_timing_reset(self.handle))

    def take_flags(self) -> int:
        f = ctypes.c_uint32(0)
        check(lib().pw_runtime_take_flags(self.handle, ctypes.byref(f)))
        return f.value

    # ------------------------------------------------------------------ binding
    def bind_projection(self, weight: np.ndarray, scale: np.ndarray, layout: int = LAYOUT_PLAIN,
                        scan_codes: bool = True) -> Projection:
        w = np.ascontiguousarray(weight, dtype=np.uint8)
        s = np.ascontiguousarray(scale, dtype=np.float32)
        if w.ndim != 2:
            raise ValueError("weight must be [rows, columns]")
        desc = _abi.ProjectionDesc(_region(w), _region(s), w.shape[0], w.shape[1], layout, 0)
        h = ctypes.c_void_p()
        check(lib().pw_projection_bind(self.handle, ctypes.byref(desc), int(scan_codes), ctypes.byref(h)))
        return Projection(h.value, w.shape[0], w.shape[1], layout)

    def bind_segments(self, segments: Iterable, scan_codes: bool = True) -> Projection:
        segs = [(np.ascontiguousarray(w, np.uint8), np.ascontiguousarray(s, np.float32)) for w, s in segments]
        columns = segs[0][0].shape[1]
        arr = (_abi.SegmentDesc * len(segs))()
        for i, (w, s) in enumerate(segs):
            arr[i] = _abi.SegmentDesc(_region(w), _region(s), w.shape[0])
        h = ctypes.c_void_p()
        check(lib().pw_projection_bind_segments(self.handle, arr, len(segs), columns, int(scan_codes),
                                                ctypes.byref(h)))
        return Projection(h.value, sum(w.shape[0] for w, _ in segs), columns)

    def bind_projection_device(self, weight, scale, rows: int, columns: int) -> Projection:
        h = ctypes.c_void_p()
        check(lib().pw_projection_bind_device(self.handle, _ptr(weight), _ptr(scale), rows, columns,
                                              ctypes.byref(h)))
        return Projection(h.value, rows, columns)

    def expert_bank_from_safetensors(self, files: Sequence["Safetensors"], layer: int, n_experts: int,
                                     hidden: int, intermediate: int, scan_codes: bool = True) -> ExpertBank:
        """One layer's routed experts from checkpoint files, copied once into a device bank it owns."""
        arr = (ctypes.c_void_p * len(files))(*[f.handle for f in files])
        h = ctypes.c_void_p()
        check(lib().pw_expert_bank_from_safetensors(self.handle, arr, len(files), layer, n_experts, hidden,
                                                    intermediate, int(scan_codes), ctypes.byref(h)))
        return ExpertBank(h.value, n_experts, hidden, intermediate)

    def bind_bf16(self, weight: np.ndarray) -> Projection:
        """A checkpoint BF16 weight [rows, columns] (uint16 bits) copied into HBM once."""
        w = np.ascontiguousarray(weight, dtype=np.uint16)
        if w.ndim != 2:
            raise ValueError("weight must be [rows, columns]")
        h = ctypes.c_void_p()
        check(lib().pw_bf16_bind(self.handle, ctypes.byref(_region(w)), w.shape[0], w.shape[1], ctypes.byref(h)))
        return Projection(h.value, w.shape[0], w.shape[1])

    def bind_bf16_device(self, weight, rows: int, columns: int) -> Projection:
        h = ctypes.c_void_p()
        check(lib().pw_bf16_bind_device(self.handle, _ptr(weight), rows, columns, ctypes.byref(h)))
        return Projection(h.value, rows, columns)

    def expert_bank(self, gates: Sequence[Projection], ups: Sequence[Projection],
                    downs: Sequence[Projection]) -> ExpertBank:
        n = len(gates)
        g = (ctypes.c_void_p * n)(*[p.handle for p in gates])
        u = (ctypes.c_void_p * n)(*[p.handle for p in ups])
        d = (ctypes.c_void_p * n)(*[p.handle for p in downs])
        h = ctypes.c_void_p()
        check(lib().pw_expert_bank_create(self.handle, n, g, u, d, ctypes.byref(h)))
        return ExpertBank(h.value, n, gates[0].columns, gates[0].rows, keep=(gates, ups, downs))

    # ---------------------------------------------------------- host-memory calls
    def execute_fp8_linear(self, input: np.ndarray, binding: Projection, full_qkv_layout: bool = False,
                           mode: int = MODE_B) -> WideLinearExecution:
        """execute_fp8_linear (src/wide_metal_moe.rs:241-385); mode B is the reference's mode."""
        if full_qkv_layout and binding.layout != LAYOUT_FULL_QKV_TP4:
            raise _abi.PwError(-2, "wide FP8 linear layout mismatch")
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        if x.shape[1] != binding.columns:
            raise _abi.PwError(-1, "wide row shape mismatch")
        rows = x.shape[0]
        out = np.zeros((rows, binding.rows), np.float32)
        st = _abi.LinearStats()
        check(lib().pw_fp8_linear(self.handle, mode, x.ctypes.data_as(_abi._f32p), rows, binding.handle,
                                  out.ctypes.data_as(_abi._f32p), ctypes.byref(st)))
        return WideLinearExecution(out, st.wall_ms, st.mapped_source_bytes, st.resident_source_bytes)

    def execute_bf16_linear(self, input: np.ndarray, binding: Projection) -> WideLinearExecution:
        """execute_bf16_linear (src/wide_metal_moe.rs:728-834): f32 rows -> bf16-rounded f32."""
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        if x.shape[1] != binding.columns:
            raise _abi.PwError(-1, "wide row shape mismatch")
        rows = x.shape[0]
        out = np.zeros((rows, binding.rows), np.float32)
        st = _abi.LinearStats()
        check(lib().pw_bf16_linear(self.handle, x.ctypes.data_as(_abi._f32p), rows, binding.handle,
                                   out.ctypes.data_as(_abi._f32p), ctypes.byref(st)))
        return WideLinearExecution(out, st.wall_ms, st.mapped_source_bytes, st.resident_source_bytes)

    def execute(self, input: np.ndarray, experts: Sequence[WideExpertBinding],
                mode: int = MODE_B) -> WideMoeExecution:
        """execute (src/wide_metal_moe.rs:836-842); mode B is the reference's mode."""
        return self._execute(input, experts, mode, False)

    def execute_fused_gate_up(self, input: np.ndarray, experts: Sequence[WideExpertBinding],
                              mode: int = MODE_B) -> WideMoeExecution:
        """execute_fused_gate_up (src/wide_metal_moe.rs:844-850)."""
        return self._execute(input, experts, mode, True)

    def _execute(self, input, experts, mode, fused):
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        rows, hidden = x.shape
        arr = (_abi.ExpertBindingC * len(experts))()
        keep = []
        for i, b in enumerate(experts):
            pos = np.ascontiguousarray(b.positions, dtype=np.uint32)
            w = np.ascontiguousarray(b.route_weights, dtype=np.float32)
            keep += [pos, w]
            arr[i] = _abi.ExpertBindingC(b.expert, len(pos), pos.ctypes.data_as(_abi._u32p),
                                         w.ctypes.data_as(_abi._f32p), b.gate.handle, b.up.handle,
                                         b.down.handle)
        out = np.zeros((rows, hidden), np.float32)
        st = _abi.MoeStats()
        check(lib().pw_moe_execute(self.handle, mode, int(fused), x.ctypes.data_as(_abi._f32p), rows, arr,
                                   len(experts), out.ctypes.data_as(_abi._f32p), ctypes.byref(st)))
        del keep
        return WideMoeExecution(out, st.wall_ms, st.unique_experts, st.expert_rows,
                                st.mapped_source_bytes, st.resident_source_bytes)

    # -------------------------------------------------------- device-memory calls
    def fp8_linear_device(self, proj: Projection, x, rows: int, out, mode: int = MODE_A,
                          x_dtype: int = DTYPE_BF16, out_dtype: int = DTYPE_F32, round_output: bool = True,
                          stream: Optional[int] = None):
        check(lib().pw_fp8_linear_device(self.handle, mode, _ptr(x), x_dtype, rows, proj.handle, _ptr(out),
                                         out_dtype, int(round_output), stream or 0))

    def bf16_linear_device(self, proj: Projection, x, rows: int, out, x_dtype: int = DTYPE_F32,
                           out_dtype: int = DTYPE_F32, round_output: bool = True, stream: Optional[int] = None):
        check(lib().pw_bf16_linear_device(self.handle, _ptr(x), x_dtype, rows, proj.handle, _ptr(out), out_dtype,
                                          int(round_output), stream or 0))

    def quantize_fp8_group128_device(self, x, rows: int, cols: int, codes, scales,
                                     x_dtype: int = DTYPE_F32, stream: Optional[int] = None):
        """dynamic_fp8_quantized_group128 on device rows -> codes [rows, cols], scales [rows, cols/128]."""
        check(lib().pw_quantize_fp8_group128_device(self.handle, _ptr(x), x_dtype, rows, cols, _ptr(codes),
                                                    _ptr(scales), stream or 0))

    def swiglu_staged_device(self, gate, up, count: int, out, form: int = 0, stream: Optional[int] = None):
        """bf16_staged_swiglu on device f32 arrays; form 0 evaluates the silu in place (the decode
        kernels' form), form 1 looks it up in the runtime's table (the prefill kernels' form)."""
        check(lib().pw_swiglu_staged_device(self.handle, _ptr(gate), _ptr(up), count, _ptr(out), form,
                                            stream or 0))

    def moe_layer_device(self, bank: ExpertBank, x, rows: int, route_ids, route_weights, out,
                         mode: int = MODE_A, x_dtype: int = DTYPE_BF16, out_dtype: int = DTYPE_BF16,
                         stream: Optional[int] = None):
        check(lib().pw_moe_layer_device(self.handle, bank.handle, mode, _ptr(x), x_dtype, rows,
                                        _ptr(route_ids), _ptr(route_weights), _ptr(out), out_dtype,
                                        stream or 0))

    def moe_layer_routed_device(self, bank: ExpertBank, x, rows: int, router_weight, bias, route_ids, route_weights,
                                out, mode: int = MODE_A, x_dtype: int = DTYPE_BF16, w_dtype: int = DTYPE_BF16,
                                out_dtype: int = DTYPE_BF16, stream: Optional[int] = None):
        """route_mlp over the bank's experts, then the routed layer on those routes (one call); the
        routes are also written to route_ids / route_weights [rows x 8]."""
        check(lib().pw_moe_layer_routed_device(self.handle, bank.handle, mode, _ptr(x), x_dtype, rows,
                                               _ptr(router_weight), w_dtype, _ptr(bias), _ptr(route_ids),
                                               _ptr(route_weights), _ptr(out), out_dtype, stream or 0))

    def moe_layer_device_noalloc(self, bank: ExpertBank, x, rows: int, route_ids, route_weights, out,
                                 mode: int = MODE_A, x_dtype: int = DTYPE_BF16, out_dtype: int = DTYPE_BF16,
                                 stream: Optional[int] = None):
        """moe_layer_device on the library's static scratch (no device allocation): rows <= 8."""
        check(lib().pw_moe_layer_device_noalloc(self.handle, bank.handle, mode, _ptr(x), x_dtype, rows,
                                                _ptr(route_ids), _ptr(route_weights), _ptr(out), out_dtype,
                                                stream or 0))

    def moe_prefill_device(self, bank: ExpertBank, x, rows: int, route_ids, route_weights, out,
                           x_dtype: int = DTYPE_BF16, out_dtype: int = DTYPE_BF16, stream: Optional[int] = None):
        """Mode B routed-MoE layer over up to 4096 token rows (grouped FP8 GEMM), device buffers."""
        check(lib().pw_moe_prefill_device(self.handle, bank.handle, _ptr(x), x_dtype, rows, _ptr(route_ids),
                                          _ptr(route_weights), _ptr(out), out_dtype, stream or 0))

    def moe_schedule_device(self, bank: ExpertBank, rows: int, route_ids, route_weights, expert_offsets,
                            positions, weights, row_slots, stream: Optional[int] = None):
        """The device routed schedule: expert_offsets [E + 1], positions / weights / row_slots [rows x 8]."""
        check(lib().pw_moe_schedule_device(self.handle, bank.handle, _ptr(route_ids), _ptr(route_weights), rows,
                                           _ptr(expert_offsets), _ptr(positions), _ptr(weights), _ptr(row_slots),
                                           stream or 0))

    def route_device(self, x, rows: int, hidden: int, router_weight, experts: int, bias, route_ids, route_weights,
                     x_dtype: int = DTYPE_BF16, w_dtype: int = DTYPE_BF16, scores=None, tie_rows=None,
                     stream: Optional[int] = None):
        """route_mlp on device buffers -> route_ids / route_weights [rows x 8] (and scores)."""
        check(lib().pw_route_device(self.handle, _ptr(x), x_dtype, rows, hidden, _ptr(router_weight), w_dtype,
                                    experts, _ptr(bias), _ptr(route_ids), _ptr(route_weights),
                                    _ptr(scores) if scores is not None else None,
                                    _ptr(tie_rows) if tie_rows is not None else None, stream or 0))

    def expert_forward_device(self, bank: ExpertBank, expert: int, x, rows: int, out, mode: int = MODE_A,
                              x_dtype: int = DTYPE_BF16, out_dtype: int = DTYPE_BF16,
                              stream: Optional[int] = None):
        check(lib().pw_expert_forward_device(self.handle, bank.handle, expert, mode, _ptr(x), x_dtype, rows,
                                             _ptr(out), out_dtype, stream or 0))

    # ------------------------------------------------------------ synthetic data
    def synth_scales(self, scales, count: int, seed: int, log2_lo: float = -10.0, log2_hi: float = -6.0):
        check(lib().pw_synth_scales(self.handle, _ptr(scales), count, seed, log2_lo, log2_hi))

    def synth_fp8(self, w, scales, rows: int, cols: int, seed: int):
        check(lib().pw_synth_fp8(self.handle, _ptr(w), _ptr(scales), rows, cols, seed))

    def synth_normal_bf16(self, x, count: int, seed: int, stddev: float = 1.0):
        check(lib().pw_synth_normal_bf16(self.handle, _ptr(x), count, seed, stddev))


# ------------------------------------------------------------------ routing (host)
def topk_unsorted(values: np.ndarray, top_k: int = 8) -> np.ndarray:
    """pw_pytorch_topk_unsorted_f32 (src/pytorch_topk.cpp:8-30), libc++ nth_element order."""
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(top_k, np.uint32)
    rc = lib().pw_pytorch_topk_unsorted_f32(v.ctypes.data_as(_abi._f32p), v.size, top_k,
                                            out.ctypes.data_as(_abi._u32p))
    if rc != 0:
        raise _abi.PwError(-1, f"top-k failed ({rc})")
    return out


def noaux_routes(scores: np.ndarray, bias: np.ndarray):
    """pytorch_noaux_routes (src/text_endpoint.rs:4394-4473) -> (selected, weights, tie_rows)."""
    s = np.ascontiguousarray(np.atleast_2d(scores), np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    rows, experts = s.shape
    sel = np.zeros((rows, 8), np.uint32)
    w = np.zeros((rows, 8), np.float32)
    ties = ctypes.c_uint64(0)
    check(lib().pw_noaux_routes(s.ctypes.data_as(_abi._f32p), b.ctypes.data_as(_abi._f32p), rows, experts,
                                sel.ctypes.data_as(_abi._u32p), w.ctypes.data_as(_abi._f32p), ctypes.byref(ties)))
    return sel, w, ties.value


def route_from_logits(logits: np.ndarray, bias: np.ndarray):
    """route_mlp after the router GEMM (src/text_endpoint.rs:4342-4380) -> (scores, selected, weights, ties)."""
    lg = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    rows, experts = lg.shape
    scores = np.zeros_like(lg)
    sel = np.zeros((rows, 8), np.uint32)
    w = np.zeros((rows, 8), np.float32)
    ties = ctypes.c_uint64(0)
    check(lib().pw_route_from_logits(lg.ctypes.data_as(_abi._f32p), b.ctypes.data_as(_abi._f32p), rows, experts,
                                     scores.ctypes.data_as(_abi._f32p), sel.ctypes.data_as(_abi._u32p),
                                     w.ctypes.data_as(_abi._f32p), ctypes.byref(ties)))
    return scores, sel, w, ties.value


def full_qkv_source_row(r: int) -> int:
    return lib().pw_full_qkv_source_row(r)


def full_qkv_scale_row(r: int) -> int:
    return lib().pw_full_qkv_scale_row(r)


def swa_qkv_source_row(r: int) -> int:
    return lib().pw_swa_qkv_source_row(r)
