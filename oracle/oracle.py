"""ctypes loader for the C oracle (test infrastructure only).

Only the tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` import this
module. It is the checker that the HIP product path is compared against and never part of it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libpw_oracle.so")
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_sz = ctypes.c_size_t


class PwoExpert(ctypes.Structure):
    _fields_ = [
        ("gate_w", _u8p), ("gate_s", _f32p),
        ("up_w", _u8p), ("up_s", _f32p),
        ("down_w", _u8p), ("down_s", _f32p),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.pwo_decode_e4m3fn.argtypes = [ctypes.c_uint8]
        L.pwo_decode_e4m3fn.restype = ctypes.c_float
        L.pwo_round_bf16.argtypes = [ctypes.c_float]
        L.pwo_round_bf16.restype = ctypes.c_float
        L.pwo_encode_e4m3fn.argtypes = [ctypes.c_float, _u8p]
        L.pwo_encode_e4m3fn.restype = ctypes.c_int
        L.pwo_sleef_expf_u10.argtypes = [ctypes.c_float]
        L.pwo_sleef_expf_u10.restype = ctypes.c_float
        L.pwo_sigmoid_f32.argtypes = [ctypes.c_float]
        L.pwo_sigmoid_f32.restype = ctypes.c_float
        L.pwo_dynamic_fp8.argtypes = [_f32p, _sz, _sz, _u8p, _f32p, _f32p]
        L.pwo_gemm_mode_a.argtypes = [_u8p, _f32p, _sz, _sz, _f32p, _sz, _f32p]
        L.pwo_gemm_mode_b_equation.argtypes = [_u8p, _f32p, _sz, _sz, _u8p, _f32p, _sz, _f32p]
        L.pwo_fp8_linear_mode_b.argtypes = [_u8p, _f32p, _sz, _sz, _f32p, _sz, _f32p]
        L.pwo_bf16_linear.argtypes = [_u16p, _sz, _sz, _f32p, _sz, _f32p, _f32p]
        L.pwo_swiglu_f32.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.pwo_swiglu_f32.restype = None
        L.pwo_swiglu_bf16_staged.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.pwo_swiglu_bf16_staged.restype = None
        L.pwo_topk_unsorted.argtypes = [_f32p, _sz, _sz, _u32p]
        L.pwo_noaux_routes.argtypes = [_f32p, _f32p, _sz, _sz, _u32p, _f32p, _u64p]
        L.pwo_router_logits_t256.argtypes = [_f32p, _sz, _f32p, _sz, _sz, _f32p]
        L.pwo_router_logits_t256.restype = None
        L.pwo_route.argtypes = [_f32p, _sz, _f32p, _f32p, _sz, _sz, _f32p, _f32p, _u32p, _f32p, _u64p]
        for name in ("pwo_moe_layer_mode_a", "pwo_moe_layer_mode_b"):
            getattr(L, name).argtypes = [_f32p, _sz, _sz, _sz, ctypes.POINTER(PwoExpert), _sz,
                                         _u32p, _f32p, _sz, _f32p, _f32p]
        L.pwo_expert_mode_a.argtypes = [_f32p, _sz, _sz, _sz, ctypes.POINTER(PwoExpert), _f32p, _f32p]
        for name in ("pwo_full_qkv_source_row", "pwo_full_qkv_scale_row", "pwo_swa_qkv_source_row"):
            getattr(L, name).argtypes = [ctypes.c_int64]
            getattr(L, name).restype = ctypes.c_int64
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def decode_e4m3fn(b: int) -> float:
    return lib().pwo_decode_e4m3fn(b)


def round_bf16(v: float) -> float:
    return lib().pwo_round_bf16(v)


def encode_e4m3fn(v: float):
    out = ctypes.c_uint8(0)
    rc = lib().pwo_encode_e4m3fn(v, ctypes.byref(out))
    return None if rc != 0 else out.value


def sleef_expf_u10(v: float) -> float:
    return lib().pwo_sleef_expf_u10(v)


def sigmoid_f32(v: float) -> float:
    return lib().pwo_sigmoid_f32(v)


def dynamic_fp8(x: np.ndarray):
    x = _c(x, np.float32)
    rows, cols = x.shape
    codes = np.zeros((rows, cols), np.uint8)
    scales = np.zeros((rows, cols // 128), np.float32)
    deq = np.zeros((rows, cols), np.float32)
    rc = lib().pwo_dynamic_fp8(_p(x, _f32p), rows, cols, _p(codes, _u8p), _p(scales, _f32p), _p(deq, _f32p))
    if rc != 0:
        raise ValueError(f"dynamic_fp8 failed: {rc}")
    return codes, scales, deq


def gemm_mode_a(w: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = _c(w, np.uint8); s = _c(s, np.float32); x = _c(np.atleast_2d(x), np.float32)
    n, k = w.shape
    y = np.zeros((x.shape[0], n), np.float32)
    rc = lib().pwo_gemm_mode_a(_p(w, _u8p), _p(s, _f32p), n, k, _p(x, _f32p), x.shape[0], _p(y, _f32p))
    if rc != 0:
        raise ValueError(f"gemm_mode_a failed: {rc}")
    return y


def bf16_linear(w_bits: np.ndarray, x: np.ndarray, raw: bool = False):
    """W [n, k] bf16 bits (uint16), x [rows, k] f32 -> bf16-rounded y [rows, n] (and the raw sums)."""
    w = _c(w_bits, np.uint16); x = _c(np.atleast_2d(x), np.float32)
    n, k = w.shape
    y = np.zeros((x.shape[0], n), np.float32)
    y_raw = np.zeros_like(y)
    rc = lib().pwo_bf16_linear(_p(w, _u16p), n, k, _p(x, _f32p), x.shape[0], _p(y, _f32p), _p(y_raw, _f32p))
    if rc != 0:
        raise ValueError(f"bf16_linear failed: {rc}")
    return (y, y_raw) if raw else y


def gemm_mode_b_equation(w, s, q, a) -> np.ndarray:
    w = _c(w, np.uint8); s = _c(s, np.float32); q = _c(q, np.uint8); a = _c(a, np.float32)
    n, k = w.shape
    y = np.zeros((q.shape[0], n), np.float32)
    rc = lib().pwo_gemm_mode_b_equation(_p(w, _u8p), _p(s, _f32p), n, k, _p(q, _u8p), _p(a, _f32p),
                                        q.shape[0], _p(y, _f32p))
    if rc != 0:
        raise ValueError(f"gemm_mode_b_equation failed: {rc}")
    return y


def fp8_linear_mode_b(w, s, x) -> np.ndarray:
    w = _c(w, np.uint8); s = _c(s, np.float32); x = _c(np.atleast_2d(x), np.float32)
    n, k = w.shape
    y = np.zeros((x.shape[0], n), np.float32)
    rc = lib().pwo_fp8_linear_mode_b(_p(w, _u8p), _p(s, _f32p), n, k, _p(x, _f32p), x.shape[0], _p(y, _f32p))
    if rc != 0:
        raise ValueError(f"fp8_linear_mode_b failed: {rc}")
    return y


def swiglu_f32(g, u):
    g = _c(g, np.float32); u = _c(u, np.float32)
    out = np.zeros_like(g)
    lib().pwo_swiglu_f32(_p(g, _f32p), _p(u, _f32p), _p(out, _f32p), g.size)
    return out


def swiglu_bf16_staged(g, u):
    g = _c(g, np.float32); u = _c(u, np.float32)
    out = np.zeros_like(g)
    lib().pwo_swiglu_bf16_staged(_p(g, _f32p), _p(u, _f32p), _p(out, _f32p), g.size)
    return out


def topk_unsorted(values, k=8):
    v = _c(values, np.float32)
    sel = np.zeros(k, np.uint32)
    rc = lib().pwo_topk_unsorted(_p(v, _f32p), v.size, k, _p(sel, _u32p))
    if rc != 0:
        raise ValueError(f"topk failed: {rc}")
    return sel


def noaux_routes(scores, bias):
    scores = _c(np.atleast_2d(scores), np.float32); bias = _c(bias, np.float32)
    rows, experts = scores.shape
    sel = np.zeros((rows, 8), np.uint32)
    w = np.zeros((rows, 8), np.float32)
    ties = ctypes.c_uint64(0)
    rc = lib().pwo_noaux_routes(_p(scores, _f32p), _p(bias, _f32p), rows, experts, _p(sel, _u32p),
                                _p(w, _f32p), ctypes.byref(ties))
    if rc != 0:
        raise ValueError(f"noaux routes failed: {rc}")
    return sel, w, ties.value


def router_logits_t256(x, router_w):
    x = _c(np.atleast_2d(x), np.float32); r = _c(router_w, np.float32)
    out = np.zeros((x.shape[0], r.shape[0]), np.float32)
    lib().pwo_router_logits_t256(_p(x, _f32p), x.shape[0], _p(r, _f32p), r.shape[0], r.shape[1], _p(out, _f32p))
    return out


def route(x, router_w, bias):
    x = _c(np.atleast_2d(x), np.float32); r = _c(router_w, np.float32); b = _c(bias, np.float32)
    rows, experts, k = x.shape[0], r.shape[0], r.shape[1]
    logits = np.zeros((rows, experts), np.float32)
    scores = np.zeros((rows, experts), np.float32)
    sel = np.zeros((rows, 8), np.uint32)
    w = np.zeros((rows, 8), np.float32)
    ties = ctypes.c_uint64(0)
    rc = lib().pwo_route(_p(x, _f32p), rows, _p(r, _f32p), _p(b, _f32p), experts, k, _p(logits, _f32p),
                         _p(scores, _f32p), _p(sel, _u32p), _p(w, _f32p), ctypes.byref(ties))
    if rc != 0:
        raise ValueError(f"route failed: {rc}")
    return logits, scores, sel, w, ties.value


def _expert_array(experts: dict, n_experts: int):
    """experts: {id: (gate_w, gate_s, up_w, up_s, down_w, down_s)} numpy arrays."""
    arr = (PwoExpert * n_experts)()
    keep = []
    for e, (gw, gs, uw, us, dw, ds) in experts.items():
        t = [_c(gw, np.uint8), _c(gs, np.float32), _c(uw, np.uint8), _c(us, np.float32),
             _c(dw, np.uint8), _c(ds, np.float32)]
        keep.extend(t)
        arr[e] = PwoExpert(_p(t[0], _u8p), _p(t[1], _f32p), _p(t[2], _u8p), _p(t[3], _f32p),
                           _p(t[4], _u8p), _p(t[5], _f32p))
    return arr, keep


def moe_layer(mode: str, x, experts: dict, n_experts: int, selected, weights, hidden=None, inter=None,
              raw=False):
    """Routed MoE layer; returns the bf16-rounded output, plus the f32 combine when raw=True."""
    x = _c(np.atleast_2d(x), np.float32)
    rows = x.shape[0]
    hidden = hidden or x.shape[1]
    any_e = next(iter(experts.values()))
    inter = inter or any_e[0].shape[0]
    sel = _c(selected, np.uint32); w = _c(weights, np.float32)
    arr, keep = _expert_array(experts, n_experts)
    out = np.zeros((rows, hidden), np.float32)
    out_raw = np.zeros((rows, hidden), np.float32)
    fn = lib().pwo_moe_layer_mode_a if mode == "a" else lib().pwo_moe_layer_mode_b
    rc = fn(_p(x, _f32p), rows, hidden, inter, arr, n_experts, _p(sel, _u32p), _p(w, _f32p),
            sel.shape[1], _p(out, _f32p), _p(out_raw, _f32p))
    del keep
    if rc != 0:
        raise ValueError(f"moe_layer_mode_{mode} failed: {rc}")
    return (out, out_raw) if raw else out


def expert_mode_a(x, expert):
    x = _c(np.atleast_2d(x), np.float32)
    rows, hidden = x.shape
    arr, keep = _expert_array({0: expert}, 1)
    inter = expert[0].shape[0]
    out32 = np.zeros((rows, hidden), np.float32)
    outbf = np.zeros((rows, hidden), np.float32)
    rc = lib().pwo_expert_mode_a(_p(x, _f32p), rows, hidden, inter, arr, _p(out32, _f32p), _p(outbf, _f32p))
    del keep
    if rc != 0:
        raise ValueError(f"expert_mode_a failed: {rc}")
    return out32, outbf


def full_qkv_source_row(r: int) -> int:
    return lib().pwo_full_qkv_source_row(r)


def full_qkv_scale_row(r: int) -> int:
    return lib().pwo_full_qkv_scale_row(r)


def swa_qkv_source_row(r: int) -> int:
    return lib().pwo_swa_qkv_source_row(r)


# ------------------------------------------------------------------ the reference's CPU BLAS path
def decode_fp8_matrix_f32(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """f32 copy of a block-FP8 matrix, dec(w[r, c]) * s[r / 128, c / 128] rounded to f32
    (src/lib.rs:2003-2015; the reference makes these copies once, when it loads a layer)."""
    lut = np.array([decode_e4m3fn(b) for b in range(256)], np.float32)
    rows, cols = w.shape
    full = np.repeat(np.repeat(np.asarray(s, np.float32), 128, axis=0)[:rows], 128, axis=1)[:, :cols]
    return lut[w] * full


def expert_blas_f32(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """One expert on the reference's CPU BLAS path (src/lib.rs:5807-5850): f32 SGEMMs against the
    dequantised weights (x . G^T, x . U^T), silu(g) * u as g / (1 + exp(-g)) * u in f32, then
    h . D^T. Summation order is the BLAS library's, so this agrees with the mode-A layer to f32
    rounding, not bit for bit."""
    x = np.asarray(x, np.float32)
    g = x @ gate.T
    u = x @ up.T
    with np.errstate(over="ignore"):
        h = (g / (np.float32(1.0) + np.exp(-g))) * u
    return h @ down.T


def moe_layer_blas(x: np.ndarray, dequantised: dict, selected: np.ndarray, weights: np.ndarray,
                   pool=None) -> np.ndarray:
    """The reference's CPU BLAS routed layer (src/lib.rs:5807-5862) over f32-dequantised experts
    {id: (gate, up, down)}: per expert in ascending id, gather its token rows in ascending order,
    run expert_blas_f32, and add y * route weight into the f32 block. With a thread pool the experts
    run concurrently and are still combined in ascending id, so the block is the same either way."""
    x = np.asarray(x, np.float32)
    selected = np.asarray(selected)
    rows = x.shape[0]
    plan = []
    for e in sorted(set(selected.reshape(-1).tolist())):
        pos, slot = np.nonzero(selected == e)
        order = np.argsort(pos, kind="stable")
        plan.append((e, pos[order], np.asarray(weights, np.float32)[pos[order], slot[order]]))

    def run(item):
        e, pos, _ = item
        return expert_blas_f32(x[pos], *dequantised[e])

    outs = list(pool.map(run, plan)) if pool is not None else [run(p) for p in plan]
    block = np.zeros((rows, x.shape[1]), np.float32)
    for (e, pos, wts), y in zip(plan, outs):
        for l, p in enumerate(pos.tolist()):
            block[p] = block[p] + y[l] * wts[l]
    return block


def _round_bf16_np(v: np.ndarray) -> np.ndarray:
    """round_bf16 (src/text_endpoint.rs:2960-2971) on a finite f32 array."""
    b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def fp8_linear_blas(x: np.ndarray, dequantised_w: np.ndarray) -> np.ndarray:
    """fp8_linear (src/text_endpoint.rs:3053-3108) against an f32-dequantised weight: the dynamic
    FP8 activations' dequantised values (dynamic_fp8, the C restatement of :3008-3051), one f32
    SGEMM (the BLAS library's summation order), every output rounded to bf16."""
    _, _, deq = dynamic_fp8(np.asarray(x, np.float32))
    return _round_bf16_np(deq @ dequantised_w.T)


def expert_blas_mode_b(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """One expert of routed_mlp_traced (src/text_endpoint.rs:5290-5381) on BLAS: fp8_linear gate and
    up, the bf16-staged SwiGLU (:5336-5343, the C restatement), fp8_linear down."""
    g = fp8_linear_blas(x, gate)
    u = fp8_linear_blas(x, up)
    return fp8_linear_blas(swiglu_bf16_staged(g, u), down)


def moe_layer_blas_mode_b(x: np.ndarray, dequantised: dict, selected: np.ndarray, weights: np.ndarray,
                          pool=None):
    """routed_mlp_traced (src/text_endpoint.rs:5290-5381) over f32-dequantised experts: experts in
    ascending id, each on its token rows in ascending order (expert_blas_mode_b), out[pos] += y * w in
    f32, bf16 at the end. Returns (bf16-rounded output, the f32 block). With a thread pool the experts
    run concurrently and are still combined in ascending id."""
    x = np.asarray(x, np.float32)
    selected = np.asarray(selected)
    plan = []
    for e in sorted(set(selected.reshape(-1).tolist())):
        pos, slot = np.nonzero(selected == e)
        order = np.argsort(pos, kind="stable")
        plan.append((e, pos[order], np.asarray(weights, np.float32)[pos[order], slot[order]]))

    def run(item):
        e, pos, _ = item
        return expert_blas_mode_b(x[pos], *dequantised[e])

    outs = list(pool.map(run, plan)) if pool is not None else [run(p) for p in plan]
    block = np.zeros((x.shape[0], x.shape[1]), np.float32)
    for (e, pos, wts), y in zip(plan, outs):
        for l, p in enumerate(pos.tolist()):
            block[p] = block[p] + y[l] * wts[l]
    return _round_bf16_np(block), block
