"""CPU tests of the C-ABI library: it loads, exports every declared entry point, and its host-side
routing and layout code matches the golden vectors and the oracle. No GPU compute is called."""
import ctypes
import json
import os
import re

import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pwfp8.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pw_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    declared = header_functions()
    assert len(declared) >= 25
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_abi.SIGNATURES) == declared
    assert lib.pw_abi_version() == 1


def test_runtime_create_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    rc = _abi.lib().pw_runtime_create(0, 0, ctypes.byref(h))
    assert rc == -5 and h.value is None
    assert _abi.lib().pw_last_error()


def test_null_arguments_are_rejected():
    lib = _abi.lib()
    assert lib.pw_runtime_create(0, 0, None) == -1
    assert lib.pw_fp8_linear(None, 0, None, 1, None, None, None) == -1
    assert lib.pw_moe_execute(None, 0, 0, None, 1, None, 0, None, None) == -1


def _load(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


def _f32(bits):
    return np.array([b & 0xFFFFFFFF for b in bits], np.uint32).view(np.float32)


def test_product_topk_matches_golden_orders(golden_dir):
    fx = _load(golden_dir, "pw0063-topk-order.json")
    assert P.topk_unsorted(_f32(fx["corrected_f32_u32"])).tolist() == fx["selected_experts"]
    ties = _load(golden_dir, "pw0157-pytorch-topk-ties.json")
    for case in ties["cases"]:
        assert P.topk_unsorted(_f32(case["corrected_f32_u32"])).tolist() == case["selected_experts"]


def _ref_topk(values, count, top_k, out):
    """Calls the library through the reference's own FFI name and signature (src/text_endpoint.rs:
    2466-2474): (*const f32, usize, usize, *mut u32) -> i32."""
    fn = _abi.lib().pw_pytorch_topk_unsorted_f32
    return fn(values, ctypes.c_size_t(count), ctypes.c_size_t(top_k), out)


def test_reference_topk_symbol_return_codes():
    """src/pytorch_topk.cpp:7-30: -1 for a null values or selected pointer, top_k == 0 or
    top_k >= count; -2 when the (value, index) buffer cannot be made; 0 otherwise."""
    v = np.arange(16, dtype=np.float32)
    out = np.full(16, 0xDEADBEEF, np.uint32)
    vp, op = v.ctypes.data_as(_abi._f32p), out.ctypes.data_as(_abi._u32p)
    assert _ref_topk(None, 16, 4, op) == -1
    assert _ref_topk(vp, 16, 4, None) == -1
    assert _ref_topk(vp, 16, 0, op) == -1
    assert _ref_topk(vp, 16, 16, op) == -1
    assert _ref_topk(vp, 16, 17, op) == -1
    assert _ref_topk(vp, 0, 1, op) == -1
    assert (out == 0xDEADBEEF).all()  # rejected calls write nothing
    # 2^62 pairs exceed std::vector's max_size: the library throws inside and returns -2 before it
    # reads a single value (the reference's vector<pair<float, int64_t>>(count) throws the same way)
    assert _ref_topk(vp, 1 << 62, 8, op) == -2
    assert (out == 0xDEADBEEF).all()
    assert _ref_topk(vp, 16, 15, op) == 0
    assert sorted(out[:15].tolist()) == list(range(1, 16))
    assert out[15] == 0xDEADBEEF  # only top_k indices are written


def test_reference_topk_symbol_golden_orders_and_any_k(golden_dir):
    """The reference's name gives the libc++ partition orders of pw0063 and pw0157; for other k the
    selected set is the k largest values (brute force) and the order is the oracle's nth_element."""
    def call(v, k):
        v = np.ascontiguousarray(v, np.float32)
        out = np.zeros(k, np.uint32)
        assert _ref_topk(v.ctypes.data_as(_abi._f32p), v.size, k, out.ctypes.data_as(_abi._u32p)) == 0
        return out

    fx = _load(golden_dir, "pw0063-topk-order.json")
    assert call(_f32(fx["corrected_f32_u32"]), 8).tolist() == fx["selected_experts"]
    for case in _load(golden_dir, "pw0157-pytorch-topk-ties.json")["cases"]:
        assert call(_f32(case["corrected_f32_u32"]), 8).tolist() == case["selected_experts"]
    rng = np.random.default_rng(11)
    for n in (2, 3, 7, 8, 9, 40, 256):
        for trial in range(6):
            v = (rng.integers(0, 5, n) if trial % 2 else rng.standard_normal(n)).astype(np.float32)
            for k in sorted(k for k in {1, 2, n // 2, n - 1} if 0 < k < n):
                got = call(v, k)
                assert len(set(got.tolist())) == k
                assert np.array_equal(np.sort(v[got])[::-1], np.sort(v)[::-1][:k])
                assert got.tolist() == O.topk_unsorted(v, k).tolist()


def test_product_topk_matches_oracle_on_random_and_tied_rows():
    rng = np.random.default_rng(5)
    for trial in range(400):
        if trial % 2:
            v = rng.integers(0, 6, 256).astype(np.float32)  # heavy ties exercise every branch
        else:
            v = rng.standard_normal(256).astype(np.float32)
        assert P.topk_unsorted(v).tolist() == O.topk_unsorted(v).tolist()
    for n in (9, 10, 17, 33):
        v = rng.integers(0, 3, n).astype(np.float32)
        assert P.topk_unsorted(v).tolist() == O.topk_unsorted(v).tolist()


def test_product_routes_bit_exact_with_oracle():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)  # bf16-valued activations
    r = (rng.standard_normal((256, 4096)) * 0.02).astype(np.float32)
    r = (r.view(np.uint32) & 0xFFFF0000).view(np.float32)
    bias = rng.uniform(-0.01, 0.01, 256).astype(np.float32)
    logits, scores, sel, w, ties = O.route(x, r, bias)
    s2, sel2, w2, ties2 = P.route_from_logits(logits, bias)
    assert np.array_equal(s2.view(np.uint32), scores.view(np.uint32))
    assert np.array_equal(sel2, sel)
    assert np.array_equal(w2.view(np.uint32), w.view(np.uint32))
    assert ties == ties2


def test_product_noaux_tie_counting(golden_dir):
    ties = _load(golden_dir, "pw0157-pytorch-topk-ties.json")
    for case in ties["cases"]:
        v = _f32(case["corrected_f32_u32"])
        _, _, n = P.noaux_routes(np.ones(256, np.float32), (v - np.float32(1)).astype(np.float32))
        assert n == 1


def test_product_routes_reject_nonfinite():
    with pytest.raises(P.PwError):
        P.noaux_routes(np.full((1, 256), np.nan, np.float32), np.zeros(256, np.float32))


def test_product_qkv_maps_match_oracle():
    for r in list(range(0, 13568, 7)) + [13567, 13568, -1]:
        assert P.full_qkv_source_row(r) == O.full_qkv_source_row(r)
        assert P.full_qkv_scale_row(r) == O.full_qkv_scale_row(r)
    for r in list(range(0, 14848, 7)) + [14847, 14848, -1]:
        assert P.swa_qkv_source_row(r) == O.swa_qkv_source_row(r)
