"""Cross-checks the oracle's top-k against the reference's own src/pytorch_topk.cpp.

The reference source is compiled from its single file into oracle/_ref/ (make -C oracle ref).
It builds here with libstdc++, not the libc++ that produced the golden orders, so only the
selected SET and the argument checks are compared; the slot ORDER is pinned by the golden
vectors in test_oracle_golden.py.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O

REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                   "libpw_topk_ref.so")

pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref not built")


def _ref_topk(values, k=8):
    lib = ctypes.CDLL(REF)
    fn = lib.pw_pytorch_topk_unsorted_f32
    fn.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_size_t, ctypes.c_size_t,
                   ctypes.POINTER(ctypes.c_uint32)]
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(k, np.uint32)
    rc = fn(v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), v.size, k,
            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return rc, out


def test_reference_topk_set_matches_oracle():
    rng = np.random.default_rng(123)
    for _ in range(300):
        v = rng.standard_normal(256).astype(np.float32)
        rc, ref = _ref_topk(v)
        assert rc == 0
        assert set(ref.tolist()) == set(O.topk_unsorted(v).tolist())


def test_reference_topk_argument_checks():
    rc, _ = _ref_topk(np.zeros(8, np.float32), k=8)  # top_k >= count
    assert rc == -1
    with pytest.raises(ValueError):
        O.topk_unsorted(np.zeros(8, np.float32), k=8)
