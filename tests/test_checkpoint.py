"""Checkpoint files (safetensors) through the C ABI on the CPU: the header parser follows
MappedSafetensors::open (src/lib.rs:783-905) — length prefix, JSON object of {dtype, shape,
data_offsets}, __metadata__, size checks, no overlaps, no duplicate names — and is checked against
files written by this test and by the safetensors package itself."""
import json
import struct

import numpy as np
import pytest

import prismwing_amd as P
from helpers import write_safetensors


def test_reads_tensors_written_by_the_safetensors_package(tmp_path):
    st_np = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(1)
    tensors = {"a.weight": rng.standard_normal((3, 5)).astype(np.float32),
               "b": rng.integers(0, 255, (7,)).astype(np.uint8),
               "c.bias": rng.integers(-9, 9, (2, 2, 2)).astype(np.int32)}
    path = str(tmp_path / "pkg.safetensors")
    st_np.save_file(tensors, path, metadata={"format": "np"})
    with P.Safetensors(path) as f:
        assert len(f) == 3
        for name, arr in tensors.items():
            dtype, shape, data = f.tensor(name)
            assert shape == arr.shape
            assert dtype == {np.float32: "F32", np.uint8: "U8", np.int32: "I32"}[arr.dtype.type]
            assert data == arr.tobytes()
        with pytest.raises(P.PwError, match="absent"):
            f.tensor("missing")


def test_fp8_and_scale_tensors(tmp_path):
    w = np.arange(256 * 128, dtype=np.uint32).astype(np.uint8).reshape(256, 128)
    s = np.full((2, 1), 0.5, np.float32)
    path = write_safetensors(tmp_path / "x.safetensors", {
        "m.weight": ("F8_E4M3", w.shape, w.tobytes()), "m.weight_scale_inv": ("F32", s.shape, s.tobytes())},
        metadata={"k": "v"})
    with P.Safetensors(str(path)) as f:
        assert f.tensor("m.weight") == ("F8_E4M3", (256, 128), w.tobytes())
        assert f.tensor("m.weight_scale_inv") == ("F32", (2, 1), s.tobytes())


def _bad(tmp_path, name, **kw):
    path = str(tmp_path / f"{name}.safetensors")
    kw.setdefault("tensors", {"t": ("F32", (2,), b"\0" * 8)})
    write_safetensors(path, kw.pop("tensors"), **kw)
    return path


@pytest.mark.parametrize("case", ["short", "zero_len", "unaligned_len", "len_past_file", "malformed", "trailing",
                                  "not_object", "duplicate", "unknown_dtype", "zero_dim", "size_mismatch",
                                  "past_payload", "overlap", "no_tensors", "metadata_not_object", "reversed"])
def test_malformed_files_fail_closed(tmp_path, case):
    path = str(tmp_path / f"{case}.safetensors")
    if case == "short":
        open(path, "wb").write(b"\x08" + b"\0" * 9)
    elif case == "zero_len":
        open(path, "wb").write(struct.pack("<Q", 0) + b"{}      ")
    elif case == "unaligned_len":
        open(path, "wb").write(struct.pack("<Q", 3) + b"{} " + b"\0" * 8)
    elif case == "len_past_file":
        open(path, "wb").write(struct.pack("<Q", 64) + b"{}      ")
    elif case == "malformed":
        _bad(tmp_path, case, raw_header='{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]')
    elif case == "trailing":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}} x')
    elif case == "not_object":
        _bad(tmp_path, case, raw_header='[1, 2]')
    elif case == "duplicate":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
                                        '"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}')
    elif case == "unknown_dtype":
        _bad(tmp_path, case, tensors={"t": ("Q7", (2,), b"\0" * 8)})
    elif case == "zero_dim":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[0],"data_offsets":[0,0]}}')
    elif case == "size_mismatch":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}')
    elif case == "past_payload":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}')
    elif case == "overlap":
        _bad(tmp_path, case, tensors={"t": ("F32", (2,), b"\0" * 8), "u": ("F32", (2,), b"\0" * 8)},
             raw_header='{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
                        '"u":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}')
    elif case == "no_tensors":
        _bad(tmp_path, case, raw_header='{"__metadata__":{"a":"b"}}')
    elif case == "metadata_not_object":
        _bad(tmp_path, case, raw_header='{"__metadata__":[1],"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}')
    elif case == "reversed":
        _bad(tmp_path, case, raw_header='{"t":{"dtype":"F32","shape":[2],"data_offsets":[8,0]}}')
    with pytest.raises(P.PwError, match="LAYOUT"):
        P.Safetensors(path)


def test_missing_file(tmp_path):
    with pytest.raises(P.PwError, match="ARGUMENT"):
        P.Safetensors(str(tmp_path / "absent.safetensors"))


def test_json_escapes_in_names(tmp_path):
    header = {"café.😀.w": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}
    path = str(tmp_path / "esc.safetensors")
    write_safetensors(path, {}, raw_header=json.dumps(header, ensure_ascii=True))
    with open(path, "ab") as f:
        f.write(b"\1\2\3\4")
    with P.Safetensors(path) as f:
        assert f.tensor("café.😀.w".encode("utf-16", "surrogatepass").decode("utf-16")) == \
            ("U8", (4,), b"\1\2\3\4")
