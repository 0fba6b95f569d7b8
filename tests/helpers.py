"""Test helpers: seeded data in the reference's formats and the parity metrics the tests use."""
from __future__ import annotations

import numpy as np

# e4m3fn magnitudes of codes 0..0x7e (0x7f is NaN), exact in f64
_MAG = np.array([(m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
                 for e in range(16) for m in range(8)][:0x7F])


def decode_table() -> np.ndarray:
    t = np.concatenate([_MAG, [np.nan], -_MAG, [np.nan]])
    return t


def encode_e4m3(values: np.ndarray) -> np.ndarray:
    """Nearest e4m3fn code with ties to the even code, saturating at +-448 (table search in f64)."""
    v = np.asarray(values, np.float64)
    a = np.minimum(np.abs(v), 448.0)
    hi = np.clip(np.searchsorted(_MAG, a), 1, len(_MAG) - 1)
    lo = hi - 1
    dlo, dhi = a - _MAG[lo], _MAG[hi] - a
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    return (pick | np.where(np.signbit(v), 0x80, 0)).astype(np.uint8)


def log_uniform_scales(rng, rows: int, cols: int) -> np.ndarray:
    """[ceil(rows/128), cols/128] scales, log-uniform in [2^-10, 2^-6]."""
    return (2.0 ** rng.uniform(-10, -6, size=((rows + 127) // 128, cols // 128))).astype(np.float32)


def fp8_weight(rng, rows: int, cols: int, scales: np.ndarray) -> np.ndarray:
    """N(0,1) / block scale quantised to e4m3 with saturation."""
    z = rng.standard_normal((rows, cols))
    s = np.repeat(np.repeat(scales.astype(np.float64), 128, 0)[:rows], 128, 1)
    return encode_e4m3(z / s)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 RNE, widened back to f32 (finite inputs)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_normal(rng, shape, std=1.0) -> np.ndarray:
    return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def normwise(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| — the parity metric for f32 accumulation-order differences."""
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.linalg.norm(got.astype(np.float64) - ref) / max(np.linalg.norm(ref.astype(np.float64)), 1e-30))


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def dequant(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Dequantised f64 weight dec(W) * S[r/128, c/128]."""
    rows, cols = w.shape
    return decode_table()[w] * np.repeat(np.repeat(s.astype(np.float64), 128, 0)[:rows], 128, 1)


def condition(w: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_c |W[r, c] x[p, c]| per output [rows, n]: the scale of f32 reordering error."""
    return np.abs(np.asarray(x, np.float64)) @ np.abs(dequant(w, s)).T


def within_bf16_cond(got: np.ndarray, ref_bf16: np.ndarray, cond: np.ndarray, rel: float = 1e-5) -> bool:
    """bf16 outputs agree up to one rounding step plus an f32 summation-order error bounded by
    rel * sum|terms| (element-wise relative error is ill-conditioned where terms cancel)."""
    d = np.abs(got.astype(np.float64) - ref_bf16.astype(np.float64))
    bound = bf16_ulp(np.maximum(np.abs(got), np.abs(ref_bf16))) * 1.0000001 + rel * cond
    return bool(np.all(d <= bound))


def within_one_bf16_ulp(got: np.ndarray, ref: np.ndarray) -> bool:
    """bf16 outputs differ from the reference's bf16 outputs by at most one rounding step."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return bool(np.all(d <= bf16_ulp(np.maximum(np.abs(got), np.abs(ref))) * 1.0000001))


def write_safetensors(path, tensors, metadata=None, header_pad=True, raw_header=None):
    """Writes a safetensors file: tensors maps name -> (dtype string, shape, bytes), payloads packed in
    the given order. raw_header replaces the JSON header text (for malformed-file tests)."""
    import json
    import struct
    header, payload, off = {}, b"", 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dtype, shape, data) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        payload += data
        off += len(data)
    text = raw_header if raw_header is not None else json.dumps(header, separators=(",", ":"))
    hb = text.encode()
    if header_pad:
        hb += b" " * ((-len(hb)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + payload)
    return path
