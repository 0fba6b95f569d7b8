"""GPU parity of the block-scaled FP8 projections (modes A and B, plain / segmented / TP4 layouts)
against the C oracle, through the C ABI.

Tolerances: mode A f32 accumulation <= 1e-3 max|d|/max|ref| on the f32
result before the final bf16 round (in practice ~1e-7: products are exact, only the summation
order differs), and bf16 outputs within one bf16 rounding step plus 1e-5 * sum|terms| of the
oracle's; mode B <= 2e-2 max|d|/max|ref|. Integer work (codes, scales) is bit-exact.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from helpers import (bf16_normal, bf16_round, condition, decode_table, dequant, encode_e4m3, fp8_weight,
                     from_bf16_bits, log_uniform_scales, normwise, rel_l2, to_bf16_bits,
                     within_bf16_cond)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def run_device(rt, proj, x, mode=P.MODE_A, x_dtype=P.DTYPE_BF16, out_dtype=P.DTYPE_F32_RAW):
    """Device-resident projection on torch's stream; returns numpy f32 [rows, proj.rows]."""
    torch = _torch()
    rows = x.shape[0]
    if x_dtype == P.DTYPE_BF16:
        xt = torch.from_numpy(to_bf16_bits(x).view(np.int16)).cuda()
    else:
        xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    if out_dtype == P.DTYPE_BF16:
        out = torch.empty((rows, proj.rows), dtype=torch.int16, device="cuda")
    else:
        out = torch.empty((rows, proj.rows), dtype=torch.float32, device="cuda")
    rt.fp8_linear_device(proj, xt, rows, out, mode=mode, x_dtype=x_dtype, out_dtype=out_dtype,
                         stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    host = out.cpu().numpy()
    return from_bf16_bits(host.view(np.uint16)) if out_dtype == P.DTYPE_BF16 else host


def test_fp8_hardware_decode_all_bytes_mode_a(rt):
    """v_cvt_scalef32_pk_bf16_fp8 reads OCP e4m3fn: every finite byte decodes to the oracle value."""
    codes = np.arange(256, dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    w = np.repeat(codes[:, None], 256, axis=1)  # row r is all byte r
    s = np.ones((2, 2), np.float32)
    proj = rt.bind_projection(w, s)
    for col in (0, 77, 200):
        x = np.zeros((1, 256), np.float32)
        x[0, col] = 1.0
        y = run_device(rt, proj, x)[0]
        want = np.array([O.decode_e4m3fn(int(c)) for c in codes], np.float32)
        assert np.array_equal(y.view(np.uint32) & 0x7FFFFFFF, want.view(np.uint32) & 0x7FFFFFFF)
        assert np.array_equal(np.signbit(y[want != 0]), np.signbit(want[want != 0]))


def test_fp8_hardware_decode_all_bytes_mode_b(rt):
    """The FP8 MFMA reads OCP e4m3fn codes: x one-hot 448 quantises to code 0x7e, scale 1."""
    codes = np.arange(256, dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    w = np.repeat(codes[:, None], 128, axis=1)
    proj = rt.bind_projection(w, np.ones((2, 1), np.float32))
    x = np.zeros((1, 128), np.float32)
    x[0, 5] = 448.0
    y = run_device(rt, proj, x, mode=P.MODE_B, x_dtype=P.DTYPE_F32)[0]
    want = np.array([O.decode_e4m3fn(int(c)) * 448.0 for c in codes], np.float32)
    assert np.array_equal(y, want)


def test_closed_form_row_and_column_blocks(rt):
    w = np.full((256, 256), 0x38, np.uint8)
    s = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    proj = rt.bind_projection(w, s)
    for mode in (P.MODE_A, P.MODE_B):
        y = rt.execute_fp8_linear(np.ones((1, 256), np.float32), proj, mode=mode).output[0]
        assert np.all(y[:128] == 384.0) and np.all(y[128:] == 896.0)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8, 16, 17, 32])
@pytest.mark.parametrize("x_kind", ["bf16", "f32"])
def test_mode_a_matches_oracle(rt, rows, x_kind):
    rng = np.random.default_rng(100 + rows)
    n, k = 200, 512  # partial 16-row tile and partial 128-row scale block
    s = log_uniform_scales(rng, n, k)
    w = fp8_weight(rng, n, k, s)
    x = bf16_normal(rng, (rows, k)) if x_kind == "bf16" else rng.standard_normal((rows, k)).astype(np.float32)
    ref = O.gemm_mode_a(w, s, x)
    proj = rt.bind_projection(w, s)
    got = run_device(rt, proj, x, x_dtype=P.DTYPE_BF16 if x_kind == "bf16" else P.DTYPE_F32)
    assert normwise(got, ref) <= 2e-6  # exact products, f32 accumulation order only
    host = rt.execute_fp8_linear(x, proj, mode=P.MODE_A).output
    assert within_bf16_cond(host, bf16_round(ref), condition(w, s, x))


@pytest.mark.parametrize("n,k", [(200, 512), (2048, 4096)])
def test_mode_a_f32_row_split_in_staging(rt, n, k):
    """One f32 row is split into its bf16 planes inside the projection's staging; two rows go
    through the separate split launch. The same row alone and as both rows of a pair gives the same
    raw f32 bits."""
    rng = np.random.default_rng(n + k)
    s = log_uniform_scales(rng, n, k)
    w = fp8_weight(rng, n, k, s)
    x = rng.standard_normal((1, k)).astype(np.float32)
    proj = rt.bind_projection(w, s)
    one = run_device(rt, proj, x, x_dtype=P.DTYPE_F32)
    two = run_device(rt, proj, np.concatenate([x, x]), x_dtype=P.DTYPE_F32)
    assert np.array_equal(one[0].view(np.uint32), two[0].view(np.uint32))
    assert np.array_equal(one[0].view(np.uint32), two[1].view(np.uint32))
    # the f32 summation order against the oracle's: 2e-6 at K = 512, more room at K = 4096
    assert normwise(one, O.gemm_mode_a(w, s, x)) <= (2e-6 if k <= 512 else 1e-5)


def test_real_checkpoint_gemv_fixture(rt, golden_dir):
    with open(os.path.join(golden_dir, "mtp-gate-fp8-gemv.json")) as f:
        fx = json.load(f)
    w = np.array(fx["raw_u8"], np.uint8)
    s = np.array(fx["scale_inv"], np.float32).reshape(1, -1)
    x = np.array(fx["input"], np.float32).reshape(1, -1)
    proj = rt.bind_projection(w, s)
    got = run_device(rt, proj, x, x_dtype=P.DTYPE_F32)[0]
    # the reference's Metal harness bound for this fixture (tools/test_all.sh:9-21)
    assert np.all(np.abs(got - np.array(fx["expected_f32"], np.float32)) < 2e-6)


def test_projection_2048x4096_width1(rt):
    """A single block-scaled FP8 projection GEMV at 2048 x 4096, width 1, bf16 output."""
    rng = np.random.default_rng(0x50570000)
    s = log_uniform_scales(rng, 2048, 4096)
    w = fp8_weight(rng, 2048, 4096, s)
    x = bf16_normal(rng, (1, 4096))
    ref = O.gemm_mode_a(w, s, x)
    proj = rt.bind_projection(w, s)
    raw = run_device(rt, proj, x)
    assert normwise(raw, ref) <= 1e-3 and rel_l2(raw, ref) <= 1e-5
    out = run_device(rt, proj, x, out_dtype=P.DTYPE_BF16)
    assert within_bf16_cond(out, bf16_round(ref), condition(w, s, x))


def test_quantiser_bit_exact(rt, golden_dir):
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.standard_normal((4, 512)) * 10, rng.standard_normal((2, 512)) * 1e-3,
                        np.zeros((1, 512))]).astype(np.float32)
    x[1, :128] = 0.0
    x[1, 5] = -0.0
    x[2, 130] = 1e-12
    with open(os.path.join(golden_dir, "pw0053-dynamic-fp8-activation.json")) as f:
        fx = json.load(f)
    fixture_rows = np.array([b & 0xFFFFFFFF for b in np.array(fx["input_f32_bits"]).reshape(-1)],
                            np.uint32).view(np.float32).reshape(2, 256)
    for data in (x, fixture_rows):
        codes_ref, scales_ref, _ = O.dynamic_fp8(data)
        codes, scales = quantize_device(rt, data)
        assert np.array_equal(codes, codes_ref)
        assert np.array_equal(scales.view(np.uint32), scales_ref.view(np.uint32))


def _encoder_sweep_values():
    """f32 values with |x| <= 448 that decide e4m3fn round-to-nearest-even: every bit pattern with
    its low 11 bits clear (all codes and all exact ties between codes are among them), each tie
    and its neighbours 1 and 2 ulp away, and 2^20 random patterns; both signs, zeros included."""
    lim = 0x43E00000  # 448.0f
    coarse = np.arange(0, lim + 1, 2048, dtype=np.int64)
    mags = np.array([O.decode_e4m3fn(c) for c in range(0x7F)], np.float64)
    mids = ((mags[:-1] + mags[1:]) / 2).astype(np.float32).view(np.uint32).astype(np.int64)
    ties = (mids[:, None] + np.arange(-2, 3)).reshape(-1)
    rand = np.random.default_rng(21).integers(0, lim + 1, 1 << 20, dtype=np.int64)
    bits = np.unique(np.concatenate([coarse, ties, rand]))
    vals = bits[(bits >= 0) & (bits <= lim)].astype(np.uint32).view(np.float32)
    return np.concatenate([vals, -vals])


def test_quantiser_encoder_sweep(rt):
    """Groups whose first value is 448 have scale exactly 1, so their codes are the e4m3fn
    encodings of the values themselves: the device encoder against the oracle's on ~3.2M values."""
    vals = _encoder_sweep_values()
    per = 127
    n = -(-vals.size // per)
    body = np.zeros(n * per, np.float32)
    body[:vals.size] = vals
    x = np.concatenate([np.full((n, 1), 448.0, np.float32), body.reshape(n, per)], axis=1)
    codes_ref, scales_ref, _ = O.dynamic_fp8(x)
    codes, scales = quantize_device(rt, x)
    assert np.all(scales_ref == 1.0) and np.array_equal(scales.view(np.uint32), scales_ref.view(np.uint32))
    assert np.array_equal(codes, codes_ref)


def _bf16_division_sweep():
    """bf16 groups whose first value is the group absmax m (sign alternating) and whose other 127
    values are bf16 numbers with |a| <= m: for 1,528 absmaxes (every bf16 exponent with six
    mantissas, subnormals and values below the 1e-10 scale clamp), every bf16 magnitude from m down
    twenty binades (quotients a / scale from 448 to below the smallest e4m3 subnormal), both signs."""
    ms = [(e << 7) | mant for e in range(1, 255) for mant in (0x00, 0x01, 0x3F, 0x40, 0x55, 0x7F)]
    ms += [0x0001, 0x0040, 0x007F, 0x2EDB, 0x2E00]  # subnormal bf16 and absmaxes under 1e-10
    groups = []
    for mb in ms:
        e = mb >> 7
        lo = max(0, (e - 20)) << 7
        mags = np.arange(lo, mb + 1, dtype=np.uint32)
        vals = np.concatenate([mags, mags | 0x8000])
        pad = (-vals.size) % 127
        vals = np.concatenate([vals, np.zeros(pad, np.uint32)]).reshape(-1, 127)
        head = np.full((vals.shape[0], 1), mb, np.uint32)
        head[1::2] |= 0x8000
        groups.append(np.concatenate([head, vals], axis=1))
    bits = np.concatenate(groups).astype(np.uint16)
    return bits.reshape(-1, 512) if bits.shape[0] % 4 == 0 else np.concatenate(
        [bits, np.zeros(((-bits.shape[0]) % 4, 128), np.uint16)]).reshape(-1, 512)


def test_quantiser_bf16_division_sweep(rt):
    """bf16 activations are quantised through one correctly rounded reciprocal per group (a
    Markstein-corrected quotient): codes and scales equal the oracle's IEEE division bit for bit
    over ~8.6M values around every binade of the absmax."""
    torch = _torch()
    bits = _bf16_division_sweep()
    rows, k = bits.shape
    x32 = (bits.astype(np.uint32) << 16).view(np.float32)
    codes_ref, scales_ref, _ = O.dynamic_fp8(x32)
    xt = torch.from_numpy(bits.view(np.int16)).cuda()
    codes = torch.empty((rows, k), dtype=torch.uint8, device="cuda")
    scales = torch.empty((rows, k // 128), dtype=torch.float32, device="cuda")
    rt.quantize_fp8_group128_device(xt, rows, k, codes, scales, x_dtype=P.DTYPE_BF16,
                                    stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), scales_ref.view(np.uint32))
    got = codes.cpu().numpy()
    bad = np.argwhere(got != codes_ref)
    assert bad.size == 0, (bad[:4], x32[tuple(bad[0])] if bad.size else None)


def quantize_device(rt, data):
    torch = _torch()
    rows, k = data.shape
    xt = torch.from_numpy(np.ascontiguousarray(data, np.float32)).cuda()
    codes = torch.empty((rows, k), dtype=torch.uint8, device="cuda")
    scales = torch.empty((rows, k // 128), dtype=torch.float32, device="cuda")
    rt.quantize_fp8_group128_device(xt, rows, k, codes, scales, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    return codes.cpu().numpy(), scales.cpu().numpy()


def test_quantiser_rejects_misaligned_buffers(rt):
    torch = _torch()
    base = torch.zeros(2 * 128 + 8, dtype=torch.float32, device="cuda")
    codes = torch.empty((2, 128), dtype=torch.uint8, device="cuda")
    scales = torch.empty((2, 1), dtype=torch.float32, device="cuda")
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.quantize_fp8_group128_device(base[1:257], 2, 128, codes, scales)
    raw = torch.empty(2 * 128 + 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.quantize_fp8_group128_device(base[:256], 2, 128, raw[4:260], scales)


def test_quantiser_flags_nonfinite(rt):
    torch = _torch()
    data = np.ones((1, 128), np.float32)
    data[0, 17] = np.inf
    xt = torch.from_numpy(data).cuda()
    codes = torch.empty((1, 128), dtype=torch.uint8, device="cuda")
    scales = torch.empty((1, 1), dtype=torch.float32, device="cuda")
    rt.quantize_fp8_group128_device(xt, 1, 128, codes, scales, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 2  # PW_FLAG_QUANT_NONFINITE
    assert rt.take_flags() == 0


@pytest.mark.parametrize("active", [2, 9, 26, 32])
def test_mode_b_reference_probe(rt, active):
    """The reference's block-scaled probe (src/wide_metal_moe.rs:387-532): codes and scales equal
    the CPU quantiser, projection within 0.01 of the CPU block equation."""
    rows, cols = 128, 256
    x = ((np.arange(active * cols) * 29 % 401 - 200) / 37).astype(np.float32).reshape(active, cols)
    q, a, _ = O.dynamic_fp8(x)
    w = ((np.arange(rows * cols) * 37 + 11) % 0x7F).astype(np.uint8).reshape(rows, cols)
    s = (0.003 + np.arange(2) * 0.0017).astype(np.float32).reshape(1, 2)
    ref = O.gemm_mode_b_equation(w, s, q, a)
    proj = rt.bind_projection(w, s)
    got = run_device(rt, proj, x, mode=P.MODE_B, x_dtype=P.DTYPE_F32)
    codes, scales = quantize_device(rt, x)
    assert np.array_equal(codes, q) and np.array_equal(scales.view(np.uint32), a.view(np.uint32))
    assert np.max(np.abs(got - ref)) <= 0.01


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_mode_b_matches_fp8_linear(rt, rows):
    rng = np.random.default_rng(200 + rows)
    n, k = 384, 1024
    s = log_uniform_scales(rng, n, k)
    w = fp8_weight(rng, n, k, s)
    x = bf16_normal(rng, (rows, k))
    ref = O.fp8_linear_mode_b(w, s, x)
    proj = rt.bind_projection(w, s)
    got = rt.execute_fp8_linear(x, proj, mode=P.MODE_B).output
    assert normwise(got, ref) <= 2e-2
    _, _, xd = O.dynamic_fp8(x)
    assert within_bf16_cond(got, ref, np.abs(xd.astype(np.float64)) @ np.abs(dequant(w, s)).T)


def _segments(rng, rows_list, k=4096):
    segs = []
    for rows in rows_list:
        s = log_uniform_scales(rng, rows, k)
        segs.append((fp8_weight(rng, rows, k, s), s))
    return segs


@pytest.mark.parametrize("k_rows", [768, 1000])
@pytest.mark.parametrize("width", [1, 8])
def test_qkv_segments_nonuniform_scales(rt, k_rows, width):
    """Separate q [12288], k [768 or 1000 (partial trailing block)], v [512] x 4096 tensors, each
    with its own ceil(rows/128) x 32 scale grid, output concatenated."""
    rng = np.random.default_rng(0x50570003 + k_rows + width)
    segs = _segments(rng, [12288, k_rows, 512])
    x = bf16_normal(rng, (width, 4096))
    ref = np.concatenate([O.gemm_mode_a(w, s, x) for w, s in segs], axis=1)
    proj = rt.bind_segments(segs)
    assert proj.rows == 12288 + k_rows + 512
    raw = run_device(rt, proj, x)
    assert normwise(raw, ref) <= 1e-3 and rel_l2(raw, ref) <= 1e-5
    out = run_device(rt, proj, x, out_dtype=P.DTYPE_BF16)
    cond = np.concatenate([condition(w, s, x) for w, s in segs], axis=1)
    assert within_bf16_cond(out, bf16_round(ref), cond)


@pytest.mark.parametrize("layout", [P.LAYOUT_FULL_QKV_TP4, P.LAYOUT_SWA_QKV_TP4])
def test_tp4_qkv_layouts(rt, layout):
    """The checkpoint's four TP shards deinterleaved on one device (src/text_endpoint.rs:3174-3242)
    checked against an f64 brute force that applies the reference's row and scale-row maps."""
    rng = np.random.default_rng(7 + layout)
    rows, srows = (13568, 108) if layout == P.LAYOUT_FULL_QKV_TP4 else (14848, 116)
    w = rng.integers(0, 0x7F, size=(rows, 4096), dtype=np.uint8) | (rng.integers(0, 2, size=(rows, 4096), dtype=np.uint8) << 7)
    s = (2.0 ** rng.uniform(-10, -6, size=(srows, 32))).astype(np.float32)
    x = bf16_normal(rng, (8, 4096))
    proj = rt.bind_projection(w, s, layout=layout)
    got = run_device(rt, proj, x)
    src = np.array([(O.full_qkv_source_row if layout == P.LAYOUT_FULL_QKV_TP4 else O.swa_qkv_source_row)(r)
                    for r in range(rows)])
    srow = (np.array([O.full_qkv_scale_row(r) for r in range(rows)]) if layout == P.LAYOUT_FULL_QKV_TP4
            else src // 128)
    dec = decode_table()[w[src]].astype(np.float32)
    wd = dec * np.repeat(s[srow], 128, axis=1)
    ref = x.astype(np.float64) @ wd.T.astype(np.float64)
    assert normwise(got, ref) <= 1e-5


@pytest.mark.parametrize("layout", [P.LAYOUT_FULL_QKV_TP4, P.LAYOUT_SWA_QKV_TP4])
@pytest.mark.parametrize("rows", [1, 8])
def test_tp4_qkv_mode_b_as_the_reference_calls_it(rt, layout, rows):
    """The reference's attention projection: execute_fp8_linear(.., full_qkv_layout = true) in
    mode B on the TP4 layout (full_qkv_fp8_gemm8_sglang_blockscaled; the SWA form is picked by its
    14848 x 4096 shape, src/wide_metal_moe.rs:241-350). CPU authority: decode_full_qkv_weight
    (src/text_endpoint.rs:3260-3314) and fp8_linear (:3053-3108), i.e. the dynamically quantised
    input times the deinterleaved dequantised weight, rounded to bf16. Outputs within one bf16
    rounding step plus 1e-5 of the sum of |terms| (f32 order and the FP8 MFMA's block sums)."""
    rng = np.random.default_rng(70 + layout + rows)
    n, srows = (13568, 108) if layout == P.LAYOUT_FULL_QKV_TP4 else (14848, 116)
    s = (2.0 ** rng.uniform(-10, -6, size=(srows, 32))).astype(np.float32)
    w = encode_e4m3(rng.standard_normal((n, 4096)) / np.repeat(np.repeat(s.astype(np.float64), 128, 0), 128, 1)[:n])
    x = bf16_normal(rng, (rows, 4096))
    proj = rt.bind_projection(w, s, layout=layout)
    got = rt.execute_fp8_linear(x, proj, full_qkv_layout=layout == P.LAYOUT_FULL_QKV_TP4, mode=P.MODE_B).output
    src = np.array([(O.full_qkv_source_row if layout == P.LAYOUT_FULL_QKV_TP4 else O.swa_qkv_source_row)(r)
                    for r in range(n)])
    srow = (np.array([O.full_qkv_scale_row(r) for r in range(n)]) if layout == P.LAYOUT_FULL_QKV_TP4
            else src // 128)
    wd = decode_table()[w[src]] * np.repeat(s[srow].astype(np.float64), 128, axis=1)
    _, _, xd = O.dynamic_fp8(x)
    exact = xd.astype(np.float64) @ wd.T
    ref = bf16_round(exact.astype(np.float32))
    assert got.shape == (rows, n)
    assert normwise(got, exact) <= 2e-2
    assert within_bf16_cond(got, ref, np.abs(xd.astype(np.float64)) @ np.abs(wd).T)


def test_fail_closed_validation(rt):
    w = np.full((128, 128), 0x38, np.uint8)
    s = np.ones((1, 1), np.float32)
    proj = rt.bind_projection(w, s)
    bad = np.ones((1, 128), np.float32)
    bad[0, 3] = np.nan
    with pytest.raises(P.PwError, match="NONFINITE"):
        rt.execute_fp8_linear(bad, proj, mode=P.MODE_A)
    w2 = w.copy()
    w2[3, 9] = 0x7F
    with pytest.raises(P.PwError, match="non-finite FP8 weight"):
        rt.bind_projection(w2, s)
    with pytest.raises(P.PwError, match="LAYOUT"):
        rt.bind_projection(w, np.ones((2, 1), np.float32))
    with pytest.raises(P.PwError, match="NONFINITE"):
        rt.bind_projection(w, np.full((1, 1), np.inf, np.float32))
