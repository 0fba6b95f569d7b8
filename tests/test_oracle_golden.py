"""Pins the C oracle against the reference's golden vectors, known answers and brute force.

Each check is chosen so that a plausible slip in the restatement (dropped term, wrong sign,
wrong index, transposed operand, wrong tie rule) fails it.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O


def load(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


def f32(bits):
    return np.array([b & 0xFFFFFFFF for b in bits], dtype=np.uint32).view(np.float32)


def bits(x):
    return np.array([x], dtype=np.float32).view(np.uint32)[0]


# ---------------------------------------------------------------- a1 decode
def test_decode_all_256_bytes(golden_dir):
    fx = load(golden_dir, "f8-e4m3fn-all-bytes.json")
    assert fx["semantic"] == "f8_e4m3fn_exhaustive_f32_bits"
    for b in range(256):
        got = bits(O.decode_e4m3fn(b))
        want = fx["expected_f32_bits"][b] & 0xFFFFFFFF
        if b in (0x7F, 0xFF):
            assert math.isnan(O.decode_e4m3fn(b)) and math.isnan(f32([want])[0])
            assert (got >> 31) == (want >> 31)
        else:
            assert got == want, hex(b)


def test_real_block_dequant(golden_dir):
    fx = load(golden_dir, "mtp-gate-fp8-block.json")
    for raw_row, dec_row, deq_row in zip(fx["raw_u8"], fx["decoded_fp8"], fx["dequantized"]):
        for b, d, q in zip(raw_row, dec_row, deq_row):
            v = O.decode_e4m3fn(b)
            assert v == d
            assert abs(np.float32(v) * np.float32(fx["scale_inv"]) - q) < 1e-9


# ---------------------------------------------------------------- a2 bf16
def test_bf16_boundary(golden_dir):
    fx = load(golden_dir, "pw0054-bf16-boundary.json")
    inputs = f32(fx["input_f32_bits"])
    for x, want16, wide in zip(inputs, fx["bf16_u16"], fx["widened_f32_bits"]):
        got = np.float32(O.round_bf16(float(x)))
        gb = bits(got)
        if np.isfinite(x):
            assert (gb >> 16) == want16
            assert gb == (wide & 0xFFFFFFFF)
        elif np.isnan(x):
            assert np.isnan(got) and (gb >> 31) == (bits(x) >> 31)
        else:
            assert gb == bits(x)


def test_bf16_nan_payload_quieted():
    # signalling NaN 0x7f800001 must become a quiet NaN with payload bit 0x40 set
    got = bits(np.float32(O.round_bf16(float(f32([0x7F800001])[0]))))
    assert got == 0x7FC00000


# ---------------------------------------------------------------- a3 quantiser
def test_dynamic_fp8_fixture(golden_dir):
    fx = load(golden_dir, "pw0053-dynamic-fp8-activation.json")
    assert fx["semantic"] == "dynamic_fp8_e4m3fn_per_token_group_128"
    x = f32(np.array(fx["input_f32_bits"]).reshape(-1).tolist()).reshape(fx["rows"], fx["columns"])
    codes, scales, deq = O.dynamic_fp8(x)
    want_scales = f32(np.array(fx["scale_f32_bits"]).reshape(-1).tolist())
    assert np.array_equal(scales.reshape(-1).view(np.uint32), want_scales.view(np.uint32))
    assert np.array_equal(codes.reshape(-1), np.array(fx["encoded_u8"]).reshape(-1).astype(np.uint8))
    want_deq = f32(np.array(fx["dequantized_f32_bits"]).reshape(-1).tolist())
    assert np.array_equal(deq.reshape(-1).view(np.uint32), want_deq.view(np.uint32))


def test_dynamic_fp8_rejects_bad_input():
    with pytest.raises(ValueError):
        O.dynamic_fp8(np.zeros((1, 127), np.float32))
    bad = np.zeros((1, 128), np.float32)
    bad[0, 3] = np.nan
    with pytest.raises(ValueError):
        O.dynamic_fp8(bad)


def _nearest_code_f64(values):
    """Independent nearest-e4m3 search in f64 (exact distances), ties to the even code."""
    cand = np.array([O.decode_e4m3fn(c) for c in range(0x7F)], dtype=np.float64)
    mag = np.abs(values.astype(np.float64))[:, None]
    dist = np.abs(mag - cand[None, :])
    best = dist.min(axis=1, keepdims=True)
    ties = dist == best
    # among tied candidates prefer an even code, else the lowest
    even = ties & (np.arange(0x7F)[None, :] % 2 == 0)
    pick = np.where(even.any(axis=1), even.argmax(axis=1), ties.argmax(axis=1))
    neg = np.signbit(values)
    return (pick | np.where(neg, 0x80, 0)).astype(np.uint8)


def test_encoder_brute_force_near_every_midpoint():
    pos = np.array([O.decode_e4m3fn(c) for c in range(0x7F)], dtype=np.float32)
    probes = []
    for lo, hi in zip(pos[:-1], pos[1:]):
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        for d in range(-6, 7):
            probes.append(np.nextafter(mid, np.float32(np.inf) if d > 0 else np.float32(-np.inf),
                                       dtype=np.float32) if d else mid)
            v = mid
            for _ in range(abs(d)):
                v = np.nextafter(v, np.float32(np.inf) if d > 0 else np.float32(-np.inf), dtype=np.float32)
            probes.append(v)
    probes.extend(pos.tolist())
    rng = np.random.default_rng(7)
    probes.extend((rng.random(2000) * 448).astype(np.float32).tolist())
    probes.extend((rng.random(500) * 2.0 ** -6).astype(np.float32).tolist())  # subnormal range
    probes = np.array(probes, dtype=np.float32)
    probes = np.concatenate([probes, -probes])
    want = _nearest_code_f64(probes)
    got = np.array([O.encode_e4m3fn(float(v)) for v in probes], dtype=np.uint8)
    assert np.array_equal(got, want)
    assert O.encode_e4m3fn(448.5) is None and O.encode_e4m3fn(float("nan")) is None
    assert O.encode_e4m3fn(-0.0) == 0x80 and O.encode_e4m3fn(0.0) == 0


# ---------------------------------------------------------------- a4 mode A
def test_real_fp8_gemv(golden_dir):
    fx = load(golden_dir, "mtp-gate-fp8-gemv.json")
    w = np.array(fx["raw_u8"], dtype=np.uint8)
    s = np.array(fx["scale_inv"], dtype=np.float32).reshape(1, -1)
    x = np.array(fx["input"], dtype=np.float32)
    y = O.gemm_mode_a(w, s, x)[0]
    assert np.all(np.abs(y - np.array(fx["expected_f32"], np.float32)) < 2e-7)


def test_closed_form_row_and_column_blocks():
    w = np.full((256, 256), 0x38, np.uint8)  # e4m3 1.0
    s = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    y = O.gemm_mode_a(w, s, np.ones(256, np.float32))[0]
    assert np.all(y[:128] == 384.0) and np.all(y[128:] == 896.0)
    bad_x = np.ones(256, np.float32); bad_x[0] = np.nan
    with pytest.raises(ValueError):
        O.gemm_mode_a(w, s, bad_x)
    bad_s = s.copy(); bad_s[0, 0] = np.nan
    with pytest.raises(ValueError):
        O.gemm_mode_a(w, bad_s, np.ones(256, np.float32))
    bad_w = w.copy(); bad_w.flat[123] = 0x7F
    with pytest.raises(ValueError):
        O.gemm_mode_a(bad_w, s, np.ones(256, np.float32))


def test_width_specialised_fixture_pattern():
    # src/lib.rs:4650-4763: weights 0xb8/0x38 by index % 3, scale 0.5, input ((i % 13) - 6) * 0.01
    w = np.where(np.arange(128 * 128) % 3 == 0, 0xB8, 0x38).astype(np.uint8).reshape(128, 128)
    s = np.array([[0.5]], np.float32)
    x = (((np.arange(8 * 128) % 13) - 6) * 0.01).astype(np.float32).reshape(8, 128)
    dec = np.where(w == 0xB8, -1.0, 1.0)
    for active in range(1, 9):
        y = O.gemm_mode_a(w, s, x[:active])
        want = (x[:active].astype(np.float64) @ (dec * 0.5).T)
        assert np.max(np.abs(y - want)) <= 2e-5


def _random_fp8(rng, shape):
    w = rng.integers(0, 256, size=shape, dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x7E
    return w


def _dec_table():
    return np.array([O.decode_e4m3fn(b) for b in range(256)], np.float64)


def test_mode_a_brute_force_f64_with_partial_row_block():
    rng = np.random.default_rng(11)
    n, k, rows = 200, 384, 3  # 200 rows -> partial trailing 128-row block
    w = _random_fp8(rng, (n, k))
    s = (2.0 ** rng.uniform(-10, -6, size=(2, 3))).astype(np.float32)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    y = O.gemm_mode_a(w, s, x)
    W = _dec_table()[w] * np.repeat(np.repeat(s.astype(np.float64), 128, 0)[:n], 128, 1)
    want = x.astype(np.float64) @ W.T
    assert np.max(np.abs(y - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))
    # scaling one block's scale must move only that block's rows
    s2 = s.copy(); s2[1, 2] *= 2
    y2 = O.gemm_mode_a(w, s2, x)
    assert np.array_equal(y2[:, :128], y[:, :128])
    assert not np.array_equal(y2[:, 128:], y[:, 128:])


# ---------------------------------------------------------------- a5 mode B
def test_mode_b_equation_probe_inputs():
    # src/wide_metal_moe.rs:387-421 probe: rows 128, columns 256
    rows, cols = 128, 256
    for active in (2, 9, 26, 32):
        x = ((np.arange(active * cols) * 29 % 401 - 200) / 37).astype(np.float32).reshape(active, cols)
        q, a, _ = O.dynamic_fp8(x)
        w = ((np.arange(rows * cols) * 37 + 11) % 0x7F).astype(np.uint8).reshape(rows, cols)
        s = (0.003 + np.arange(2) * 0.0017).astype(np.float32).reshape(1, 2)
        y = O.gemm_mode_b_equation(w, s, q, a)
        dec = _dec_table()
        want = np.zeros((active, rows))
        for b in range(2):
            blk = slice(b * 128, (b + 1) * 128)
            want += (dec[q[:, blk]] @ dec[w[:, blk]].T) * s[0, b] * a[:, b:b + 1]
        assert np.max(np.abs(y - want)) <= 0.01


def test_mode_b_equation_equals_mode_a_on_exact_codes():
    rng = np.random.default_rng(3)
    w = _random_fp8(rng, (128, 256))
    s = np.array([[0.25, 0.5]], np.float32)
    q = _random_fp8(rng, (4, 256))
    a = np.ones((4, 2), np.float32)
    yb = O.gemm_mode_b_equation(w, s, q, a)
    xa = _dec_table()[q].astype(np.float32)
    ya = O.gemm_mode_a(w, s, xa)
    assert np.max(np.abs(yb - ya)) <= 1e-5 * np.max(np.abs(ya))


def test_fp8_linear_mode_b_brute_force():
    rng = np.random.default_rng(5)
    n, k, rows = 256, 256, 3
    w = _random_fp8(rng, (n, k))
    s = (2.0 ** rng.uniform(-10, -6, size=(2, 2))).astype(np.float32)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    y = O.fp8_linear_mode_b(w, s, x)
    _, _, xd = O.dynamic_fp8(x)
    W = _dec_table()[w] * np.repeat(np.repeat(s.astype(np.float64), 128, 0), 128, 1)
    want = xd.astype(np.float64) @ W.T
    # bf16 output: within one bf16 ulp of the f64 value
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    assert np.all(np.abs(y - want) <= ulp)
    assert np.array_equal(y, np.vectorize(O.round_bf16, otypes=[np.float32])(y))


# ---------------------------------------------------------------- a7 SwiGLU
def test_swiglu_fixture(golden_dir):
    fx = load(golden_dir, "swiglu-f32.json")
    got = O.swiglu_f32(np.array(fx["gate"], np.float32), np.array(fx["up"], np.float32))
    want = np.array(fx["expected_f64"])
    # f32 evaluation of the f64 oracle: 4 f32 ulps relative, or the reference's 1e-15 absolute
    # (gate = -100 underflows to -0 in f32 where f64 gives -3.7e-42)
    tol = np.maximum(4 * np.finfo(np.float32).eps * np.abs(want), 1e-15)
    assert np.all(np.abs(got - want) <= tol)


def test_swiglu_staged_is_bf16_and_close():
    rng = np.random.default_rng(9)
    g = rng.standard_normal(1000).astype(np.float32) * 3
    u = rng.standard_normal(1000).astype(np.float32)
    h = O.swiglu_bf16_staged(g, u)
    assert np.array_equal(h.view(np.uint32) & 0xFFFF, np.zeros(1000, np.uint32))
    ref = O.swiglu_f32(g, u)
    assert np.max(np.abs(h - ref)) <= 0.02 * np.max(np.abs(ref))


# ---------------------------------------------------------------- a9 router
def test_router_sigmoid_fixture(golden_dir):
    fx = load(golden_dir, "pw0062-router-sigmoid.json")
    for lb, sb in zip(fx["logit_f32_u32"], fx["score_f32_u32"]):
        assert bits(np.float32(O.sigmoid_f32(float(f32([lb])[0])))) == sb


def test_sleef_boundaries_fixture(golden_dir):
    fx = load(golden_dir, "pw0068-sleef-boundaries.json")
    for ib, eb, sb in zip(fx["input_f32_u32"], fx["exp_f32_u32"], fx["sigmoid_of_negated_input_f32_u32"]):
        v = float(f32([ib])[0])
        assert bits(np.float32(O.sleef_expf_u10(v))) == eb
        assert bits(np.float32(O.sigmoid_f32(-v))) == sb


def test_sleef_exp_accuracy_sweep():
    xs = np.linspace(-87, 88, 20001).astype(np.float32)
    got = np.array([O.sleef_expf_u10(float(v)) for v in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 2.5 * 2 ** -23


def test_topk_order_fixture(golden_dir):
    fx = load(golden_dir, "pw0063-topk-order.json")
    v = f32(fx["corrected_f32_u32"])
    assert O.topk_unsorted(v).tolist() == fx["selected_experts"]


def test_topk_tie_fixtures(golden_dir):
    fx = load(golden_dir, "pw0157-pytorch-topk-ties.json")
    assert fx["standard_library"] == "libc++" and fx["top_k"] == 8 and fx["width"] == 256
    for case in fx["cases"]:
        v = f32(case["corrected_f32_u32"])
        assert O.topk_unsorted(v).tolist() == case["selected_experts"], case["name"]
        scores = np.ones(256, np.float32)
        correction = (v - np.float32(1.0)).astype(np.float32)
        _, _, ties = O.noaux_routes(scores, correction)
        assert ties == 1, case["name"]


def test_topk_set_is_the_top_values_for_distinct_inputs():
    rng = np.random.default_rng(1)
    for _ in range(200):
        v = rng.standard_normal(256).astype(np.float32)
        sel = O.topk_unsorted(v)
        assert set(sel.tolist()) == set(np.argsort(-v)[:8].tolist())


def test_noaux_weights_and_rejection():
    rng = np.random.default_rng(2)
    scores = (1 / (1 + np.exp(-rng.standard_normal((8, 256))))).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, 256).astype(np.float32)
    sel, w, ties = O.noaux_routes(scores, bias)
    assert ties == 0
    for p in range(8):
        assert abs(float(np.sum(w[p], dtype=np.float32)) - 1.0) <= 1e-6
        corrected = scores[p] + bias
        assert set(sel[p].tolist()) == set(np.argsort(-corrected)[:8].tolist())
        # weights use the uncorrected score
        chosen = scores[p, sel[p]].astype(np.float64)
        assert np.allclose(w[p], chosen / chosen.sum(), rtol=1e-6)
    with pytest.raises(ValueError):
        O.noaux_routes(np.full((1, 256), np.nan, np.float32), bias)


def test_router_logits_t256_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    r = (rng.standard_normal((16, 4096)) * 0.02).astype(np.float32)
    got = O.router_logits_t256(x, r)
    want = x.astype(np.float64) @ r.T.astype(np.float64)
    assert np.max(np.abs(got - want)) < 1e-5


def _one_logit(entries, k=4096):
    """Logit of one row against one expert with x[c] = a, w[c] = b for (c, a, b) in entries."""
    x = np.zeros((1, k), np.float32)
    r = np.zeros((1, k), np.float32)
    for c, a, b in entries:
        x[0, c], r[0, c] = a, b
    return float(O.router_logits_t256(x, r)[0, 0])


def test_router_logits_t256_order_known_answers():
    """Sums whose f32 value is fixed by the declared order (2^24 + 1 rounds to 2^24)."""
    big = float(2 ** 24)
    # fused multiply-add: -(1 + 2^-11) + (1 + 2^-12)^2 = 2^-24 exactly; a rounded product gives 0
    assert _one_logit([(0, 1.0, -(1 + 2 ** -11)), (1, 1 + 2 ** -12, 1 + 2 ** -12)]) == 2 ** -24
    # one thread: columns 0, 1 of the first group, then column 2048 of its next group -> 0
    assert _one_logit([(0, 1.0, big), (1, 1.0, 1.0), (2048, 1.0, -big)]) == 0.0
    # halving tree: threads 0 and 32 meet first, thread 1 joins at offset 1 -> 1 (a lane-serial sum gives 0)
    assert _one_logit([(0, 1.0, big), (8, 1.0, 1.0), (256, 1.0, -big)]) == 1.0
    # waves: (w0 + w1) + (w2 + w3) with w = 2^24, 1, 1, -2^24 -> 1 (serial 0, exact 2)
    assert _one_logit([(0, 1.0, big), (512, 1.0, 1.0), (1024, 1.0, 1.0), (1536, 1.0, -big)]) == 1.0
    # a hidden size that is not a multiple of 2048: thread 1's second group starts at 2056
    assert _one_logit([(8, 1.0, big), (2056, 1.0, 1.0), (2057, 1.0, -big)], k=2064) == 0.0


# ---------------------------------------------------------------- a12 QKV maps
def test_full_qkv_maps_known_answers():
    src = {0: 0, 3071: 3071, 3072: 3392, 12287: 13247, 12288: 3072, 12480: 6464, 13055: 13439,
           13056: 3264, 13567: 13567}
    for r, want in src.items():
        assert O.full_qkv_source_row(r) == want
    assert O.full_qkv_source_row(13568) == -1
    sc = {0: 0, 3071: 23, 3072: 27, 12287: 104, 12288: 24, 12415: 24, 12416: 25, 12479: 25,
          12480: 51, 13055: 106, 13056: 26, 13567: 107}
    for r, want in sc.items():
        assert O.full_qkv_scale_row(r) == want
    assert O.full_qkv_scale_row(13568) == -1
    assert {O.full_qkv_scale_row(r) for r in range(13568)} == set(range(108))


def test_swa_qkv_maps_known_answers():
    src = {0: 0, 3071: 3071, 3072: 3712, 12287: 14207, 12288: 3072, 12671: 3455, 12672: 6784,
           13823: 14591, 13824: 3456, 14079: 3711, 14080: 7168, 14847: 14847}
    for r, want in src.items():
        assert O.swa_qkv_source_row(r) == want
    assert O.swa_qkv_source_row(14848) == -1


# ---------------------------------------------------------------- f3 BF16 linear
def _bf16_bits(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_bf16_linear_sequential_unfused_known_answers():
    """Sums whose f32 value fixes the restatement: separate multiply and add, sequential columns."""
    a = 1 + 2 ** -7
    b = 1 + 2 ** -17
    # (1 + 2^-7)(1 + 2^-17) = 1 + 2^-7 + 2^-17 + 2^-24 rounds (tie to even) to 1 + 2^-7 + 2^-17, so the
    # unfused sum is exactly 0; a fused multiply-add would leave 2^-24
    w = _bf16_bits([[1.0, a]])
    x = np.array([[-(1 + 2 ** -7 + 2 ** -17), b]], np.float32)
    y, raw = O.bf16_linear(w, x, raw=True)
    assert raw[0, 0] == 0.0 and y[0, 0] == 0.0
    # sequential order: 2^24 + 1 rounds back to 2^24 twice (exact sum 2^24 + 2)
    w = _bf16_bits([[1.0, 1.0, 1.0]])
    y, raw = O.bf16_linear(w, np.array([[2.0 ** 24, 1.0, 1.0]], np.float32), raw=True)
    assert raw[0, 0] == 2.0 ** 24
    # output rounding to bf16, ties to even: 1 + 2^-8 -> 1, 1 + 3 * 2^-8 -> 1 + 2^-6
    w = _bf16_bits([[1.0, 1.0]])
    y = O.bf16_linear(w, np.array([[1.0, 2.0 ** -8], [1.0, 3 * 2.0 ** -8]], np.float32))
    assert y[0, 0] == 1.0 and y[1, 0] == 1 + 2 ** -6


def test_bf16_linear_equals_mode_a_on_e4m3_values_with_unit_scales():
    """bf16 weights holding e4m3 values are the mode A projection with unit scales, bit for bit."""
    rng = np.random.default_rng(8)
    n, k = 130, 256
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C
    dec = np.vectorize(O.decode_e4m3fn, otypes=[np.float32])(codes)
    x = rng.standard_normal((3, k)).astype(np.float32)
    ya = O.gemm_mode_a(codes, np.ones((2, 2), np.float32), x)
    _, raw = O.bf16_linear(_bf16_bits(dec), x, raw=True)
    assert np.array_equal(ya.view(np.uint32), raw.view(np.uint32))


def test_bf16_linear_f64_brute_force():
    rng = np.random.default_rng(9)
    w = _bf16_bits(rng.standard_normal((70, 384)).astype(np.float32) * 0.05)
    x = rng.standard_normal((4, 384)).astype(np.float32)
    y, raw = O.bf16_linear(w, x, raw=True)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = x.astype(np.float64) @ wf.T
    assert np.max(np.abs(raw - want)) <= 1e-5 * np.max(np.abs(want))
    assert np.array_equal(y.view(np.uint32), np.vectorize(O.round_bf16, otypes=[np.float32])(raw).view(np.uint32))
    with pytest.raises(ValueError):
        O.bf16_linear(w, np.full((1, 384), np.nan, np.float32))
