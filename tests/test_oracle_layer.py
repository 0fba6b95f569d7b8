"""Pins the oracle's routed-MoE layer, its one-expert forward and its bf16-staged SwiGLU.

Each check is chosen so that a dropped rounding, a swapped operand, a wrong index or a changed
stage order fails at least one of them:

- the reference's tiny noaux-tc MoE fixture (an f64 expert mixture, `moe-noaux-tc-swiglu.json`,
  checked by the reference at src/lib.rs:7966-7982) through both layer modes, each fixture weight
  carried exactly by its own 128 x 128 block (code +-1.0, block scale |w|);
- f64 brute force of the mode-A layer and of the one-expert forward on tiny FP8 shapes, composed in
  numpy from dequantised weights;
- bit equality of both layer modes with the reference's routed composition (routed_mlp_traced,
  src/text_endpoint.rs:5290-5381): experts in ascending id, token rows gathered in ascending order,
  gate, up, SwiGLU, down, `out[pos] += y * w` in f32, bf16 at the end; built here from the
  separately pinned projection and SwiGLU functions;
- one-hot route weights reproduce the routed expert's own output bit for bit, and a token that
  names one expert twice is rejected (src/text_endpoint.rs:13610-13654);
- known answers of the staged SwiGLU where dropping any one of its four roundings changes the
  output bits (the reference's case is src/staged_metal_expert.rs:2826-2831).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O
from helpers import (STAGED_CASES, STAGES, bf16_normal, bf16_round, closed_form_mode_b, dequant, fp8_weight,
                     log_uniform_scales, staged_swiglu_independent)


def _bits(x):
    return int(np.array([x], np.float32).view(np.uint32)[0])


def _f32(bits):
    return float(np.array([bits], np.uint32).view(np.float32)[0])


# ------------------------------------------------------------------ the tiny noaux-tc fixture
def _embed(matrix):
    """Logical [rows][cols] f64 weights as block-FP8: weight (i, j) is code +-1.0 at (128 i, 128 j)
    of a [128 rows x 128 cols] tensor whose block (i, j) scale is |w|; all other codes are zero."""
    rows, cols = len(matrix), len(matrix[0])
    w = np.zeros((128 * rows, 128 * cols), np.uint8)
    s = np.zeros((rows, cols), np.float32)
    for i, row in enumerate(matrix):
        for j, v in enumerate(row):
            w[128 * i, 128 * j] = 0xB8 if v < 0 else 0x38
            s[i, j] = abs(v)
    return w, s


def _tiny_fixture(golden_dir):
    with open(os.path.join(golden_dir, "moe-noaux-tc-swiglu.json")) as f:
        fx = json.load(f)
    assert fx["semantic"] == "mimo_v2_noaux_tc_swiglu_moe" and fx["normalize_topk"]
    assert fx["routed_scaling_factor"] == 1.0
    experts = {}
    for e, ex in enumerate(fx["experts"]):
        gw, gs = _embed(ex["gate"])
        uw, us = _embed(ex["up"])
        dw, ds = _embed(ex["down"])
        experts[e] = (gw, gs, uw, us, dw, ds)
    h = fx["hidden_size"]
    x = np.zeros((len(fx["inputs"]), 128 * h), np.float32)
    for p, row in enumerate(fx["inputs"]):
        x[p, ::128] = row
    sel = np.array([r["topk_indices"] for r in fx["expected"]], np.uint32)
    w = np.array([r["topk_weights"] for r in fx["expected"]], np.float32)
    want = np.array([r["output"] for r in fx["expected"]], np.float64)
    return fx, experts, x, sel, w, want


def test_tiny_noaux_fixture_mode_a(golden_dir):
    fx, experts, x, sel, w, want = _tiny_fixture(golden_dir)
    out, raw = O.moe_layer("a", x, experts, len(experts), sel, w, raw=True)
    got = raw[:, ::128].astype(np.float64)
    # f32 arithmetic on f64 data: a few f32 roundings per term (the outputs are ~1e-3, and a
    # swapped gate/up, a transposed down or a weight on the wrong expert moves them by > 1e-4)
    assert np.max(np.abs(got - want)) <= 1e-9, (got, want)
    assert not np.any(np.delete(raw, np.s_[::128], axis=1)), "columns outside the embedding must stay zero"
    assert np.array_equal(out.view(np.uint32), bf16_round(raw).view(np.uint32))


def test_tiny_noaux_fixture_mode_b(golden_dir):
    fx, experts, x, sel, w, want = _tiny_fixture(golden_dir)
    _, raw = O.moe_layer("b", x, experts, len(experts), sel, w, raw=True)
    got = raw[:, ::128].astype(np.float64)
    # mode B rounds every projection and SwiGLU stage to bf16 (relative 2^-9 each) and re-quantises
    # the hidden to e4m3 (one nonzero value per group here, so exactly)
    assert np.max(np.abs(got - want)) <= 2e-2 * np.max(np.abs(want))


def test_tiny_noaux_fixture_route_weights_are_normalised_scores(golden_dir):
    """The fixture's weights are the selected uncorrected sigmoid scores over their sum (the
    noaux-tc weight rule the oracle's router restates); the selection uses score + bias."""
    with open(os.path.join(golden_dir, "moe-noaux-tc-swiglu.json")) as f:
        fx = json.load(f)
    for inp, exp in zip(fx["inputs"], fx["expected"]):
        logits = np.array(fx["router_weight"]) @ np.array(inp)
        scores = np.array([O.sigmoid_f32(float(np.float32(v))) for v in logits], np.float64)
        chosen = scores[exp["topk_indices"]]
        assert np.allclose(exp["topk_weights"], chosen / chosen.sum(), rtol=1e-6, atol=0)
        corrected = scores + np.array(fx["correction_bias"])
        size = len(scores) // fx["groups"]

        def group_score(g):
            best = sorted(corrected[g * size:(g + 1) * size], reverse=True)
            return best[0] + best[1]

        kept = sorted(range(fx["groups"]), key=lambda g: (-group_score(g), g))[:fx["topk_group"]]
        candidates = [e for e in range(len(scores)) if e // size in kept]
        assert sorted(candidates, key=lambda e: (-corrected[e], e))[:fx["top_k"]] == exp["topk_indices"]


# ------------------------------------------------------------------ random tiny FP8 layers
def _bank(rng, n_experts, hidden, inter):
    experts = {}
    for e in range(n_experts):
        gs, us = log_uniform_scales(rng, inter, hidden), log_uniform_scales(rng, inter, hidden)
        ds = log_uniform_scales(rng, hidden, inter)
        experts[e] = (fp8_weight(rng, inter, hidden, gs), gs, fp8_weight(rng, inter, hidden, us), us,
                      fp8_weight(rng, hidden, inter, ds), ds)
    return experts


def _routes(rng, rows, n_experts, top_k=8):
    sel = np.stack([rng.permutation(n_experts)[:top_k] for _ in range(rows)]).astype(np.uint32)
    w = rng.uniform(0.05, 1.0, (rows, top_k)).astype(np.float32)
    return sel, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def _expert_f64(ex, x):
    gw, gs, uw, us, dw, ds = ex
    g = x.astype(np.float64) @ dequant(gw, gs).T
    u = x.astype(np.float64) @ dequant(uw, us).T
    return (g / (1.0 + np.exp(-g)) * u) @ dequant(dw, ds).T


def _compose(mode, x, experts, sel, w):
    """The reference's routed composition from the pinned projection and SwiGLU functions."""
    rows = x.shape[0]
    block = np.zeros_like(x, dtype=np.float32)
    for e in sorted(set(sel.reshape(-1).tolist())):
        pos = [p for p in range(rows) if e in sel[p].tolist()]
        wts = [w[p, sel[p].tolist().index(e)] for p in pos]
        xs = x[pos]
        gw, gs, uw, us, dw, ds = experts[e]
        if mode == "a":
            h = O.swiglu_f32(O.gemm_mode_a(gw, gs, xs), O.gemm_mode_a(uw, us, xs))
            y = O.gemm_mode_a(dw, ds, h)
        else:
            h = O.swiglu_bf16_staged(O.fp8_linear_mode_b(gw, gs, xs), O.fp8_linear_mode_b(uw, us, xs))
            y = O.fp8_linear_mode_b(dw, ds, h)
        for l, p in enumerate(pos):
            block[p] = block[p] + y[l] * np.float32(wts[l])
    return bf16_round(block), block


@pytest.mark.parametrize("rows", [1, 2, 5])
def test_mode_a_layer_f64_brute_force(rows):
    rng = np.random.default_rng(100 + rows)
    hidden, inter, n_exp = 256, 256, 10
    experts = _bank(rng, n_exp, hidden, inter)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    out, raw = O.moe_layer("a", x, experts, n_exp, sel, w, raw=True)
    want = np.zeros((rows, hidden))
    for p in range(rows):
        for e, wt in zip(sel[p].tolist(), w[p].tolist()):
            want[p] += wt * _expert_f64(experts[e], x[p:p + 1])[0]
    assert np.max(np.abs(raw - want)) <= 2e-5 * np.max(np.abs(want))
    assert np.array_equal(out.view(np.uint32), bf16_round(raw).view(np.uint32))


@pytest.mark.parametrize("rows", [1, 3])
def test_mode_b_layer_f64_brute_force(rows):
    rng = np.random.default_rng(200 + rows)
    hidden, inter, n_exp = 256, 128, 9
    experts = _bank(rng, n_exp, hidden, inter)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    out = O.moe_layer("b", x, experts, n_exp, sel, w)
    # the reference's mode-B stages with f64 sums: dynamically quantised input (the quantiser is
    # pinned by pw0053) -> gate, up rounded to bf16 -> silu rounded to bf16 -> product rounded to bf16
    # -> quantised hidden -> down rounded to bf16 -> weighted sum
    def bf(v):
        return bf16_round(np.asarray(v, np.float32)).astype(np.float64)

    xd = O.dynamic_fp8(x)[2].astype(np.float64)
    want = np.zeros((rows, hidden))
    for p in range(rows):
        for e, wt in zip(sel[p].tolist(), w[p].tolist()):
            gw, gs, uw, us, dw, ds = experts[e]
            g = bf(xd[p] @ dequant(gw, gs).T)
            u = bf(xd[p] @ dequant(uw, us).T)
            h = bf(bf(g / (1.0 + np.exp(-g))) * u)
            hd = O.dynamic_fp8(h.astype(np.float32)[None])[2][0].astype(np.float64)
            want[p] += np.float64(wt) * bf(hd @ dequant(dw, ds).T)
    # left: f32 sums that round to the other bf16 value than their f64 sums, and the hidden codes
    # that follow them; a dropped expert (weight ~1/8) or a swapped projection moves this by > 0.1
    assert np.linalg.norm(out - want) <= 2e-3 * np.linalg.norm(want)


@pytest.mark.parametrize("mode", ["a", "b"])
@pytest.mark.parametrize("rows", [1, 4, 7])
def test_layer_equals_routed_composition_bit_for_bit(mode, rows):
    rng = np.random.default_rng(300 + rows + (mode == "b"))
    hidden, inter, n_exp = 256, 256, 12
    experts = _bank(rng, n_exp, hidden, inter)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    out, raw = O.moe_layer(mode, x, experts, n_exp, sel, w, raw=True)
    want, want_raw = _compose(mode, x, experts, sel, w)
    assert np.array_equal(raw.view(np.uint32), want_raw.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    # the combine order is ascending expert id: a slot-order accumulation differs in some bits
    slot_order = np.zeros_like(x)
    for p in range(rows):
        for e, wt in zip(sel[p].tolist(), w[p].tolist()):
            _, one = _compose(mode, x[p:p + 1], experts, np.array([[e]], np.uint32), np.array([[1.0]], np.float32))
            slot_order[p] = slot_order[p] + one[0] * np.float32(wt)
    if rows > 1 or sel.shape[1] > 1:
        assert not np.array_equal(raw.view(np.uint32), slot_order.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 3])
def test_one_expert_forward_f64_brute_force(rows):
    rng = np.random.default_rng(400 + rows)
    hidden, inter = 384, 256
    ex = _bank(rng, 1, hidden, inter)[0]
    x = bf16_normal(rng, (rows, hidden))
    out32, outbf = O.expert_mode_a(x, ex)
    want = _expert_f64(ex, x)
    assert np.max(np.abs(out32 - want)) <= 2e-5 * np.max(np.abs(want))
    assert np.array_equal(outbf.view(np.uint32), bf16_round(out32).view(np.uint32))


@pytest.mark.parametrize("mode", ["a", "b"])
def test_one_hot_route_weights_reconstruct_the_expert(mode):
    """src/text_endpoint.rs:13610-13638: weights (1, 0, ..., 0) give the first routed expert's
    bf16 output exactly."""
    rng = np.random.default_rng(500 + (mode == "b"))
    hidden, inter, n_exp, rows = 256, 128, 10, 4
    experts = _bank(rng, n_exp, hidden, inter)
    x = bf16_normal(rng, (rows, hidden))
    sel, _ = _routes(rng, rows, n_exp)
    w = np.zeros(sel.shape, np.float32)
    w[:, 0] = 1.0
    out = O.moe_layer(mode, x, experts, n_exp, sel, w)
    for p in range(rows):
        e = int(sel[p, 0])
        if mode == "a":
            _, want = O.expert_mode_a(x[p:p + 1], experts[e])
        else:
            want, _ = _compose("b", x[p:p + 1], experts, np.array([[e]], np.uint32), np.array([[1.0]], np.float32))
        assert np.array_equal(out[p].view(np.uint32), want[0].view(np.uint32)), (p, e)


def test_layer_rejects_non_bijective_routes():
    """src/text_endpoint.rs:13640-13654: a token naming one expert twice is not a placement
    bijection; out-of-range experts and non-finite weights are rejected as well."""
    rng = np.random.default_rng(600)
    n_exp = 20
    experts = _bank(rng, n_exp, 128, 128)
    x = bf16_normal(rng, (2, 128))
    sel = np.array([[0, 1, 2, 3, 4, 5, 6, 7], [8, 9, 10, 11, 12, 13, 14, 15]], np.uint32)
    w = np.full((2, 8), 0.125, np.float32)
    O.moe_layer("a", x, experts, n_exp, sel, w)
    for mode in ("a", "b"):
        # expert 9 twice for token 1: two placements for two rows, so only the pair check sees it
        dup = sel.copy()
        dup[1, 3] = 9
        with pytest.raises(ValueError):
            O.moe_layer(mode, x, experts, n_exp, dup, w)
        bad = sel.copy()
        bad[0, 0] = n_exp
        with pytest.raises(ValueError):
            O.moe_layer(mode, x, experts, n_exp, bad, w)
        nan_w = w.copy()
        nan_w[1, 2] = np.nan
        with pytest.raises(ValueError):
            O.moe_layer(mode, x, experts, n_exp, sel, nan_w)


# ------------------------------------------------------------------ staged SwiGLU known answers
@pytest.mark.parametrize("case", STAGED_CASES, ids=lambda c: hex(c["g"]))
def test_staged_swiglu_known_answers(case):
    """The oracle gives the expected bits; the independent evaluation gives them too with every
    rounding in place, and taking out the named rounding gives the `dropped` bits instead, so a
    staged SwiGLU missing that rounding would fail here."""
    g = np.array([_f32(case["g"])], np.float32)
    u = np.array([_f32(case["u"])], np.float32)
    got = _bits(O.swiglu_bf16_staged(g, u)[0])
    assert got == case["out"], hex(got)
    assert staged_swiglu_independent(case["g"], case["u"]) == case["out"]
    for stage in STAGES:
        alt = staged_swiglu_independent(case["g"], case["u"], drop=stage)
        if stage in case["dropped"]:
            assert alt == case["dropped"][stage] and alt != case["out"], (stage, hex(alt))
    # together the cases pin all four roundings
    assert {st for c in STAGED_CASES for st in c["dropped"]} == set(STAGES)


def test_staged_swiglu_rounds_every_stage():
    """Every output is a bf16 value, and the silu is rounded before the product: the reference's
    assertion staged(g, u) == round(round(silu(g)) * u) on its own case."""
    g, u = 1.03125, 0.71484375
    silu = bf16_round(np.array([g / (1.0 + math.exp(-g))], np.float32))
    want = bf16_round(silu * np.float32(u))[0]
    assert O.swiglu_bf16_staged(np.array([g], np.float32), np.array([u], np.float32))[0] == want
    rng = np.random.default_rng(9)
    h = O.swiglu_bf16_staged(rng.standard_normal(4096).astype(np.float32) * 3,
                             rng.standard_normal(4096).astype(np.float32))
    assert not np.any(h.view(np.uint32) & 0xFFFF)


# ------------------------------------------------------------------ the CPU BLAS restatement
# (the CPU-baseline leg times it; src/lib.rs:2003-2015 and 5807-5862)
def test_decode_fp8_matrix_f32_rounds_each_product_once():
    """dec(w) * s is one f32 rounding of the exact product (f64 holds it exactly); a partial
    trailing 128-row block and a partial 128-column block take their block's scale."""
    rng = np.random.default_rng(700)
    s = log_uniform_scales(rng, 300, 256)
    w = fp8_weight(rng, 300, 256, s)
    got = O.decode_fp8_matrix_f32(w, s)
    assert got.shape == (300, 256) and got.dtype == np.float32
    assert np.array_equal(got, dequant(w, s).astype(np.float32))
    # the element at (299, 200) lives in block (2, 1)
    assert got[299, 200] == np.float32(O.decode_e4m3fn(int(w[299, 200])) * np.float64(s[2, 1]))
    # a partial trailing 128-column block
    got2 = O.decode_fp8_matrix_f32(w[:, :200], s)
    assert np.array_equal(got2, got[:, :200])


@pytest.mark.parametrize("rows", [1, 4])
def test_blas_layer_f64_brute_force(rows):
    rng = np.random.default_rng(710 + rows)
    hidden, inter, n_exp = 256, 256, 10
    experts = _bank(rng, n_exp, hidden, inter)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    deq = {e: (O.decode_fp8_matrix_f32(ex[0], ex[1]), O.decode_fp8_matrix_f32(ex[2], ex[3]),
               O.decode_fp8_matrix_f32(ex[4], ex[5])) for e, ex in experts.items()}
    got = O.moe_layer_blas(x, deq, sel, w)
    want = np.zeros((rows, hidden))
    for p in range(rows):
        for e, wt in zip(sel[p].tolist(), w[p].tolist()):
            want[p] += wt * _expert_f64(experts[e], x[p:p + 1])[0]
    # f32 weight copies (one rounding per weight) and f32 sums: ~1e-6 relative; a swapped gate/up,
    # a transposed projection or a weight on the wrong token moves the output by far more
    assert np.max(np.abs(got - want)) <= 2e-5 * np.max(np.abs(want))
    _, raw = O.moe_layer("a", x, experts, n_exp, sel, w, raw=True)
    assert np.max(np.abs(got - raw)) <= 2e-5 * np.max(np.abs(raw))


def test_blas_layer_thread_pool_and_one_hot():
    """Experts run concurrently but combine in ascending id: same bits as the serial loop; one-hot
    weights give the first routed expert's own output for that token (its rows gathered as the
    layer gathers them: BLAS may sum a one-row product in another order)."""
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(720)
    hidden, inter, n_exp, rows = 256, 128, 12, 5
    experts = _bank(rng, n_exp, hidden, inter)
    deq = {e: (O.decode_fp8_matrix_f32(ex[0], ex[1]), O.decode_fp8_matrix_f32(ex[2], ex[3]),
               O.decode_fp8_matrix_f32(ex[4], ex[5])) for e, ex in experts.items()}
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    serial = O.moe_layer_blas(x, deq, sel, w)
    with ThreadPoolExecutor(4) as pool:
        pooled = O.moe_layer_blas(x, deq, sel, w, pool=pool)
    assert np.array_equal(serial.view(np.uint32), pooled.view(np.uint32))
    one = np.zeros_like(w)
    one[:, 0] = 1.0
    got = O.moe_layer_blas(x, deq, sel, one)
    for p in range(rows):
        e = int(sel[p, 0])
        pos = sorted({q for q in range(rows) if e in sel[q].tolist()})
        want = O.expert_blas_f32(x[pos], *deq[e])[pos.index(p)]
        assert np.array_equal(got[p], want), p


# ------------------------------------------------------------------ the mode-B CPU BLAS restatement
# (the prefill's and mode-B decode's CPU-baseline legs time it; routed_mlp_traced and fp8_linear,
# src/text_endpoint.rs:5290-5381, :3053-3108)
def _deq_bank(experts):
    return {e: (O.decode_fp8_matrix_f32(ex[0], ex[1]), O.decode_fp8_matrix_f32(ex[2], ex[3]),
                O.decode_fp8_matrix_f32(ex[4], ex[5])) for e, ex in experts.items()}


def test_blas_mode_b_layer_bit_exact_on_closed_form():
    """On closed-form mode-B data every projection sum is exact in f32 in any order, so the BLAS
    restatement (BLAS summation order) must give the scalar oracle's layer bit for bit: a missing
    activation quantisation, bf16 rounding or staged SwiGLU rounding, a swapped gate/up or a
    transposed projection changes these bits."""
    experts, x, sel, w = closed_form_mode_b(0x50570100, 256, 12)
    x, sel, w = x[:24], sel[:24], w[:24]
    got, got_raw = O.moe_layer_blas_mode_b(x, _deq_bank(experts), sel, w)
    want, want_raw = O.moe_layer("b", x, experts, 12, sel, w, raw=True)
    assert np.array_equal(got_raw.view(np.uint32), want_raw.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 9])
def test_blas_mode_b_layer_matches_oracle(rows):
    """Random FP8 data: BLAS sums in another order than the oracle's sequential loop, so a bf16
    rounding or an e4m3 re-quantisation may land on the other side; within the mode-B tolerance,
    and bit-equal through a thread pool (experts combined in ascending id either way)."""
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(730 + rows)
    hidden, inter, n_exp = 512, 256, 12
    experts = _bank(rng, n_exp, hidden, inter)
    deq = _deq_bank(experts)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = _routes(rng, rows, n_exp)
    got, _ = O.moe_layer_blas_mode_b(x, deq, sel, w)
    want = O.moe_layer("b", x, experts, n_exp, sel, w)
    assert np.max(np.abs(got - want)) <= 2e-2 * np.max(np.abs(want))
    with ThreadPoolExecutor(4) as pool:
        pooled, _ = O.moe_layer_blas_mode_b(x, deq, sel, w, pool=pool)
    assert np.array_equal(pooled.view(np.uint32), got.view(np.uint32))
