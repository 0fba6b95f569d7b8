"""Bit-level GPU parity checks: cases where the product's result is fixed exactly, so that a dropped
rounding, a truncated operand or a changed stage order fails.

- bf16 round-to-nearest-even of the product's epilogues against the reference's `pw0054` vectors
  (src/text_endpoint.rs:14106-14170), sent through a projection whose sum equals its input;
- the bf16-staged SwiGLU (kernels/block_fp8_gemv.metal:139-160) in its in-place and table forms over
  every bf16 gate, and its known answers;
- closed-form mode-B layers (every f32 sum exact in any order) through the host `execute`, the
  device layer, the one-expert forward and the prefill, each equal to the oracle bit for bit;
- the mode-B layer against the same layer composed from the product's separate projection and
  SwiGLU calls, bit for bit (the reference's fused-vs-unfused check, src/wide_metal_moe.rs:709-724);
- the mode-A f32 hidden (three exact bf16 planes), exposed through an identity down projection.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from helpers import (STAGED_CASES, STAGES, _unit_codes, bf16_normal, bf16_round, closed_form_mode_b, decode_table,
                     fp8_weight, log_uniform_scales, staged_swiglu_independent, to_bf16_bits)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _stream():
    return _torch().cuda.current_stream().cuda_stream


def _f32_bits(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


# ------------------------------------------------------------------ bf16 rounding of the epilogues
def _identity_projection(rt, n=128):
    w = np.zeros((n, n), np.uint8)
    w[np.arange(n), np.arange(n)] = 0x38  # e4m3 1.0 on the diagonal, scale 1: y[r] = x[r]
    return rt.bind_projection(w, np.ones((1, 1), np.float32))


# f32 activations reach the bf16 MFMA as three bf16 planes, whose finest step is 2^-133 (the
# smallest bf16 subnormal): values of magnitude 2^-110 and above are carried exactly, smaller ones to
# within 2^-133
PLANES_EXACT_FROM = 2.0 ** -110


def test_product_bf16_rounding_matches_pw0054(rt, golden_dir):
    """Each finite pw0054 input x goes through y = x . I (f32 input split into three bf16 planes,
    products by 1.0): the raw f32 output must be x itself and the bf16 output the fixture's bf16_u16
    (round_bf16, src/text_endpoint.rs:2960-2971). Inputs below 2^-110 in magnitude are held to the
    planes' 2^-133 resolution instead, and -0 is left out (a sum that starts at +0, here and in the
    reference's mapped_fp8_gemv, cannot end at -0)."""
    torch = _torch()
    with open(os.path.join(golden_dir, "pw0054-bf16-boundary.json")) as f:
        fx = json.load(f)
    bits = np.array([b & 0xFFFFFFFF for b in fx["input_f32_bits"]], np.uint32)
    want16 = np.array(fx["bf16_u16"], np.uint16)
    x = bits.view(np.float32)
    keep = np.isfinite(x) & ((want16 & 0x7F80) != 0x7F80) & (bits != 0x80000000)
    xs, want16 = x[keep], want16[keep]
    pad = (-xs.size) % 128
    xv = np.concatenate([xs, np.zeros(pad, np.float32)]).reshape(-1, 128)
    proj = _identity_projection(rt)
    got16, got32 = [], []
    for r0 in range(0, xv.shape[0], 32):
        chunk = np.ascontiguousarray(xv[r0:r0 + 32])
        xt = torch.from_numpy(chunk).cuda()
        y16 = torch.empty(chunk.shape, dtype=torch.int16, device="cuda")
        y32 = torch.empty(chunk.shape, dtype=torch.float32, device="cuda")
        for out, dt in ((y16, P.DTYPE_BF16), (y32, P.DTYPE_F32_RAW)):
            rt.fp8_linear_device(proj, xt, chunk.shape[0], out, mode=P.MODE_A, x_dtype=P.DTYPE_F32, out_dtype=dt,
                                 stream=_stream())
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        got16.append(y16.cpu().numpy().view(np.uint16))
        got32.append(y32.cpu().numpy())
    got16 = np.concatenate(got16).reshape(-1)[:xs.size]
    got32 = np.concatenate(got32).reshape(-1)[:xs.size]
    big = (np.abs(xs) >= PLANES_EXACT_FROM) | (xs == 0)
    assert big.sum() > 450
    assert np.array_equal(got32[big].view(np.uint32), xs[big].view(np.uint32)), "three-plane split is not exact"
    assert np.all(np.abs(got32[~big].astype(np.float64) - xs[~big]) <= 2.0 ** -133)
    got16, want16, xs = got16[big], want16[big], xs[big]
    bad = np.nonzero(got16 != want16)[0]
    assert bad.size == 0, [(hex(int(xs.view(np.uint32)[i])), hex(int(got16[i])), hex(int(want16[i]))) for i in bad[:8]]


def test_host_projection_fails_closed_when_the_output_rounds_to_infinity(rt):
    """The reference rounds the projection to bf16 and rejects a non-finite result; an input whose
    bf16 round overflows must make the host call fail, not return a finite value."""
    proj = _identity_projection(rt)
    x = np.zeros((1, 128), np.float32)
    x[0, 5] = np.float32(3.4e38)
    with pytest.raises(P.PwError):
        rt.execute_fp8_linear(x, proj, mode=P.MODE_A)


# ------------------------------------------------------------------ staged SwiGLU
def _swiglu_device(rt, g, u, form):
    torch = _torch()
    gt = torch.from_numpy(np.ascontiguousarray(g, np.float32)).cuda()
    ut = torch.from_numpy(np.ascontiguousarray(u, np.float32)).cuda()
    out = torch.empty_like(gt)
    rt.swiglu_staged_device(gt, ut, g.size, out, form=form, stream=_stream())
    torch.cuda.synchronize()
    return out.cpu().numpy(), rt.take_flags()


def test_staged_swiglu_every_bf16_gate(rt):
    """All 65,536 bf16 gates with up = 1 (finite ones): the table form equals the in-place form bit
    for bit, and both equal the exact silu rounded to bf16 wherever the exact value is more than
    four f32 steps from a bf16 rounding boundary (an exp one step off may round those either way)."""
    b = np.arange(65536, dtype=np.uint32)
    g = (b << 16).view(np.float32)
    g = g[np.isfinite(g)]
    u = np.ones_like(g)
    inplace, f0 = _swiglu_device(rt, g, u, 0)
    table, f1 = _swiglu_device(rt, g, u, 1)
    assert f0 == 0 and f1 == 0
    assert np.array_equal(inplace.view(np.uint32), table.view(np.uint32))
    gd = g.astype(np.float64)
    with np.errstate(over="ignore"):
        e = np.exp(np.minimum(-gd, 700.0))
    # the reference evaluates e^-g in f32: past 2^128 it is infinite and the silu is -0
    exact = np.where(e >= 2.0 ** 128, -0.0, gd / (1.0 + e))
    f = exact.astype(np.float32)
    low = (f.view(np.uint32) & 0xFFFF).astype(np.int64)
    decided = np.abs(low - 0x8000) > 4
    want = bf16_round(f)
    assert decided.sum() > 65000
    diff = np.nonzero(decided & (inplace.view(np.uint32) != want.view(np.uint32)))[0]
    assert diff.size == 0, [(float(g[i]), float(inplace[i]), float(want[i])) for i in diff[:8]]


@pytest.mark.parametrize("form", [0, 1])
def test_staged_swiglu_known_answers(rt, form):
    """Both device forms on the staged-SwiGLU known answers (the reference's case first,
    src/staged_metal_expert.rs:2826-2831): each output equals the independent evaluation
    (bf16 rounding in numpy, silu in f64, helpers.staged_swiglu_independent) with every rounding in
    place, and differs from the same evaluation with the case's named rounding taken out, so a
    device form missing that rounding fails here."""
    g = _f32_bits([c["g"] for c in STAGED_CASES])
    u = _f32_bits([c["u"] for c in STAGED_CASES])
    out, flags = _swiglu_device(rt, g, u, form)
    assert flags == 0
    got = out.view(np.uint32).tolist()
    for c, bits in zip(STAGED_CASES, got):
        assert bits == staged_swiglu_independent(c["g"], c["u"]) == c["out"], (hex(c["g"]), hex(bits))
        for stage in c["dropped"]:
            assert bits != staged_swiglu_independent(c["g"], c["u"], drop=stage), (hex(c["g"]), stage)
    assert {st for c in STAGED_CASES for st in c["dropped"]} == set(STAGES)


def test_staged_swiglu_flags_nonfinite(rt):
    g = np.array([1.0, np.inf, 2.0], np.float32)
    _, flags = _swiglu_device(rt, g, np.ones(3, np.float32), 0)
    assert flags & P.FLAG_SWIGLU_NONFINITE


# ------------------------------------------------------------------ closed-form mode-B layers
def _bank_from(rt, experts, n):
    projs = {e: (rt.bind_projection(v[0], v[1]), rt.bind_projection(v[2], v[3]), rt.bind_projection(v[4], v[5]))
             for e, v in experts.items()}
    bank = rt.expert_bank([projs[e][0] for e in range(n)], [projs[e][1] for e in range(n)],
                          [projs[e][2] for e in range(n)])
    return projs, bank


def _bindings(projs, sel, w):
    out = []
    for e in sorted(set(sel.reshape(-1).tolist())):
        pos, slot = np.nonzero(sel == e)
        order = np.argsort(pos, kind="stable")
        out.append(P.WideExpertBinding(e, pos[order].astype(np.uint32), w[pos[order], slot[order]].astype(np.float32),
                                       *projs[e]))
    return out


def _device_layer(rt, bank, x, sel, w, out_dtype, prefill=False):
    torch = _torch()
    rows = x.shape[0]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    ids = torch.from_numpy(sel.astype(np.int32)).cuda()
    wts = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    out = torch.empty((rows, x.shape[1]), dtype=torch.int16 if out_dtype == P.DTYPE_BF16 else torch.float32,
                      device="cuda")
    if prefill:
        rt.moe_prefill_device(bank, xt, rows, ids, wts, out, x_dtype=P.DTYPE_F32, out_dtype=out_dtype,
                              stream=_stream())
    else:
        rt.moe_layer_device(bank, xt, rows, ids, wts, out, mode=P.MODE_B, x_dtype=P.DTYPE_F32, out_dtype=out_dtype,
                            stream=_stream())
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    o = out.cpu().numpy()
    return (o.view(np.uint16).astype(np.uint32) << 16).view(np.float32) if out_dtype == P.DTYPE_BF16 else o


@pytest.fixture(scope="module")
def closed_form(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570100, 256, 12)
    projs, bank = _bank_from(rt, experts, 12)
    return experts, x, sel, w, projs, bank


def _same_bits(got, want):
    d = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert d[0].size == 0, f"{d[0].size} values differ, first at {d[0][0], d[1][0]}: {got[d][0]} vs {want[d][0]}"


@pytest.mark.parametrize("rows", [1, 5, 32])
def test_closed_form_mode_b_execute_bit_exact(rt, closed_form, rows):
    experts, x, sel, w, projs, _ = closed_form
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want = O.moe_layer("b", x, experts, 12, sel, w)
    got = rt.execute(x, _bindings(projs, sel, w), mode=P.MODE_B).output
    _same_bits(got, want)


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_closed_form_mode_b_device_layer_bit_exact(rt, closed_form, rows):
    experts, x, sel, w, _, bank = closed_form
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 12, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16), want)


@pytest.mark.parametrize("rows", [1, 40, 192, 256])
def test_closed_form_prefill_bit_exact(rt, closed_form, rows):
    """The grouped FP8 GEMM prefill (table silu, fused SwiGLU re-quantisation, each hidden group's
    maximum at another of its 128 rows) on closed-form data, up to 256 rows (117 to 141 placements
    per expert at 192 rows: one full 128-slot m-tile or a second with a few slots; 152 to 187 at
    256 rows: two m-tiles each)."""
    experts, x, sel, w, _, bank = closed_form
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 12, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW, prefill=True), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16, prefill=True), want)


@pytest.fixture(scope="module")
def closed_form_two_step(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570300, 144, 8, hidden=512, inter=512)
    projs, bank = _bank_from(rt, experts, 8)
    return experts, x, sel, w, projs, bank


@pytest.mark.parametrize("rows", [9, 144])
def test_closed_form_prefill_two_steps_bit_exact(rt, closed_form_two_step, rows):
    """Hidden 512, intermediate 512, top-8 of 8 experts: two 256-column K steps per projection (the
    gate/up workgroups start at either step and wrap); 144 rows give each expert a full 128-slot
    m-tile and a 16-slot one. Bit for bit the oracle's layer."""
    experts, x, sel, w, _, bank = closed_form_two_step
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 8, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW, prefill=True), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16, prefill=True), want)


@pytest.fixture(scope="module")
def closed_form_wide(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570400, 40, 8, hidden=4096, inter=512)
    projs, bank = _bank_from(rt, experts, 8)
    return experts, x, sel, w, projs, bank


@pytest.mark.parametrize("rows", [1, 40])
def test_closed_form_prefill_production_steps_bit_exact(rt, closed_form_wide, rows):
    """Hidden 4096 (the production hidden size), intermediate 512, top-8 of 8 experts: the gate/up
    GEMM's sixteen 256-column K steps, each workgroup starting at its own step and wrapping, and
    the down GEMM's sixteen 256-row n-tiles of two K steps, four per workgroup with the next
    n-tile's first weights loaded during the last steps of the one before. Bit for bit the
    oracle's layer."""
    experts, x, sel, w, _, bank = closed_form_wide
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 8, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW, prefill=True), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16, prefill=True), want)


@pytest.fixture(scope="module")
def closed_form_production(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570500, 24, 8, hidden=4096, inter=2048)
    projs, bank = _bank_from(rt, experts, 8)
    return experts, x, sel, w, projs, bank


def test_closed_form_prefill_production_shape_bit_exact(rt, closed_form_production):
    """The production expert shape, hidden 4096 and intermediate 2048, top-8 of 8 experts over 24
    rows: the gate/up GEMM's sixteen rotated 256-column K steps over 4096 stacked gate and up rows,
    and the down GEMM at its real K of 2048 (eight 256-column steps, four 256-row n-tiles per
    workgroup). Bit for bit the oracle's layer, raw f32 and bf16."""
    experts, x, sel, w, _, bank = closed_form_production
    want, want_raw = O.moe_layer("b", x, experts, 8, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW, prefill=True), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16, prefill=True), want)
    # the mode-B decode layer on the first eight rows, the same bits
    want8, want8_raw = O.moe_layer("b", x[:8], experts, 8, sel[:8], w[:8], raw=True)
    _same_bits(_device_layer(rt, bank, x[:8], sel[:8], w[:8], P.DTYPE_F32_RAW), want8_raw)


def test_closed_form_mode_b_device_layer_wide_hidden_bit_exact(rt, closed_form_wide):
    """The mode-B decode layer (eight rows) on the hidden-4096 closed form, bit for bit."""
    experts, x, sel, w, _, bank = closed_form_wide
    x, sel, w = x[:8], sel[:8], w[:8]
    want, want_raw = O.moe_layer("b", x, experts, 8, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW), want_raw)


@pytest.fixture(scope="module")
def closed_form_odd(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570200, 96, 12, hidden=384)
    projs, bank = _bank_from(rt, experts, 12)
    return experts, x, sel, w, projs, bank


@pytest.mark.parametrize("rows", [1, 96])
def test_closed_form_prefill_odd_blocks_bit_exact(rt, closed_form_odd, rows):
    """Hidden 384 (an odd count of 128-column blocks): the prefill's gate/up takes one-block K
    steps with 128-row tiles (hidden 256 takes two-block steps with 256-row tiles); bit for bit the
    oracle's layer."""
    experts, x, sel, w, _, bank = closed_form_odd
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 12, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW, prefill=True), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16, prefill=True), want)


@pytest.mark.parametrize("rows", [1, 8])
def test_closed_form_mode_b_expert_forward_bit_exact(rt, closed_form, rows):
    torch = _torch()
    experts, x, _, _, _, bank = closed_form
    e = 3
    want = O.moe_layer("b", x[:rows], experts, 12, np.full((rows, 1), e, np.uint32), np.ones((rows, 1), np.float32))
    xt = torch.from_numpy(np.ascontiguousarray(x[:rows])).cuda()
    out = torch.empty((rows, x.shape[1]), dtype=torch.float32, device="cuda")
    rt.expert_forward_device(bank, e, xt, rows, out, mode=P.MODE_B, x_dtype=P.DTYPE_F32, out_dtype=P.DTYPE_F32,
                             stream=_stream())
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    _same_bits(out.cpu().numpy(), want)


def _expert_forward(rt, bank, e, x, out_dtype):
    torch = _torch()
    rows = x.shape[0]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out = torch.empty((rows, x.shape[1]), dtype=torch.int16 if out_dtype == P.DTYPE_BF16 else torch.float32,
                      device="cuda")
    rt.expert_forward_device(bank, e, xt, rows, out, mode=P.MODE_B, x_dtype=P.DTYPE_F32, out_dtype=out_dtype,
                             stream=_stream())
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    o = out.cpu().numpy()
    return (o.view(np.uint16).astype(np.uint32) << 16).view(np.float32) if out_dtype == P.DTYPE_BF16 else o


@pytest.mark.parametrize("rows", [1, 8, 16, 17])
def test_closed_form_mode_b_expert_forward_production_bit_exact(rt, closed_form_production, rows):
    """The one-expert forward in mode B at the production expert shape (hidden 4096, intermediate
    2048): up to 16 rows run as whole-K workgroups (gate/up of 8 + 8 stacked rows, the down writing
    the output rows), 17 rows take the split kernels. Bit for bit the oracle's layer, f32 (also as
    F32_RAW, which in mode B is the rounded expert output) and bf16."""
    experts, x, _, _, _, bank = closed_form_production
    e = 5
    xr = x[:rows]
    want = O.moe_layer("b", xr, experts, 8, np.full((rows, 1), e, np.uint32), np.ones((rows, 1), np.float32))
    for dt in (P.DTYPE_F32, P.DTYPE_F32_RAW, P.DTYPE_BF16):
        _same_bits(_expert_forward(rt, bank, e, xr, dt), want)


@pytest.mark.parametrize("rows", [1, 16, 17])
def test_closed_form_mode_b_device_layer_production_rows_bit_exact(rt, closed_form_production, rows):
    """The mode-B decode layer at the production expert shape with one row (one-row experts: 8 + 8
    stacked gate/up rows per workgroup), sixteen rows (sixteen rows per expert in LDS) and seventeen
    (the split kernels), top-8 of 8 experts; bit for bit the oracle's layer."""
    experts, x, sel, w, _, bank = closed_form_production
    x, sel, w = x[:rows], sel[:rows], w[:rows]
    want, want_raw = O.moe_layer("b", x, experts, 8, sel, w, raw=True)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_F32_RAW), want_raw)
    _same_bits(_device_layer(rt, bank, x, sel, w, P.DTYPE_BF16), want)


@pytest.fixture(scope="module")
def closed_form_dense(rt):
    experts, x, sel, w = closed_form_mode_b(0x50570600, 8, 1, hidden=1024, inter=16384, top_k=1, down_block_step=8)
    projs, bank = _bank_from(rt, experts, 1)
    return experts, x, projs, bank


@pytest.mark.parametrize("rows", [1, 8])
def test_closed_form_mode_b_dense_mlp_bit_exact(rt, closed_form_dense, rows):
    """The dense layer-0 MLP's intermediate 16384 as a one-expert bank in mode B (hidden 1024 keeps
    the fixture small): the down's K of 16384 runs as four K shares whose sums are added in share
    order by the output rounding (the down weights hold codes in every eighth 128-column block, four
    blocks per share, which keeps every sum exact). Bit for bit the oracle's layer, f32 and bf16."""
    experts, x, _, bank = closed_form_dense
    xr = x[:rows]
    want = O.moe_layer("b", xr, experts, 1, np.zeros((rows, 1), np.uint32), np.ones((rows, 1), np.float32))
    for dt in (P.DTYPE_F32, P.DTYPE_BF16):
        _same_bits(_expert_forward(rt, bank, 0, xr, dt), want)


# ------------------------------------------------------------------ layer vs separate calls
@pytest.mark.parametrize("rows", [1, 5, 8])
def test_mode_b_layer_equals_unfused_calls(rt, rows):
    """The routed layer (gate and up in one pass with the SwiGLU fused) equals the same experts run
    as separate projection calls, the separate staged SwiGLU and a host combine in ascending expert
    id, bit for bit. Shapes where the two paths add the same block partials in the same order
    (hidden 512: four 128-column blocks, one per wave; intermediate 256: two)."""
    torch = _torch()
    rng = np.random.default_rng(900 + rows)
    hidden, inter, n = 512, 256, 12
    experts = {}
    for e in range(n):
        gs, us = log_uniform_scales(rng, inter, hidden), log_uniform_scales(rng, inter, hidden)
        ds = log_uniform_scales(rng, hidden, inter)
        experts[e] = (fp8_weight(rng, inter, hidden, gs), gs, fp8_weight(rng, inter, hidden, us), us,
                      fp8_weight(rng, hidden, inter, ds), ds)
    projs, _ = _bank_from(rt, experts, n)
    x = bf16_normal(rng, (rows, hidden))
    sel = np.stack([rng.permutation(n)[:8] for _ in range(rows)]).astype(np.uint32)
    w = rng.uniform(0.05, 1.0, (rows, 8)).astype(np.float32)
    layer = rt.execute(x, _bindings(projs, sel, w), mode=P.MODE_B).output
    block = np.zeros((rows, hidden), np.float32)
    for e in sorted(set(sel.reshape(-1).tolist())):
        pos = [p for p in range(rows) if e in sel[p].tolist()]
        g = rt.execute_fp8_linear(x[pos], projs[e][0], mode=P.MODE_B).output
        u = rt.execute_fp8_linear(x[pos], projs[e][1], mode=P.MODE_B).output
        h, flags = _swiglu_device(rt, g, u, 0)
        assert flags == 0
        y = rt.execute_fp8_linear(h.reshape(len(pos), inter), projs[e][2], mode=P.MODE_B).output
        for l, p in enumerate(pos):
            block[p] = block[p] + y[l] * w[p, sel[p].tolist().index(e)]
    _same_bits(layer, bf16_round(block))


# ------------------------------------------------------------------ mode-A hidden
@pytest.mark.parametrize("hidden,inter,rows", [(4096, 2048, 1), (4096, 2048, 8), (256, 256, 3)])
def test_mode_a_hidden_through_identity_down(rt, hidden, inter, rows):
    """An expert whose down projection is the identity returns its f32 SwiGLU hidden
    (g / (1 + e^-g)) * u unrounded: the three bf16 planes must carry it exactly. Gate/up sums are
    exact (e4m3 activations and weights in [1, 2), power-of-two scales), so the only difference
    from the oracle is the exp (a few f32 steps); dropping the lowest plane moves values by up to
    2^-16 relative. Hidden 4096 takes the whole-K fused gate/up kernel, 256 the split-K one."""
    torch = _torch()
    rng = np.random.default_rng(hidden + rows)
    gw, uw = _unit_codes(rng, (inter, hidden), 0.3), _unit_codes(rng, (inter, hidden), 0.3)
    gs = (2.0 ** rng.integers(-7, -5, (inter // 128, hidden // 128))).astype(np.float32)
    us = (2.0 ** rng.integers(-7, -5, (inter // 128, hidden // 128))).astype(np.float32)
    dw = np.zeros((hidden, inter), np.uint8)
    dw[np.arange(inter), np.arange(inter)] = 0x38
    ds = np.ones((hidden // 128, inter // 128), np.float32)
    ex = (gw, gs, uw, us, dw, ds)
    _, bank = _bank_from(rt, {0: ex}, 1)
    xs = decode_table()[_unit_codes(rng, (rows, hidden), 0.2)].astype(np.float32)
    xt = torch.from_numpy(to_bf16_bits(xs).view(np.int16)).cuda()
    out = torch.empty((rows, hidden), dtype=torch.float32, device="cuda")
    rt.expert_forward_device(bank, 0, xt, rows, out, mode=P.MODE_A, x_dtype=P.DTYPE_BF16, out_dtype=P.DTYPE_F32_RAW,
                             stream=_stream())
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    got = out.cpu().numpy()
    g = O.gemm_mode_a(gw, gs, xs)
    u = O.gemm_mode_a(uw, us, xs)
    h = O.swiglu_f32(g, u)
    assert not np.any(got[:, inter:])
    ulp = np.spacing(np.abs(h)).astype(np.float64)
    err = np.abs(got[:, :inter].astype(np.float64) - h) / ulp
    assert err.max() <= 4, err.max()
