"""GPU parity of the on-device router (route_mlp, src/text_endpoint.rs:4342-4473) through the C ABI.

Routes are integer work and must match the C oracle bit for bit: selected expert ids in libc++
nth_element order, renormalised weights, sigmoid scores and tie counts. The oracle's logits use the
same declared summation order (256 partial fused multiply-add sums over 8-column groups, halving
trees per wave, then (w0 + w1) + (w2 + w3)), and its top-k order is pinned by the reference's
golden orders (pw0063, pw0157). The device splits nth_element's partitions across a wave; the
pattern tests drive its guard, fallback and already-sorted branches.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import workloads as WL

pytestmark = pytest.mark.gpu


def _bf16_dev(torch, a):
    return torch.from_numpy(WL.bf16_bits_np(a).view(np.int16)).cuda()


def _device_route(rt, torch, x, rw, bias, x_f32=False, w_f32=False):
    rows, hidden = x.shape
    experts = rw.shape[0]
    xt = torch.from_numpy(x.astype(np.float32)).cuda() if x_f32 else _bf16_dev(torch, x)
    wt = torch.from_numpy(rw.astype(np.float32)).cuda() if w_f32 else _bf16_dev(torch, rw)
    bt = torch.from_numpy(bias.astype(np.float32)).cuda()
    ids = torch.zeros((rows, 8), dtype=torch.int32, device="cuda")
    wts = torch.zeros((rows, 8), dtype=torch.float32, device="cuda")
    scores = torch.zeros((rows, experts), dtype=torch.float32, device="cuda")
    ties = torch.zeros(1, dtype=torch.int32, device="cuda")
    rt.route_device(xt, rows, hidden, wt, experts, bt, ids, wts, x_dtype=P.DTYPE_F32 if x_f32 else P.DTYPE_BF16,
                    w_dtype=P.DTYPE_F32 if w_f32 else P.DTYPE_BF16, scores=scores, tie_rows=ties,
                    stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    flags = rt.take_flags()
    return (ids.cpu().numpy().astype(np.uint32), wts.cpu().numpy(), scores.cpu().numpy(), int(ties.item()), flags)


@pytest.mark.parametrize("rows,zipf", [(1, False), (2, False), (3, True), (8, False), (8, True), (12, False),
                                       (32, False), (300, True)])
def test_device_routes_bit_exact(rt, rows, zipf):
    """Scores, routes, weights and ties bit-exact with the oracle: 1, 2, 3 (four loaded rows, the
    last reread) and 8 rows per scores workgroup, and 12 rows (a chunk of eight, then one of four)."""
    import torch
    x = WL.activations(rows, WL.SEED_BASE + 60 + rows)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, bias)
    assert flags == 0
    _, ref_scores, ref_sel, ref_w, ref_ties = O.route(x, rw, bias)
    assert np.array_equal(scores.view(np.uint32), ref_scores.view(np.uint32))
    assert np.array_equal(ids, ref_sel)
    assert np.array_equal(wts.view(np.uint32), ref_w.view(np.uint32))
    assert ties == ref_ties


def test_device_routes_f32_inputs(rt):
    """f32 activations and f32 router weights (the checkpoint stores the router in F32)."""
    import torch
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    rw = (rng.standard_normal((256, 4096)) * 0.02).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, 256).astype(np.float32)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, bias, x_f32=True, w_f32=True)
    assert flags == 0
    _, ref_scores, ref_sel, ref_w, ref_ties = O.route(x, rw, bias)
    assert np.array_equal(ids, ref_sel)
    assert np.array_equal(wts.view(np.uint32), ref_w.view(np.uint32))
    assert np.array_equal(scores.view(np.uint32), ref_scores.view(np.uint32))


def test_device_routes_with_ties(rt):
    """Logits equal to chosen values (one-hot activation on column 0), with repeated values at the
    top-8 boundary: the selection order is the libc++ partition order and ties are counted."""
    import torch
    rows, hidden, experts = 6, 256, 64
    rng = np.random.default_rng(5)
    x = np.zeros((rows, hidden), np.float32)
    x[:, 0] = 1.0
    rw = np.zeros((experts, hidden), np.float32)
    levels = np.array([0.5, 0.25, 0.125, 0.0625, -0.5], np.float32)
    rw[:, 0] = levels[rng.integers(0, levels.size, experts)]
    bias = np.zeros(experts, np.float32)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, bias, x_f32=True, w_f32=True)
    _, ref_scores, ref_sel, ref_w, ref_ties = O.route(x, rw, bias)
    assert flags == 0
    assert np.array_equal(ids, ref_sel)
    assert np.array_equal(wts.view(np.uint32), ref_w.view(np.uint32))
    assert ties == ref_ties and ties == rows


def _pattern(kind, experts, rng):
    if kind == "random":
        return rng.standard_normal(experts).astype(np.float32)
    if kind == "levels":
        return np.array([0.5, 0.25, -0.125, 1.0], np.float32)[rng.integers(0, 4, experts)]
    if kind == "equal":
        return np.full(experts, 0.75, np.float32)
    if kind == "ascending":
        return np.linspace(-2, 2, experts).astype(np.float32)
    if kind == "descending":
        return np.linspace(2, -2, experts).astype(np.float32)
    if kind == "one_high":
        v = np.full(experts, -1.0, np.float32)
        v[experts // 2] = 3.0
        return v
    raise ValueError(kind)


KINDS = ["random", "levels", "equal", "ascending", "descending", "one_high"]


@pytest.mark.parametrize("experts", [9, 100, 257, 1024])
@pytest.mark.parametrize("hidden", [8, 2056])
def test_device_routes_patterns(rt, experts, hidden):
    """Row r has logits = pattern r exactly (x one-hot on column r): ties everywhere, all-equal rows,
    sorted rows, expert counts that are not multiples of the wave, hidden sizes off the 2048 stride."""
    import torch
    rng = np.random.default_rng(experts * 7 + hidden)
    rows = len(KINDS)
    x = np.zeros((rows, hidden), np.float32)
    rw = np.zeros((experts, hidden), np.float32)
    for r, kind in enumerate(KINDS):
        x[r, r] = 1.0
        rw[:, r] = _pattern(kind, experts, rng)
    bias = np.zeros(experts, np.float32)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, bias, x_f32=True, w_f32=True)
    assert flags == 0
    _, ref_scores, ref_sel, ref_w, ref_ties = O.route(x, rw, bias)
    assert np.array_equal(scores.view(np.uint32), ref_scores.view(np.uint32))
    assert np.array_equal(ids, ref_sel)
    assert np.array_equal(wts.view(np.uint32), ref_w.view(np.uint32))
    assert ties == ref_ties


def test_device_routes_many_rows_ragged(rt):
    """1000 rows (125 row chunks), 300 experts, bf16, hidden 4104 (not a multiple of 2048)."""
    import torch
    rng = np.random.default_rng(21)
    x = WL.bf16_round_np(rng.standard_normal((1000, 4104)).astype(np.float32))
    rw = WL.bf16_round_np((rng.standard_normal((300, 4104)) * 0.02).astype(np.float32))
    bias = rng.uniform(-0.01, 0.01, 300).astype(np.float32)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, bias)
    assert flags == 0
    _, ref_scores, ref_sel, ref_w, ref_ties = O.route(x, rw, bias)
    assert np.array_equal(scores.view(np.uint32), ref_scores.view(np.uint32))
    assert np.array_equal(ids, ref_sel)
    assert np.array_equal(wts.view(np.uint32), ref_w.view(np.uint32))
    assert ties == ref_ties


def test_device_router_rejects_bad_hidden(rt):
    import torch
    x = torch.zeros((4, 260), dtype=torch.int16, device="cuda")
    wt = torch.zeros((16, 260), dtype=torch.int16, device="cuda")
    bt = torch.zeros(16, dtype=torch.float32, device="cuda")
    ids = torch.zeros((4, 8), dtype=torch.int32, device="cuda")
    wts = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.route_device(x, 4, 260, wt, 16, bt, ids, wts)


def test_device_router_feeds_the_layer(rt):
    """Device routes drive the decode layer without a host round trip: same output as host routes."""
    import torch
    bank = WL.synth_bank(rt, n_experts=16, hidden=256, inter=128, seed=WL.SEED_BASE + 70)
    rows = 8
    x = WL.activations(rows, WL.SEED_BASE + 71, hidden=256)
    rng = np.random.default_rng(12)
    rw = WL.bf16_round_np((rng.standard_normal((16, 256)) * 0.02).astype(np.float32))
    bias = rng.uniform(-0.01, 0.01, 16).astype(np.float32)
    xt = _bf16_dev(torch, x)
    wt = _bf16_dev(torch, rw)
    bt = torch.from_numpy(bias).cuda()
    ids = torch.zeros((rows, 8), dtype=torch.int32, device="cuda")
    wts = torch.zeros((rows, 8), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rt.route_device(xt, rows, 256, wt, 16, bt, ids, wts, stream=stream)
    out_dev = torch.empty((rows, 256), dtype=torch.int16, device="cuda")
    rt.moe_layer_device(bank.bank, xt, rows, ids, wts, out_dev, mode=P.MODE_A, stream=stream)
    _, _, sel, w, _ = O.route(x, rw, bias)
    ids_h = torch.from_numpy(sel.astype(np.int32)).cuda()
    w_h = torch.from_numpy(w).cuda()
    out_host = torch.empty((rows, 256), dtype=torch.int16, device="cuda")
    rt.moe_layer_device(bank.bank, xt, rows, ids_h, w_h, out_host, mode=P.MODE_A, stream=stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    assert torch.equal(out_dev, out_host)


def test_device_router_flags_nonfinite_bias(rt):
    import torch
    x = WL.activations(4, WL.SEED_BASE + 72)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    bias = bias.copy()
    bias[17] = np.nan
    ids, wts, _, _, flags = _device_route(rt, torch, x, rw, bias)
    assert flags & P.FLAG_ROUTE
    assert (ids == 256).all() and (wts == 0).all()


def test_device_route_weights_known_answer(rt):
    """The device router's route weights on the known-answer rows of tests/helpers.py, which pin the
    reference's denominator (pytorch_sum_eight folded left to right over the selected scores in
    partition order, + 1e-20; src/text_endpoint.rs:4382-4390, :4450-4452): a tree or plain sum, a
    sum in expert-id order or a missing 1e-20 would change these bits. Logits enter exactly through
    a one-hot activation row and f32 router weights whose column 0 holds them."""
    import torch
    from helpers import ROUTE_WEIGHT_ROWS, route_weight_row_logits
    rows, hidden = len(ROUTE_WEIGHT_ROWS), 64
    x = np.zeros((rows, hidden), np.float32)
    rw = np.zeros((256, hidden), np.float32)
    for r, row in enumerate(ROUTE_WEIGHT_ROWS):
        x[r, r] = 1.0
        rw[:, r] = route_weight_row_logits(row)
    ids, wts, scores, ties, flags = _device_route(rt, torch, x, rw, np.zeros(256, np.float32), x_f32=True,
                                                  w_f32=True)
    assert flags == 0 and ties == 0
    for r, row in enumerate(ROUTE_WEIGHT_ROWS):
        assert ids[r].tolist() == row["selected"]
        assert scores[r][ids[r]].view(np.uint32).tolist() == row["score_bits"]
        assert wts[r].view(np.uint32).tolist() == row["weight_bits"]


@pytest.fixture(scope="module")
def router_full_bank(rt):
    return WL.synth_bank(rt, n_experts=256, seed=WL.SEED_BASE + 2)


def _routed_vs_two_calls(rt, torch, bank, x, rw, bias, mode, out_dtype=P.DTYPE_F32_RAW, w_f32=False):
    """(routes and output of pw_moe_layer_routed_device, the same of pw_route_device then
    pw_moe_layer_device, the device flags)."""
    rows, hidden = x.shape
    experts = rw.shape[0]
    xt = _bf16_dev(torch, x)
    wt = torch.from_numpy(rw.astype(np.float32)).cuda() if w_f32 else _bf16_dev(torch, rw)
    bt = torch.from_numpy(bias.astype(np.float32)).cuda()
    odt = torch.float32 if out_dtype != P.DTYPE_BF16 else torch.int16
    stream = torch.cuda.current_stream().cuda_stream
    res = []
    for fused in (True, False):
        ids = torch.full((rows, 8), -1, dtype=torch.int32, device="cuda")
        wts = torch.full((rows, 8), 7.0, dtype=torch.float32, device="cuda")
        out = torch.full((rows, hidden), 7, dtype=odt, device="cuda")
        wd = P.DTYPE_F32 if w_f32 else P.DTYPE_BF16
        if fused:
            rt.moe_layer_routed_device(bank.bank, xt, rows, wt, bt, ids, wts, out, mode=mode, w_dtype=wd,
                                       out_dtype=out_dtype, stream=stream)
        else:
            rt.route_device(xt, rows, hidden, wt, experts, bt, ids, wts, w_dtype=wd, stream=stream)
            rt.moe_layer_device(bank.bank, xt, rows, ids, wts, out, mode=mode, out_dtype=out_dtype, stream=stream)
        torch.cuda.synchronize()
        res.append((ids.cpu().numpy().astype(np.uint32), wts.cpu().numpy(), out.cpu().numpy()))
    return res[0], res[1], rt.take_flags()


@pytest.mark.parametrize("rows,mode", [(1, 0), (1, 1), (5, 0), (8, 0), (8, 1), (9, 0), (32, 1)])
def test_routed_layer_equals_router_then_layer(rt, router_full_bank, rows, mode):
    """pw_moe_layer_routed_device on the 256-expert bank at hidden 4096: the routes it writes equal
    the oracle's and pw_route_device's bit for bit, and its output equals pw_route_device followed by
    pw_moe_layer_device byte for byte -- the one-token mode A path (selection, then the schedule-free
    layer), the one-launch selection and schedule (2..8 rows), and the separate selection (9, 32)."""
    import torch
    x = WL.activations(rows, WL.SEED_BASE + 80 + rows)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=rows == 5)
    (fi, fw, fo), (ti, tw, to), flags = _routed_vs_two_calls(rt, torch, router_full_bank, x, rw, bias, mode)
    assert flags == 0
    _, _, ref_sel, ref_w, _ = O.route(x, rw, bias)
    assert np.array_equal(fi, ref_sel) and np.array_equal(fi, ti)
    assert np.array_equal(fw.view(np.uint32), ref_w.view(np.uint32)) and np.array_equal(fw.view(np.uint32),
                                                                                          tw.view(np.uint32))
    assert np.array_equal(fo.view(np.uint32), to.view(np.uint32))
    assert np.all(np.isfinite(fo)) and np.any(fo)


@pytest.mark.parametrize("experts", [16, 100, 300])
def test_routed_layer_expert_counts(rt, experts):
    """Banks of 16, 100 (the one-launch selection with one and two 64-expert registers per lane) and
    300 experts (above the one-launch bound: the separate selection kernel), hidden 256: the same
    routes and bytes as the two calls, f32 router weights, modes A and B, bf16 output."""
    import torch
    bank = WL.synth_bank(rt, n_experts=experts, hidden=256, inter=128, seed=WL.SEED_BASE + 85 + experts)
    rng = np.random.default_rng(experts)
    for rows, mode in ((3, 0), (8, 1), (1, 1)):
        x = WL.activations(rows, WL.SEED_BASE + 86 + rows, hidden=256)
        rw = (rng.standard_normal((experts, 256)) * 0.05).astype(np.float32)
        bias = rng.uniform(-0.01, 0.01, experts).astype(np.float32)
        (fi, fw, fo), (ti, tw, to), flags = _routed_vs_two_calls(rt, torch, bank, x, rw, bias, mode,
                                                                 out_dtype=P.DTYPE_BF16, w_f32=True)
        assert flags == 0
        assert np.array_equal(fi, ti) and np.array_equal(fw.view(np.uint32), tw.view(np.uint32))
        assert np.array_equal(fo, to)
        _, _, ref_sel, ref_w, _ = O.route(x, rw, bias)
        assert np.array_equal(fi, ref_sel)


def test_routed_layer_rejects_a_failed_row(rt, router_full_bank):
    """A NaN bias fails every row's routing: FLAG_ROUTE, ids E, zero weights, and the layer rejects the
    batch (FLAG_SCHEDULE) and writes zeros, on the one-launch path and the one-token path."""
    import torch
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    bias = bias.copy()
    bias[3] = np.nan
    for rows, mode in ((8, 0), (1, 0), (12, 1)):
        x = WL.activations(rows, WL.SEED_BASE + 90 + rows)
        (fi, fw, fo), _, flags = _routed_vs_two_calls(rt, torch, router_full_bank, x, rw, bias, mode)
        assert flags & P.FLAG_ROUTE and flags & P.FLAG_SCHEDULE
        assert (fi == 256).all() and not np.any(fw) and not np.any(fo.view(np.uint32))


@pytest.mark.parametrize("mode", [0, 1])
def test_routed_layer_tied_and_untied_rows(rt, mode):
    """The one-launch schedule finds each row's expert set without the partition when the row's
    top-8 boundary is untied, and partitions the rows whose boundary is tied (one-hot activations
    over five logit levels); the route order and weights come from the separate weights launch.
    Six rows, three of each kind, 64 experts, hidden 256, modes A and B: the same routes, weights and
    output bytes as pw_route_device then pw_moe_layer_device, the oracle's routes and tie count."""
    import torch
    hidden, experts, rows = 256, 64, 6
    bank = WL.synth_bank(rt, n_experts=experts, hidden=hidden, inter=128, seed=WL.SEED_BASE + 95)
    rng = np.random.default_rng(95)
    x = WL.activations(rows, WL.SEED_BASE + 96, hidden=hidden)
    x[:3] = 0.0
    x[:3, 0] = 1.0
    rw = (rng.standard_normal((experts, hidden)) * 0.05).astype(np.float32)
    levels = np.array([0.5, 0.25, 0.125, 0.0625, -0.5], np.float32)
    rw[:, 0] = levels[rng.integers(0, levels.size, experts)]
    bias = np.zeros(experts, np.float32)
    (fi, fw, fo), (ti, tw, to), flags = _routed_vs_two_calls(rt, torch, bank, x, rw, bias, mode,
                                                             out_dtype=P.DTYPE_BF16, w_f32=True)
    assert flags == 0
    _, _, ref_sel, ref_w, ref_ties = O.route(WL.bf16_round_np(x), rw, bias)
    assert ref_ties == 3
    assert np.array_equal(fi, ti) and np.array_equal(fi, ref_sel)
    assert np.array_equal(fw.view(np.uint32), tw.view(np.uint32))
    assert np.array_equal(fw.view(np.uint32), ref_w.view(np.uint32))
    assert np.array_equal(fo, to) and np.any(fo)
    # one-token batches of a tied and an untied row (mode A: the schedule-free one-token layer)
    for r in (0, 3):
        (fi, fw, fo), (ti, tw, to), flags = _routed_vs_two_calls(rt, torch, bank, x[r:r + 1], rw, bias, mode,
                                                                 out_dtype=P.DTYPE_BF16, w_f32=True)
        assert flags == 0
        assert np.array_equal(fi, ti) and np.array_equal(fi, ref_sel[r:r + 1])
        assert np.array_equal(fw.view(np.uint32), tw.view(np.uint32))
        assert np.array_equal(fo, to) and np.any(fo)


def test_routed_layer_rejects_zero_route_weights(rt):
    """Logits near -256 make every sigmoid score 0 while the biases (distinct) still rank the experts,
    so the expert sets are found without a tie, but the weights are 0 / 1e-20 = 0 and fail the
    reference's sum check: the weights launch must reject the batch it did not schedule itself --
    FLAG_ROUTE and FLAG_SCHEDULE, ids E, zero weights, zero output, as pw_route_device then
    pw_moe_layer_device give."""
    import torch
    hidden, experts, rows = 256, 64, 2
    bank = WL.synth_bank(rt, n_experts=experts, hidden=hidden, inter=128, seed=WL.SEED_BASE + 97)
    v = WL.activations(1, WL.SEED_BASE + 98, hidden=hidden)[0]
    x = np.stack([v, v])
    vb = (WL.bf16_bits_np(v).astype(np.uint32) << 16).view(np.float32)
    assert float(np.dot(vb.astype(np.float64), vb)) > 120.0
    rw = np.tile(-vb, (experts, 1)).astype(np.float32)
    bias = np.random.default_rng(97).permutation(experts).astype(np.float32) * np.float32(1e-3)
    for mode, n in ((0, 2), (1, 2), (0, 1), (1, 1)):
        (fi, fw, fo), (ti, tw, to), flags = _routed_vs_two_calls(rt, torch, bank, x[:n], rw, bias, mode, w_f32=True)
        assert flags & P.FLAG_ROUTE and flags & P.FLAG_SCHEDULE
        assert (fi == experts).all() and (ti == experts).all()
        assert not np.any(fw) and not np.any(tw)
        assert not np.any(fo.view(np.uint32)) and not np.any(to.view(np.uint32))
