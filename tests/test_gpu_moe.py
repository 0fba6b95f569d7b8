"""GPU parity of the routed-MoE path (schedule, fused gate/up + SwiGLU, down, combine) against the
C oracle, through the C ABI: the reference's execute/execute_fused_gate_up host surface and the
device-resident layer on a full 256-expert bank.

Tolerances: mode A products are exact (e4m3 weights times bf16 activation planes), so the f32
combine before the final bf16 round may differ from the oracle only by summation order: each
element within 1e-8 of its condition scale C (the sum of the magnitudes of every term whose
rounding reaches it, `helpers.moe_condition`; observed at most 1.6e-9 C on MI355X), and bf16
outputs within one rounding step of that. Mode B <= 2e-2 max|d|/max|ref| (block sums come from the
FP8 MFMA, which truncates products 14 bits below a block's largest). Routes, placement counts and
the schedule are integer work and bit-exact.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import workloads as WL
from helpers import (bf16_normal, fp8_weight, log_uniform_scales, moe_condition, normwise, rel_l2,
                     within_bf16_cond)

pytestmark = pytest.mark.gpu

# mode A: |got - oracle| <= COND_REL * C per element on the f32 combine; bf16 outputs may also sit
# on the other side of one bf16 rounding boundary
COND_REL = 1e-8


def check_mode_a(got, ref, cond, raw):
    """got/ref f32 combines (raw) or bf16-valued outputs against the oracle's, element-wise."""
    if raw:
        d = np.abs(got.astype(np.float64) - ref)
        assert np.all(d <= COND_REL * cond), float((d / np.maximum(cond, 1e-30)).max())
    else:
        assert within_bf16_cond(got, ref, cond, rel=COND_REL)


def make_experts(rng, n, hidden, inter):
    ex = {}
    for e in range(n):
        gs = log_uniform_scales(rng, inter, hidden)
        us = log_uniform_scales(rng, inter, hidden)
        ds = log_uniform_scales(rng, hidden, inter)
        ex[e] = (fp8_weight(rng, inter, hidden, gs), gs, fp8_weight(rng, inter, hidden, us), us,
                 fp8_weight(rng, hidden, inter, ds), ds)
    return ex


def random_routes(rng, rows, n_experts):
    logits = rng.standard_normal((rows, n_experts)).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, n_experts).astype(np.float32)
    scores = np.vectorize(O.sigmoid_f32, otypes=[np.float32])(logits)
    sel, w, _ = O.noaux_routes(scores, bias)
    return sel, w


def bindings_from_routes(projs, sel, w):
    """BTreeMap schedule of src/text_endpoint.rs:4767-4775: experts ascending, positions ascending."""
    out = []
    for e in sorted(set(sel.reshape(-1).tolist())):
        pos, wts = np.nonzero(sel == e)
        order = np.argsort(pos, kind="stable")
        g, u, d = projs[e]
        out.append(P.WideExpertBinding(e, pos[order].astype(np.uint32),
                                       w[pos[order], wts[order]].astype(np.float32), g, u, d))
    return out


@pytest.fixture(scope="module")
def small_layer(rt):
    rng = np.random.default_rng(42)
    hidden, inter, n = 512, 256, 12
    experts = make_experts(rng, n, hidden, inter)
    projs = {e: (rt.bind_projection(v[0], v[1]), rt.bind_projection(v[2], v[3]), rt.bind_projection(v[4], v[5]))
             for e, v in experts.items()}
    return experts, projs, hidden, inter, n


@pytest.mark.parametrize("rows", [1, 5, 8])
@pytest.mark.parametrize("mode", [P.MODE_A, P.MODE_B])
def test_execute_matches_oracle(rt, small_layer, rows, mode):
    experts, projs, hidden, inter, n = small_layer
    rng = np.random.default_rng(rows * 10 + mode)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = random_routes(rng, rows, n)
    res = rt.execute(x, bindings_from_routes(projs, sel, w), mode=mode)
    ref = O.moe_layer("a" if mode == P.MODE_A else "b", x, experts, n, sel, w)
    assert res.unique_experts == len(set(sel.reshape(-1).tolist()))
    assert res.expert_rows == rows * 8
    if mode == P.MODE_A:
        check_mode_a(res.output, ref, moe_condition(x, experts, sel, w), raw=False)
    else:
        assert normwise(res.output, ref) <= 2e-2


@pytest.fixture(scope="module")
def wide_layer(rt):
    rng = np.random.default_rng(64)
    hidden, inter, n = 256, 128, 64
    experts = make_experts(rng, n, hidden, inter)
    projs = {e: (rt.bind_projection(v[0], v[1]), rt.bind_projection(v[2], v[3]), rt.bind_projection(v[4], v[5]))
             for e, v in experts.items()}
    return experts, projs, hidden, inter, n


@pytest.mark.parametrize("rows", [64, 128])
@pytest.mark.parametrize("mode", [P.MODE_A, P.MODE_B])
def test_execute_layer_major_slices(rt, wide_layer, rows, mode):
    """The reference's layer-major prefill drives execute with 128-row slices (LAYER_MAJOR_ROWS,
    src/wide_metal_moe.rs:11, checked at :858): 64 and 128 rows over 64 experts, each expert at
    most 32 placements."""
    experts, projs, hidden, inter, n = wide_layer
    rng = np.random.default_rng(rows + mode)
    x = bf16_normal(rng, (rows, hidden))
    sel, w = random_routes(rng, rows, n)
    assert np.bincount(sel.reshape(-1), minlength=n).max() <= 32
    res = rt.execute(x, bindings_from_routes(projs, sel, w), mode=mode)
    ref = O.moe_layer("a" if mode == P.MODE_A else "b", x, experts, n, sel, w)
    assert res.expert_rows == rows * 8
    if mode == P.MODE_A:
        check_mode_a(res.output, ref, moe_condition(x, experts, sel, w), raw=False)
    else:
        assert normwise(res.output, ref) <= 2e-2 and rel_l2(res.output, ref) <= 5e-3


def test_thirty_two_rows_per_expert(rt, small_layer):
    """The reference's widest specialisation (MAX_EXPERT_ROWS = 32, src/wide_metal_moe.rs:12)."""
    experts, projs, hidden, inter, n = small_layer
    rng = np.random.default_rng(4)
    rows = 32
    x = rng.standard_normal((rows, hidden)).astype(np.float32)  # f32 activations (three-plane split path)
    sel = np.tile(np.arange(8, dtype=np.uint32), (rows, 1))
    w = np.full((rows, 8), 0.125, np.float32)
    for mode in (P.MODE_A, P.MODE_B):
        res = rt.execute(x, bindings_from_routes(projs, sel, w), mode=mode)
        ref = O.moe_layer("a" if mode == P.MODE_A else "b", x, experts, n, sel, w)
        if mode == P.MODE_A:
            check_mode_a(res.output, ref, moe_condition(x, experts, sel, w), raw=False)
        else:
            assert normwise(res.output, ref) <= 2e-2


def test_slot_order_does_not_change_output(rt, small_layer):
    """Placements are combined in ascending expert id whatever the route-slot order."""
    experts, projs, hidden, inter, n = small_layer
    rng = np.random.default_rng(5)
    x = bf16_normal(rng, (4, hidden))
    sel, w = random_routes(rng, 4, n)
    base = rt.execute(x, bindings_from_routes(projs, sel, w), mode=P.MODE_A).output
    perm = np.stack([rng.permutation(8) for _ in range(4)])
    sel2 = np.take_along_axis(sel, perm, 1)
    w2 = np.take_along_axis(w, perm, 1)
    again = rt.execute(x, bindings_from_routes(projs, sel2, w2), mode=P.MODE_A).output
    assert np.array_equal(base.view(np.uint32), again.view(np.uint32))


def test_schedule_validation_fails_closed(rt, small_layer):
    experts, projs, hidden, inter, n = small_layer
    x = np.ones((2, hidden), np.float32)
    g, u, d = projs[0]
    mk = lambda pos, wts, e=0: P.WideExpertBinding(e, np.array(pos, np.uint32), np.array(wts, np.float32), *projs[e])
    full = [mk([0, 1], [0.125, 0.125], e) for e in range(8)]
    assert rt.execute(x, full, mode=P.MODE_A).expert_rows == 16
    with pytest.raises(P.PwError, match="SCHEDULE"):
        rt.execute(x, full[:7], mode=P.MODE_A)  # 14 placements for 2 rows
    with pytest.raises(P.PwError, match="SCHEDULE"):
        rt.execute(x, full[:7] + [mk([0, 2], [0.1, 0.1], 7)], mode=P.MODE_A)  # position >= rows
    with pytest.raises(P.PwError, match="SCHEDULE"):
        rt.execute(x, full[:7] + [mk([0, 1], [0.1, np.nan], 7)], mode=P.MODE_A)
    with pytest.raises(P.PwError, match="SCHEDULE"):
        rt.execute(x, full[:6] + [mk([0, 0], [0.1, 0.1], 6), mk([1, 1], [0.1, 0.1], 7)], mode=P.MODE_A)
    bad = x.copy()
    bad[1, 3] = np.inf
    with pytest.raises(P.PwError, match="NONFINITE"):
        rt.execute(bad, full, mode=P.MODE_A)


def test_complete_expert_widths(rt):
    """One routed expert (gate/up [2 x 2048 x 4096], down [4096 x 2048]) at widths 1, 2, 4, 8."""
    import torch
    bank = WL.synth_bank(rt, n_experts=1, seed=WL.SEED_BASE + 1)
    host = bank.expert_host(0)
    for width in (1, 2, 4, 8):
        x = WL.activations(width, WL.SEED_BASE + 10 + width)
        xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
        out = torch.empty((width, 4096), dtype=torch.float32, device="cuda")
        rt.expert_forward_device(bank.bank, 0, xt, width, out, mode=P.MODE_A, out_dtype=P.DTYPE_F32_RAW,
                                 stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        raw = out.cpu().numpy()
        ref32, ref16 = O.expert_mode_a(x, host)
        one = np.zeros((width, 1), np.uint32)
        cond = moe_condition(x, {0: host}, one, np.ones((width, 1), np.float32))
        check_mode_a(raw, ref32, cond, raw=True)
        out16 = torch.empty((width, 4096), dtype=torch.float32, device="cuda")
        rt.expert_forward_device(bank.bank, 0, xt, width, out16, mode=P.MODE_A, out_dtype=P.DTYPE_F32,
                                 stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        check_mode_a(out16.cpu().numpy(), ref16, cond, raw=False)


@pytest.fixture(scope="module")
def full_bank(rt):
    return WL.synth_bank(rt, n_experts=256, seed=WL.SEED_BASE + 2)


@pytest.mark.parametrize("zipf", [False, True])
def test_decode_layer_256_experts_width8(rt, full_bank, zipf):
    """Width-8 routed-MoE decode layer: top-8 of 256 experts, hidden 4096, intermediate 2048."""
    import torch
    x = WL.activations(8, WL.SEED_BASE + 2)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    _, _, sel, w, ties = O.route(x, rw, bias)
    ids = torch.from_numpy(sel.astype(np.int32)).cuda()
    wts = torch.from_numpy(w).cuda()
    xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
    used = sorted(set(sel.reshape(-1).tolist()))
    experts = {e: full_bank.expert_host(e) for e in used}
    stream = torch.cuda.current_stream().cuda_stream
    for mode in (P.MODE_A, P.MODE_B):
        raw = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
        out = torch.empty((8, 4096), dtype=torch.int16, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, 8, ids, wts, raw, mode=mode, out_dtype=P.DTYPE_F32_RAW, stream=stream)
        rt.moe_layer_device(full_bank.bank, xt, 8, ids, wts, out, mode=mode, out_dtype=P.DTYPE_BF16, stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        ref, ref_raw = O.moe_layer("a" if mode == P.MODE_A else "b", x, experts, 256, sel, w, raw=True)
        got16 = (out.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        if mode == P.MODE_A:
            cond = moe_condition(x, experts, sel, w)
            check_mode_a(raw.cpu().numpy(), ref_raw, cond, raw=True)
            check_mode_a(got16, ref, cond, raw=False)
        else:
            assert normwise(got16, ref) <= 2e-2 and rel_l2(got16, ref) <= 5e-3


def test_decode_layer_is_deterministic(rt, full_bank):
    """The width-8 layer gives the same raw f32 bits for the same batch twice, modes A and B, with a
    different batch (other routes, so another schedule and other pieces) run in between."""
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    batches = []
    for seed in (WL.SEED_BASE + 2, WL.SEED_BASE + 40):
        x = WL.activations(8, seed)
        _, _, sel, w, _ = O.route(x, rw, bias)
        batches.append((torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda(),
                        torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda()))

    def layer(b, mode):
        xt, ids, wts = b
        raw = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, 8, ids, wts, raw, mode=mode, out_dtype=P.DTYPE_F32_RAW, stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        return raw.cpu().numpy()

    for mode in (P.MODE_A, P.MODE_B):
        first = layer(batches[0], mode)
        layer(batches[1], mode)
        again = layer(batches[0], mode)
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32))
        assert np.all(np.isfinite(first)) and np.any(first)


def test_whole_k_gateup_matches_split_k(rt, full_bank):
    """At hidden 4096 a batch of up to 8 bf16 rows takes the whole-K gate/up kernel (SwiGLU fused, no
    split partials in memory); 9 rows take the split-K kernel plus the SwiGLU kernel. Each token's
    result depends only on its own row and routes, and both paths add the same eight K-split sums
    in the same order, so the first 8 rows of a 9-row batch equal the 8-row batch bit for bit."""
    import torch
    x = WL.activations(9, WL.SEED_BASE + 80)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    _, _, sel, w, _ = O.route(x, rw, bias)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for rows in (8, 9):
        xt = torch.from_numpy(WL.bf16_bits_np(x[:rows]).view(np.int16)).cuda()
        ids = torch.from_numpy(sel[:rows].astype(np.int32)).cuda()
        wts = torch.from_numpy(w[:rows]).cuda()
        raw = torch.empty((rows, 4096), dtype=torch.float32, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, rows, ids, wts, raw, mode=P.MODE_A, out_dtype=P.DTYPE_F32_RAW,
                            stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        outs.append(raw.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1][:8].view(np.uint32))
    used = sorted(set(sel.reshape(-1).tolist()))
    experts = {e: full_bank.expert_host(e) for e in used}
    _, ref_raw = O.moe_layer("a", x, experts, 256, sel, w, raw=True)
    check_mode_a(outs[1], ref_raw, moe_condition(x, experts, sel, w), raw=True)


@pytest.mark.parametrize("width", [5, 6, 8])
def test_pieces_match_one_workgroup_schedule(rt, full_bank, width):
    """A decode batch of 5 to 8 rows runs both projections on pieces of at most four slots of an
    expert (its one-wave schedule cuts them). With every token on the same eight experts (width
    slots each: pieces of 4 + 1, 4 + 2, 4 + 4), the first rows of a 9-row batch (one-workgroup
    schedule, no pieces) equal the smaller batch bit for bit."""
    import torch
    x = WL.activations(9, WL.SEED_BASE + 130)
    sel = np.tile(np.array([17, 3, 250, 99, 128, 64, 5, 200], np.uint32), (9, 1))
    w = np.random.default_rng(5).uniform(0.01, 0.3, (9, 8)).astype(np.float32)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for rows in (width, 9):
        xt = torch.from_numpy(WL.bf16_bits_np(x[:rows]).view(np.int16)).cuda()
        ids = torch.from_numpy(sel[:rows].astype(np.int32)).cuda()
        wts = torch.from_numpy(w[:rows]).cuda()
        raw = torch.empty((rows, 4096), dtype=torch.float32, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, rows, ids, wts, raw, mode=P.MODE_A, out_dtype=P.DTYPE_F32_RAW,
                            stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        outs.append(raw.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1][:width].view(np.uint32))
    experts = {e: full_bank.expert_host(e) for e in sorted(set(sel.reshape(-1).tolist()))}
    _, ref_raw = O.moe_layer("a", x[:width], experts, 256, sel[:width], w[:width], raw=True)
    check_mode_a(outs[0], ref_raw, moe_condition(x[:width], experts, sel[:width], w[:width]), raw=True)


@pytest.mark.parametrize("x_f32", [False, True])
def test_one_token_equals_two_copies(rt, full_bank, x_f32):
    """Each token's result depends only on its own row and routes: a two-row batch holding the
    same token twice (every routed expert then has two placements) gives the one-row result in both
    rows, bit for bit, and that result matches the oracle. The one-row layer reads its eight routes
    in the fused gate/up and the one-token down+combine (no schedule launch); the two-row layer
    goes through the schedule, so the two paths are held to the same bits."""
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    for seed in (0, 1, 2):
        x = WL.activations(1, WL.SEED_BASE + 120 + seed)
        _, _, sel, w, _ = O.route(x, rw, bias)
        for out_dtype in (P.DTYPE_F32_RAW, P.DTYPE_BF16):
            outs = []
            for rows in (1, 2):
                xr = np.repeat(x, rows, axis=0)
                xt = (torch.from_numpy(np.ascontiguousarray(xr)).cuda() if x_f32
                      else torch.from_numpy(WL.bf16_bits_np(xr).view(np.int16)).cuda())
                ids = torch.from_numpy(np.repeat(sel, rows, axis=0).astype(np.int32)).cuda()
                wts = torch.from_numpy(np.repeat(w, rows, axis=0)).cuda()
                out = torch.empty((rows, 4096), dtype=torch.float32 if out_dtype == P.DTYPE_F32_RAW else torch.int16,
                                  device="cuda")
                rt.moe_layer_device(full_bank.bank, xt, rows, ids, wts, out, mode=P.MODE_A,
                                    x_dtype=P.DTYPE_F32 if x_f32 else P.DTYPE_BF16, out_dtype=out_dtype,
                                    stream=stream)
                torch.cuda.synchronize()
                assert rt.take_flags() == 0
                outs.append(out.cpu().numpy())
            bits = [o.view(np.uint32) if out_dtype == P.DTYPE_F32_RAW else o.view(np.uint16) for o in outs]
            assert np.array_equal(bits[0][0], bits[1][0]) and np.array_equal(bits[0][0], bits[1][1])
        experts = {e: full_bank.expert_host(e) for e in sorted(set(sel.reshape(-1).tolist()))}
        _, ref_raw = O.moe_layer("a", x, experts, 256, sel, w, raw=True)
        xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
        raw = torch.empty((1, 4096), dtype=torch.float32, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, 1, torch.from_numpy(sel.astype(np.int32)).cuda(),
                            torch.from_numpy(w).cuda(), raw, mode=P.MODE_A, out_dtype=P.DTYPE_F32_RAW, stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        check_mode_a(raw.cpu().numpy(), ref_raw, moe_condition(x, experts, sel, w), raw=True)


def test_device_layer_rejects_misaligned_activations(rt, full_bank):
    import torch
    x = torch.zeros(4096 + 8, dtype=torch.int16, device="cuda")[1:4097].view(1, 4096)
    ids = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
    ids[0] = torch.arange(8, dtype=torch.int32)
    w = torch.full((1, 8), 0.125, dtype=torch.float32, device="cuda")
    out = torch.empty((1, 4096), dtype=torch.int16, device="cuda")
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.moe_layer_device(full_bank.bank, x, 1, ids, w, out)


@pytest.mark.parametrize("mode", [0, 1], ids=["mode_a", "mode_b"])
@pytest.mark.parametrize("rows", [1, 8, 9])
def test_device_layer_rejects_bad_routes(rt, full_bank, rows, mode):
    """Route buffers with an expert id outside the bank, one token naming an expert twice, or a NaN
    weight raise the schedule error bit (src/wide_metal_moe.rs:858-938 rejects such schedules) from
    both schedule kernels (8 rows: one wave; 9 rows: one workgroup) and from the one-token mode A
    layer's own route checks (1 row, no schedule) without faulting; every rejected call writes an
    all-zero output, whichever path took it, and the next valid call gives the same bytes as before."""
    import torch
    x = WL.activations(rows, WL.SEED_BASE + 90)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    _, _, sel, w, _ = O.route(x, rw, bias)
    xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
    stream = torch.cuda.current_stream().cuda_stream

    def run(ids, wts):
        out = torch.empty((rows, 4096), dtype=torch.float32, device="cuda")
        rt.moe_layer_device(full_bank.bank, xt, rows, torch.from_numpy(ids.astype(np.int32)).cuda(),
                            torch.from_numpy(wts).cuda(), out, mode=mode, out_dtype=P.DTYPE_F32_RAW,
                            stream=stream)
        torch.cuda.synchronize()
        return out.cpu().numpy(), rt.take_flags()

    clean, flags = run(sel, w)
    assert flags == 0
    assert np.any(clean != 0)
    bad_id = sel.copy()
    bad_id[rows - 1, 3] = 256
    twice = sel.copy()
    twice[0, 1] = twice[0, 0]
    nan_w = w.copy()
    nan_w[min(1, rows - 1), 5] = np.nan
    for ids, wts in ((bad_id, w), (twice, w), (sel, nan_w)):
        out, flags = run(ids, wts)
        assert flags & P.FLAG_SCHEDULE
        assert not np.any(out.view(np.uint32)), "a rejected batch writes zeros"
    again, flags = run(sel, w)
    assert flags == 0
    assert np.array_equal(clean.view(np.uint32), again.view(np.uint32))


def test_calls_on_two_streams_are_ordered(rt, full_bank):
    """Calls share the runtime's scratch: layers enqueued alternately on two streams with no host
    wait between them still give their one-stream results, bit for bit (each call's stream waits
    for the previous call's work)."""
    import torch
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    batches = []
    for seed in (140, 141):
        x = WL.activations(8, WL.SEED_BASE + seed)
        _, _, sel, w, _ = O.route(x, rw, bias)
        batches.append((torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda(),
                        torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda()))

    def run(b, out, stream):
        rt.moe_layer_device(full_bank.bank, b[0], 8, b[1], b[2], out, mode=P.MODE_A, out_dtype=P.DTYPE_F32_RAW,
                            stream=stream)

    ref = []
    for b in batches:
        out = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
        run(b, out, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref.append(out.cpu().numpy())
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.empty((8, 4096), dtype=torch.float32, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    for _ in range(3):
        run(batches[0], outs[0], s1.cuda_stream)
        run(batches[1], outs[1], s2.cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    for o, r in zip(outs, ref):
        assert np.array_equal(o.cpu().numpy().view(np.uint32), r.view(np.uint32))
