"""GPU parity of the routed-MoE prefill (mode B grouped block-FP8 GEMM) through the C ABI.

The reference runs its layer-major prefill as 128-row slices through the wide MoE runtime
(src/text_endpoint.rs:4951-5287); every placement depends only on its own token row, so the
prefill over all rows must agree with the C oracle's mode B layer on the same rows and with the
decode-path layer run on 32-row chunks. Tolerance: mode B <= 2e-2 max|d|/max|ref| (the
reference's own mode B gate, src/wide_metal_moe.rs:394-421 uses 0.01 on its probe inputs).
Schedules and tile tables are integer work: the flags word stays zero.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import workloads as WL
from helpers import normwise, rel_l2

pytestmark = pytest.mark.gpu

MODE_B_TOL = 2e-2


def _dev(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t if dtype is None else t.to(dtype)).cuda()


def _bf16_dev(torch, x):
    return torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()


def _from_bf16(t):
    return (t.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)


def _prefill(rt, torch, bank, x, sel, w, out_dtype=P.DTYPE_BF16, x_f32=False):
    rows = x.shape[0]
    xt = _dev(torch, x.astype(np.float32)) if x_f32 else _bf16_dev(torch, x)
    ids = _dev(torch, sel.astype(np.int32))
    wts = _dev(torch, w.astype(np.float32))
    out = torch.empty((rows, bank.bank.hidden), dtype=torch.int16 if out_dtype == P.DTYPE_BF16 else torch.float32,
                      device="cuda")
    rt.moe_prefill_device(bank.bank, xt, rows, ids, wts, out, x_dtype=P.DTYPE_F32 if x_f32 else P.DTYPE_BF16,
                          out_dtype=out_dtype, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    return _from_bf16(out) if out_dtype == P.DTYPE_BF16 else out.cpu().numpy()


def _routes(rng, rows, n_experts):
    logits = rng.standard_normal((rows, n_experts)).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, n_experts).astype(np.float32)
    sel, w, _ = P.route_from_logits(logits, bias)[1:]
    return sel, w


class _SmallBank:
    def __init__(self, rt, n, hidden, inter, seed):
        self.dev = WL.synth_bank(rt, n_experts=n, hidden=hidden, inter=inter, seed=seed)
        self.bank = self.dev.bank
        self.hidden = hidden
        self.experts = {e: self.dev.expert_host(e) for e in range(n)}
        self.n = n


@pytest.fixture(scope="module")
def small_bank(rt):
    return _SmallBank(rt, 16, 256, 128, WL.SEED_BASE + 40)


@pytest.mark.parametrize("rows", [1, 7, 64, 200, 300])
def test_prefill_matches_oracle(rt, small_bank, rows):
    """Random top-8 of 16 experts: 8 * rows / 16 placements per expert (100 at 200 rows: one 128-slot
    m-tile with seven 16-token tiles; 150 at 300 rows: two m-tiles)."""
    import torch
    rng = np.random.default_rng(100 + rows)
    x = WL.activations(rows, WL.SEED_BASE + 50 + rows, hidden=256)
    sel, w = _routes(rng, rows, small_bank.n)
    got = _prefill(rt, torch, small_bank, x, sel, w)
    ref = O.moe_layer("b", x, small_bank.experts, small_bank.n, sel, w)
    assert normwise(got, ref) <= MODE_B_TOL
    assert rel_l2(got, ref) <= 5e-3


def test_prefill_skewed_routes_f32_input(rt, small_bank):
    """Every token on the same eight experts (count = rows = 300: three 128-slot m-tiles each, the
    last one partial), f32 input."""
    import torch
    rows = 300
    rng = np.random.default_rng(7)
    x = rng.standard_normal((rows, 256)).astype(np.float32)
    sel = np.tile(np.array([3, 1, 4, 15, 9, 2, 6, 5], np.uint32), (rows, 1))
    w = rng.uniform(0.01, 0.3, (rows, 8)).astype(np.float32)
    got = _prefill(rt, torch, small_bank, x, sel, w, out_dtype=P.DTYPE_F32, x_f32=True)
    ref = O.moe_layer("b", x, small_bank.experts, small_bank.n, sel, w)
    assert normwise(got, ref) <= MODE_B_TOL
    assert rel_l2(got, ref) <= 5e-3


@pytest.fixture(scope="module")
def full_bank(rt):
    return WL.synth_bank(rt, n_experts=256, seed=WL.SEED_BASE + 2)


def _decode_chunks(rt, torch, bank, x, sel, w, chunk=32):
    rows = x.shape[0]
    out = torch.empty((rows, 4096), dtype=torch.int16, device="cuda")
    xt = _bf16_dev(torch, x)
    ids = _dev(torch, sel.astype(np.int32))
    wts = _dev(torch, w.astype(np.float32))
    stream = torch.cuda.current_stream().cuda_stream
    for r0 in range(0, rows, chunk):
        n = min(chunk, rows - r0)
        rt.moe_layer_device(bank.bank, xt[r0:], n, ids[r0:], wts[r0:], out[r0:], mode=P.MODE_B,
                            out_dtype=P.DTYPE_BF16, stream=stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    return _from_bf16(out)


@pytest.mark.parametrize("rows,zipf", [(2048, False), (2048, True), (4096, False)])
def test_prefill_matches_decode_chunks(rt, full_bank, rows, zipf):
    """2048 tokens (and the 4096-row maximum), top-8 of 256 experts (16 384 / 32 768 placements):
    the prefill agrees with the decode layer run on 32-row chunks (the same mode B numerics per
    placement, summed in another order) within the mode B tolerance, and with the oracle on eight
    rows spread over the batch plus the token rows of the first and last slot of every 128-slot
    m-tile of the busiest expert (587 placements in five m-tiles under Zipf routing)."""
    import torch
    x = WL.activations(rows, WL.SEED_BASE + 4)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    sel, w, _ = WL.route_host(x, rw, bias)
    counts = np.bincount(sel.reshape(-1), minlength=256)
    assert counts.sum() == rows * 8
    got = _prefill(rt, torch, full_bank, x, sel, w)
    dec = _decode_chunks(rt, torch, full_bank, x, sel, w)
    assert normwise(got, dec) <= MODE_B_TOL
    assert rel_l2(got, dec) <= 2e-3
    # oracle rows (only their experts are fetched): eight spread over the batch, and the first and
    # last slot of each m-tile of the busiest expert (its slots hold its token rows in ascending order)
    hot = int(np.argmax(counts))
    hot_rows = np.nonzero(np.any(sel == hot, axis=1))[0]
    assert hot_rows.size == counts[hot]
    m_tiles = -(-hot_rows.size // 128)
    ends = [hot_rows[min(128 * t + k, hot_rows.size - 1)] for t in range(m_tiles) for k in (0, 127)]
    pick = np.unique(np.concatenate([np.linspace(0, rows - 1, 8).astype(np.int64), ends]))
    print(f"oracle rows {pick.size}: busiest expert {hot}, {counts[hot]} placements, {m_tiles} m-tiles", flush=True)
    used = sorted(set(sel[pick].reshape(-1).tolist()))
    experts = {e: full_bank.expert_host(e) for e in used}
    ref = O.moe_layer("b", x[pick], experts, 256, sel[pick], w[pick])
    assert normwise(got[pick], ref) <= MODE_B_TOL


@pytest.mark.parametrize("zipf", [False, True])
def test_prefill_is_deterministic(rt, full_bank, zipf):
    """The same 2048-token batch gives the same raw f32 bits twice, with another batch (300 rows, a
    different schedule, m-tile table and scratch contents) run on the runtime in between: no result
    depends on the timing of the plan launch's quantiser workgroups, the rotated K order of the
    gate/up workgroups or what the scratch held before."""
    import torch
    x = WL.activations(2048, WL.SEED_BASE + 4)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3, zipf=zipf)
    sel, w, _ = WL.route_host(x, rw, bias)
    first = _prefill(rt, torch, full_bank, x, sel, w, out_dtype=P.DTYPE_F32_RAW)
    _prefill(rt, torch, full_bank, x[:300][::-1].copy(), sel[:300], w[:300], out_dtype=P.DTYPE_F32_RAW)
    again = _prefill(rt, torch, full_bank, x, sel, w, out_dtype=P.DTYPE_F32_RAW)
    assert np.array_equal(first.view(np.uint32), again.view(np.uint32))
    assert np.all(np.isfinite(first)) and np.any(first)


def test_prefill_rejects_bad_arguments(rt, small_bank):
    import torch
    x = torch.zeros((8, 256), dtype=torch.int16, device="cuda")
    ids = torch.zeros((8, 8), dtype=torch.int32, device="cuda")
    w = torch.zeros((8, 8), dtype=torch.float32, device="cuda")
    out = torch.zeros((8, 256), dtype=torch.int16, device="cuda")
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.moe_prefill_device(small_bank.bank, x, 0, ids, w, out)
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.moe_prefill_device(small_bank.bank, x, 4097, ids, w, out)


def test_prefill_rejected_routes_write_zeros(rt, small_bank):
    """An expert id outside the bank, an expert named twice by one token, or a NaN weight raise the
    schedule error bit (src/wide_metal_moe.rs:858-938) for short (one-workgroup schedule) and long
    (three-launch schedule) batches; the output is all zeros, and the next valid batch gives its
    bytes again."""
    import torch
    for rows in (40, 300):
        rng = np.random.default_rng(900 + rows)
        x = WL.activations(rows, WL.SEED_BASE + 95, hidden=256)
        sel, w = _routes(rng, rows, small_bank.n)
        clean = _prefill(rt, torch, small_bank, x, sel, w, out_dtype=P.DTYPE_F32_RAW)
        assert np.any(clean)
        bad_id = sel.copy()
        bad_id[rows - 1, 3] = small_bank.n
        twice = sel.copy()
        twice[rows // 2, 1] = twice[rows // 2, 0]
        nan_w = w.copy()
        nan_w[1, 5] = np.nan
        for ids, wts in ((bad_id, w), (twice, w), (sel, nan_w)):
            xt = _bf16_dev(torch, x)
            out = torch.full((rows, 256), 7.0, dtype=torch.float32, device="cuda")
            rt.moe_prefill_device(small_bank.bank, xt, rows, _dev(torch, ids.astype(np.int32)),
                                  _dev(torch, wts.astype(np.float32)), out, out_dtype=P.DTYPE_F32_RAW,
                                  stream=torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            assert rt.take_flags() & P.FLAG_SCHEDULE
            assert not np.any(out.cpu().numpy().view(np.uint32)), "a rejected batch writes zeros"
        again = _prefill(rt, torch, small_bank, x, sel, w, out_dtype=P.DTYPE_F32_RAW)
        assert np.array_equal(clean.view(np.uint32), again.view(np.uint32))


def test_prefill_token_results_do_not_depend_on_the_batch(rt, full_bank):
    """1024 token rows with their routes give the same raw f32 bits inside two batches: after 1024
    other tokens under Zipf routing (busy experts take several m-tiles, so every later expert's
    m-tiles sit elsewhere in the grid, and the shared tokens' slots move), and alone. Each gate/up
    tile's K order depends only on its expert and n-tile group."""
    import torch
    shared = WL.activations(1024, WL.SEED_BASE + 96)
    rw_u, bias_u = WL.router_inputs(WL.SEED_BASE + 3)
    sel_s, w_s, _ = WL.route_host(shared, rw_u, bias_u)
    other = WL.activations(1024, WL.SEED_BASE + 97)
    rw_z, bias_z = WL.router_inputs(WL.SEED_BASE + 3, zipf=True)
    sel_o, w_o, _ = WL.route_host(other, rw_z, bias_z)
    assert np.bincount(sel_o.reshape(-1), minlength=256).max() > 128
    alone = _prefill(rt, torch, full_bank, shared, sel_s, w_s, out_dtype=P.DTYPE_F32_RAW)
    mixed = _prefill(rt, torch, full_bank, np.concatenate([other, shared]), np.concatenate([sel_o, sel_s]),
                     np.concatenate([w_o, w_s]), out_dtype=P.DTYPE_F32_RAW)
    assert np.array_equal(mixed[1024:].view(np.uint32), alone.view(np.uint32))
    assert np.all(np.isfinite(alone)) and np.any(alone)
