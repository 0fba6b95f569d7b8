"""GPU routed schedule against the reference's BTreeMap<expert, [(position, weight)]>
(src/text_endpoint.rs:4767-4775) through pw_moe_schedule_device.

The schedule is integer work and bit-exact: per-expert slot offsets (placement counts), the token
row and router weight of every slot (experts ascending, rows ascending within an expert) and each
token's eight slots in ascending expert id (the combine order, src/text_endpoint.rs:5365-5373).
Row counts cover every schedule kernel: up to 8 rows one wave, 9..128 one workgroup, more rows
three launches over many workgroups. Rejected routes (src/wide_metal_moe.rs:858-938) raise the
schedule bit; the long-batch schedule then leaves the placement tables zero.
"""
import numpy as np
import pytest

import prismwing_amd as P
from prismwing_amd import workloads as WL

pytestmark = pytest.mark.gpu


def host_schedule(sel, w, n_experts):
    """The BTreeMap order restated on the host: placements sorted by (expert, token row)."""
    rows = sel.shape[0]
    e = sel.reshape(-1).astype(np.int64)
    p = np.repeat(np.arange(rows), 8)
    order = np.lexsort((p, e))                  # slot -> placement index
    slot = np.empty(rows * 8, np.int64)
    slot[order] = np.arange(rows * 8)
    offsets = np.concatenate([[0], np.cumsum(np.bincount(e, minlength=n_experts))]).astype(np.uint32)
    positions = p[order].astype(np.uint32)
    weights = w.reshape(-1)[order].astype(np.float32)
    by_expert = np.argsort(sel, axis=1, kind="stable")
    row_slots = np.take_along_axis(slot.reshape(rows, 8), by_expert, axis=1).reshape(-1).astype(np.uint32)
    return offsets, positions, weights, row_slots


def distinct_routes(rng, rows, n_experts, zipf=False):
    """Eight distinct experts per row (Gumbel top-8), uniform or Zipf(1.1)-skewed popularity."""
    logp = -1.1 * np.log(np.arange(1, n_experts + 1)) if zipf else np.zeros(n_experts)
    keys = logp[None, :] + rng.gumbel(size=(rows, n_experts))
    sel = np.argsort(-keys, axis=1)[:, :8].astype(np.uint32)
    w = rng.uniform(0.01, 0.3, (rows, 8)).astype(np.float32)
    return sel, w


@pytest.fixture(scope="module")
def bank256(rt):
    # the schedule reads only the bank's pointer table: tiny expert shapes
    return WL.synth_bank(rt, n_experts=256, hidden=128, inter=128, seed=WL.SEED_BASE + 70)


def device_schedule(rt, bank, sel, w):
    import torch
    rows = sel.shape[0]
    E = bank.bank.n_experts
    ids = torch.from_numpy(np.ascontiguousarray(sel.astype(np.int32))).cuda()
    wts = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    off = torch.full((E + 1,), 0x7EEEEEEE, dtype=torch.int32, device="cuda")
    pos = torch.full((rows * 8,), 0x7EEEEEEE, dtype=torch.int32, device="cuda")
    pw = torch.full((rows * 8,), -1.0, dtype=torch.float32, device="cuda")
    rs = torch.full((rows * 8,), 0x7EEEEEEE, dtype=torch.int32, device="cuda")
    rt.moe_schedule_device(bank.bank, rows, ids, wts, off, pos, pw, rs,
                           stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    flags = rt.take_flags()
    return (off.cpu().numpy().view(np.uint32), pos.cpu().numpy().view(np.uint32), pw.cpu().numpy(),
            rs.cpu().numpy().view(np.uint32), flags)


def check_equal(got, want):
    off, pos, pw, rs, flags = got
    assert flags == 0
    assert np.array_equal(off, want[0])
    assert np.array_equal(pos, want[1])
    assert np.array_equal(pw.view(np.uint32), want[2].view(np.uint32))
    assert np.array_equal(rs, want[3])


@pytest.mark.parametrize("rows", [1, 3, 8, 9, 64, 128, 129, 300, 2048, 4096])
def test_schedule_matches_btreemap(rt, bank256, rows):
    rng = np.random.default_rng(500 + rows)
    sel, w = distinct_routes(rng, rows, 256)
    check_equal(device_schedule(rt, bank256, sel, w), host_schedule(sel, w, 256))


@pytest.mark.parametrize("n_experts", [9, 64, 1000, 1024])
def test_schedule_wave_expert_counts(rt, n_experts):
    """The one-wave schedule (up to 8 rows) over banks of 9 to 1024 experts (one to 32 words of its
    routed-id bitmap, token-row masks at every id): routes spread over the whole id range, every
    row on the eight highest ids (one expert per row rank, eight rows each), and a row naming an
    expert twice (rejected, then the valid routes again)."""
    bank = WL.synth_bank(rt, n_experts=n_experts, hidden=128, inter=128, seed=WL.SEED_BASE + 72 + n_experts)
    for rows in (1, 5, 8):
        rng = np.random.default_rng(n_experts * 10 + rows)
        sel, w = distinct_routes(rng, rows, n_experts)
        check_equal(device_schedule(rt, bank, sel, w), host_schedule(sel, w, n_experts))
        top = np.tile(np.arange(n_experts - 1, n_experts - 9, -1, dtype=np.uint32), (rows, 1))
        check_equal(device_schedule(rt, bank, top, w), host_schedule(top, w, n_experts))
    twice = sel.copy()
    twice[rows - 1, 7] = twice[rows - 1, 2]
    assert device_schedule(rt, bank, twice, w)[4] & P.FLAG_SCHEDULE
    check_equal(device_schedule(rt, bank, sel, w), host_schedule(sel, w, n_experts))


@pytest.mark.parametrize("rows", [100, 2048])
def test_schedule_zipf_routes(rt, bank256, rows):
    rng = np.random.default_rng(900 + rows)
    sel, w = distinct_routes(rng, rows, 256, zipf=True)
    check_equal(device_schedule(rt, bank256, sel, w), host_schedule(sel, w, 256))


@pytest.mark.parametrize("rows", [40, 300, 4096])
def test_schedule_every_row_on_eight_experts(rt, bank256, rows):
    """Counts = rows for eight experts (more than 16 slots each), the other 248 unrouted."""
    rng = np.random.default_rng(rows)
    sel = np.tile(np.array([200, 3, 77, 255, 0, 128, 31, 32], np.uint32), (rows, 1))
    w = rng.uniform(0.01, 0.3, (rows, 8)).astype(np.float32)
    check_equal(device_schedule(rt, bank256, sel, w), host_schedule(sel, w, 256))


def test_schedule_matches_router_routes(rt):
    """Routes from the reference router (sigmoid + bias, top-8 of 256) on the 2048-token workload."""
    bank = WL.synth_bank(rt, n_experts=256, hidden=128, inter=128, seed=WL.SEED_BASE + 71)
    x = WL.activations(2048, WL.SEED_BASE + 4)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    sel, w, _ = WL.route_host(x, rw, bias)
    check_equal(device_schedule(rt, bank, sel, w), host_schedule(sel, w, 256))


@pytest.mark.parametrize("rows", [8, 100, 300])
def test_schedule_rejects_bad_routes(rt, bank256, rows):
    """An id outside the bank, a token naming one expert twice or a NaN weight raise the schedule
    bit from each schedule kernel; the long-batch schedule leaves its tables zero. The next valid
    call gives the host schedule again."""
    rng = np.random.default_rng(rows + 1)
    sel, w = distinct_routes(rng, rows, 256)
    bad_id = sel.copy()
    bad_id[rows - 1, 3] = 256
    twice = sel.copy()
    twice[0, 1] = twice[0, 0]
    nan_w = w.copy()
    nan_w[rows // 2, 5] = np.nan
    for ids, wts in ((bad_id, w), (twice, w), (sel, nan_w)):
        off, pos, pw, rs, flags = device_schedule(rt, bank256, ids, wts)
        assert flags & P.FLAG_SCHEDULE
        assert off[-1] <= rows * 8 and np.all(np.diff(off.astype(np.int64)) >= 0)
        if rows > 128:
            assert not pos.any() and not pw.view(np.uint32).any() and not rs.any()
    check_equal(device_schedule(rt, bank256, sel, w), host_schedule(sel, w, 256))
