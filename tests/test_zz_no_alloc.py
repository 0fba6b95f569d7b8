"""The decode-layer entry point that allocates nothing (pw_moe_layer_device_noalloc) against the
allocating one (pw_moe_layer_device), through the C ABI: same kernels, so the same bytes, on two
calls in a row with the second one smaller (its static scratch keeps the first call's contents),
in both modes; and requests beyond its limits fail with a clear error."""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import workloads as WL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bank(rt):
    return WL.synth_bank(rt, n_experts=256, seed=WL.SEED_BASE + 2)


def _inputs(torch, rows, seed, f32=False):
    x = WL.activations(rows, WL.SEED_BASE + seed)
    rw, bias = WL.router_inputs(WL.SEED_BASE + 3)
    _, _, sel, w, _ = O.route(x, rw, bias)
    xt = torch.from_numpy(x).cuda() if f32 else torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda()
    return xt, torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda()


@pytest.mark.parametrize("mode", [P.MODE_A, P.MODE_B])
@pytest.mark.parametrize("out_dtype", [P.DTYPE_F32_RAW, P.DTYPE_BF16])
def test_noalloc_layer_equals_allocating_layer(rt, bank, mode, out_dtype):
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    for rows, seed, f32 in ((8, 150, False), (3, 151, False), (5, 152, True), (1, 153, False), (1, 154, True)):
        xt, ids, wts = _inputs(torch, rows, seed, f32)
        x_dtype = P.DTYPE_F32 if f32 else P.DTYPE_BF16
        dt = torch.float32 if out_dtype == P.DTYPE_F32_RAW else torch.int16
        want = torch.empty((rows, 4096), dtype=dt, device="cuda")
        got = torch.full((rows, 4096), 7, dtype=dt, device="cuda")
        rt.moe_layer_device(bank.bank, xt, rows, ids, wts, want, mode=mode, x_dtype=x_dtype, out_dtype=out_dtype,
                            stream=stream)
        rt.moe_layer_device_noalloc(bank.bank, xt, rows, ids, wts, got, mode=mode, x_dtype=x_dtype,
                                    out_dtype=out_dtype, stream=stream)
        torch.cuda.synchronize()
        assert rt.take_flags() == 0
        a, b = want.cpu().numpy(), got.cpu().numpy()
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (rows, mode, out_dtype)


def test_noalloc_layer_rejects_requests_beyond_its_scratch(rt, bank):
    import torch
    xt, ids, wts = _inputs(torch, 9, 153)
    out = torch.empty((9, 4096), dtype=torch.int16, device="cuda")
    with pytest.raises(P.PwError, match="1 to 8 token rows"):
        rt.moe_layer_device_noalloc(bank.bank, xt, 9, ids, wts, out)
    # a bank with an intermediate size above 2048
    g = rt.bind_projection(np.full((4096, 128), 0x38, np.uint8), np.ones((32, 1), np.float32))
    d = rt.bind_projection(np.full((128, 4096), 0x38, np.uint8), np.ones((1, 32), np.float32))
    wide = rt.expert_bank([g], [g], [d])
    x = torch.zeros((1, 128), dtype=torch.int16, device="cuda")
    ids1 = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
    w1 = torch.full((1, 8), 0.125, dtype=torch.float32, device="cuda")
    out1 = torch.empty((1, 128), dtype=torch.int16, device="cuda")
    with pytest.raises(P.PwError, match="intermediate 2048"):
        rt.moe_layer_device_noalloc(wide, x, 1, ids1, w1, out1)


@pytest.mark.parametrize("mode", [P.MODE_A, P.MODE_B])
def test_noalloc_layer_under_graph_capture(rt, bank, mode):
    """The entry point is for callers under HIP graph capture: after eager calls on two other streams
    (so the runtime's last call sits on a stream outside the capture), one call captured on a fresh
    stream is not ordered against that stream (a wait on an event recorded outside the capture is a
    cross-boundary dependency the capture rejects), and every replay of the graph gives the eager
    call's bytes. Between replays the program runs its own eager layer calls (on the same static
    scratch) and synchronises; those keep their bytes too."""
    import torch
    s_eager, s_other, s_cap = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    xt, ids, wts = _inputs(torch, 8, 160)
    x2, ids2, wts2 = _inputs(torch, 8, 161)
    want = torch.empty((8, 4096), dtype=torch.int16, device="cuda")
    other = torch.empty((8, 4096), dtype=torch.int16, device="cuda")
    rt.moe_layer_device_noalloc(bank.bank, xt, 8, ids, wts, want, mode=mode, stream=s_eager.cuda_stream)
    rt.moe_layer_device_noalloc(bank.bank, x2, 8, ids2, wts2, other, mode=mode, stream=s_other.cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    got = torch.full((8, 4096), 7, dtype=torch.int16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s_cap, capture_error_mode="thread_local"):
        rt.moe_layer_device_noalloc(bank.bank, xt, 8, ids, wts, got, mode=mode, stream=s_cap.cuda_stream)
    torch.cuda.synchronize()
    assert torch.all(got == 7), "capturing enqueues nothing"
    for replay in range(3):
        got.fill_(7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {replay}"
        again = torch.empty_like(other)
        rt.moe_layer_device_noalloc(bank.bank, x2, 8, ids2, wts2, again, mode=mode, stream=s_other.cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(again, other), f"eager call after replay {replay}"
    assert rt.take_flags() == 0
