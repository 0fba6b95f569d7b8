"""GPU parity of the BF16 wide linear (execute_bf16_linear, src/wide_metal_moe.rs:728-834; CPU twin
bf16_linear, src/text_endpoint.rs:3347-3380) through the C ABI.

Products of bf16 weights and bf16 activation planes are exact in f32, so only the f32 summation
order differs from the oracle's sequential sum: the raw sums are held to 2e-6 max|d|/max|ref| (at
K = 8192 against the f64 sum, since the oracle's own sequential error reaches a few 1e-6 there), and
the bf16-rounded outputs to one rounding step of the largest element (8e-3), as for mode A.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from prismwing_amd import workloads as WL
from helpers import normwise

pytestmark = pytest.mark.gpu

RAW_TOL = 2e-6
BF16_OUT = 8e-3


def _weights(rng, n, k, scale=0.05):
    return (rng.standard_normal((n, k)).astype(np.float32) * scale).view(np.uint32).__rshift__(16).astype(np.uint16)


def _device(torch, rt, proj, x, rows, out_dtype, x_bf16=False):
    xt = torch.from_numpy(WL.bf16_bits_np(x).view(np.int16)).cuda() if x_bf16 else torch.from_numpy(x).cuda()
    dt = torch.int16 if out_dtype == P.DTYPE_BF16 else torch.float32
    out = torch.empty((rows, proj.rows), dtype=dt, device="cuda")
    rt.bf16_linear_device(proj, xt, rows, out, x_dtype=P.DTYPE_BF16 if x_bf16 else P.DTYPE_F32,
                          out_dtype=out_dtype, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    got = out.cpu().numpy()
    if out_dtype == P.DTYPE_BF16:
        got = (got.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return got


@pytest.mark.parametrize("rows", [1, 5, 8])
def test_host_call_matches_oracle(rt, rows):
    """The reference-shaped synchronous call: f32 rows, 300 output rows (a partial 64-row group),
    1024 columns."""
    rng = np.random.default_rng(30 + rows)
    w = _weights(rng, 300, 1024)
    x = rng.standard_normal((rows, 1024)).astype(np.float32)
    proj = rt.bind_bf16(w)
    res = rt.execute_bf16_linear(x, proj)
    ref = O.bf16_linear(w, x)
    assert res.output.shape == (rows, 300)
    assert normwise(res.output, ref) <= BF16_OUT
    assert res.resident_source_bytes == w.nbytes


@pytest.mark.parametrize("rows,x_bf16", [(1, False), (8, False), (8, True), (20, False), (32, True)])
def test_device_raw_sums_match_oracle(rt, rows, x_bf16):
    """Raw f32 sums (before the bf16 round), f32 inputs (three planes) and bf16 inputs, widths up to
    32 (two 16-token MFMA tiles), K = 1536 (three 512-column splits)."""
    import torch
    rng = np.random.default_rng(40 + rows)
    w = _weights(rng, 256, 1536)
    x = rng.standard_normal((rows, 1536)).astype(np.float32)
    if x_bf16:
        x = WL.bf16_round_np(x)
    proj = rt.bind_bf16(w)
    got = _device(torch, rt, proj, x, rows, P.DTYPE_F32_RAW, x_bf16)
    ref, ref_raw = O.bf16_linear(w, x, raw=True)
    assert normwise(got, ref_raw) <= RAW_TOL
    got16 = _device(torch, rt, proj, x, rows, P.DTYPE_BF16, x_bf16)
    assert normwise(got16, ref) <= BF16_OUT


@pytest.mark.parametrize("rows", [1, 8])
def test_o_proj_shape(rt, rows):
    """The attention output projection: [4096 x 8192] bf16 weights bound no-copy from device memory."""
    import torch
    rng = np.random.default_rng(50 + rows)
    w = _weights(rng, 4096, 8192, scale=0.02)
    x = rng.standard_normal((rows, 8192)).astype(np.float32)
    wt = torch.from_numpy(w.view(np.int16)).cuda()
    proj = rt.bind_bf16_device(wt, 4096, 8192)
    got = _device(torch, rt, proj, x, rows, P.DTYPE_F32_RAW)
    ref, ref_raw = O.bf16_linear(w, x, raw=True)
    # at K = 8192 the oracle's sequential f32 sum carries its own error of a few 1e-6: both are held
    # against the f64 sum, the device to 2e-6 and the oracle to 1e-5
    exact = x.astype(np.float64) @ (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).T
    assert normwise(got, exact) <= RAW_TOL
    assert normwise(ref_raw, exact) <= 1e-5
    got32 = _device(torch, rt, proj, x, rows, P.DTYPE_F32)
    assert normwise(got32, ref) <= BF16_OUT


@pytest.mark.parametrize("rows", [1, 8])
def test_lm_head_shape(rt, rows):
    """The LM head the reference runs through the same wide linear (src/text_endpoint.rs:5673-5705):
    [152576 x 4096] bf16 weights (1.25 GB, generated on the device), every output row computed and
    2048 of them, spread over the matrix and including its last 64-row group, checked against the
    f64 sum and the oracle."""
    import torch
    vocab, hidden = 152576, 4096
    gen = torch.Generator(device="cuda").manual_seed(60 + rows)
    wt = (torch.randn((vocab, hidden), generator=gen, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
    rng = np.random.default_rng(61 + rows)
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    proj = rt.bind_bf16_device(wt, vocab, hidden)
    got = _device(torch, rt, proj, x, rows, P.DTYPE_F32_RAW)
    got32 = _device(torch, rt, proj, x, rows, P.DTYPE_F32)
    pick = np.unique(np.concatenate([np.linspace(0, vocab - 1, 1984).astype(np.int64), np.arange(vocab - 64, vocab)]))
    w = wt[torch.from_numpy(pick).cuda()].cpu().numpy().view(np.uint16)
    exact = x.astype(np.float64) @ (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).T
    assert normwise(got[:, pick], exact) <= RAW_TOL
    ref, _ = O.bf16_linear(w, x, raw=True)
    assert normwise(got32[:, pick], ref) <= BF16_OUT
    assert np.all(np.isfinite(got))


def test_closed_form_exact_outputs(rt):
    """Weights and inputs that are small powers of two: every sum is exact in any order, so the
    device output equals the oracle's bit for bit."""
    rng = np.random.default_rng(60)
    k = 512
    wv = np.ldexp(1.0, rng.integers(-6, 1, (128, k))).astype(np.float32) * rng.choice([-1, 1], (128, k))
    xv = np.ldexp(1.0, rng.integers(-6, 1, (3, k))).astype(np.float32)
    w = _bf16_bits_of(wv)
    proj = rt.bind_bf16(w)
    res = rt.execute_bf16_linear(xv, proj)
    ref = O.bf16_linear(w, xv)
    assert np.array_equal(res.output.view(np.uint32), ref.view(np.uint32))


def _bf16_bits_of(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_fail_closed(rt):
    rng = np.random.default_rng(70)
    w = _weights(rng, 64, 256)
    proj = rt.bind_bf16(w)
    with pytest.raises(P.PwError, match="NONFINITE"):
        rt.execute_bf16_linear(np.full((1, 256), np.nan, np.float32), proj)
    with pytest.raises(P.PwError, match="ARGUMENT"):
        rt.execute_fp8_linear(np.zeros((1, 256), np.float32), proj)
    with pytest.raises(P.PwError, match="LAYOUT"):
        rt.bind_bf16(_weights(rng, 64, 200))
    # an infinite weight makes a non-finite output: the reference's error bit 32
    w_inf = w.copy()
    w_inf[3, 0] = 0x7F80
    proj_inf = rt.bind_bf16(w_inf)
    with pytest.raises(P.PwError, match="GPU_FLAGS"):
        rt.execute_bf16_linear(np.ones((1, 256), np.float32), proj_inf)
    assert rt.take_flags() == 0
