"""GPU parity of the dense layer-0 FP8 MLP (dense_mlp, src/text_endpoint.rs:4266-4340: gate and up
[16384 x 4096] through wide_fp8_linear, bf16-staged SwiGLU, down [4096 x 16384]) run as a one-expert
bank through pw_expert_forward_device, at the real shapes.

Mode B (the reference's mode) against the oracle's fp8_linear composition: <= 2e-2
max|d|/max|ref| (the reference's own mode B gate is 0.01 on its probe inputs). Mode A against the
oracle's f32 expert: <= 1e-3 on the f32 result and one bf16 step (8e-3) on bf16 outputs.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from helpers import bf16_normal, normwise

pytestmark = pytest.mark.gpu

H, I = 4096, 16384


@pytest.fixture(scope="module")
def dense(rt):
    import torch
    mats = {}
    for i, (name, rows, cols) in enumerate((("gate", I, H), ("up", I, H), ("down", H, I))):
        w = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
        s = torch.empty((rows // 128, cols // 128), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        rt.synth_scales(s, s.numel(), 900 + 2 * i)
        rt.synth_fp8(w, s, rows, cols, 901 + 2 * i)
        torch.cuda.synchronize()
        mats[name] = (w, s, rt.bind_projection_device(w, s, rows, cols))
    bank = rt.expert_bank([mats["gate"][2]], [mats["up"][2]], [mats["down"][2]])
    host = {k: (v[0].cpu().numpy(), v[1].cpu().numpy()) for k, v in mats.items()}
    return bank, host, mats


def _run(rt, torch, bank, x, mode, out_dtype):
    rows = x.shape[0]
    xt = torch.from_numpy(x).cuda()
    dt = torch.int16 if out_dtype == P.DTYPE_BF16 else torch.float32
    out = torch.empty((rows, H), dtype=dt, device="cuda")
    rt.expert_forward_device(bank, 0, xt, rows, out, mode=mode, x_dtype=P.DTYPE_F32, out_dtype=out_dtype,
                             stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    got = out.cpu().numpy()
    if out_dtype == P.DTYPE_BF16:
        got = (got.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return got


@pytest.mark.parametrize("rows", [2, 9])
def test_dense_mlp_mode_b(rt, dense, rows):
    import torch
    bank, host, _ = dense
    x = bf16_normal(np.random.default_rng(rows), (rows, H))
    got = _run(rt, torch, bank, x, P.MODE_B, P.DTYPE_BF16)
    gate = O.fp8_linear_mode_b(*host["gate"], x)
    up = O.fp8_linear_mode_b(*host["up"], x)
    ref = O.fp8_linear_mode_b(*host["down"], O.swiglu_bf16_staged(gate, up))
    assert normwise(got, ref) <= 2e-2


@pytest.mark.parametrize("rows", [1, 8])
def test_dense_mlp_mode_a(rt, dense, rows):
    import torch
    bank, host, _ = dense
    x = bf16_normal(np.random.default_rng(20 + rows), (rows, H))
    expert = (*host["gate"], *host["up"], *host["down"])
    ref32, refbf = O.expert_mode_a(x, expert)
    assert normwise(_run(rt, torch, bank, x, P.MODE_A, P.DTYPE_F32_RAW), ref32) <= 1e-3
    assert normwise(_run(rt, torch, bank, x, P.MODE_A, P.DTYPE_BF16), refbf) <= 8e-3
