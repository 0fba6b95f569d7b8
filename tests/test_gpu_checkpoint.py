"""GPU parity of the checkpoint-bound expert bank: one layer's routed experts read from safetensors
shards (names of src/text_endpoint.rs:4785-4845, validation of src/lib.rs:1217-1270) and copied into
HBM once must drive the decode layer to the same bytes as a bank bound from the same arrays, and
match the C oracle (mode A <= 1e-3 on the f32 combine). Malformed experts fail closed."""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from helpers import bf16_normal, fp8_weight, log_uniform_scales, normwise, write_safetensors

pytestmark = pytest.mark.gpu

H, I, E, LAYER = 256, 128, 9, 3


def _experts(seed):
    rng = np.random.default_rng(seed)
    ex = {}
    for e in range(E):
        gs, us, ds = log_uniform_scales(rng, I, H), log_uniform_scales(rng, I, H), log_uniform_scales(rng, H, I)
        ex[e] = (fp8_weight(rng, I, H, gs), gs, fp8_weight(rng, I, H, us), us, fp8_weight(rng, H, I, ds), ds)
    return ex


def _tensors(ex, experts):
    t = {}
    for e in experts:
        gw, gs, uw, us, dw, ds = ex[e]
        for name, w, s in (("gate", gw, gs), ("up", uw, us), ("down", dw, ds)):
            key = f"model.layers.{LAYER}.mlp.experts.{e}.{name}_proj.weight"
            t[key] = ("F8_E4M3", w.shape, np.ascontiguousarray(w).tobytes())
            t[key + "_scale_inv"] = ("F32", s.shape, np.ascontiguousarray(s, np.float32).tobytes())
    return t


def _layer(rt, torch, bank, x, sel, w, out_dtype=P.DTYPE_F32_RAW):
    rows = x.shape[0]
    xt = torch.from_numpy(x).cuda()
    ids = torch.from_numpy(sel.astype(np.int32)).cuda()
    wts = torch.from_numpy(w.astype(np.float32)).cuda()
    out = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    rt.moe_layer_device(bank, xt, rows, ids, wts, out, mode=P.MODE_A, x_dtype=P.DTYPE_F32, out_dtype=out_dtype,
                        stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rt.take_flags() == 0
    return out.cpu().numpy()


def test_checkpoint_bank_matches_bound_bank_and_oracle(rt, tmp_path):
    import torch
    ex = _experts(5)
    # two shards, experts split across them, plus an unrelated tensor
    a = write_safetensors(tmp_path / "shard0.safetensors", {**_tensors(ex, range(0, 5)),
                                                            "model.norm.weight": ("BF16", (H,), b"\0" * 2 * H)})
    b = write_safetensors(tmp_path / "shard1.safetensors", _tensors(ex, range(5, E)))
    files = [P.Safetensors(str(a)), P.Safetensors(str(b))]
    bank = rt.expert_bank_from_safetensors(files, LAYER, E, H, I)
    for f in files:  # the bank owns its copy: the files may close
        f.close()
    projs = [[rt.bind_projection(ex[e][2 * m], ex[e][2 * m + 1]) for m in range(3)] for e in range(E)]
    bound = rt.expert_bank([p[0] for p in projs], [p[1] for p in projs], [p[2] for p in projs])
    rng = np.random.default_rng(6)
    rows = 6
    x = bf16_normal(rng, (rows, H))
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    _, sel, w, _ = P.route_from_logits(logits, np.zeros(E, np.float32))
    got = _layer(rt, torch, bank, x, sel, w)
    ref_bound = _layer(rt, torch, bound, x, sel, w)
    assert np.array_equal(got.view(np.uint32), ref_bound.view(np.uint32))
    _, ref_raw = O.moe_layer("a", x, ex, E, sel, w, raw=True)
    assert normwise(got, ref_raw) <= 1e-3


@pytest.mark.parametrize("case", ["absent", "dtype", "shape", "scale_grid", "nan_code", "inf_scale"])
def test_checkpoint_bank_fails_closed(rt, tmp_path, case):
    ex = _experts(7)
    t = _tensors(ex, range(E))
    key = f"model.layers.{LAYER}.mlp.experts.4.up_proj.weight"
    want = "LAYOUT"
    if case == "absent":
        del t[key + "_scale_inv"]
    elif case == "dtype":
        t[key] = ("U8",) + t[key][1:]
    elif case == "shape":
        t[key] = ("F8_E4M3", (H, I), t[key][2])
    elif case == "scale_grid":
        t[key + "_scale_inv"] = ("F32", (2, 1), b"\0" * 8)
    elif case == "nan_code":
        data = bytearray(t[key][2])
        data[77] = 0x7F
        t[key] = (t[key][0], t[key][1], bytes(data))
        want = "NONFINITE"
    elif case == "inf_scale":
        s = np.frombuffer(t[key + "_scale_inv"][2], np.float32).copy()
        s[0] = np.inf
        t[key + "_scale_inv"] = ("F32", t[key + "_scale_inv"][1], s.tobytes())
        want = "NONFINITE"
    path = write_safetensors(tmp_path / f"{case}.safetensors", t)
    with P.Safetensors(str(path)) as f:
        with pytest.raises(P.PwError, match=want):
            rt.expert_bank_from_safetensors([f], LAYER, E, H, I)
