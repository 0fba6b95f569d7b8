"""The test helpers' vectorised e4m3 encoder agrees with the oracle's literal search."""
import numpy as np

import oracle as O
from helpers import closed_form_mode_b, decode_table, encode_e4m3, exact_in_f32, fp8_blocks_exact


def test_helper_encoder_matches_oracle():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(3000) * 50, rng.standard_normal(1000) * 0.01,
                        [0.0, -0.0, 448.0, -448.0, 2 ** -9 / 2, 3 * 2 ** -10]]).astype(np.float32)
    got = encode_e4m3(v)
    want = np.array([O.encode_e4m3fn(float(x)) for x in v], np.uint8)
    assert np.array_equal(got, want)
    assert np.array_equal(encode_e4m3(np.array([1000.0, -1e9])), np.array([0x7E, 0xFE], np.uint8))
    t = decode_table()
    assert t[0x38] == 1.0 and t[0xB8] == -1.0 and np.isnan(t[0x7F])


def test_fp8_window_rule_matches_the_measured_mfma_sums():
    """The window rule reproduces what the FP8 MFMA gave on MI355X for one 128-product block:
    448 + 2^-3 exact, 448 + 2^-6 and 448 + 2^-9 truncated to 448, 64 + 7 * 2^-9 to 64 + 2^-7,
    1 + 2^-9 exact, 1 + 2^-18 truncated to 1; zero products do not widen the window."""
    q = np.zeros((1, 128))
    q[0, :6] = [448.0, 1.0, 2.0 ** -9, 2.0 ** -6, 2.0 ** -3, 64.0]
    q[0, 6] = 7 * 2.0 ** -9

    def exact(cols):
        w = np.zeros((1, 128))
        for c, v in cols.items():
            w[0, c] = v
        return fp8_blocks_exact(q, w)

    assert exact({0: 1.0, 4: 1.0}) and exact({1: 1.0, 2: 1.0}) and exact({1: 1.0, 3: 1.0})
    assert not exact({0: 1.0, 3: 1.0}) and not exact({0: 1.0, 2: 1.0}) and not exact({5: 1.0, 6: 1.0})
    assert not exact({1: 1.0, 2: 2.0 ** -9})
    assert exact({0: 0.0, 1: 1.0, 2: 1.0})


def test_exact_in_f32_bound():
    assert exact_in_f32(np.array([[2.0 ** 23, 1.0]]), np.array([[1.0, 1.0]]))
    assert not exact_in_f32(np.array([[2.0 ** 24, 1.0]]), np.array([[1.0, 1.0]]))


def test_closed_form_layer_data_meets_its_preconditions():
    """The closed-form mode-B data the GPU tests use (seed and size as there): every gate, up and
    down sum is exact in f32 in any order and inside the FP8 MFMA window, hidden groups have
    absmax 448, and the oracle's layer runs on it."""
    experts, x, sel, w = closed_form_mode_b(0x50570100, 256, 12, check=True)
    out = O.moe_layer("b", x[:8], experts, 12, sel[:8], w[:8])
    assert np.all(np.isfinite(out)) and np.any(out)


def test_closed_form_two_step_layer_meets_its_preconditions():
    """The hidden-512, intermediate-512 closed form (two K steps per projection, several n-tiles
    per prefill workgroup) at the GPU test's seed and size."""
    experts, x, sel, w = closed_form_mode_b(0x50570300, 144, 8, hidden=512, inter=512, check=True)
    out = O.moe_layer("b", x[:2], experts, 8, sel[:2], w[:2])
    assert np.all(np.isfinite(out)) and np.any(out)


def test_closed_form_odd_hidden_blocks_meets_its_preconditions():
    """The hidden-384 closed form (three 128-column blocks: the prefill's one-block K steps and its
    separate SwiGLU kernel) at the GPU test's seed and size."""
    experts, x, sel, w = closed_form_mode_b(0x50570200, 96, 12, hidden=384, check=True)
    out = O.moe_layer("b", x[:4], experts, 12, sel[:4], w[:4])
    assert np.all(np.isfinite(out)) and np.any(out)


def test_closed_form_wide_hidden_meets_its_preconditions():
    """The hidden-4096, intermediate-512 closed form (the prefill gate/up's sixteen rotated K steps,
    the down projection's four n-tiles per workgroup) at the GPU test's seed and size."""
    experts, x, sel, w = closed_form_mode_b(0x50570400, 40, 8, hidden=4096, inter=512, check=True)
    out = O.moe_layer("b", x[:2], experts, 8, sel[:2], w[:2])
    assert np.all(np.isfinite(out)) and np.any(out)


def test_closed_form_production_shape_meets_its_preconditions():
    """The hidden-4096, intermediate-2048 closed form (the production expert shape: the prefill
    gate/up's sixteen rotated K steps over 4096 stacked rows, the down GEMM's eight 256-column K
    steps) at the GPU test's seed and size."""
    experts, x, sel, w = closed_form_mode_b(0x50570500, 24, 8, hidden=4096, inter=2048, check=True)
    out = O.moe_layer("b", x[:1], experts, 8, sel[:1], w[:1])
    assert np.all(np.isfinite(out)) and np.any(out)


def test_closed_form_dense_intermediate_meets_its_preconditions():
    """The intermediate-16384 closed form of the dense-MLP test (hidden 1024, one expert, down codes
    in every eighth 128-column block) at the GPU test's seed and size."""
    experts, x, sel, w = closed_form_mode_b(0x50570600, 8, 1, hidden=1024, inter=16384, top_k=1, check=True,
                                            down_block_step=8)
    out = O.moe_layer("b", x[:1], experts, 1, sel[:1], np.ones((1, 1), np.float32))
    assert np.all(np.isfinite(out)) and np.any(out)
