"""The test helpers' vectorised e4m3 encoder agrees with the oracle's literal search."""
import numpy as np

import oracle as O
from helpers import decode_table, encode_e4m3


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
