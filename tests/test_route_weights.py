"""Known answers for the route-weight denominator of pytorch_noaux_routes
(src/text_endpoint.rs:4382-4390, :4450-4452): weights = s_i / (pytorch_sum_eight(s) + 1e-20), where
pytorch_sum_eight folds (s0 + s4, s1 + s5, s2 + s6, s3 + s7) left to right from 0 over the selected
scores in nth_element's partition order.

The rows (tests/helpers.py ROUTE_WEIGHT_ROWS) were chosen so that a tree order, a plain left-to-right
sum, a sum in expert-id order and (second row) a missing 1e-20 each change the weight bits; the test
first proves that with IEEE f32 arithmetic, then holds the oracle and the library's host routing to
the frozen bits. The device router is held to the same rows in tests/test_gpu_router.py.
"""
import numpy as np
import pytest

import oracle as O
import prismwing_amd as P
from helpers import ROUTE_WEIGHT_ROWS, route_weight_alternatives, route_weight_row_logits


def _u32(a):
    return np.asarray(a, np.float32).view(np.uint32).tolist()


@pytest.mark.parametrize("row", ROUTE_WEIGHT_ROWS, ids=["ordinary", "tiny-scores"])
def test_frozen_bits_discriminate_every_alternative_order(row):
    scores = np.array(row["score_bits"], np.uint32).view(np.float32)
    alt = route_weight_alternatives(scores, row["selected"])
    assert _u32(alt["reference"]) == row["weight_bits"]
    for name in ("tree", "plain", "id_order", "no_eps"):
        same = _u32(alt[name]) == row["weight_bits"]
        assert same == (name not in row["differs"]), name
    # the selected order is not ascending id, so the id-order slip is a real alternative
    assert row["selected"] != sorted(row["selected"])


@pytest.mark.parametrize("row", ROUTE_WEIGHT_ROWS, ids=["ordinary", "tiny-scores"])
def test_oracle_route_weights_known_answer(row):
    logits = route_weight_row_logits(row)
    scores = np.array([O.sigmoid_f32(float(v)) for v in logits], np.float32)
    sel, w, ties = O.noaux_routes(scores[None, :], np.zeros(256, np.float32))
    assert sel[0].tolist() == row["selected"]
    assert _u32(scores[sel[0]]) == row["score_bits"]
    assert _u32(w[0]) == row["weight_bits"]
    assert ties == 0
    # the whole route through the oracle's logits: a one-hot activation row times f32 router weights
    # whose column 0 holds the logits gives them exactly
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = 1.0
    rw = np.zeros((256, 64), np.float32)
    rw[:, 0] = logits
    lg, sc, sel2, w2, _ = O.route(x, rw, np.zeros(256, np.float32))
    assert np.array_equal(lg[0].view(np.uint32), logits.view(np.uint32))
    assert sel2[0].tolist() == row["selected"] and _u32(w2[0]) == row["weight_bits"]


@pytest.mark.parametrize("row", ROUTE_WEIGHT_ROWS, ids=["ordinary", "tiny-scores"])
def test_product_host_route_weights_known_answer(row):
    logits = route_weight_row_logits(row)
    scores, sel, w, ties = P.route_from_logits(logits[None, :], np.zeros(256, np.float32))
    assert sel[0].tolist() == row["selected"]
    assert _u32(scores[0][sel[0]]) == row["score_bits"]
    assert _u32(w[0]) == row["weight_bits"]
    assert ties == 0
    sel2, w2, _ = P.noaux_routes(scores, np.zeros(256, np.float32))
    assert sel2[0].tolist() == row["selected"] and _u32(w2[0]) == row["weight_bits"]
