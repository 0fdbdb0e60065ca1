"""CPU pins of the product-key route oracle (oracle/routes.py) and the
argument checks of cowsdm_product_key_routes (no kernel is launched)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import scipy.special

from copy_on_write_sdm_amd import _native as nat
from oracle import routes


@pytest.mark.parametrize("slots,selected", [(16, 1), (16, 4), (16, 16), (256, 4),
                                            (256, 16), (1024, 32), (4096, 16), (65536, 16)])
def test_shortlist_equals_brute_force(slots, selected):
    # fp32 addition is monotone in each operand, so a pair outside either
    # half's shortlist can never enter the top `selected` of all N sums
    rng = np.random.default_rng(slots + selected)
    projected = rng.standard_normal((3, 2, 2 * int(np.sqrt(slots))), dtype=np.float32)
    weights, indices = routes.product_key_routes(projected, slots, selected)
    bw, bi = routes.brute_force_routes(projected, slots, selected)
    np.testing.assert_array_equal(indices, bi)
    np.testing.assert_array_equal(weights, bw)
    assert np.all(np.diff(indices, axis=-1) > 0)


def test_weights_are_softmax_of_selected_scores():
    rng = np.random.default_rng(7)
    projected = rng.standard_normal((4, 1, 32), dtype=np.float32)
    weights, indices = routes.product_key_routes(projected, 256, 16)
    first, second = projected[..., :16], projected[..., 16:]
    scores = (np.take_along_axis(first, indices // 16, -1)
              + np.take_along_axis(second, indices % 16, -1))
    expected = scipy.special.softmax(scores.astype(np.float64), axis=-1)
    np.testing.assert_allclose(weights, expected, rtol=1e-6, atol=1e-8)


def test_hand_computed_case():
    # first = [1, 3], second = [2, 0.5]: slots 0..3 score 3, 1.5, 5, 3.5
    projected = np.array([[[1.0, 3.0, 2.0, 0.5]]], dtype=np.float32)
    weights, indices = routes.product_key_routes(projected, 4, 2)
    assert indices.tolist() == [[[2, 3]]]
    np.testing.assert_allclose(weights[0, 0], [1 / (1 + np.exp(-1.5)), 1 / (1 + np.exp(1.5))],
                               rtol=1e-6)
    weights, indices = routes.product_key_routes(projected, 4, 1)
    assert indices.tolist() == [[[2]]] and weights.tolist() == [[[1.0]]]


def test_equal_scores_take_the_lowest_position():
    # pair positions (a, b) over the shortlists: (3+2) slot 2, then the tie
    # (3+0) slot 3 at position 1 against (1+2) slot 0 at position 2
    projected = np.array([[[1.0, 3.0, 2.0, 0.0]]], dtype=np.float32)
    assert routes.product_key_routes(projected, 4, 2)[1].tolist() == [[[2, 3]]]


def test_argument_errors_without_launching():
    lib = nat.lib()
    f = lib.cowsdm_product_key_routes
    assert f(None, 0, 256, 16, None, None, None) == 0
    assert f(None, 4, 255, 16, None, None, None) == -1
    assert b"do not match" in lib.cowsdm_last_error_string()
    assert f(None, 4, 256, 0, None, None, None) == -1
    assert f(None, 4, 256, 257, None, None, None) == -1
    assert b"between one and slots" in lib.cowsdm_last_error_string()
    assert f(None, 4, 2048 * 2048, 16, None, None, None) == -2
    assert f(None, 4, 4096, 33, None, None, None) == -2
    assert f(None, 4, 1024, 33, None, None, None) == -2   # K = 33 routes
    assert b"routes per row" in lib.cowsdm_last_error_string()
    assert f(None, 4, 49, 49, None, None, None) == -2     # K = min(49, 7 * 7)
    assert f(None, 4, 256, 16, None, None, None) == -1
    assert b"null" in lib.cowsdm_last_error_string()
    assert f(None, -1, 256, 16, None, None, None) == -1
