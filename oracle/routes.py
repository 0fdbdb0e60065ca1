"""numpy restatement of product-key route selection -- TEST INFRASTRUCTURE.

Follows copy_on_write_sdm/sdm.py:96-159 (product_key_routes): shortlist each
half of the projection to its top min(selected, root) scores (:118-127), rank
the pair sums (:128-152), map pairs to slots first*root + second (:153-155),
sort by slot (:156-157) and take the softmax of the selected scores (:158).
Scores stay float32 (the pair sum is one float32 add); the softmax is taken
in float64 and rounded once.  Equal scores are taken lowest position first
(a stable sort), the order the HIP kernel uses; torch.topk leaves it open.

Pinned in tests/test_routes_oracle.py by a brute-force top-k over all N slot
sums (the product-key shortlist must not change the answer), a hand-computed
case and scipy's softmax.
"""

from __future__ import annotations

import math

import numpy as np


def _top(scores: np.ndarray, count: int) -> tuple[np.ndarray, np.ndarray]:
    order = np.argsort(-scores, axis=-1, kind="stable")[..., :count]
    return np.take_along_axis(scores, order, axis=-1), order


def _softmax(values: np.ndarray) -> np.ndarray:
    v = values.astype(np.float64)
    e = np.exp(v - v.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def product_key_routes(projected: np.ndarray, slots: int,
                       selected: int) -> tuple[np.ndarray, np.ndarray]:
    """(weights float32, indices int64), each [..., K] (sdm.py:96-159)."""

    projected = np.asarray(projected, dtype=np.float32)
    root = math.isqrt(slots)
    assert root * root == slots and projected.shape[-1] == 2 * root
    first, second = projected[..., :root], projected[..., root:]
    sub = min(selected, root)
    first_values, first_indices = _top(first, sub)
    second_values, second_indices = _top(second, sub)
    lead = projected.shape[:-1]
    pair_scores = (first_values[..., :, None] + second_values[..., None, :]).reshape(
        *lead, sub * sub)
    pair_first = np.repeat(first_indices, sub, axis=-1)
    pair_second = np.tile(second_indices, (1,) * len(lead) + (sub,))
    final = min(selected, sub * sub)
    values, positions = _top(pair_scores, final)
    indices = (np.take_along_axis(pair_first, positions, axis=-1).astype(np.int64) * root
               + np.take_along_axis(pair_second, positions, axis=-1))
    order = np.argsort(indices, axis=-1, kind="stable")
    indices = np.take_along_axis(indices, order, axis=-1)
    values = np.take_along_axis(values, order, axis=-1)
    return _softmax(values), indices


def brute_force_routes(projected: np.ndarray, slots: int,
                       selected: int) -> tuple[np.ndarray, np.ndarray]:
    """Top ``selected`` of all N slot scores first[i] + second[j], no shortlist."""

    projected = np.asarray(projected, dtype=np.float32)
    root = math.isqrt(slots)
    first, second = projected[..., :root], projected[..., root:]
    full = (first[..., :, None] + second[..., None, :]).reshape(*projected.shape[:-1], slots)
    values, slot_ids = _top(full, min(selected, slots))
    order = np.argsort(slot_ids, axis=-1, kind="stable")
    return (_softmax(np.take_along_axis(values, order, axis=-1)),
            np.take_along_axis(slot_ids, order, axis=-1).astype(np.int64))
