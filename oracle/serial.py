"""Independent formulations of SDM used to pin ``oracle.state``.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* ``serial_gated_delta_recurrence`` restates copy_on_write_sdm/sdm.py:464-529
  in float64: dense per-token route vectors over all N slots, decay only where
  the route weight is nonzero, retrieval as a sum over N.
* ``serial_copy_on_write_recurrence`` restates sdm.py:365-461: a private
  overlay plus an active mask over shared M0; it must equal the dense form.
* ``loop_step`` is one SDM token written as scalar Python loops straight from
  the update rule, for tiny inputs.
"""

from __future__ import annotations

import math

import numpy as np


def dense_routes(indices: np.ndarray, weights: np.ndarray, slots: int) -> np.ndarray:
    """Scatter sparse routes [B,T,K] into dense route vectors [B,T,N]
    (sdm.py:162-172)."""

    b, t, k = indices.shape
    out = np.zeros((b, t, slots), dtype=np.float64)
    bi = np.arange(b)[:, None, None]
    ti = np.arange(t)[None, :, None]
    np.add.at(out, (np.broadcast_to(bi, indices.shape), np.broadcast_to(ti, indices.shape), indices),
              weights.astype(np.float64))
    return out


def serial_gated_delta_recurrence(
    initial_memory, write_routes, values, input_gate, forget_log_gate, read_routes,
    *, erase_gate=None,
):
    """sdm.py:464-529 in float64.  Returns (readings [B,T,D], final memory,
    per-step memories [B,T,N,D])."""

    memory = np.asarray(initial_memory, dtype=np.float64).copy()
    readings, states = [], []
    for position in range(write_routes.shape[1]):
        writes = write_routes[:, position].astype(np.float64)
        decay = np.exp(forget_log_gate[:, position].astype(np.float64))[:, None, None]
        selected = writes != 0.0
        decayed = np.where(selected[..., None], memory * decay, memory)
        retrieved = np.sum(writes[..., None] * decayed, axis=1)
        write = input_gate[:, position].astype(np.float64)[:, None]
        erase = write if erase_gate is None else erase_gate[:, position].astype(np.float64)[:, None]
        delta = write * values[:, position].astype(np.float64) - erase * retrieved
        memory = decayed + writes[..., None] * delta[:, None, :]
        readings.append(np.sum(read_routes[:, position].astype(np.float64)[..., None] * memory, axis=1))
        states.append(memory.copy())
    return np.stack(readings, axis=1), memory, np.stack(states, axis=1)


def serial_copy_on_write_recurrence(
    initial_memory, write_routes, values, input_gate, forget_log_gate, read_routes,
    *, erase_gate=None,
):
    """sdm.py:365-461 in float64: overlay + active mask over shared M0.
    Returns (readings, final effective memory, final active mask)."""

    shared = np.asarray(initial_memory, dtype=np.float64)
    overlay = np.zeros_like(shared)
    active = np.zeros(shared.shape[:2], dtype=bool)
    readings = []
    for position in range(write_routes.shape[1]):
        writes = write_routes[:, position].astype(np.float64)
        selected = writes != 0.0
        memory = np.where(active[..., None], overlay, shared)
        decay = np.exp(forget_log_gate[:, position].astype(np.float64))[:, None, None]
        decayed = np.where(selected[..., None], memory * decay, memory)
        retrieved = np.sum(writes[..., None] * decayed, axis=1)
        write = input_gate[:, position].astype(np.float64)[:, None]
        erase = write if erase_gate is None else erase_gate[:, position].astype(np.float64)[:, None]
        delta = write * values[:, position].astype(np.float64) - erase * retrieved
        updated = decayed + writes[..., None] * delta[:, None, :]
        overlay = np.where(selected[..., None], updated, overlay)
        active = active | selected
        memory = np.where(active[..., None], overlay, shared)
        readings.append(np.sum(read_routes[:, position].astype(np.float64)[..., None] * memory, axis=1))
    return np.stack(readings, axis=1), memory, active


def loop_step(table, write_idx, write_w, value, ig, eg, flg, read_idx, read_w):
    """One SDM token for one bank with scalar loops (float64).

    table: list of N rows (lists of D floats), mutated in place.
    M[i] <- a*M[i] + w_i * (ig*v - eg * sum_j w_j a*M[j]) for written i,
    then reading = sum_r rw_r * M[r].
    """

    a = math.exp(flg)
    width = len(value)
    decayed = {i: [a * x for x in table[i]] for i in write_idx}
    retrieved = [0.0] * width
    for i, w in zip(write_idx, write_w):
        for d in range(width):
            retrieved[d] += w * decayed[i][d]
    for i, w in zip(write_idx, write_w):
        table[i] = [decayed[i][d] + w * (ig * value[d] - eg * retrieved[d]) for d in range(width)]
    reading = [0.0] * width
    for i, w in zip(read_idx, read_w):
        for d in range(width):
            reading[d] += w * table[i][d]
    return reading
