"""GPU parity of the dense-route recurrence (csrc/recurrence.hip:
sdm.py:534-607 through _NativeSDMRecurrence.forward, sdm.py:779-861) and of
dense_sparse_routes (sdm.py:162-172).

* Against ``oracle.serial.serial_gated_delta_recurrence`` (float64, the
  reference's token-serial loop sdm.py:464-529) on the kernel's own float32
  inputs: readings, per-token memories and the final memory within
  rtol 1e-4 / atol 2e-5 (the kernel sums over N in float32 with fused
  multiply-adds, in its own order; the reference's Triton kernel fixes no
  order either).
* Exact properties: prefix causality (the reference's own
  test_prefix_causality_is_exact), a shorter run's final memory equal bit
  for bit to the longer run's memory at that token, rows no route writes
  keep their initial memory bit for bit.
* dense_sparse_routes bit for bit against a numpy scatter.
* The prefill handoff: the recurrence's final memory packed by
  pack_prefill_layer materialises back bit for bit, and agrees (tolerance)
  with the sparse decode kernel's prefill of the same routes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import synthetic
from oracle import serial

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 2e-5


def _inputs(batch, time, slots, width, *, k=4, seed=0, distinct_erase=True):
    rng = np.random.default_rng(seed)
    m0 = (rng.standard_normal((batch, slots, width)) * 0.5).astype(np.float32)
    k = min(k, slots)
    idx = np.stack([np.stack([rng.choice(slots, k, replace=False) for _ in range(time)])
                    for _ in range(batch)]).reshape(batch, time, k)
    w = rng.random((batch, time, k)).astype(np.float32)
    w /= w.sum(-1, keepdims=True)
    w[..., 0] *= np.where(rng.random((batch, time)) < 0.2, -1.0, 1.0).astype(np.float32)
    ridx = np.stack([np.stack([rng.choice(slots, k, replace=False) for _ in range(time)])
                     for _ in range(batch)]).reshape(batch, time, k)
    rw = rng.random((batch, time, k)).astype(np.float32)
    wr = serial.dense_routes(idx, w, slots).astype(np.float32)
    rr = serial.dense_routes(ridx, rw, slots).astype(np.float32)
    values = rng.standard_normal((batch, time, width)).astype(np.float32)
    ig = (1.0 / (1.0 + np.exp(-rng.standard_normal((batch, time))))).astype(np.float32)
    eg = ((1.0 / (1.0 + np.exp(-rng.standard_normal((batch, time))))).astype(np.float32)
          if distinct_erase else ig.copy())
    flg = (-rng.random((batch, time)) * 2.0).astype(np.float32)
    return dict(initial_memory=m0, write_routes=wr, values=values, input_gate=ig,
                erase_gate=eg, forget_log_gate=flg, read_routes=rr)


def _gpu(arrays, device):
    return {k: torch.from_numpy(v).to(device) for k, v in arrays.items()}


def _oracle(a):
    return serial.serial_gated_delta_recurrence(
        a["initial_memory"], a["write_routes"], a["values"], a["input_gate"],
        a["forget_log_gate"], a["read_routes"], erase_gate=a["erase_gate"])


# (batch, time, slots, width): config 3's shape at a short prefix, odd N and
# D (scalar loads, a partial column block), every rows-per-lane variant
# (N = 16 .. 1024), one token, one slot
SHAPES = [(4, 24, 256, 128), (3, 37, 64, 128), (2, 11, 100, 20), (2, 9, 1024, 8),
          (2, 13, 512, 36), (3, 7, 16, 16), (2, 5, 32, 64), (1, 1, 1, 1), (2, 6, 250, 12)]


@pytest.mark.parametrize("batch,time,slots,width", SHAPES)
def test_recurrence_matches_serial_oracle(device, batch, time, slots, width):
    print(f"recurrence B={batch} T={time} N={slots} D={width}", flush=True)
    a = _inputs(batch, time, slots, width, seed=slots + width)
    g = _gpu(a, device)
    readings, final, states = cow.sdm_recurrence(**g, return_states=True)
    want_r, want_m, want_s = _oracle(a)
    np.testing.assert_allclose(readings.cpu().numpy(), want_r, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(final.cpu().numpy(), want_m, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(states.cpu().numpy(), want_s, rtol=RTOL, atol=ATOL)
    assert torch.equal(states[:, -1], final)
    # without the per-token memories: the same readings and final memory
    r2, m2 = cow.sdm_recurrence(**g)
    assert torch.equal(r2, readings) and torch.equal(m2, final)


def test_erase_gate_defaults_to_input_gate(device):
    a = _inputs(2, 9, 64, 32, seed=3, distinct_erase=False)
    g = _gpu(a, device)
    readings, final = cow.gated_delta_recurrence(
        g["initial_memory"], g["write_routes"], g["values"], g["input_gate"],
        g["forget_log_gate"], g["read_routes"])
    r2, m2 = cow.sdm_recurrence(**g)
    assert torch.equal(readings, r2) and torch.equal(final, m2)
    want_r, want_m, _ = _oracle(a)
    np.testing.assert_allclose(readings.cpu().numpy(), want_r, rtol=RTOL, atol=ATOL)


def test_prefix_causality_is_exact(device):
    """Changing tokens from position 5 on leaves the readings before it bit
    for bit unchanged (the reference's test_native_sdm.py:89-101)."""

    a = _inputs(2, 9, 64, 16, seed=9)
    b = {k: v.copy() for k, v in a.items()}
    rng = np.random.default_rng(1)
    for name in ("write_routes", "read_routes", "values", "input_gate", "erase_gate",
                 "forget_log_gate"):
        b[name][:, 5:] = rng.permutation(b[name][:, 5:].ravel()).reshape(b[name][:, 5:].shape)
    ra, _ = cow.sdm_recurrence(**_gpu(a, device))
    rb, _ = cow.sdm_recurrence(**_gpu(b, device))
    assert torch.equal(ra[:, :5], rb[:, :5])
    assert not torch.equal(ra[:, 5:], rb[:, 5:])


def test_shorter_run_is_the_longer_runs_prefix(device):
    a = _inputs(3, 20, 256, 64, seed=4)
    g = _gpu(a, device)
    readings, _, states = cow.sdm_recurrence(**g, return_states=True)
    t0 = 7
    part = {k: (v[:, :t0].contiguous() if k != "initial_memory" else v) for k, v in g.items()}
    r0, m0 = cow.sdm_recurrence(**part)
    assert torch.equal(r0, readings[:, :t0])
    assert torch.equal(m0, states[:, t0 - 1])


def test_unwritten_rows_keep_initial_memory(device):
    a = _inputs(2, 15, 128, 32, seed=5)
    g = _gpu(a, device)
    _, final = cow.sdm_recurrence(**g)
    written = (a["write_routes"] != 0).any(axis=1)                  # [B, N]
    m0 = g["initial_memory"]
    untouched = torch.from_numpy(~written).to(device)
    assert bool(untouched.any())
    assert torch.equal(final[untouched], m0[untouched])


def test_zero_tokens_return_the_initial_memory(device):
    a = _inputs(2, 1, 64, 16, seed=6)
    g = {k: (v[:, :0].contiguous() if k != "initial_memory" else v) for k, v in _gpu(a, device).items()}
    readings, final = cow.sdm_recurrence(**g)
    assert readings.shape == (2, 0, 16)
    assert torch.equal(final, g["initial_memory"])


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_dense_sparse_routes_match_numpy(device, index_dtype):
    rng = np.random.default_rng(7)
    slots, rows, k = 256, 40, 16
    idx = np.stack([rng.choice(slots, k, replace=False) for _ in range(rows)]).reshape(5, 8, k)
    w = rng.standard_normal((5, 8, k)).astype(np.float32)
    idx[0, 0, 3] = idx[0, 0, 1]               # a repeated index: the last weight wins
    want = np.zeros((5, 8, slots), np.float32)
    for (i, j), _ in np.ndenumerate(idx[..., 0]):
        for q in range(k):
            want[i, j, idx[i, j, q]] = w[i, j, q]
    got = cow.dense_sparse_routes(torch.from_numpy(w).to(device),
                                  torch.from_numpy(idx).to(device, index_dtype), slots)
    assert np.array_equal(got.cpu().numpy(), want)
    with pytest.raises(ValueError, match="outside"):
        bad = idx.copy()
        bad[2, 3, 0] = slots
        cow.dense_sparse_routes(torch.from_numpy(w).to(device),
                                torch.from_numpy(bad).to(device, index_dtype), slots)
    with pytest.raises(ValueError, match="must align"):
        cow.dense_sparse_routes(torch.from_numpy(w).to(device),
                                torch.from_numpy(idx[..., :3]).to(device, index_dtype), slots)
    # rows with no routes scatter nothing: all-zero dense vectors, even
    # where the output memory held other values before
    filler = torch.full((5, 8, slots), 7.0, device=device)
    del filler
    empty = cow.dense_sparse_routes(torch.zeros(5, 8, 0, device=device),
                                    torch.zeros(5, 8, 0, device=device, dtype=index_dtype), slots)
    assert empty.shape == (5, 8, slots)
    assert not empty.any()


def test_argument_errors(device):
    g = _gpu(_inputs(2, 3, 16, 8, seed=8), device)
    with pytest.raises(ValueError, match="do not align"):
        cow.sdm_recurrence(**{**g, "input_gate": g["input_gate"][:, :2].contiguous()})
    with pytest.raises(ValueError, match="must be contiguous"):
        cow.sdm_recurrence(**{**g, "values": g["values"].transpose(0, 1).contiguous()
                              .transpose(0, 1)})
    big = _gpu(_inputs(1, 2, 1025, 4, k=2, seed=8), device)
    with pytest.raises(ValueError, match="at most 1,024 slots"):
        cow.sdm_recurrence(**big)
    with pytest.raises(ValueError, match="do not align"):      # the reference's dtypes
        cow.sdm_recurrence(**{k: v.double() for k, v in g.items()})
    with pytest.raises(TypeError, match="float32"):
        cow.sdm_recurrence(**{k: v.to(torch.bfloat16) for k, v in g.items()})
    with pytest.raises(RuntimeError, match="no CPU path"):
        cow.sdm_recurrence(**{k: v.cpu() for k, v in g.items()})


def test_prefill_handoff_from_the_recurrence(device):
    """Sparse prefill routes scattered to dense vectors, the recurrence's
    final memory packed into copy-on-write state (inference.py:314-366):
    the packed state materialises to that memory bit for bit, and the
    memory agrees with the sparse decode kernel's prefill of the same
    routes (a different summation order: tolerance)."""

    banks, slots, width, prefix, writes, reads = 8, 256, 128, 48, 4, 16
    m0 = synthetic.make_initial_memory(1, 1, slots, width, seed=11, device=device)[0]
    routes = synthetic.make_steps(steps=prefix, layers=1, banks=banks, slots=slots, width=width,
                                  writes=writes, reads=reads, seed=12, device=device)

    def per_bank(t):                      # [T, 1, B, ...] -> [B, T, ...]
        return t[:, 0].transpose(0, 1).contiguous()

    wr = cow.dense_sparse_routes(per_bank(routes.write_weights), per_bank(routes.write_indices),
                                 slots)
    rr = cow.dense_sparse_routes(per_bank(routes.read_weights), per_bank(routes.read_indices),
                                 slots)
    initial = m0.expand(banks, -1, -1).contiguous()
    gates = per_bank(routes.input_gate)
    readings, final = cow.gated_delta_recurrence(initial, wr, per_bank(routes.values), gates,
                                                 per_bank(routes.forget_log_gate), rr)
    # the sparse decode kernel's prefill of the same routes
    table = initial.clone()
    cow.DecodeTrace(memories=[table], write_indices=routes.write_indices,
                    write_weights=routes.write_weights, values=routes.values,
                    input_gate=routes.input_gate, forget_log_gate=routes.forget_log_gate,
                    read_indices=routes.read_indices,
                    read_weights=routes.read_weights).launch(prefix, start=0)
    torch.cuda.synchronize()
    np.testing.assert_allclose(final.cpu().numpy(), table.cpu().numpy(), rtol=RTOL, atol=ATOL)
    state = cow.pack_prefill_layer(m0, final.reshape(banks, 1, slots, width),
                                   per_bank(routes.write_indices).reshape(banks, prefix, 1, writes),
                                   capacity_rows=None, decode_capacity=prefix + 16,
                                   growth_quantum_rows=banks * writes * 4)
    assert torch.equal(state.materialize_dense(), final)
    state.validate_invariants()
