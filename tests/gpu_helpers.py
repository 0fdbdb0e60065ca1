"""Shared helpers of the GPU parity tests: move inputs, snapshot states."""

from __future__ import annotations

import numpy as np
import torch

from copy_on_write_sdm_amd import synthetic
from oracle import state as ref


def to_device(inputs: dict, device) -> dict:
    return {k: v.to(device) for k, v in inputs.items()}


def to_numpy(inputs: dict) -> dict:
    return {k: v.cpu().numpy() for k, v in inputs.items()}


def snapshot(state) -> dict:
    """Exact host copy of a product state's allocator-visible tensors."""

    free = int(state.free_count.item())
    mapping = state.direct_map().cpu().numpy()
    values = state.values.cpu().numpy()
    live = mapping[mapping >= 0]
    return {
        "map": mapping,
        "free_count": free,
        "free_rows": state.free_rows.cpu().numpy()[:free],
        "live_values": values[live],
        "overflow": int(state.overflow_flag.item()),
        "capacity": state.capacity_rows,
        "templates": state.template_indices.cpu().numpy(),
    }


def assert_state_equal(state, oracle: ref.OracleState, *, permuted: bool = False) -> None:
    """Map, free stack, live rows, counters: all bit-exact.  permuted: the
    physical rows of first touches may be assigned in another order (decode
    traces claim them with an atomic add, as the reference's proven kernel
    does); the same logical rows are private, they use the same set of
    physical rows and hold the same values, and the free stack is identical."""

    got = snapshot(state)
    assert got["capacity"] == oracle.capacity_rows
    assert got["free_count"] == oracle.free_count
    want_map = oracle.logical_to_physical
    live = want_map[want_map >= 0]
    if permuted:
        assert np.array_equal(got["map"] >= 0, want_map >= 0)
        assert np.array_equal(np.sort(got["map"][got["map"] >= 0]), np.sort(live))
    else:
        assert np.array_equal(got["map"], want_map)
    assert np.array_equal(got["free_rows"], oracle.free_rows[: oracle.free_count])
    assert np.array_equal(got["live_values"], oracle.values[live])
    assert got["overflow"] == oracle.overflow_flag
    assert np.array_equal(got["templates"], oracle.template_indices)
    assert state.growth_events == oracle.growth_events
    assert state.growth_rows_added == oracle.growth_rows_added
    assert state.growth_rows_copied == oracle.growth_rows_copied
    assert state.capacity_is_proven == oracle.capacity_is_proven
    assert (state.proven_maximum_additional_allocations
            == oracle.proven_maximum_additional_allocations)


def assert_states_match(a, b) -> None:
    """Two product states equal up to the order in which first touches were
    given physical rows: same private logical rows and values, same set of
    physical rows, identical free stacks and flags."""

    x, y = snapshot(a), snapshot(b)
    assert x["capacity"] == y["capacity"]
    assert x["free_count"] == y["free_count"]
    assert np.array_equal(x["free_rows"], y["free_rows"])
    assert np.array_equal(x["map"] >= 0, y["map"] >= 0)
    assert np.array_equal(np.sort(x["map"][x["map"] >= 0]), np.sort(y["map"][y["map"] >= 0]))
    assert np.array_equal(x["live_values"], y["live_values"])
    assert x["overflow"] == y["overflow"]
    assert torch.equal(a.materialize_dense(), b.materialize_dense())


def make_case(*, banks, slots, width, writes, reads, steps, seed, index_dtype=torch.int32,
              distribution="uniform"):
    m0 = synthetic.make_initial_memory(1, 1, slots, width, seed=seed)[0]
    batch = synthetic.make_steps(steps=steps, layers=1, banks=banks, slots=slots, width=width,
                                 writes=writes, reads=reads, seed=seed + 1,
                                 index_dtype=index_dtype, distribution=distribution)
    return m0, [batch.step(s, 0) for s in range(steps)]


def assert_states_identical(a, b) -> None:
    """Two product states equal bit for bit: maps (physical rows included),
    free stacks, live rows, flags, capacities, growth counters and proofs."""

    x, y = snapshot(a), snapshot(b)
    assert x["capacity"] == y["capacity"]
    assert x["free_count"] == y["free_count"]
    assert np.array_equal(x["map"], y["map"])
    assert np.array_equal(x["free_rows"], y["free_rows"])
    assert np.array_equal(x["live_values"], y["live_values"])
    assert x["overflow"] == y["overflow"]
    assert (a.growth_events, a.growth_rows_added, a.growth_rows_copied) == (
        b.growth_events, b.growth_rows_added, b.growth_rows_copied)
    assert a.capacity_is_proven == b.capacity_is_proven
    assert (a.proven_maximum_additional_allocations
            == b.proven_maximum_additional_allocations)


def oracle_decode_loop(oracles, batch, steps, *, start=0, need=None):
    """The reference's decode loop on oracle states (inference.py:538-566):
    per step and layer, prepare_step_capacity(need) when the state has a
    growth quantum (allocator.py:745-773), then the packed step.  ``batch``
    is a synthetic.StepBatch on any device.  Returns the readings
    [steps, L, B, D]."""

    out = []
    for s in range(start, start + steps):
        row = []
        for l, orc in enumerate(oracles):
            if orc.growth_quantum_rows and need is not None:
                ref.prepare_step_capacity(orc, need)
            x = {k: v.cpu().numpy() for k, v in batch.step(s, l).items()}
            reading, _ = ref.packed_step(orc, **x, validate_routes=False)
            row.append(reading)
        out.append(np.stack(row))
    return np.stack(out)
