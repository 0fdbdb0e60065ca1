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
    mapping = state.logical_to_physical.cpu().numpy()
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


def assert_state_equal(state, oracle: ref.OracleState) -> None:
    """Map, free stack, live rows, counters: all bit-exact."""

    got = snapshot(state)
    assert got["capacity"] == oracle.capacity_rows
    assert got["free_count"] == oracle.free_count
    assert np.array_equal(got["map"], oracle.logical_to_physical)
    assert np.array_equal(got["free_rows"], oracle.free_rows[: oracle.free_count])
    live = oracle.logical_to_physical[oracle.logical_to_physical >= 0]
    assert np.array_equal(got["live_values"], oracle.values[live])
    assert got["overflow"] == oracle.overflow_flag
    assert np.array_equal(got["templates"], oracle.template_indices)
    assert state.growth_events == oracle.growth_events
    assert state.growth_rows_added == oracle.growth_rows_added
    assert state.growth_rows_copied == oracle.growth_rows_copied
    assert state.capacity_is_proven == oracle.capacity_is_proven
    assert (state.proven_maximum_additional_allocations
            == oracle.proven_maximum_additional_allocations)


def make_case(*, banks, slots, width, writes, reads, steps, seed, index_dtype=torch.int32,
              distribution="uniform"):
    m0 = synthetic.make_initial_memory(1, 1, slots, width, seed=seed)[0]
    batch = synthetic.make_steps(steps=steps, layers=1, banks=banks, slots=slots, width=width,
                                 writes=writes, reads=reads, seed=seed + 1,
                                 index_dtype=index_dtype, distribution=distribution)
    return m0, [batch.step(s, 0) for s in range(steps)]
