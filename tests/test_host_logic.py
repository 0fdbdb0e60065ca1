"""Host-side logic of the product package -- CPU only, no kernel launches.

The capacity arithmetic must agree with the oracle's restatement of
allocator.py:629-655, 706-708, 745-773 and 792-795; argument errors must be
raised with the reference's messages before any device work; and the product
must refuse CPU tensors instead of falling back to a CPU path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import allocator as alloc
from oracle import state as ref


@settings(max_examples=300, deadline=None)
@given(active=st.integers(0, 5000), banks=st.integers(1, 64), slots=st.integers(1, 256),
       capacity=st.one_of(st.none(), st.integers(1, 20000)), quantum=st.integers(0, 2048),
       future=st.one_of(st.none(), st.integers(0, 100000)))
def test_handoff_capacity_matches_oracle(active, banks, slots, capacity, quantum, future):
    def run(fn):
        try:
            return fn(active, banks, slots, capacity, quantum, future)
        except ValueError as exc:
            return str(exc)

    assert run(alloc.handoff_capacity) == run(ref.handoff_capacity)


@settings(max_examples=300, deadline=None)
@given(active=st.integers(0, 10**6), headroom=st.integers(0, 10**5), quantum=st.integers(1, 4096))
def test_trim_target_matches_oracle(active, headroom, quantum):
    assert alloc.trim_target(active, headroom, quantum) == ref.trim_target(active, headroom,
                                                                           quantum)


@settings(max_examples=300, deadline=None)
@given(minimum=st.integers(1, 10**7), quantum=st.integers(1, 4096))
def test_growth_target_is_quantum_ceiling(minimum, quantum):
    target = alloc.growth_target(minimum, quantum)
    assert target % quantum == 0 and minimum <= target < minimum + quantum


def _cpu_state(banks=3, slots=16, width=8, capacity=48, quantum=0):
    """A state object over CPU tensors, built directly (allocate() refuses
    CPU tensors); used only to exercise host-side checks."""

    return cow.PackedSDMCopyOnWriteState(
        shared_initial_memory=torch.zeros(1, slots, width),
        template_indices=torch.zeros(banks, dtype=torch.int64),
        values=torch.zeros(capacity, width),
        logical_to_physical=torch.full((banks, slots), -1, dtype=torch.int32),
        free_rows=torch.arange(capacity, dtype=torch.int32),
        free_count=torch.tensor(capacity, dtype=torch.int32),
        overflow_flag=torch.zeros((), dtype=torch.int32),
        growth_quantum_rows=quantum,
    )


def _inputs(banks=3, writes=2, reads=4, width=8):
    return dict(
        write_indices=torch.tensor([[2, 5], [1, 7], [4, 10]])[:banks, :writes],
        write_weights=torch.full((banks, writes), 0.5),
        values=torch.zeros(banks, width),
        input_gate=torch.full((banks,), 0.5),
        forget_log_gate=torch.zeros(banks),
        read_indices=torch.zeros(banks, reads, dtype=torch.int64),
        read_weights=torch.full((banks, reads), 0.25),
    )


def test_cpu_tensors_are_refused_not_computed():
    state = _cpu_state()
    with pytest.raises(RuntimeError, match="HIP device"):
        cow.packed_sdm_cow_step(state, **_inputs())
    with pytest.raises(RuntimeError, match="HIP device"):
        cow.dense_sdm_sparse_step(torch.zeros(3, 16, 8), **_inputs())
    with pytest.raises(RuntimeError, match="HIP device"):
        cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(1, 16, 8), banks=2, capacity_rows=4)


def test_backend_names():
    state = _cpu_state()
    with pytest.raises(RuntimeError, match="Triton SDM COW backend is unavailable"):
        cow.packed_sdm_cow_step(state, **_inputs(), backend="triton")
    # "torch" runs the HIP kernels too: CPU tensors are refused, not computed
    with pytest.raises(RuntimeError, match="HIP device"):
        cow.packed_sdm_cow_step(state, **_inputs(), backend="torch")
    with pytest.raises(ValueError, match="allocator backend must be"):
        cow.packed_sdm_cow_step(state, **_inputs(), backend="cuda")


def test_shape_errors_use_reference_messages():
    state = _cpu_state()
    bad = _inputs()
    bad["write_indices"] = bad["write_indices"].float()
    with pytest.raises(ValueError, match="write indices must be integer"):
        cow.packed_sdm_cow_step(state, **bad)
    bad = _inputs()
    bad["read_indices"] = bad["read_indices"][:2]
    with pytest.raises(ValueError, match="read indices must be integer"):
        cow.packed_sdm_cow_step(state, **bad)
    bad = _inputs()
    bad["values"] = torch.zeros(3, 7)
    with pytest.raises(ValueError, match="route weights and values do not align"):
        cow.packed_sdm_cow_step(state, **bad)
    bad = _inputs()
    bad["input_gate"] = torch.zeros(3, 1)
    with pytest.raises(ValueError, match="native SDM input gate must be"):
        cow.packed_sdm_cow_step(state, **bad)
    bad = _inputs()
    with pytest.raises(ValueError, match="gates must align"):
        cow.packed_sdm_cow_step(state, **bad, erase_gate=torch.zeros(2))
    with pytest.raises(ValueError, match="dense SDM memory must be"):
        cow.dense_sdm_sparse_step(torch.zeros(3, 16), **_inputs())


def test_allocate_argument_errors():
    with pytest.raises(ValueError, match=r"\[H,N,D\] or \[N,D\]"):
        cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(8), banks=1, capacity_rows=1)
    with pytest.raises(ValueError, match="must be positive"):
        cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(4, 8), banks=0, capacity_rows=1)
    with pytest.raises(ValueError, match="quantum cannot be negative"):
        cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(4, 8), banks=1, capacity_rows=1,
                                               growth_quantum_rows=-1)
    with pytest.raises(ValueError, match="float16, bfloat16, or float32"):
        cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(4, 8), banks=1, capacity_rows=1,
                                               state_dtype=torch.float64)


def test_capacity_proof_without_growth_matches_oracle():
    """prepare_step_capacity branches that need no slab growth."""

    state = _cpu_state(capacity=48, quantum=16)
    oracle = ref.allocate(np.zeros((1, 16, 8), np.float32), banks=3, capacity_rows=48,
                          growth_quantum_rows=16)
    for demand, free in [(6, 48), (6, 48), (30, 40), (6, 20), (0, 20), (10, 12)]:
        state.free_count.fill_(free)
        oracle.free_count = free
        assert state.prepare_step_capacity(demand) == ref.prepare_step_capacity(oracle, demand)
        assert (state.proven_maximum_additional_allocations
                == oracle.proven_maximum_additional_allocations)
        assert state.capacity_is_proven and oracle.capacity_is_proven
    with pytest.raises(ValueError, match="cannot be negative"):
        state.prepare_step_capacity(-1)
    fixed = _cpu_state(quantum=0)
    with pytest.raises(ValueError, match="no decode proof"):
        fixed.prepare_step_capacity(4)
    fixed.capacity_is_proven = True
    assert fixed.prepare_step_capacity(4) == 0


def test_lifecycle_argument_errors():
    state = _cpu_state(quantum=16)
    with pytest.raises(ValueError, match="trim headroom cannot be negative"):
        state.trim_capacity(headroom_rows=-1)
    with pytest.raises(ValueError, match="trimming requires copy-on-write"):
        _cpu_state(quantum=0).trim_capacity()
    with pytest.raises(ValueError, match="growth is disabled"):
        _cpu_state(quantum=0).grow_capacity(100)
    assert state.grow_capacity(10) == 0
    with pytest.raises(ValueError, match="released bank indices must be integer"):
        state.release(torch.zeros(2, 2, dtype=torch.int64))
    with pytest.raises(ValueError, match="retained bank indices must be integer"):
        state.retain_banks(torch.zeros(2))
    assert int(state.release(torch.zeros(0, dtype=torch.int64))) == 0


def test_paged_map_page_sizes():
    """Pages hold a power of two of 2 to 64 slots dividing N."""

    from copy_on_write_sdm_amd.allocator import PagedSlotMap

    assert PagedSlotMap._shift(16, 65536) == 4
    assert PagedSlotMap._shift(2, 4) == 1
    assert PagedSlotMap._shift(64, 128) == 6
    for bad, slots in ((1, 64), (3, 63), (128, 1024), (16, 40), (0, 16)):
        with pytest.raises(ValueError, match="power of two"):
            PagedSlotMap._shift(bad, slots)


def test_zipf_seed_shares_hot_slots_across_calls():
    """make_steps(zipf_seed=...) draws the per-(layer, head) Zipf permutation
    from its own generator: a prefill and a decode drawn with different seeds
    write the same hot slots, and calls without it keep drawing the
    permutation from the call's generator."""
    import torch
    from copy_on_write_sdm_amd.synthetic import make_steps

    kw = dict(steps=64, layers=2, banks=4, slots=64, width=4, writes=4, reads=8,
              distribution="zipf", zipf_exponent=2.4, heads=2)
    a = make_steps(seed=1, zipf_seed=11, **kw).write_indices.long()
    b = make_steps(seed=2, zipf_seed=11, **kw).write_indices.long()
    c = make_steps(seed=2, zipf_seed=12, **kw).write_indices.long()

    def hottest(w):
        counts = torch.zeros(w.shape[1], w.shape[2], kw["slots"], dtype=torch.long)
        for t in range(w.shape[0]):
            counts.scatter_add_(2, w[t], torch.ones_like(w[t]))
        return counts.argmax(dim=2)

    assert torch.equal(hottest(a), hottest(b))
    assert not torch.equal(hottest(b), hottest(c))
    # banks of one head share its permutation (bank = request * heads + head)
    h = hottest(a)
    assert torch.equal(h[:, 0], h[:, 2]) and torch.equal(h[:, 1], h[:, 3])
    # without zipf_seed the call's own generator draws it: same seed, same routes
    d = make_steps(seed=3, **kw).write_indices
    assert torch.equal(d, make_steps(seed=3, **kw).write_indices)
