"""GPU parity of the fused packed step and the dense-table control.

Bar: readings, map, free stack, live slab rows and diagnostics are bit-exact
against the CPU oracle (oracle/state.py, allocator.py:1466-1525 semantics,
bank-major pops), and the packed and dense GPU kernels agree bit for bit.
The oracle itself is pinned in tests/test_oracle_pins.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import _native as nat
import reference_cases as rc
from gpu_helpers import assert_state_equal, make_case, to_device, to_numpy
from oracle import state as ref

pytestmark = pytest.mark.gpu


def _trace(device, *, banks, slots, width, writes, reads, steps, seed,
           index_dtype=torch.int32, capacity=None, distribution="uniform"):
    m0, seq = make_case(banks=banks, slots=slots, width=width, writes=writes, reads=reads,
                        steps=steps, seed=seed, index_dtype=index_dtype,
                        distribution=distribution)
    capacity = capacity or banks * slots
    print(f"trace B={banks} N={slots} D={width} W={writes} R={reads} T={steps} "
          f"seed={seed} idx={index_dtype}", flush=True)
    state = cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=banks,
                                                   capacity_rows=capacity)
    state.capacity_is_proven = True
    oracle = ref.allocate(m0.numpy(), banks=banks, capacity_rows=capacity)
    oracle.capacity_is_proven = True
    dense = m0.expand(banks, -1, -1).clone(memory_format=torch.contiguous_format).to(device)
    for s, inputs in enumerate(seq):
        gpu = to_device(inputs, device)
        reading, diag = cow.packed_sdm_cow_step(state, **gpu, validate_routes=False)
        dense_reading = cow.dense_sdm_sparse_step(dense, **gpu, validate_routes=False)
        want, wdiag = ref.packed_step(oracle, **to_numpy(inputs))
        got = reading.cpu().numpy()
        if not np.array_equal(got, want):
            diff = np.abs(got - want).max()
            raise AssertionError(f"step {s}: reading differs from oracle (max abs {diff})")
        assert torch.equal(reading, dense_reading), f"step {s}: packed != dense"
        assert np.array_equal(diag.first_touches_by_sequence.cpu().numpy(),
                              wdiag.first_touches_by_sequence)
        assert np.array_equal(diag.repeated_writes_by_sequence.cpu().numpy(),
                              wdiag.repeated_writes_by_sequence)
        assert int(diag.allocated_rows_after_step) == wdiag.allocated_rows_after_step
    assert_state_equal(state, oracle)
    materialized = state.materialize_dense()
    assert np.array_equal(materialized.cpu().numpy(), ref.materialize_dense(oracle))
    assert torch.equal(materialized, dense)
    state.validate_invariants()
    return state, oracle


@pytest.mark.parametrize("backend", ["auto", "torch"])
def test_reference_known_answers(device, backend):
    """tests/test_allocator.py:65-82 on the GPU path, also with the backend
    the reference's test names ("torch": the same kernels, with the torch
    path's exhaustion check before every step)."""

    initial, steps = rc.reference_case(2)
    packed = cow.PackedSDMCopyOnWriteState.allocate(
        initial.to(device), banks=rc.BANKS, capacity_rows=rc.BANKS * rc.SLOTS)
    dense = initial.expand(rc.BANKS, -1, -1).clone().to(device)
    oracle = ref.allocate(initial.numpy(), banks=rc.BANKS, capacity_rows=rc.BANKS * rc.SLOTS)
    firsts = []
    for inputs in steps:
        gpu = to_device(inputs, device)
        dense_read = cow.dense_sdm_sparse_step(dense, **gpu, backend=backend)
        packed_read, diag = cow.packed_sdm_cow_step(packed, **gpu, backend=backend)
        want, _ = ref.packed_step(oracle, **to_numpy(inputs))
        assert torch.equal(dense_read, packed_read)
        assert torch.equal(dense, packed.materialize_dense())
        assert np.array_equal(packed_read.cpu().numpy(), want)
        firsts.append((int(diag.first_touches_by_sequence.sum()),
                       int(packed.allocated_rows_tensor())))
    assert firsts == [(rc.FIRST_STEP_FIRST_TOUCHES, rc.FIRST_STEP_ALLOCATED),
                      (rc.REPEAT_STEP_FIRST_TOUCHES, rc.REPEAT_STEP_ALLOCATED)]
    b, s = rc.UNTOUCHED_PROBE
    assert torch.equal(packed.materialize_dense()[b, s].cpu(), initial[0, s])
    assert_state_equal(packed, oracle)


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_baseline_shape_trace(device, index_dtype):
    """Benchmark layer shape: B=64, N=256, D=128, top-4 write, top-16 read."""

    _trace(device, banks=64, slots=256, width=128, writes=4, reads=16, steps=24, seed=21,
           index_dtype=index_dtype)


@pytest.mark.parametrize("banks,slots,width,writes,reads", [
    (1, 8, 8, 1, 1),          # smallest
    (5, 64, 64, 4, 16),       # partial last block, one float per lane
    (7, 48, 130, 7, 33),      # W=7 (16-row path), 3 read batches, 2 width chunks
    (4, 64, 256, 16, 64),     # float4 lanes, 16 writes, 64 reads
    (3, 128, 5, 3, 100),      # odd width, 2 read registers per lane
    (2, 300, 384, 64, 256),   # W=64, R=256, 2 float4 chunks
    (130, 64, 32, 4, 16),     # 130 banks: look-back across >2 windows
])
def test_shapes(device, banks, slots, width, writes, reads):
    _trace(device, banks=banks, slots=slots, width=width, writes=writes, reads=reads,
           steps=6, seed=banks * 7 + writes)


def test_many_banks_lookback(device):
    """1000 banks: the bank-order scan spans 16 look-back windows."""

    _trace(device, banks=1000, slots=64, width=64, writes=4, reads=8, steps=4, seed=5)


def test_read_after_write_same_slots(device):
    """Every read slot is also written this step: reads must see the update."""

    banks, slots, width = 8, 32, 128
    m0, seq = make_case(banks=banks, slots=slots, width=width, writes=4, reads=4, steps=5,
                        seed=31)
    for inputs in seq:
        inputs["read_indices"] = inputs["write_indices"].flip(-1).contiguous()
    state = cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=banks,
                                                   capacity_rows=banks * slots)
    oracle = ref.allocate(m0.numpy(), banks=banks, capacity_rows=banks * slots)
    for inputs in seq:
        reading, _ = cow.packed_sdm_cow_step(state, **to_device(inputs, device))
        want, _ = ref.packed_step(oracle, **to_numpy(inputs))
        assert np.array_equal(reading.cpu().numpy(), want)
    assert_state_equal(state, oracle)


def test_explicit_erase_gate_and_templates(device):
    """Two memory heads (templates) and a separate erase gate."""

    banks, slots, width, heads = 6, 32, 64, 2
    m0 = torch.randn(heads, slots, width, generator=torch.Generator().manual_seed(3)) * 0.02
    templates = torch.arange(heads).repeat(banks // heads)
    _, seq = make_case(banks=banks, slots=slots, width=width, writes=4, reads=8, steps=6,
                       seed=41)
    state = cow.PackedSDMCopyOnWriteState.allocate(
        m0.to(device), banks=banks, capacity_rows=banks * slots,
        template_indices=templates.to(device))
    oracle = ref.allocate(m0.numpy(), banks=banks, capacity_rows=banks * slots,
                          template_indices=templates.numpy())
    gen = torch.Generator().manual_seed(9)
    for inputs in seq:
        erase = torch.sigmoid(torch.randn(banks, generator=gen))
        reading, _ = cow.packed_sdm_cow_step(state, **to_device(inputs, device),
                                             erase_gate=erase.to(device))
        want, _ = ref.packed_step(oracle, **to_numpy(inputs), erase_gate=erase.numpy())
        assert np.array_equal(reading.cpu().numpy(), want)
    assert_state_equal(state, oracle)
    assert np.array_equal(state.materialize_dense().cpu().numpy(), ref.materialize_dense(oracle))


def test_layers_launch_equals_per_layer_calls(device):
    layers, banks, slots, width = 7, 16, 64, 128
    from copy_on_write_sdm_amd import synthetic

    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=8, device=device)
    batch = synthetic.make_steps(steps=5, layers=layers, banks=banks, slots=slots, width=width,
                                 writes=4, reads=16, seed=9, device=device)
    fused = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks,
                                                    capacity_rows=banks * slots)
             for l in range(layers)]
    single = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks,
                                                     capacity_rows=banks * slots)
              for l in range(layers)]
    for st in fused + single:
        st.capacity_is_proven = True
    dense = [m0[l].expand(banks, -1, -1).clone(memory_format=torch.contiguous_format) for l in range(layers)]
    for s in range(5):
        outs = cow.packed_sdm_cow_step_layers(
            fused, batch.write_indices[s], batch.write_weights[s], batch.values[s],
            batch.input_gate[s], batch.forget_log_gate[s], batch.read_indices[s],
            batch.read_weights[s])
        douts = cow.dense_sdm_sparse_step_layers(
            dense, batch.write_indices[s], batch.write_weights[s], batch.values[s],
            batch.input_gate[s], batch.forget_log_gate[s], batch.read_indices[s],
            batch.read_weights[s])
        for l in range(layers):
            one, _ = cow.packed_sdm_cow_step(single[l], **batch.step(s, l),
                                             validate_routes=False)
            assert torch.equal(outs[l], one)
            assert torch.equal(douts[l], one)
    for a, b in zip(fused, single):
        assert torch.equal(a.logical_to_physical, b.logical_to_physical)
        assert torch.equal(a.free_rows[: int(a.free_count)], b.free_rows[: int(b.free_count)])
        assert torch.equal(a.materialize_dense(), b.materialize_dense())


def test_unproven_exhaustion_raises_without_mutation(device):
    initial, steps = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=5)
    before = state.logical_to_physical.clone()
    with pytest.raises(ValueError, match="physical slab is exhausted"):
        cow.packed_sdm_cow_step(state, **to_device(steps[0], device))
    assert torch.equal(state.logical_to_physical, before)
    assert int(state.free_count) == 5


def test_torch_backend_checks_exhaustion_on_proven_state(device):
    """The reference's torch path asserts the free stack covers the step's
    first touches whether or not a proof exists (allocator.py:1474): with
    backend="torch" a proven state too small for the step raises before
    anything changes."""

    initial, steps = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=5)
    state.capacity_is_proven = True
    before = state.logical_to_physical.clone()
    with pytest.raises(ValueError, match="physical slab is exhausted"):
        cow.packed_sdm_cow_step(state, **to_device(steps[0], device), validate_routes=False,
                                backend="torch")
    assert torch.equal(state.logical_to_physical, before)
    assert int(state.free_count) == 5 and int(state.overflow_flag) == 0


def test_proven_overflow_latches_and_spares_later_banks(device):
    """Capacity 5 with 2+2+2 first touches: banks 0 and 1 fit (bank-major),
    bank 2 does not; the overflow flag latches, bank 2 is untouched."""

    initial, steps = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=5)
    state.capacity_is_proven = True
    cow.packed_sdm_cow_step(state, **to_device(steps[0], device), validate_routes=False)
    mapping = state.logical_to_physical.cpu()
    assert int(state.overflow_flag) == 1
    assert int(state.free_count) == 1
    assert [int(mapping[0, 2]), int(mapping[0, 5]), int(mapping[1, 1]), int(mapping[1, 7])] == [
        4, 3, 2, 1]
    assert (mapping[2] == -1).all()
    with pytest.raises(AssertionError, match="recorded a slab overflow"):
        state.validate_invariants()


def test_route_validation_errors(device):
    initial, steps = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=48)
    good = to_device(steps[0], device)
    cases = [
        ("write_indices", [[2, 2], [1, 7], [4, 10]], "write one logical slot twice"),
        ("write_indices", [[2, 16], [1, 7], [4, 10]], "write index lies outside"),
        ("write_indices", [[2, -1], [1, 7], [4, 10]], "write index lies outside"),
        ("read_indices", [[0, 1, 2, 16], [3, 4, 5, 6], [6, 7, 8, 9]], "read index lies outside"),
    ]
    for key, value, message in cases:
        bad = dict(good)
        bad[key] = torch.tensor(value, dtype=torch.int64, device=device)
        with pytest.raises(ValueError, match=message):
            cow.packed_sdm_cow_step(state, **bad)
        dense = initial.expand(rc.BANKS, -1, -1).clone(memory_format=torch.contiguous_format).to(device)
        with pytest.raises(ValueError, match=message):
            cow.dense_sdm_sparse_step(dense, **bad)
    assert (state.logical_to_physical == -1).all()
    state.validate_invariants()


def test_unvalidated_bad_routes_skip_the_bank_and_flag(device):
    """With validate_routes=False an out-of-range index never reaches memory:
    the bank is skipped and the sticky error word makes validation fail."""

    initial, steps = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=48)
    state.capacity_is_proven = True
    bad = to_device(steps[0], device)
    bad["write_indices"] = torch.tensor([[2, 5], [1, 1 << 30], [4, 10]], device=device)
    cow.packed_sdm_cow_step(state, **bad, validate_routes=False)
    assert (state.logical_to_physical[1] == -1).all()
    assert int((state.logical_to_physical >= 0).sum()) == 4
    with pytest.raises(AssertionError, match="recorded errors"):
        state.validate_invariants()


def test_zipf_routes_large_address_space(device):
    """Config-5-like skewed routes at N=65536 (one layer, reduced batch)."""

    _trace(device, banks=8, slots=65536, width=128, writes=4, reads=16, steps=8, seed=77,
           distribution="zipf", capacity=1024)


def test_fault_bits_raise_at_the_proofs_read(device):
    """A step whose bounded wait gave up (or that found the state corrupt)
    latches COWSDM_ERR_LOOKBACK / _CORRUPT; the next read the decode loop
    makes anyway (the proof's free-count read, single and batched) raises.
    The fault is set from the host: no kernel is made to stop."""

    initial, _ = rc.reference_case(1)
    state = cow.PackedSDMCopyOnWriteState.allocate(initial.to(device), banks=rc.BANKS,
                                                   capacity_rows=8, growth_quantum_rows=8)
    state.prepare_step_capacity(4)       # a clean word: the proof reads and passes
    for bit in (nat.ERR_LOOKBACK, nat.ERR_CORRUPT):
        state.ensure_scratch()[nat.SCRATCH_ERRORS] = bit
        state.proven_maximum_additional_allocations = 0
        with pytest.raises(RuntimeError, match="stopped on a fault"):
            state.prepare_step_capacity(4)
        with pytest.raises(RuntimeError, match="stopped on a fault"):
            cow.PackedSDMCopyOnWriteState.prepare_step_capacity_layers([state], 4)
    # a route error alone (the bank was skipped) does not stop the loop
    state.ensure_scratch()[nat.SCRATCH_ERRORS] = nat.ERR_WRITE_INDEX
    state.proven_maximum_additional_allocations = 0
    state.prepare_step_capacity(4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_precision_inputs(device, dtype):
    """Route weights, values and gates in float16/bfloat16 (the reference
    model's activations): both steps compute in float32 from the widened
    inputs, as both reference backends do (allocator.py:1136-1139, 1490-1521),
    so the state equals the oracle's step on the widened inputs bit for bit
    and the reading is that step's reading rounded to the values' dtype."""

    banks, slots, width = 8, 64, 128
    m0, steps = make_case(banks=banks, slots=slots, width=width, writes=4, reads=16, steps=6,
                          seed=51)
    packed = cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=banks,
                                                    capacity_rows=banks * slots)
    dense = m0.expand(banks, -1, -1).clone().to(device)
    oracle = ref.allocate(m0.numpy(), banks=banks, capacity_rows=banks * slots)
    floats = ("write_weights", "values", "input_gate", "forget_log_gate", "read_weights")
    for inputs in steps:
        narrow = {k: (v.to(dtype) if k in floats else v) for k, v in inputs.items()}
        widened = {k: (v.float() if k in floats else v) for k, v in narrow.items()}
        got, _ = cow.packed_sdm_cow_step(packed, **to_device(narrow, device))
        got_dense = cow.dense_sdm_sparse_step(dense, **to_device(narrow, device))
        assert got.dtype == dtype and got_dense.dtype == dtype
        want, _ = ref.packed_step(oracle, **to_numpy(widened))
        want = torch.from_numpy(want).to(dtype)
        assert torch.equal(got.cpu(), want)
        assert torch.equal(got_dense.cpu(), want)
        assert torch.equal(dense, packed.materialize_dense())
    assert_state_equal(packed, oracle)
