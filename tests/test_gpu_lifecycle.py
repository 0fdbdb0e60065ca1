"""GPU parity of the state lifecycle: allocate, prefill handoff, growth and
the capacity proof, release, bank retention, trim, admission, invariant
checks, and a continuous-batching scenario (release, compact, trim, admit).

Bar: map, free stack, live slab rows, counters and returned values equal
the CPU oracle (oracle/state.py restating allocator.py:506-1095) exactly.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import synthetic
from gpu_helpers import assert_state_equal, make_case, to_device, to_numpy
from oracle import state as ref

pytestmark = pytest.mark.gpu


def _pair(device, *, banks=6, slots=64, width=32, writes=4, reads=8, steps=10, seed=3,
          quantum=16, capacity=None):
    """A GPU state and an oracle state driven through the same decode steps
    with per-step capacity proofs (slab growth on)."""

    m0, seq = make_case(banks=banks, slots=slots, width=width, writes=writes, reads=reads,
                        steps=steps, seed=seed)
    capacity = capacity or quantum
    st = cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=banks,
                                                capacity_rows=capacity,
                                                growth_quantum_rows=quantum)
    orc = ref.allocate(m0.numpy(), banks=banks, capacity_rows=capacity,
                       growth_quantum_rows=quantum)
    for inputs in seq:
        assert st.prepare_step_capacity(banks * writes) == ref.prepare_step_capacity(
            orc, banks * writes)
        reading, _ = cow.packed_sdm_cow_step(st, **to_device(inputs, device),
                                             validate_routes=False)
        want, _ = ref.packed_step(orc, **to_numpy(inputs))
        assert np.array_equal(reading.cpu().numpy(), want)
        assert_state_equal(st, orc)
    return st, orc, m0


def test_allocate_matches_oracle(device):
    m0 = torch.randn(2, 16, 8)
    st = cow.PackedSDMCopyOnWriteState.allocate(
        m0.to(device), banks=4, capacity_rows=10,
        template_indices=torch.tensor([0, 1, 1, 0], device=device))
    orc = ref.allocate(m0.numpy(), banks=4, capacity_rows=10,
                       template_indices=np.array([0, 1, 1, 0]))
    assert_state_equal(st, orc)
    assert st.validate_invariants() == ref.validate_invariants(orc)
    assert int(st.scratch.abs().sum()) == 0
    with pytest.raises(ValueError, match="template index lies outside"):
        cow.PackedSDMCopyOnWriteState.allocate(
            m0.to(device), banks=2, capacity_rows=4,
            template_indices=torch.tensor([0, 2], device=device))
    with pytest.raises(ValueError, match="require explicit mapping"):
        cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=2, capacity_rows=4)


def test_decode_with_growth_matches_oracle(device):
    st, orc, _ = _pair(device, steps=12)
    assert st.growth_events >= 2
    assert np.array_equal(st.materialize_dense().cpu().numpy(), ref.materialize_dense(orc))
    assert st.validate_invariants() == ref.validate_invariants(orc)


def test_reference_growth_known_answer(device):
    st = cow.PackedSDMCopyOnWriteState.allocate(torch.zeros(1, 16, 4, device=device), banks=2,
                                                capacity_rows=4, growth_quantum_rows=4)
    before = st.materialize_dense().clone()
    st.grow_capacity(5)
    assert st.capacity_rows == 8
    assert st.growth_rows_added == 4
    assert st.growth_rows_copied == 4
    assert torch.equal(st.materialize_dense(), before)
    st.validate_invariants()
    assert st.free_rows.tolist() == list(range(8))


def test_growth_within_headroom_moves_no_rows(device):
    """After a growth the slab leads a buffer with room for as much growth
    again: a later growth that fits keeps every row where it is (the slab's
    address does not change), one that does not fit moves them, and the
    state equals the oracle's after the same growths either way."""

    st, orc, _ = _pair(device, steps=4)
    width = st.width
    # the smallest growth (new buffers on the first), one that fits, one
    # past the buffer, and one that fits again
    for case in ("first", "fits", "past", "fits"):
        if case == "past":
            minimum = st.slab_buffers[0].shape[0] + 1
        else:
            minimum = st.capacity_rows + 1
        before = st.values.data_ptr()
        added = st.grow_capacity(minimum)
        assert added == ref.grow_capacity(orc, minimum)
        if case != "first":
            assert (st.values.data_ptr() == before) == (case == "fits"), case
        assert_state_equal(st, orc)
        room = st.slab_buffers[0].shape[0] - st.capacity_rows
        assert room > 0
        assert st.storage_bytes()["slab_headroom"] == room * (width * 4 + 4)
    assert st.growth_rows_copied == orc.growth_rows_copied
    st.validate_invariants()


def test_batched_proof_equals_per_state_proofs(device):
    pairs = [_pair(device, seed=s, steps=3) for s in (5, 6, 7)]
    states = [p[0] for p in pairs]
    oracles = [p[1] for p in pairs]
    for demand in (24, 24, 60, 200, 8):
        caps = cow.PackedSDMCopyOnWriteState.prepare_step_capacity_layers(states, demand)
        assert caps == [ref.prepare_step_capacity(o, demand) for o in oracles]
        for st, orc in zip(states, oracles):
            assert_state_equal(st, orc)


@pytest.mark.parametrize("order", [[2, 0], [5], [0, 1, 2, 3, 4, 5], [4, 1, 3]])
def test_release_matches_oracle(device, order):
    st, orc, _ = _pair(device)
    released = st.release(torch.tensor(order, device=device))
    assert released.dtype == torch.int64 and released.ndim == 0
    assert int(released) == ref.release(orc, np.array(order))
    assert_state_equal(st, orc)
    st.validate_invariants()


def test_release_errors(device):
    st, _, _ = _pair(device, steps=2)
    with pytest.raises(ValueError, match="invalid or duplicated"):
        st.release(torch.tensor([1, 1], device=device))
    with pytest.raises(ValueError, match="invalid or duplicated"):
        st.release(torch.tensor([6], device=device))
    empty = st.release(torch.tensor([], dtype=torch.int64, device=device))
    assert int(empty) == 0 and empty.dtype == torch.int32


def test_retain_matches_oracle(device):
    st, orc, _ = _pair(device)
    with pytest.raises(ValueError, match="released before compaction"):
        st.retain_banks(torch.tensor([0, 1], device=device))
    st.release(torch.tensor([1, 4], device=device))
    ref.release(orc, np.array([1, 4]))
    with pytest.raises(ValueError, match="invalid or duplicated"):
        st.retain_banks(torch.tensor([0, 0], device=device))
    keep = [5, 0, 3, 2]
    st.retain_banks(torch.tensor(keep, device=device, dtype=torch.int32))
    ref.retain_banks(orc, np.array(keep))
    assert_state_equal(st, orc)
    assert st.scratch.numel() == 8 + len(keep)
    st.validate_invariants()


@pytest.mark.parametrize("headroom", [0, 5, 40])
def test_trim_matches_oracle(device, headroom):
    st, orc, _ = _pair(device, steps=12)
    st.release(torch.tensor([0, 3], device=device))
    ref.release(orc, np.array([0, 3]))
    before = st.materialize_dense()
    removed = st.trim_capacity(headroom_rows=headroom)
    assert removed == ref.trim_capacity(orc, headroom_rows=headroom)
    assert_state_equal(st, orc)
    assert torch.equal(st.materialize_dense(), before)
    st.validate_invariants()


def test_trim_then_decode_matches_oracle(device):
    st, orc, _ = _pair(device, steps=8)
    st.release(torch.tensor([2], device=device))
    ref.release(orc, np.array([2]))
    st.trim_capacity(headroom_rows=3)
    ref.trim_capacity(orc, headroom_rows=3)
    _, seq = make_case(banks=6, slots=64, width=32, writes=4, reads=8, steps=4, seed=99)
    for inputs in seq:
        st.prepare_step_capacity(24)
        ref.prepare_step_capacity(orc, 24)
        r, _ = cow.packed_sdm_cow_step(st, **to_device(inputs, device), validate_routes=False)
        w, _ = ref.packed_step(orc, **to_numpy(inputs))
        assert np.array_equal(r.cpu().numpy(), w)
    assert_state_equal(st, orc)


@pytest.mark.parametrize("dst_capacity", [None, 400])
def test_append_matches_oracle(device, dst_capacity):
    dst, dorc, m0 = _pair(device, seed=11, steps=6, capacity=dst_capacity)
    src, sorc, _ = _pair(device, seed=11, steps=0)
    # same M0 object for both pools; drive the source with other routes
    _, seq = make_case(banks=6, slots=64, width=32, writes=4, reads=8, steps=5, seed=12)
    for inputs in seq:
        src.prepare_step_capacity(24)
        ref.prepare_step_capacity(sorc, 24)
        cow.packed_sdm_cow_step(src, **to_device(inputs, device), validate_routes=False)
        ref.packed_step(sorc, **to_numpy(inputs))
    sorc.shared_initial_memory = dorc.shared_initial_memory
    src.shared_initial_memory = dst.shared_initial_memory
    src_dense = src.materialize_dense()
    count = dst.append_banks_from(src)
    assert count == ref.append_banks_from(dorc, sorc)
    assert_state_equal(dst, dorc)
    assert torch.equal(dst.materialize_dense()[6:], src_dense)
    assert dst.scratch.numel() == 8 + 12
    dst.validate_invariants()


def test_append_rejects_other_initial_memory(device):
    a, _, _ = _pair(device, seed=1, steps=1)
    b, _, _ = _pair(device, seed=2, steps=1)
    with pytest.raises(ValueError, match="different learned initial memory"):
        a.append_banks_from(b)


def test_from_dense_overlay_matches_oracle(device):
    gen = torch.Generator().manual_seed(4)
    banks, slots, width = 5, 32, 16
    m0 = torch.randn(1, slots, width, generator=gen)
    dense = m0.expand(banks, -1, -1).clone()
    active = torch.rand(banks, slots, generator=gen) < 0.3
    dense[active] = torch.randn(int(active.sum()), width, generator=gen)
    tmpl = torch.zeros(banks, dtype=torch.int64)
    # (a quantum past B * N: a slab larger than the count's row lists, which
    # the handoff counts again into a larger workspace)
    for kwargs in (dict(growth_quantum_rows=8), dict(capacity_rows=80),
                   dict(capacity_rows=160, maximum_future_allocations=100), dict(),
                   dict(growth_quantum_rows=256)):
        st = cow.PackedSDMCopyOnWriteState.from_dense_overlay(
            m0.to(device), dense.to(device), active.to(device),
            template_indices=tmpl.to(device), **kwargs)
        orc = ref.from_dense_overlay(m0.numpy(), dense.numpy(), active.numpy(),
                                     template_indices=tmpl.numpy(), **kwargs)
        assert_state_equal(st, orc)
        assert torch.equal(st.materialize_dense().cpu(), dense)
    with pytest.raises(ValueError, match="smaller than the prefill working set"):
        cow.PackedSDMCopyOnWriteState.from_dense_overlay(
            m0.to(device), dense.to(device), active.to(device),
            template_indices=tmpl.to(device), capacity_rows=int(active.sum()) - 1)


def test_pack_prefill_layer_from_routes(device):
    """inference.py:314-366: the union of prefix-written slots becomes
    private; the terminal dense state is preserved."""

    batch, heads, slots, width, writes, time = 3, 2, 32, 16, 4, 7
    gen = torch.Generator().manual_seed(8)
    m0 = torch.randn(heads, slots, width, generator=gen)
    idx = torch.rand(batch, time, heads, slots, generator=gen).topk(writes, -1).indices
    final = torch.randn(batch, heads, slots, width, generator=gen)
    st = cow.pack_prefill_layer(m0.to(device), final.to(device), idx.to(device),
                                capacity_rows=None, decode_capacity=time + 5,
                                growth_quantum_rows=0)
    active = np.zeros((batch * heads, slots), bool)
    for b in range(batch):
        for h in range(heads):
            active[b * heads + h, idx[b, :, h].flatten().numpy()] = True
    assert np.array_equal(st.logical_to_physical.cpu().numpy() >= 0, active)
    dense = st.materialize_dense().cpu()
    flat = final.flatten(0, 1)
    assert torch.equal(dense[torch.from_numpy(active)], flat[torch.from_numpy(active)])
    assert st.capacity_is_proven
    assert st.proven_maximum_additional_allocations == min(batch * heads * writes * 5,
                                                           batch * heads * slots - active.sum())


def test_invariant_violations_are_reported(device):
    st, _, _ = _pair(device, steps=4)
    live = st.logical_to_physical[st.logical_to_physical >= 0]
    # two owners of one row
    bad = dataclasses.replace(st)
    bad.logical_to_physical = st.logical_to_physical.clone()
    flat = bad.logical_to_physical.view(-1)
    owners = (flat >= 0).nonzero().flatten()
    flat[owners[1]] = flat[owners[0]]
    with pytest.raises(AssertionError, match="multiple logical owners"):
        bad.validate_invariants()
    # free stack duplicate
    bad = dataclasses.replace(st)
    bad.free_rows = st.free_rows.clone()
    if int(st.free_count) >= 2:
        bad.free_rows[1] = bad.free_rows[0]
        with pytest.raises(AssertionError, match="free SDM row stack contains duplicates"):
            bad.validate_invariants()
    # coverage
    bad = dataclasses.replace(st)
    bad.free_count = st.free_count.clone() - 1
    with pytest.raises(AssertionError, match="do not cover capacity"):
        bad.validate_invariants()
    # overflow flag
    bad = dataclasses.replace(st)
    bad.overflow_flag = torch.ones((), dtype=torch.int32, device=device)
    with pytest.raises(AssertionError, match="recorded a slab overflow"):
        bad.validate_invariants()
    assert live.numel() > 0
    st.validate_invariants()


def _decode_both(states, oracles, dense, seq, device):
    for inputs_per_layer in seq:
        for st, orc, tab, inputs in zip(states, oracles, dense, inputs_per_layer):
            st.prepare_step_capacity(st.banks * 4)
            ref.prepare_step_capacity(orc, orc.banks * 4)
            gpu = to_device(inputs, device)
            r, _ = cow.packed_sdm_cow_step(st, **gpu, validate_routes=False,
                                           collect_diagnostics=False)
            rd = cow.dense_sdm_sparse_step(tab, **gpu, validate_routes=False)
            w, _ = ref.packed_step(orc, **to_numpy(inputs))
            assert torch.equal(r, rd)
            assert np.array_equal(r.cpu().numpy(), w)


def test_continuous_batching_config4(device):
    """Continuous batching (experiments/benchmark_serving.py:472-613 pattern)
    at config 4's shape (B=4, L=7, N=256, D=128): 4 requests decode 16
    steps, requests 0 and 2 are released, survivors compacted and the pools
    trimmed, 2 new requests with 128-token prefixes admitted, decode
    continues 16 steps at mixed positions.  Packed state must equal the dense
    control and the oracle throughout; released rows must equal the rows
    those requests held."""

    layers, batch, slots, width, writes, reads = 7, 4, 256, 128, 4, 16
    quantum = 16
    before, after = 16, 16      # decode steps around the lifecycle events
    layout = "B" * layers
    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=21)

    def prefill(requests, time, seed):
        routes = synthetic.make_steps(steps=time, layers=layers, banks=requests, slots=slots,
                                      width=width, writes=writes, reads=reads, seed=seed)
        states, oracles = [], []
        for l in range(layers):
            table = m0[l, 0].expand(requests, -1, -1).clone(memory_format=torch.contiguous_format).to(device)
            for t in range(time):
                cow.dense_sdm_sparse_step(table, **to_device(routes.step(t, l), device),
                                          validate_routes=False)
            st = cow.pack_prefill_layer(
                m0[l].to(device), table.view(requests, 1, slots, width),
                routes.write_indices[:, l].permute(1, 0, 2).unsqueeze(2).to(device),
                capacity_rows=None, decode_capacity=time + 8, growth_quantum_rows=quantum)
            active = st.logical_to_physical.cpu().numpy() >= 0
            orc = ref.from_dense_overlay(m0[l].numpy(), table.cpu().numpy(), active,
                                         template_indices=np.zeros(requests, np.int64),
                                         growth_quantum_rows=quantum)
            assert_state_equal(st, orc)
            states.append(st)
            oracles.append(orc)
        return states, oracles

    states, oracles = prefill(batch, 16, seed=30)
    serving = cow.FaithfulSDMDecodeState(
        layout=layout, position=16, capacity=160, activation_dtype=torch.float32,
        active_sequences=torch.ones(batch, dtype=torch.bool, device=device),
        sdm_layer_positions=tuple(range(layers)), sdm_states=tuple(states))
    dense = [st.materialize_dense() for st in states]
    steps = synthetic.make_steps(steps=before, layers=layers, banks=batch, slots=slots,
                                 width=width, writes=writes, reads=reads, seed=31)
    _decode_both(states, oracles, dense,
                 [[steps.step(s, l) for l in range(layers)] for s in range(before)], device)

    held = sum(int((st.logical_to_physical[[0, 2]] >= 0).sum()) for st in states)
    released = serving.release_and_compact([0, 2], trim=True, trim_headroom_rows=16)
    assert released == held
    want = sum(ref.release(o, np.array([0, 2])) for o in oracles)
    assert released == want
    for o in oracles:
        ref.retain_banks(o, np.array([1, 3]))
        ref.trim_capacity(o, headroom_rows=16)
    for st, o in zip(serving.sdm_states, oracles):
        assert_state_equal(st, o)
        st.validate_invariants()

    new_states, new_oracles = prefill(2, 128, seed=40)
    incoming = cow.FaithfulSDMDecodeState(
        layout=layout, position=128, capacity=160, activation_dtype=torch.float32,
        active_sequences=torch.ones(2, dtype=torch.bool, device=device),
        sdm_layer_positions=tuple(range(layers)), sdm_states=tuple(new_states))
    serving.position = 16 + before
    assert serving.admit(incoming) == 2
    assert serving.current_positions().tolist() == [16 + before] * 2 + [128, 128]
    for o, n in zip(oracles, new_oracles):
        n.shared_initial_memory = o.shared_initial_memory
        ref.append_banks_from(o, n)
    for st, o in zip(serving.sdm_states, oracles):
        assert_state_equal(st, o)
        st.validate_invariants()

    dense = [st.materialize_dense() for st in serving.sdm_states]
    more = synthetic.make_steps(steps=after, layers=layers, banks=4, slots=slots, width=width,
                                writes=writes, reads=reads, seed=41)
    _decode_both(list(serving.sdm_states), oracles, dense,
                 [[more.step(s, l) for l in range(layers)] for s in range(after)], device)
    for st, tab, o in zip(serving.sdm_states, dense, oracles):
        assert torch.equal(st.materialize_dense(), tab)
        assert_state_equal(st, o)
    usage = serving.storage_bytes()
    assert usage["sdm_logical_dense_fp32"] == layers * 4 * slots * width * 4
    live = sum(int(st.allocated_rows_tensor()) for st in serving.sdm_states)
    assert serving.release() == live
    for st in serving.sdm_states:
        assert int(st.allocated_rows_tensor()) == 0
        st.validate_invariants()
