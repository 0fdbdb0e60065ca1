"""Pins of the CPU oracle (oracle/state.py) -- CPU only.

Each check is independent of the oracle's own formulas: the reference's
known answers (copy_on_write_sdm tests/test_allocator.py:65-99), the
float64 serial recurrences of sdm.py:365-529 (dense route vectors over all
N slots), a scalar-loop restatement, closed forms and allocator invariants.
The planted-mistake tests at the end break one oracle component at a time
and show that at least one pin fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import reference_cases as rc
from oracle import serial
from oracle import state as ref


def _np(inputs: dict) -> dict:
    return {k: v.numpy() for k, v in inputs.items()}


def _random_sequence(rng, banks, slots, width, writes, reads, steps, m0_std=0.5):
    m0 = (rng.standard_normal((1, slots, width)) * m0_std).astype(np.float32)
    seq = []
    for _ in range(steps):
        wi = np.stack([np.sort(rng.permutation(slots)[:writes]) for _ in range(banks)])
        ri = np.stack([np.sort(rng.permutation(slots)[:reads]) for _ in range(banks)])
        ww = rng.standard_normal((banks, writes))
        ww = (np.exp(ww) / np.exp(ww).sum(-1, keepdims=True)).astype(np.float32)
        rw = rng.standard_normal((banks, reads))
        rw = (np.exp(rw) / np.exp(rw).sum(-1, keepdims=True)).astype(np.float32)
        seq.append({
            "write_indices": wi.astype(np.int64),
            "write_weights": ww,
            "values": rng.standard_normal((banks, width)).astype(np.float32),
            "input_gate": (1 / (1 + np.exp(-rng.standard_normal(banks)))).astype(np.float32),
            "forget_log_gate": (-rng.random(banks)).astype(np.float32),
            "read_indices": ri.astype(np.int64),
            "read_weights": rw,
        })
    return m0, seq


# ------------------------------------------------------------------ pins


def pin_reference_known_answers():
    """tests/test_allocator.py:65-82 on the oracle."""

    initial, steps = rc.reference_case(2)
    m0 = initial.numpy()
    dense = np.broadcast_to(m0, (rc.BANKS, rc.SLOTS, rc.WIDTH)).astype(np.float32).copy()
    packed = ref.allocate(m0, banks=rc.BANKS, capacity_rows=rc.BANKS * rc.SLOTS)
    counts = []
    for inputs in steps:
        x = _np(inputs)
        dense_read = ref.dense_step(dense, **x)
        packed_read, diag = ref.packed_step(packed, **x)
        assert np.array_equal(dense_read, packed_read)
        assert np.array_equal(dense, ref.materialize_dense(packed))
        counts.append((int(diag.first_touches_by_sequence.sum()), packed.allocated_rows()))
    assert counts[0] == (rc.FIRST_STEP_FIRST_TOUCHES, rc.FIRST_STEP_ALLOCATED)
    assert counts[1] == (rc.REPEAT_STEP_FIRST_TOUCHES, rc.REPEAT_STEP_ALLOCATED)
    b, s = rc.UNTOUCHED_PROBE
    assert np.array_equal(ref.materialize_dense(packed)[b, s], m0[0, s])


def pin_bank_major_pops():
    """allocator.py:1471-1481 in closed form: from a fresh stack 0..C-1 the
    k-th first touch in bank-major order gets row C-1-k."""

    initial, steps = rc.reference_case(1)
    capacity = rc.BANKS * rc.SLOTS
    packed = ref.allocate(initial.numpy(), banks=rc.BANKS, capacity_rows=capacity)
    ref.packed_step(packed, **_np(steps[0]))
    k = 0
    for bank, row in enumerate(rc.WRITE_INDICES):
        for slot in row:
            assert packed.logical_to_physical[bank, slot] == capacity - 1 - k
            k += 1
    assert packed.free_count == capacity - k


def pin_serial_recurrence(seed=0, banks=3, slots=16, width=8, writes=3, reads=5, steps=24):
    """Packed and dense sparse steps against the float64 serial recurrence
    of sdm.py:464-529 (and its copy-on-write twin, sdm.py:365-461)."""

    rng = np.random.default_rng(seed)
    m0, seq = _random_sequence(rng, banks, slots, width, writes, reads, steps)
    dense = np.broadcast_to(m0, (banks, slots, width)).astype(np.float32).copy()
    packed = ref.allocate(m0, banks=banks, capacity_rows=banks * slots)
    dense_reads, packed_reads = [], []
    for x in seq:
        dense_reads.append(ref.dense_step(dense, **x))
        packed_reads.append(ref.packed_step(packed, **x)[0])
    wi = np.stack([x["write_indices"] for x in seq], 1)
    ww = np.stack([x["write_weights"] for x in seq], 1)
    ri = np.stack([x["read_indices"] for x in seq], 1)
    rw = np.stack([x["read_weights"] for x in seq], 1)
    wroutes = serial.dense_routes(wi, ww, slots)
    rroutes = serial.dense_routes(ri, rw, slots)
    vals = np.stack([x["values"] for x in seq], 1)
    ig = np.stack([x["input_gate"] for x in seq], 1)
    fg = np.stack([x["forget_log_gate"] for x in seq], 1)
    init = np.broadcast_to(m0, (banks, slots, width))
    s_reads, s_final, _ = serial.serial_gated_delta_recurrence(init, wroutes, vals, ig, fg, rroutes)
    c_reads, c_final, _ = serial.serial_copy_on_write_recurrence(init, wroutes, vals, ig, fg,
                                                                 rroutes)
    assert np.array_equal(s_reads, c_reads) and np.array_equal(s_final, c_final)
    scale = 1.0 + np.abs(s_final).max()
    got_reads = np.stack(dense_reads, 1)
    assert np.abs(got_reads - s_reads).max() <= 1e-5 * scale
    assert np.abs(dense - s_final).max() <= 1e-5 * scale
    assert np.array_equal(np.stack(packed_reads, 1), got_reads)
    assert np.array_equal(ref.materialize_dense(packed), dense)


def pin_loop_step(seed=1):
    """One token against the scalar-loop update rule."""

    rng = np.random.default_rng(seed)
    banks, slots, width = 2, 8, 5
    m0, seq = _random_sequence(rng, banks, slots, width, 3, 4, 1)
    x = seq[0]
    dense = np.broadcast_to(m0, (banks, slots, width)).astype(np.float32).copy()
    got = ref.dense_step(dense, **x)
    for b in range(banks):
        table = [list(map(float, row)) for row in m0[0]]
        want = serial.loop_step(
            table, list(x["write_indices"][b]), list(map(float, x["write_weights"][b])),
            list(map(float, x["values"][b])), float(x["input_gate"][b]),
            float(x["input_gate"][b]), float(x["forget_log_gate"][b]),
            list(x["read_indices"][b]), list(map(float, x["read_weights"][b])))
        assert np.abs(got[b] - np.array(want)).max() <= 1e-6 * (1 + np.abs(want).max())
        assert np.abs(dense[b] - np.array(table)).max() <= 1e-6 * (1 + np.abs(table).max())


ALL_PINS = (pin_reference_known_answers, pin_bank_major_pops, pin_serial_recurrence,
            pin_loop_step)


@pytest.mark.parametrize("pin", ALL_PINS, ids=lambda f: f.__name__)
def test_oracle_passes_pin(pin):
    pin()


def test_serial_recurrence_more_shapes():
    for seed, (b, n, d, w, r) in enumerate([(1, 4, 3, 1, 1), (5, 32, 16, 4, 16), (2, 9, 7, 9, 9)]):
        pin_serial_recurrence(seed=seed + 10, banks=b, slots=n, width=d, writes=w, reads=r,
                              steps=12)


# --------------------------------------------------------- closed forms


def test_decay_factor_is_correctly_rounded_exp():
    xs = np.linspace(-3.0, 0.0, 4097).astype(np.float32)
    want = np.array([np.float32(math.exp(float(x))) for x in xs])
    assert np.array_equal(ref.decay_factor(xs), want)


def test_zero_gates_only_decay_written_rows():
    rng = np.random.default_rng(2)
    m0, seq = _random_sequence(rng, 3, 16, 8, 4, 4, 1)
    x = seq[0]
    x["input_gate"] = np.zeros(3, np.float32)
    dense = np.broadcast_to(m0, (3, 16, 8)).astype(np.float32).copy()
    before = dense.copy()
    ref.dense_step(dense, **x)
    alpha = ref.decay_factor(x["forget_log_gate"])
    for b in range(3):
        written = set(x["write_indices"][b].tolist())
        for s in range(16):
            want = before[b, s] * alpha[b] if s in written else before[b, s]
            assert np.array_equal(dense[b, s], want)


def test_full_overwrite_with_unit_gates():
    """alpha = 1, one write of weight 1, gates 1: the row becomes the value."""

    rng = np.random.default_rng(3)
    m0, seq = _random_sequence(rng, 2, 8, 6, 1, 1, 1)
    x = seq[0]
    x["write_weights"] = np.ones((2, 1), np.float32)
    x["input_gate"] = np.ones(2, np.float32)
    x["forget_log_gate"] = np.zeros(2, np.float32)
    x["read_indices"] = x["write_indices"].copy()
    x["read_weights"] = np.ones((2, 1), np.float32)
    dense = np.broadcast_to(m0, (2, 8, 6)).astype(np.float32).copy()
    reading = ref.dense_step(dense, **x)
    assert np.allclose(reading, x["values"], rtol=0, atol=4e-7 * (1 + np.abs(x["values"]).max()))


def test_one_hot_read_returns_row():
    rng = np.random.default_rng(4)
    m0, seq = _random_sequence(rng, 2, 8, 6, 2, 3, 1)
    x = seq[0]
    x["read_weights"] = np.array([[0, 1, 0], [0, 0, 1]], np.float32)
    dense = np.broadcast_to(m0, (2, 8, 6)).astype(np.float32).copy()
    reading = ref.dense_step(dense, **x)
    assert np.array_equal(reading[0], dense[0, x["read_indices"][0, 1]])
    assert np.array_equal(reading[1], dense[1, x["read_indices"][1, 2]])


def test_update_is_affine_in_values():
    rng = np.random.default_rng(5)
    m0, seq = _random_sequence(rng, 2, 8, 6, 3, 3, 1)
    x = seq[0]
    outs = []
    for v in (np.zeros_like(x["values"]), x["values"], 2 * x["values"]):
        dense = np.broadcast_to(m0, (2, 8, 6)).astype(np.float32).copy()
        outs.append(ref.dense_step(dense, **dict(x, values=v)))
    lhs = outs[2] - outs[0]
    rhs = 2 * (outs[1] - outs[0])
    assert np.abs(lhs - rhs).max() <= 1e-5 * (1 + np.abs(lhs).max())


# ----------------------------------------------------------- invariants


def test_random_trace_allocator_invariants():
    rng = np.random.default_rng(6)
    banks, slots, width, writes = 4, 32, 4, 4
    m0, seq = _random_sequence(rng, banks, slots, width, writes, 6, 40)
    st = ref.allocate(m0, banks=banks, capacity_rows=banks * slots)
    touched = [set() for _ in range(banks)]
    for x in seq:
        _, diag = ref.packed_step(st, **x)
        for b in range(banks):
            new = set(x["write_indices"][b].tolist()) - touched[b]
            assert diag.first_touches_by_sequence[b] == len(new)
            assert diag.repeated_writes_by_sequence[b] == writes - len(new)
            touched[b] |= set(x["write_indices"][b].tolist())
            assert (st.logical_to_physical[b] >= 0).sum() == len(touched[b])
        assert diag.allocated_rows_after_step == sum(len(t) for t in touched)
        ref.validate_invariants(st)


def _live_state(seed=7, banks=4, slots=16, width=4, steps=6, quantum=8):
    rng = np.random.default_rng(seed)
    m0, seq = _random_sequence(rng, banks, slots, width, 3, 3, steps)
    st = ref.allocate(m0, banks=banks, capacity_rows=quantum, growth_quantum_rows=quantum)
    for x in seq:
        ref.prepare_step_capacity(st, banks * 3)
        ref.packed_step(st, **x)
    return st


def test_release_pushes_rows_in_listed_bank_order():
    st = _live_state()
    old_free = st.free_count
    order = [2, 0]
    expected = [int(st.logical_to_physical[b, s]) for b in order for s in range(st.slots)
                if st.logical_to_physical[b, s] >= 0]
    before = ref.materialize_dense(st)
    released = ref.release(st, np.array(order))
    assert released == len(expected)
    assert st.free_count == old_free + released
    assert list(st.free_rows[old_free:old_free + released]) == expected
    assert (st.logical_to_physical[order] == -1).all()
    after = ref.materialize_dense(st)
    assert np.array_equal(after[[1, 3]], before[[1, 3]])
    ref.validate_invariants(st)


def test_release_errors():
    st = _live_state()
    with pytest.raises(ValueError, match="invalid or duplicated"):
        ref.release(st, np.array([1, 1]))
    with pytest.raises(ValueError, match="invalid or duplicated"):
        ref.release(st, np.array([9]))
    assert ref.release(st, np.array([], dtype=np.int64)) == 0


def test_retain_banks_gathers_map_rows():
    st = _live_state()
    with pytest.raises(ValueError, match="released before compaction"):
        ref.retain_banks(st, np.array([0, 1, 3]))
    ref.release(st, np.array([2]))
    rows = st.logical_to_physical[[3, 0, 1]].copy()
    values = st.values.copy()
    ref.retain_banks(st, np.array([3, 0, 1]))
    assert np.array_equal(st.logical_to_physical, rows)
    assert np.array_equal(st.values, values)
    with pytest.raises(ValueError, match="invalid or duplicated"):
        ref.retain_banks(st, np.array([0, 0, 1]))


def test_trim_repacks_live_rows_row_major():
    st = _live_state(quantum=8)
    ref.release(st, np.array([1]))
    before = ref.materialize_dense(st)
    live = int((st.logical_to_physical >= 0).sum())
    removed = ref.trim_capacity(st, headroom_rows=3)
    assert st.capacity_rows == max(8, ((live + 3 + 7) // 8) * 8)
    assert removed >= 0
    bank, slot = np.nonzero(st.logical_to_physical >= 0)
    assert list(st.logical_to_physical[bank, slot]) == list(range(live))
    assert list(st.free_rows[:st.free_count]) == list(range(live, st.capacity_rows))
    assert np.array_equal(ref.materialize_dense(st), before)
    assert not st.capacity_is_proven
    ref.validate_invariants(st)


def test_append_pops_from_top_in_row_major_order():
    dst = _live_state(seed=8)
    src = _live_state(seed=9)
    src.shared_initial_memory = dst.shared_initial_memory
    src_dense = ref.materialize_dense(src)
    dst_dense = ref.materialize_dense(dst)
    free = dst.free_count
    top = list(dst.free_rows[:free][::-1])
    count = ref.append_banks_from(dst, src)
    assert count == int((src.logical_to_physical >= 0).sum())
    merged = ref.materialize_dense(dst)
    banks = src.banks
    assert np.array_equal(merged[:-banks], dst_dense)
    # src was built on its own M0; compare live rows only
    bank, slot = np.nonzero(src.logical_to_physical >= 0)
    assert np.array_equal(merged[-banks:][bank, slot], src_dense[bank, slot])
    if count <= free:
        assert list(dst.logical_to_physical[-banks:][bank, slot]) == top[:count]
    ref.validate_invariants(dst)


def test_growth_appends_new_rows_after_old_free_entries():
    st = _live_state(quantum=8)
    free = st.free_count
    old_free_rows = list(st.free_rows[:free])
    old_capacity = st.capacity_rows
    before = ref.materialize_dense(st)
    added = ref.grow_capacity(st, old_capacity + 1)
    assert added == 8 and st.capacity_rows == old_capacity + 8
    assert list(st.free_rows[:st.free_count]) == old_free_rows + list(
        range(old_capacity, old_capacity + 8))
    assert st.growth_rows_copied == old_capacity or st.growth_events > 1
    assert np.array_equal(ref.materialize_dense(st), before)


def test_reference_growth_known_answer():
    st = ref.allocate(np.zeros((1, 16, 4), np.float32), banks=2, capacity_rows=4,
                      growth_quantum_rows=4)
    before = ref.materialize_dense(st)
    ref.grow_capacity(st, 5)
    assert st.capacity_rows == rc.GROWTH_CAPACITY_AFTER
    assert st.growth_rows_added == rc.GROWTH_ROWS_ADDED
    assert st.growth_rows_copied == rc.GROWTH_ROWS_COPIED
    assert np.array_equal(ref.materialize_dense(st), before)
    ref.validate_invariants(st)


def test_prepare_step_capacity_script():
    """Hand-computed proof sequence (allocator.py:745-773)."""

    st = ref.allocate(np.zeros((1, 8, 2), np.float32), banks=2, capacity_rows=4,
                      growth_quantum_rows=4)
    assert ref.prepare_step_capacity(st, 6) == 8      # free 4 < 6: grow to 4+6-4=6 -> 8
    assert st.proven_maximum_additional_allocations == 8 - 6
    assert st.growth_events == 1
    st.free_count = 5                                  # pretend one row was used
    assert ref.prepare_step_capacity(st, 2) == 8       # proven 2 >= 2
    assert st.proven_maximum_additional_allocations == 0
    assert ref.prepare_step_capacity(st, 2) == 8       # reconcile: free 5 >= 2
    assert st.proven_maximum_additional_allocations == 3
    unproven = ref.allocate(np.zeros((1, 8, 2), np.float32), banks=1, capacity_rows=4)
    with pytest.raises(ValueError, match="no decode proof"):
        ref.prepare_step_capacity(unproven, 1)


def test_handoff_capacity_rules():
    assert ref.handoff_capacity(10, 2, 8, None, 4, None) == (12, 0)
    assert ref.handoff_capacity(0, 2, 8, None, 4, None) == (4, 0)
    assert ref.handoff_capacity(10, 2, 8, None, 0, None) == (16, 0)
    assert ref.handoff_capacity(10, 2, 8, 16, 0, 100) == (16, 6)
    assert ref.handoff_capacity(10, 2, 8, 12, 0, 2) == (12, 2)
    with pytest.raises(ValueError, match="smaller than the prefill"):
        ref.handoff_capacity(10, 2, 8, 9, 0, None)
    with pytest.raises(ValueError, match="cannot cover the declared"):
        ref.handoff_capacity(10, 2, 8, 11, 0, 5)


def test_from_dense_overlay_keeps_prefill_state():
    rng = np.random.default_rng(11)
    banks, slots, width = 3, 8, 4
    m0 = rng.standard_normal((1, slots, width)).astype(np.float32)
    dense = np.broadcast_to(m0, (banks, slots, width)).astype(np.float32).copy()
    active = rng.random((banks, slots)) < 0.4
    dense[active] = rng.standard_normal((int(active.sum()), width)).astype(np.float32)
    st = ref.from_dense_overlay(m0, dense, active, template_indices=np.zeros(banks, np.int64),
                                growth_quantum_rows=4)
    assert np.array_equal(ref.materialize_dense(st), dense)
    bank, slot = np.nonzero(active)
    assert list(st.logical_to_physical[bank, slot]) == list(range(int(active.sum())))


def test_exhaustion_raises_before_mutation():
    initial, steps = rc.reference_case(1)
    st = ref.allocate(initial.numpy(), banks=rc.BANKS, capacity_rows=5)
    snapshot = st.copy()
    with pytest.raises(ValueError, match="exhausted"):
        ref.packed_step(st, **_np(steps[0]))
    assert np.array_equal(st.logical_to_physical, snapshot.logical_to_physical)
    assert st.free_count == snapshot.free_count


def test_route_validation_messages():
    initial, steps = rc.reference_case(1)
    st = ref.allocate(initial.numpy(), banks=rc.BANKS, capacity_rows=48)
    bad = _np(steps[0])
    bad["write_indices"] = np.array([[2, 2], [1, 7], [4, 10]])
    with pytest.raises(ValueError, match="write one logical slot twice"):
        ref.packed_step(st, **bad)
    bad["write_indices"] = np.array([[2, 16], [1, 7], [4, 10]])
    with pytest.raises(ValueError, match="write index lies outside"):
        ref.packed_step(st, **bad)


# ---------------------------------------------------- planted mistakes


def _mutant_no_erase(current, write_weights, values, input_gate, erase_gate, forget_log_gate):
    return _ORIG_GATED(current, write_weights, values, input_gate,
                       np.zeros_like(erase_gate), forget_log_gate)


def _mutant_erase_sign(current, write_weights, values, input_gate, erase_gate, forget_log_gate):
    return _ORIG_GATED(current, write_weights, values, input_gate, -erase_gate,
                       forget_log_gate)


def _mutant_no_decay(current, write_weights, values, input_gate, erase_gate, forget_log_gate):
    return _ORIG_GATED(current, write_weights, values, input_gate, erase_gate,
                       np.zeros_like(forget_log_gate))


def _mutant_reversed_read(read_weights, visible):
    return _ORIG_READ(read_weights[:, ::-1].copy(), visible)


def _mutant_pop_from_bottom(state, write_indices):
    before, first, physical, new_rows = _ORIG_RESOLVE(state, write_indices)
    ranks = np.cumsum(first.ravel().astype(np.int64)) - 1
    bottom = state.free_rows[np.clip(ranks, 0, state.capacity_rows - 1)].reshape(first.shape)
    return before, first, np.where(first, bottom, before), new_rows


def _mutant_slot_major(state, write_indices):
    before, first, physical, new_rows = _ORIG_RESOLVE(state, write_indices)
    ranks = (np.cumsum(first.T.ravel().astype(np.int64)) - 1).reshape(first.T.shape).T
    pop = np.clip(state.free_count - 1 - ranks, 0, state.capacity_rows - 1)
    return before, first, np.where(first, state.free_rows[pop], before), new_rows


_ORIG_GATED = ref.gated_delta_rows
_ORIG_READ = ref.weighted_read
_ORIG_RESOLVE = ref.resolve_writes

MUTANTS = {
    "dropped erase term": ("gated_delta_rows", _mutant_no_erase),
    "erase sign flipped": ("gated_delta_rows", _mutant_erase_sign),
    "forget decay dropped": ("gated_delta_rows", _mutant_no_decay),
    "read weights transposed": ("weighted_read", _mutant_reversed_read),
    "pops from the stack bottom": ("resolve_writes", _mutant_pop_from_bottom),
    "slot-major pop ranks": ("resolve_writes", _mutant_slot_major),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_fails_a_pin(name, monkeypatch):
    attr, fn = MUTANTS[name]
    monkeypatch.setattr(ref, attr, fn)
    failures = 0
    for pin in ALL_PINS:
        try:
            pin()
        except AssertionError:
            failures += 1
    assert failures >= 1, f"no pin catches the planted mistake: {name}"


def test_read_before_write_is_caught(monkeypatch):
    """Planted mistake: the sparse read sees the state before this token's
    write (allocator.py:1503-1516 reads after it)."""

    def packed_read_first(state, write_indices, write_weights, values, input_gate,
                          forget_log_gate, read_indices, read_weights, *, erase_gate=None,
                          validate_routes=True):
        snapshot = ref.materialize_dense(state)
        _, diag = _ORIG_PACKED(state, write_indices, write_weights, values, input_gate,
                               forget_log_gate, read_indices, read_weights,
                               erase_gate=erase_gate, validate_routes=validate_routes)
        bank = np.arange(state.banks)[:, None]
        visible = snapshot[bank, np.asarray(read_indices).astype(np.int64)]
        return ref.weighted_read(np.asarray(read_weights, np.float32), visible), diag

    monkeypatch.setattr(ref, "packed_step", packed_read_first)
    with pytest.raises(AssertionError):
        pin_serial_recurrence()


_ORIG_PACKED = ref.packed_step


def test_torch_restatement_agrees():
    """oracle.torch_port keeps torch's reductions and float32 exp; it must
    agree with the oracle within 1e-6 relative, with identical row ids."""

    from oracle import torch_port

    rng = np.random.default_rng(12)
    banks, slots, width = 4, 32, 16
    m0, seq = _random_sequence(rng, banks, slots, width, 4, 8, 30)
    st = ref.allocate(m0, banks=banks, capacity_rows=banks * slots)
    tstate = {
        "m0": torch.from_numpy(m0), "templates": torch.zeros(banks, dtype=torch.int64),
        "values": torch.zeros(banks * slots, width), "map": torch.full((banks, slots), -1,
                                                                        dtype=torch.int32),
        "free_rows": torch.arange(banks * slots, dtype=torch.int32),
        "free_count": banks * slots,
    }
    tdense = torch.from_numpy(np.broadcast_to(m0, (banks, slots, width)).copy())
    for x in seq:
        r, _ = ref.packed_step(st, **x)
        tx = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in x.items()}
        tr, _ = torch_port.packed_step(tstate, **tx)
        td = torch_port.dense_step(tdense, **tx)
        assert torch.equal(tr, td)
        scale = 1 + np.abs(r).max()
        assert np.abs(tr.numpy() - r).max() <= 1e-6 * scale
    assert np.array_equal(tstate["map"].numpy(), st.logical_to_physical)
    assert tstate["free_count"] == st.free_count
    dense = ref.materialize_dense(st)
    assert np.abs(tdense.numpy() - dense).max() <= 1e-6 * (1 + np.abs(dense).max())
