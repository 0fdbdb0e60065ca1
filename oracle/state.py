"""numpy restatement of PackedSDMCopyOnWriteState and the sparse SDM steps.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the checker the HIP
product is compared against, never part of the product.

Each function cites the reference lines it restates
(copy_on_write_sdm/allocator.py in p0rc314in/copy-on-write-sdm).  Errors are
raised with the reference's messages.  Float math is float32 with each
product and sum rounded separately, sums taken in index order starting from
the first term, and exp(forget_log_gate) computed in float64 then rounded to
float32 once.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

F32 = np.float32


def _ceil_to(value: int, quantum: int) -> int:
    return ((value + quantum - 1) // quantum) * quantum


# --------------------------------------------------------------- row math


def decay_factor(forget_log_gate: np.ndarray) -> np.ndarray:
    """exp(forget_log_gate) per bank, float64 evaluation rounded to float32.

    The reference evaluates ``forget_log_gate.float().exp()``
    (allocator.py:1490); a correctly rounded float32 exp is the value every
    faithful float32 exp approximates.
    """

    return np.exp(forget_log_gate.astype(np.float64)).astype(F32)


def gated_delta_rows(
    current: np.ndarray,
    write_weights: np.ndarray,
    values: np.ndarray,
    input_gate: np.ndarray,
    erase_gate: np.ndarray,
    forget_log_gate: np.ndarray,
) -> np.ndarray:
    """Gated-delta update of the W written rows, allocator.py:1490-1501.

    current [B,W,D] -> updated [B,W,D]:
      decayed   = current * exp(forget)
      retrieved = sum_w weight_w * decayed_w
      delta     = input_gate * value - erase_gate * retrieved
      updated_w = decayed_w + weight_w * delta
    """

    current = current.astype(F32, copy=False)
    ww = write_weights.astype(F32, copy=False)
    alpha = decay_factor(forget_log_gate)
    decayed = current * alpha[:, None, None]
    retrieved = ww[:, 0, None] * decayed[:, 0]
    for w in range(1, ww.shape[1]):
        retrieved = retrieved + ww[:, w, None] * decayed[:, w]
    delta = (
        input_gate.astype(F32)[:, None] * values.astype(F32)
        - erase_gate.astype(F32)[:, None] * retrieved
    )
    return decayed + ww[:, :, None] * delta[:, None, :]


def weighted_read(read_weights: np.ndarray, visible: np.ndarray) -> np.ndarray:
    """reading = sum_r weight_r * visible_r, allocator.py:1516 and 1631-1633."""

    rw = read_weights.astype(F32, copy=False)
    acc = rw[:, 0, None] * visible[:, 0]
    for r in range(1, rw.shape[1]):
        acc = acc + rw[:, r, None] * visible[:, r]
    return acc


# ------------------------------------------------------------------ state


@dataclass
class OracleState:
    """Fields of PackedSDMCopyOnWriteState, allocator.py:476-504."""

    shared_initial_memory: np.ndarray  # [T,N,D] float32
    template_indices: np.ndarray  # [B] int64
    values: np.ndarray  # [C,D] float32
    logical_to_physical: np.ndarray  # [B,N] int32
    free_rows: np.ndarray  # [C] int32
    free_count: int
    overflow_flag: int = 0
    capacity_is_proven: bool = False
    proven_maximum_additional_allocations: int = 0
    growth_quantum_rows: int = 0
    growth_events: int = 0
    growth_rows_added: int = 0
    growth_rows_copied: int = 0

    # properties, allocator.py:944-958
    @property
    def banks(self) -> int:
        return self.logical_to_physical.shape[0]

    @property
    def slots(self) -> int:
        return self.logical_to_physical.shape[1]

    @property
    def width(self) -> int:
        return self.values.shape[1]

    @property
    def capacity_rows(self) -> int:
        return self.values.shape[0]

    def allocated_rows(self) -> int:
        """allocated_rows_tensor, allocator.py:960-963."""

        return self.capacity_rows - self.free_count

    def copy(self) -> "OracleState":
        return OracleState(
            shared_initial_memory=self.shared_initial_memory,
            template_indices=self.template_indices.copy(),
            values=self.values.copy(),
            logical_to_physical=self.logical_to_physical.copy(),
            free_rows=self.free_rows.copy(),
            free_count=self.free_count,
            overflow_flag=self.overflow_flag,
            capacity_is_proven=self.capacity_is_proven,
            proven_maximum_additional_allocations=self.proven_maximum_additional_allocations,
            growth_quantum_rows=self.growth_quantum_rows,
            growth_events=self.growth_events,
            growth_rows_added=self.growth_rows_added,
            growth_rows_copied=self.growth_rows_copied,
        )


def allocate(
    shared_initial_memory: np.ndarray,
    *,
    banks: int,
    capacity_rows: int,
    template_indices: np.ndarray | None = None,
    growth_quantum_rows: int = 0,
) -> OracleState:
    """PackedSDMCopyOnWriteState.allocate, allocator.py:506-585."""

    m0 = np.asarray(shared_initial_memory, dtype=F32)
    if m0.ndim == 2:
        m0 = m0[None]
    if m0.ndim != 3:
        raise ValueError("shared initial memory must be [H,N,D] or [N,D]")
    templates, slots, width = m0.shape
    if banks <= 0 or capacity_rows <= 0:
        raise ValueError("banks and physical capacity must be positive")
    if growth_quantum_rows < 0:
        raise ValueError("SDM growth quantum cannot be negative")
    if template_indices is None:
        if templates != 1:
            raise ValueError("multiple initial-memory templates require explicit mapping")
        template_indices = np.zeros(banks, dtype=np.int64)
    else:
        template_indices = np.asarray(template_indices)
        if template_indices.shape != (banks,) or template_indices.dtype.kind not in "iu":
            raise ValueError("template indices must be integer [B] on the state device")
        template_indices = template_indices.astype(np.int64)
    if int(template_indices.min()) < 0 or int(template_indices.max()) >= templates:
        raise ValueError("template index lies outside shared initial memory")
    return OracleState(
        shared_initial_memory=m0,
        template_indices=template_indices,
        values=np.zeros((capacity_rows, width), dtype=F32),
        logical_to_physical=np.full((banks, slots), -1, dtype=np.int32),
        free_rows=np.arange(capacity_rows, dtype=np.int32),
        free_count=capacity_rows,
        growth_quantum_rows=growth_quantum_rows,
    )


def handoff_capacity(
    active_count: int,
    banks: int,
    slots: int,
    capacity_rows: int | None,
    growth_quantum_rows: int,
    maximum_future_allocations: int | None,
) -> tuple[int, int]:
    """Capacity rules of from_dense_overlay, allocator.py:629-655.

    Returns (selected_capacity, possible_future_allocations).
    """

    if growth_quantum_rows < 0:
        raise ValueError("SDM growth quantum cannot be negative")
    if capacity_rows is None and growth_quantum_rows:
        selected = max(growth_quantum_rows, _ceil_to(active_count, growth_quantum_rows))
    else:
        selected = banks * slots if capacity_rows is None else capacity_rows
    if selected < active_count:
        raise ValueError("SDM physical capacity is smaller than the prefill working set")
    if maximum_future_allocations is not None:
        if maximum_future_allocations < 0:
            raise ValueError("maximum future allocations cannot be negative")
        possible = min(maximum_future_allocations, banks * slots - active_count)
        if selected - active_count < possible:
            raise ValueError("SDM physical capacity cannot cover the declared decode trace")
    else:
        possible = 0
    return selected, possible


def from_dense_overlay(
    shared_initial_memory: np.ndarray,
    dense_memory: np.ndarray,
    active_slots: np.ndarray,
    *,
    template_indices: np.ndarray,
    capacity_rows: int | None = None,
    maximum_future_allocations: int | None = None,
    growth_quantum_rows: int = 0,
) -> OracleState:
    """Prefill handoff, allocator.py:587-689: active (bank, slot) pairs in
    row-major order get physical rows 0..A-1."""

    m0 = np.asarray(shared_initial_memory, dtype=F32)
    if m0.ndim == 2:
        m0 = m0[None]
    if m0.ndim != 3 or dense_memory.ndim != 3:
        raise ValueError("SDM handoff memory must be [H,N,D] and [B,N,D]")
    banks, slots, width = dense_memory.shape
    if active_slots.shape != (banks, slots) or active_slots.dtype != np.bool_ or (
        m0.shape[1:] != (slots, width)
    ):
        raise ValueError("SDM handoff state and active-slot mask do not align")
    if np.asarray(template_indices).shape != (banks,):
        raise ValueError("SDM handoff template indices must be [B] on device")
    active_count = int(active_slots.sum())
    selected, possible = handoff_capacity(
        active_count, banks, slots, capacity_rows, growth_quantum_rows,
        maximum_future_allocations,
    )
    state = allocate(
        m0,
        banks=banks,
        capacity_rows=selected,
        template_indices=template_indices,
        growth_quantum_rows=growth_quantum_rows,
    )
    if active_count:
        bank, slot = np.nonzero(active_slots)
        state.logical_to_physical[bank, slot] = np.arange(active_count, dtype=np.int32)
        state.values[:active_count] = dense_memory[bank, slot].astype(F32)
    free = selected - active_count
    state.free_rows[:free] = np.arange(active_count, selected, dtype=np.int32)
    state.free_count = free
    state.capacity_is_proven = maximum_future_allocations is not None
    state.proven_maximum_additional_allocations = possible
    validate_invariants(state)
    return state


def grow_capacity(state: OracleState, minimum_capacity_rows: int) -> int:
    """allocator.py:691-743: new ids join the top of the free stack; every
    old row is counted as copied."""

    if minimum_capacity_rows <= state.capacity_rows:
        return 0
    quantum = state.growth_quantum_rows
    if quantum <= 0:
        raise ValueError("SDM COW slab growth is disabled")
    selected = _ceil_to(minimum_capacity_rows, quantum)
    old = state.capacity_rows
    added = selected - old
    free = state.free_count
    values = np.zeros((selected, state.width), dtype=F32)
    values[:old] = state.values
    free_rows = np.zeros(selected, dtype=np.int32)
    free_rows[:free] = state.free_rows[:free]
    free_rows[free : free + added] = np.arange(old, selected, dtype=np.int32)
    state.values = values
    state.free_rows = free_rows
    state.free_count = free + added
    state.proven_maximum_additional_allocations += added
    state.overflow_flag = 0
    state.growth_events += 1
    state.growth_rows_added += added
    state.growth_rows_copied += old
    return added


def prepare_step_capacity(state: OracleState, maximum_new_rows: int) -> int:
    """Host capacity proof, allocator.py:745-773."""

    if maximum_new_rows < 0:
        raise ValueError("maximum new SDM rows cannot be negative")
    if state.growth_quantum_rows <= 0:
        if not state.capacity_is_proven:
            raise ValueError("SDM COW capacity has no decode proof")
        return 0
    if state.proven_maximum_additional_allocations < maximum_new_rows:
        free = state.free_count
        if free < maximum_new_rows:
            grow_capacity(state, state.capacity_rows + maximum_new_rows - free)
            free = state.free_count
        state.proven_maximum_additional_allocations = free
    state.proven_maximum_additional_allocations -= maximum_new_rows
    state.capacity_is_proven = True
    return state.capacity_rows


def trim_target(active_count: int, headroom_rows: int, quantum: int) -> int:
    """New capacity of trim_capacity, allocator.py:792-795."""

    return max(quantum, _ceil_to(active_count + headroom_rows, quantum))


def trim_capacity(state: OracleState, *, headroom_rows: int = 0) -> int:
    """allocator.py:775-839: repack live rows to 0..A-1 in row-major order."""

    if headroom_rows < 0:
        raise ValueError("SDM trim headroom cannot be negative")
    quantum = state.growth_quantum_rows
    if quantum <= 0:
        raise ValueError("SDM COW slab trimming requires copy-on-write capacity")
    active = state.logical_to_physical >= 0
    active_count = int(active.sum())
    selected = trim_target(active_count, headroom_rows, quantum)
    if selected >= state.capacity_rows:
        return 0
    values = np.zeros((selected, state.width), dtype=F32)
    mapping = np.full_like(state.logical_to_physical, -1)
    if active_count:
        bank, slot = np.nonzero(active)
        source = state.logical_to_physical[bank, slot].astype(np.int64)
        values[:active_count] = state.values[source]
        mapping[bank, slot] = np.arange(active_count, dtype=np.int32)
    free = selected - active_count
    free_rows = np.zeros(selected, dtype=np.int32)
    free_rows[:free] = np.arange(active_count, selected, dtype=np.int32)
    removed = state.capacity_rows - selected
    state.values = values
    state.logical_to_physical = mapping
    state.free_rows = free_rows
    state.free_count = free
    state.capacity_is_proven = False
    state.proven_maximum_additional_allocations = free
    state.overflow_flag = 0
    return removed


def append_banks_from(state: OracleState, other: OracleState) -> int:
    """allocator.py:841-914: pop destinations from the top of the free stack
    in the other map's row-major live order."""

    if (
        other.slots != state.slots
        or other.width != state.width
        or other.shared_initial_memory.shape != state.shared_initial_memory.shape
    ):
        raise ValueError("admitted SDM banks do not match the destination pool")
    if other.shared_initial_memory is not state.shared_initial_memory and not np.array_equal(
        other.shared_initial_memory, state.shared_initial_memory
    ):
        raise ValueError("admitted SDM banks use different learned initial memory")
    active = other.logical_to_physical >= 0
    active_count = int(active.sum())
    free = state.free_count
    if free < active_count:
        grow_capacity(state, state.capacity_rows + active_count - free)
        free = state.free_count
    admitted = np.full((other.banks, state.slots), -1, dtype=np.int32)
    if active_count:
        bank, slot = np.nonzero(active)
        positions = np.arange(free - 1, free - active_count - 1, -1)
        destination = state.free_rows[positions]
        source = other.logical_to_physical[bank, slot].astype(np.int64)
        state.values[destination.astype(np.int64)] = other.values[source]
        admitted[bank, slot] = destination
        state.free_count = free - active_count
    state.logical_to_physical = np.concatenate((state.logical_to_physical, admitted), axis=0)
    state.template_indices = np.concatenate((state.template_indices, other.template_indices))
    if state.growth_quantum_rows:
        state.proven_maximum_additional_allocations = min(
            state.proven_maximum_additional_allocations, state.free_count
        )
    else:
        state.capacity_is_proven = False
        state.proven_maximum_additional_allocations = 0
    return active_count


def retain_banks(state: OracleState, bank_indices: np.ndarray) -> None:
    """allocator.py:916-942: gather map rows; values never move."""

    indices = np.asarray(bank_indices).astype(np.int64)
    if indices.ndim != 1:
        raise ValueError("retained bank indices must be integer [S] on device")
    if indices.size and (
        (indices < 0).any()
        or (indices >= state.banks).any()
        or np.unique(indices).size != indices.size
    ):
        raise ValueError("retained bank index is invalid or duplicated")
    selected = np.zeros(state.banks, dtype=bool)
    selected[indices] = True
    if (state.logical_to_physical[~selected] >= 0).any():
        raise ValueError("discarded SDM banks must be released before compaction")
    state.logical_to_physical = state.logical_to_physical[indices].copy()
    state.template_indices = state.template_indices[indices].copy()


def release(state: OracleState, bank_indices: np.ndarray) -> int:
    """allocator.py:1018-1067: push live rows in (listed bank, slot) order."""

    indices = np.asarray(bank_indices).astype(np.int64)
    if indices.ndim != 1:
        raise ValueError("released bank indices must be integer [S] on device")
    if indices.size == 0:
        return 0
    if (
        (indices < 0).any()
        or (indices >= state.banks).any()
        or np.unique(indices).size != indices.size
    ):
        raise ValueError("released bank index is invalid or duplicated")
    selected = state.logical_to_physical[indices]
    flat_active = (selected >= 0).ravel()
    flat_rows = selected.ravel()
    ranks = np.cumsum(flat_active.astype(np.int64)) - 1
    released = int(flat_active.sum())
    push = np.clip(state.free_count + ranks, 0, state.capacity_rows - 1)
    state.free_rows[push[flat_active]] = flat_rows[flat_active]
    state.free_count += released
    state.logical_to_physical[indices] = -1
    return released


def materialize_dense(state: OracleState) -> np.ndarray:
    """allocator.py:1003-1016."""

    dense = state.shared_initial_memory[state.template_indices].astype(F32).copy()
    bank, slot = np.nonzero(state.logical_to_physical >= 0)
    dense[bank, slot] = state.values[state.logical_to_physical[bank, slot].astype(np.int64)]
    return dense


def validate_invariants(state: OracleState) -> dict:
    """allocator.py:1069-1095."""

    if state.overflow_flag != 0:
        raise AssertionError("SDM COW allocator recorded a slab overflow")
    mapping = state.logical_to_physical
    active = mapping[mapping >= 0].astype(np.int64)
    free = state.free_rows[: max(0, min(state.free_count, state.capacity_rows))].astype(np.int64)
    if active.size != np.unique(active).size:
        raise AssertionError("one physical SDM row has multiple logical owners")
    if free.size != np.unique(free).size:
        raise AssertionError("free SDM row stack contains duplicates")
    if active.size + free.size != state.capacity_rows:
        raise AssertionError("active and free SDM rows do not cover capacity")
    combined = np.sort(np.concatenate((active, free)))
    if not np.array_equal(combined, np.arange(state.capacity_rows)):
        raise AssertionError("active and free SDM rows do not partition the slab")
    return {
        "capacity_rows": state.capacity_rows,
        "allocated_rows": int(active.size),
        "free_rows": int(free.size),
        "exact_partition": True,
    }


# ------------------------------------------------------------------ steps


def _validate_routes(write_indices, read_indices, slots, validate_routes):
    if validate_routes:
        if ((write_indices < 0) | (write_indices >= slots)).any():
            raise ValueError("write index lies outside the logical table")
        if ((read_indices < 0) | (read_indices >= slots)).any():
            raise ValueError("read index lies outside the logical table")
        if write_indices.shape[1] > 1:
            ordered = np.sort(write_indices, axis=-1)
            if not (ordered[:, 1:] != ordered[:, :-1]).all():
                raise ValueError("one SDM step cannot write one logical slot twice")


@dataclass
class StepDiagnostics:
    """SDMCopyOnWriteStep fields, allocator.py:467-473."""

    first_touches_by_sequence: np.ndarray
    repeated_writes_by_sequence: np.ndarray
    allocated_rows_after_step: int


def resolve_writes(state: OracleState, write_indices: np.ndarray):
    """First-touch resolution with bank-major pops, allocator.py:1466-1481.

    Returns (physical_before, first_touch, physical, new_rows)."""

    bank = np.arange(state.banks)[:, None]
    before = state.logical_to_physical[bank, write_indices]
    first = before < 0
    flat_first = first.ravel()
    ranks = np.cumsum(flat_first.astype(np.int64)) - 1
    new_rows = int(flat_first.sum())
    if state.free_count < new_rows:
        raise ValueError("SDM COW physical slab is exhausted")
    pop = np.clip(state.free_count - 1 - ranks, 0, state.capacity_rows - 1)
    allocated = state.free_rows[pop].reshape(before.shape)
    physical = np.where(first, allocated, before)
    return before, first, physical, new_rows


def packed_step(
    state: OracleState,
    write_indices,
    write_weights,
    values,
    input_gate,
    forget_log_gate,
    read_indices,
    read_weights,
    *,
    erase_gate=None,
    validate_routes: bool = True,
) -> tuple[np.ndarray, StepDiagnostics]:
    """packed_sdm_cow_step, torch semantics of allocator.py:1466-1525."""

    wi = np.asarray(write_indices).astype(np.int64)
    ri = np.asarray(read_indices).astype(np.int64)
    _validate_routes(wi, ri, state.slots, validate_routes)
    ig = np.asarray(input_gate, dtype=F32)
    eg = ig if erase_gate is None else np.asarray(erase_gate, dtype=F32)
    before, first, physical, new_rows = resolve_writes(state, wi)
    bank = np.arange(state.banks)[:, None]
    tmpl = state.template_indices[:, None]
    base = state.shared_initial_memory[tmpl, wi]
    private = state.values[np.maximum(before, 0)]
    current = np.where(first[..., None], base, private)
    updated = gated_delta_rows(
        current, np.asarray(write_weights, dtype=F32), np.asarray(values, dtype=F32),
        ig, eg, np.asarray(forget_log_gate, dtype=F32),
    )
    state.logical_to_physical[bank, wi] = physical
    state.values[physical.astype(np.int64)] = updated
    state.free_count -= new_rows
    read_physical = state.logical_to_physical[bank, ri]
    visible = np.where(
        (read_physical >= 0)[..., None],
        state.values[np.maximum(read_physical, 0)],
        state.shared_initial_memory[tmpl, ri],
    )
    reading = weighted_read(np.asarray(read_weights, dtype=F32), visible)
    first_by_sequence = first.sum(axis=-1).astype(np.int64)
    return reading, StepDiagnostics(
        first_touches_by_sequence=first_by_sequence,
        repeated_writes_by_sequence=wi.shape[1] - first_by_sequence,
        allocated_rows_after_step=state.allocated_rows(),
    )


def dense_step(
    memory: np.ndarray,
    write_indices,
    write_weights,
    values,
    input_gate,
    forget_log_gate,
    read_indices,
    read_weights,
    *,
    erase_gate=None,
    validate_routes: bool = True,
) -> np.ndarray:
    """dense_sdm_sparse_step, torch semantics of allocator.py:1612-1633.
    Mutates ``memory`` [B,N,D] float32 in place."""

    wi = np.asarray(write_indices).astype(np.int64)
    ri = np.asarray(read_indices).astype(np.int64)
    _validate_routes(wi, ri, memory.shape[1], validate_routes)
    ig = np.asarray(input_gate, dtype=F32)
    eg = ig if erase_gate is None else np.asarray(erase_gate, dtype=F32)
    bank = np.arange(memory.shape[0])[:, None]
    current = memory[bank, wi]
    memory[bank, wi] = gated_delta_rows(
        current, np.asarray(write_weights, dtype=F32), np.asarray(values, dtype=F32),
        ig, eg, np.asarray(forget_log_gate, dtype=F32),
    )
    return weighted_read(np.asarray(read_weights, dtype=F32), memory[bank, ri])
