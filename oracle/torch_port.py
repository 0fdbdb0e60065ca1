"""torch CPU restatement of the reference's torch branches.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Used (1) as a second
restatement to cross-check ``oracle.state`` -- it keeps the reference's torch
reductions (``sum(dim=1)``) and float32 ``exp`` -- and (2) as the CPU
dense-table baseline that bench.py times on the host cores
(the "reference's PyTorch dense-table CPU path" of the benchmark plan).

* ``dense_step``  follows copy_on_write_sdm/allocator.py:1612-1633.
* ``packed_step`` follows allocator.py:1466-1525 on a dict-of-tensors state
  with the fields of allocator.py:492-498.
"""

from __future__ import annotations

import torch


@torch.no_grad()
def _update_rows(current, write_weights, values, input_gate, erase_gate, forget_log_gate):
    banks = current.shape[0]
    decay = forget_log_gate.float().reshape(banks, 1, 1).exp()
    decayed = current * decay
    weight = write_weights.float().unsqueeze(-1)
    retrieved = (weight * decayed).sum(dim=1)
    gate = input_gate.float().reshape(banks, 1)
    erase = gate if erase_gate is None else erase_gate.float().reshape(banks, 1)
    delta = gate * values.float() - erase * retrieved
    return decayed + weight * delta.unsqueeze(1)


@torch.no_grad()
def dense_step(memory, write_indices, write_weights, values, input_gate, forget_log_gate,
               read_indices, read_weights, *, erase_gate=None):
    """allocator.py:1612-1633; mutates ``memory`` [B,N,D]."""

    banks = memory.shape[0]
    rows = torch.arange(banks, dtype=torch.int64).unsqueeze(1)
    writes = write_indices.to(torch.int64)
    current = memory[rows, writes].float()
    memory[rows, writes] = _update_rows(
        current, write_weights, values, input_gate, erase_gate, forget_log_gate
    ).to(memory.dtype)
    reads = read_indices.to(torch.int64)
    visible = memory[rows, reads].float()
    return (read_weights.float().unsqueeze(-1) * visible).sum(dim=1).to(values.dtype)


@torch.no_grad()
def packed_step(state, write_indices, write_weights, values, input_gate, forget_log_gate,
                read_indices, read_weights, *, erase_gate=None):
    """allocator.py:1466-1525 on ``state`` = dict with keys m0 [T,N,D],
    templates [B] int64, values [C,D], map [B,N] int32, free_rows [C] int32,
    free_count (python int).  Returns (reading, first_by_sequence)."""

    m0, templates = state["m0"], state["templates"]
    slab, mapping, free_rows = state["values"], state["map"], state["free_rows"]
    banks = mapping.shape[0]
    rows = torch.arange(banks, dtype=torch.int64).unsqueeze(1)
    writes = write_indices.to(torch.int64)
    before = mapping.gather(1, writes)
    first = before < 0
    flat = first.flatten()
    ranks = flat.to(torch.int32).cumsum(0) - 1
    new_rows = int(flat.sum())
    old_free = state["free_count"]
    if old_free < new_rows:
        raise ValueError("SDM COW physical slab is exhausted")
    pop = (old_free - 1 - ranks).clamp(0, slab.shape[0] - 1)
    allocated = free_rows[pop.to(torch.int64)].reshape_as(before)
    physical = torch.where(first, allocated, before)
    base = m0[templates[:, None], writes].float()
    private = slab[before.clamp_min(0).to(torch.int64)].float()
    current = torch.where(first.unsqueeze(-1), base, private)
    updated = _update_rows(current, write_weights, values, input_gate, erase_gate, forget_log_gate)
    mapping[rows, writes] = physical
    slab[physical.to(torch.int64)] = updated.to(slab.dtype)
    state["free_count"] = old_free - new_rows
    reads = read_indices.to(torch.int64)
    read_physical = mapping.gather(1, reads)
    visible = torch.where(
        (read_physical >= 0).unsqueeze(-1),
        slab[read_physical.clamp_min(0).to(torch.int64)].float(),
        m0[templates[:, None], reads].float(),
    )
    reading = (read_weights.float().unsqueeze(-1) * visible).sum(dim=1)
    return reading.to(values.dtype), first.sum(dim=-1)
