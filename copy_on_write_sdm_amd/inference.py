"""Serving lifecycle over packed copy-on-write SDM layers.

Mirrors the SDM half of copy_on_write_sdm/inference.py: the decode-state
container with release / compact / admit / trim (inference.py:26-276), the
prefill handoff that packs the union of prefix-written rows
(inference.py:314-366) and the per-layer decode step with its capacity proof
(inference.py:538-598).  The reference's controller (LayerNorm, projections,
product-key routing) and its attention layers are not part of this package:
callers hand in the routes, values and gates the controller would produce.
Dense K/V caches, when given, are carried and compacted like the reference
does, with plain tensor indexing.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from .allocator import (
    PackedSDMCopyOnWriteState,
    dense_sdm_sparse_step,
    mark_written,
    packed_sdm_cow_step,
)


def _tensor_bytes(tensor: torch.Tensor) -> int:
    return tensor.numel() * tensor.element_size()


@dataclass
class SDMStepInputs:
    """One decode token's controller outputs for one SDM layer
    (the fields of inference.py:279-290 that reach the state step)."""

    write_indices: torch.Tensor   # [B*H, W]
    write_weights: torch.Tensor   # [B*H, W]
    values: torch.Tensor          # [B*H, D]
    input_gate: torch.Tensor      # [B*H]
    forget_log_gate: torch.Tensor # [B*H]
    read_indices: torch.Tensor    # [B*H, R]
    read_weights: torch.Tensor    # [B*H, R]
    erase_gate: torch.Tensor | None = None


@dataclass
class FaithfulSDMDecodeState:
    """Retained state for one batch of independent SDM requests
    (inference.py:26-276).  Bank ``seq * H + h`` holds request ``seq``'s
    memory head ``h`` in every layer."""

    layout: str
    position: int
    capacity: int
    activation_dtype: torch.dtype
    active_sequences: torch.Tensor
    sdm_layer_positions: tuple[int, ...]
    sdm_states: tuple[PackedSDMCopyOnWriteState, ...]
    dense_keys: tuple[torch.Tensor, ...] = ()
    dense_values: tuple[torch.Tensor, ...] = ()
    positions: torch.Tensor | None = None

    @property
    def batch(self) -> int:
        return self.active_sequences.numel()

    @property
    def device(self) -> torch.device:
        return self.active_sequences.device

    @property
    def dtype(self) -> torch.dtype:
        return self.activation_dtype

    def current_positions(self) -> torch.Tensor:
        """One decode position per live request (inference.py:59-69)."""

        if self.positions is None:
            return torch.full((self.batch,), self.position, device=self.device,
                              dtype=torch.int64)
        return self.positions

    def _banks(self, sequences: torch.Tensor, heads: int) -> torch.Tensor:
        return (sequences[:, None] * heads
                + torch.arange(heads, device=self.device)[None, :]).flatten()

    @torch.no_grad()
    def release(self, sequence_indices: torch.Tensor | Sequence[int] | None = None) -> int:
        """Release completed requests from every SDM layer; their rows return
        to each layer's shared slab (inference.py:71-114)."""

        if sequence_indices is None:
            selected = self.active_sequences.nonzero().flatten()
        else:
            selected = torch.as_tensor(sequence_indices, device=self.device,
                                       dtype=torch.int64)
        if selected.ndim != 1:
            raise ValueError("released sequence indices must be a vector")
        if selected.numel() == 0:
            return 0
        ordered = selected.sort().values
        if (
            bool((selected < 0).any())
            or bool((selected >= self.batch).any())
            or (ordered.numel() > 1 and bool((ordered[1:] == ordered[:-1]).any()))
            or not bool(self.active_sequences[selected].all())
        ):
            raise ValueError("released sequence is invalid, duplicated, or inactive")
        released = 0
        for state in self.sdm_states:
            if state.banks % self.batch:
                raise AssertionError("SDM serving banks do not divide by batch")
            heads = state.banks // self.batch
            released += int(state.release(self._banks(selected, heads)))
        self.active_sequences[selected] = False
        return released

    @torch.no_grad()
    def compact(self) -> torch.Tensor:
        """Drop released request slots; live rows never move
        (inference.py:116-159).  Returns the retained former indices."""

        previous_batch = self.batch
        retained = self.active_sequences.nonzero().flatten()
        positions = self.current_positions()
        for state in self.sdm_states:
            if previous_batch == 0:
                if state.banks != 0:
                    raise AssertionError("empty serving batch retained SDM banks")
                continue
            if state.banks % previous_batch:
                raise AssertionError("SDM serving banks do not divide by batch")
            heads = state.banks // previous_batch
            state.retain_banks(self._banks(retained, heads))
        self.dense_keys = tuple(row[retained].contiguous() for row in self.dense_keys)
        self.dense_values = tuple(row[retained].contiguous() for row in self.dense_values)
        retained_positions = positions[retained].contiguous()
        self.positions = retained_positions if self.positions is not None else None
        self.active_sequences = torch.ones(retained.numel(), device=self.device,
                                           dtype=torch.bool)
        self.position = int(retained_positions.max().item()) if retained.numel() else 0
        return retained

    @torch.no_grad()
    def admit(self, incoming: "FaithfulSDMDecodeState") -> int:
        """Admit a prefilled cohort into the same pooled slabs
        (inference.py:161-206)."""

        self.compact()
        incoming.compact()
        if (
            self.layout != incoming.layout
            or self.capacity != incoming.capacity
            or self.activation_dtype != incoming.activation_dtype
            or self.device != incoming.device
            or self.sdm_layer_positions != incoming.sdm_layer_positions
            or len(self.sdm_states) != len(incoming.sdm_states)
            or len(self.dense_keys) != len(incoming.dense_keys)
        ):
            raise ValueError("admitted faithful-SDM state is incompatible")
        admitted = incoming.batch
        for destination, source in zip(self.sdm_states, incoming.sdm_states):
            destination.append_banks_from(source)
        self.dense_keys = tuple(torch.cat((a, b), dim=0).contiguous()
                                for a, b in zip(self.dense_keys, incoming.dense_keys))
        self.dense_values = tuple(torch.cat((a, b), dim=0).contiguous()
                                  for a, b in zip(self.dense_values, incoming.dense_values))
        admitted_positions = torch.cat(
            (self.current_positions(), incoming.current_positions()), dim=0).contiguous()
        if admitted_positions.numel() and bool(
                (admitted_positions == admitted_positions[0]).all()):
            self.position = int(admitted_positions[0].item())
            self.positions = None
        else:
            self.positions = admitted_positions
        self.active_sequences = torch.ones(admitted_positions.numel(), device=self.device,
                                           dtype=torch.bool)
        if admitted_positions.numel() and self.positions is not None:
            self.position = int(admitted_positions.max().item())
        return admitted

    @torch.no_grad()
    def trim_sdm_pools(self, *, headroom_rows: int = 0) -> int:
        """Return unused slab rows after a lifecycle transition
        (inference.py:208-215)."""

        return sum(state.trim_capacity(headroom_rows=headroom_rows)
                   for state in self.sdm_states)

    @torch.no_grad()
    def release_and_compact(
        self,
        sequence_indices: torch.Tensor | Sequence[int] | None = None,
        *,
        trim: bool = False,
        trim_headroom_rows: int = 0,
    ) -> int:
        """Release, compact survivors and optionally trim (inference.py:217-231)."""

        released = self.release(sequence_indices)
        self.compact()
        if trim:
            self.trim_sdm_pools(headroom_rows=trim_headroom_rows)
        return released

    def storage_bytes(self) -> dict[str, int]:
        """Private live/reserved SDM state, shared M0 and dense K/V
        (inference.py:233-276)."""

        private_live_values = private_metadata = private_reserved = 0
        shared_initial = logical_dense = 0
        for state in self.sdm_states:
            used = state.used_bytes()
            stored = state.storage_bytes()
            private_live_values += used["live_value_bytes"]
            private_metadata += used["allocator_metadata_bytes"]
            private_reserved += stored["private_allocator_reserved_total"]
            shared_initial += stored["shared_initial_memory"]
            logical_dense += state.banks * state.slots * state.width * 4
        dense_allocated = sum(_tensor_bytes(t) for t in (*self.dense_keys, *self.dense_values))
        dense_live = sum(t[:, :, : self.position].numel() * t.element_size()
                         for t in (*self.dense_keys, *self.dense_values))
        lifecycle = _tensor_bytes(self.active_sequences) + (
            0 if self.positions is None else _tensor_bytes(self.positions))
        return {
            "sdm_private_value_live": private_live_values,
            "sdm_private_allocator_metadata": private_metadata,
            "sdm_private_live_total": private_live_values + private_metadata,
            "sdm_private_reserved_total": private_reserved,
            "sdm_logical_dense_fp32": logical_dense,
            "sdm_shared_initial_memory": shared_initial,
            "dense_kv_live": dense_live,
            "dense_kv_allocated": dense_allocated,
            "lifecycle": lifecycle,
            "per_user_live_total_excluding_shared": (
                private_live_values + private_metadata + dense_live + lifecycle),
            "total_reserved_excluding_shared": (
                private_reserved + dense_allocated + lifecycle),
        }


@torch.no_grad()
def pack_prefill_layer(
    initial_memory: torch.Tensor,
    final_memory: torch.Tensor,
    write_indices: torch.Tensor,
    *,
    capacity_rows: int | None,
    decode_capacity: int,
    growth_quantum_rows: int,
) -> PackedSDMCopyOnWriteState:
    """Prefill handoff of one SDM layer (inference.py:314-366).

    ``initial_memory`` [H,N,D] is the layer's M0, ``final_memory`` [B,H,N,D]
    the dense terminal prefill state and ``write_indices`` [B,T,H,W] the
    prefix's hard write routes.  The union of written slots per bank becomes
    private rows; everything else stays shared with M0.
    """

    batch, time, heads, writes = write_indices.shape
    if initial_memory.ndim != 3 or final_memory.shape != (
            batch, heads, initial_memory.shape[1], initial_memory.shape[2]):
        raise ValueError("SDM prefill routing does not match its controller")
    slots = initial_memory.shape[1]
    active = torch.zeros(batch * heads, slots, device=write_indices.device, dtype=torch.bool)
    mark_written(active, write_indices.permute(0, 2, 1, 3).reshape(batch * heads,
                                                                   time * writes))
    templates = torch.arange(heads, device=active.device, dtype=torch.int64).repeat(batch)
    return PackedSDMCopyOnWriteState.from_dense_overlay(
        initial_memory,
        final_memory.flatten(0, 1),
        active,
        template_indices=templates,
        capacity_rows=capacity_rows,
        state_dtype=torch.float32,
        maximum_future_allocations=(
            None if growth_quantum_rows else batch * heads * writes * (decode_capacity - time)),
        growth_quantum_rows=growth_quantum_rows,
    )


@torch.no_grad()
def decode_sdm_layer(state: PackedSDMCopyOnWriteState, step: SDMStepInputs, *,
                     backend: str = "auto") -> torch.Tensor:
    """Packed decode of one SDM layer for one token (inference.py:538-566):
    capacity proof when slab growth is enabled, then the fused step without
    route validation or diagnostics."""

    if state.growth_quantum_rows:
        state.prepare_step_capacity(state.banks * step.write_indices.shape[1])
    reading, _ = packed_sdm_cow_step(
        state, step.write_indices, step.write_weights, step.values, step.input_gate,
        step.forget_log_gate, step.read_indices, step.read_weights,
        erase_gate=step.erase_gate, backend=backend, validate_routes=False,
        collect_diagnostics=False)
    return reading


@torch.no_grad()
def decode_sdm_layer_dense(memory: torch.Tensor, step: SDMStepInputs, *,
                           backend: str = "auto") -> torch.Tensor:
    """Dense-table control decode of one SDM layer (inference.py:569-598)."""

    return dense_sdm_sparse_step(
        memory, step.write_indices, step.write_weights, step.values, step.input_gate,
        step.forget_log_gate, step.read_indices, step.read_weights,
        erase_gate=step.erase_gate, backend=backend, validate_routes=False)
