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

    # Requests are named by their index in the batch; request r owns bank
    # r * H + h of a layer with H memory heads.  Index lists are handled on
    # the host (one read of the activity mask per call) and sent to the
    # device once per layer as the bank list its state operation takes.

    def _position_list(self) -> list[int]:
        """Every live request's decode position, on the host."""

        if self.positions is None:
            return [self.position] * self.batch
        return [int(p) for p in self.positions.tolist()]

    def _heads(self, state: PackedSDMCopyOnWriteState, batch: int) -> int:
        heads, rest = divmod(state.banks, batch)
        if rest:
            raise AssertionError("SDM serving banks do not divide by batch")
        return heads

    def _bank_list(self, requests: list[int], heads: int) -> torch.Tensor:
        banks = [request * heads + head for request in requests for head in range(heads)]
        return torch.tensor(banks, device=self.device, dtype=torch.int64)

    def _requests_to_release(self, sequence_indices) -> list[int]:
        """The requests a release names, in the order given, after checking
        that they are distinct live requests of this batch."""

        live = self.active_sequences.tolist()
        if sequence_indices is None:
            return [r for r, on in enumerate(live) if on]
        if isinstance(sequence_indices, torch.Tensor):
            named = sequence_indices.detach().to("cpu", torch.int64)
        else:
            named = torch.as_tensor(sequence_indices, dtype=torch.int64)
        if named.ndim != 1:
            raise ValueError("released sequence indices must be a vector")
        requests = named.tolist()
        if (len(set(requests)) != len(requests)
                or any(not 0 <= r < len(live) or not live[r] for r in requests)):
            raise ValueError("released sequence is invalid, duplicated, or inactive")
        return requests

    @torch.no_grad()
    def release(self, sequence_indices: torch.Tensor | Sequence[int] | None = None) -> int:
        """Return the rows of finished requests to every SDM layer's shared
        slab (inference.py:71-114): all live requests when none are named.
        Their batch slots stay until ``compact``.  Returns the rows freed."""

        requests = self._requests_to_release(sequence_indices)
        if not requests:
            return 0
        freed = 0
        for state in self.sdm_states:
            banks = self._bank_list(requests, self._heads(state, self.batch))
            freed += int(state.release(banks))
        mask = torch.ones(self.batch, dtype=torch.bool)
        mask[requests] = False
        self.active_sequences &= mask.to(self.device)
        return freed

    @torch.no_grad()
    def compact(self) -> torch.Tensor:
        """Close the batch slots of released requests (inference.py:116-159):
        survivors keep their order, their rows stay where they are in the
        slabs, and each layer's map and template rows (and dense K/V batch
        rows) are renumbered.  Returns the survivors' former indices."""

        live = self.active_sequences.tolist()
        kept = [r for r, on in enumerate(live) if on]
        for state in self.sdm_states:
            if not live:
                if state.banks:
                    raise AssertionError("empty serving batch retained SDM banks")
                continue
            state.retain_banks(self._bank_list(kept, self._heads(state, len(live))))
        index = torch.tensor(kept, device=self.device, dtype=torch.int64)
        self.dense_keys = tuple(t.index_select(0, index).contiguous() for t in self.dense_keys)
        self.dense_values = tuple(t.index_select(0, index).contiguous()
                                  for t in self.dense_values)
        if self.positions is None:
            # one shared position: it stays, unless no request survives
            self.position = self.position if kept else 0
        else:
            survivors = self.positions.index_select(0, index).contiguous()
            self.positions = survivors
            self.position = int(survivors.max()) if kept else 0
        self.active_sequences = torch.ones(len(kept), device=self.device, dtype=torch.bool)
        return index

    @torch.no_grad()
    def admit(self, incoming: "FaithfulSDMDecodeState") -> int:
        """Append a prefilled cohort to this batch (inference.py:161-206):
        both batches are compacted, every SDM layer takes the cohort's banks
        into its pooled slab, and the decode positions are merged (one shared
        position when they agree).  Returns the requests admitted."""

        self.compact()
        incoming.compact()
        same = (self.layout == incoming.layout and self.capacity == incoming.capacity
                and self.activation_dtype == incoming.activation_dtype
                and self.device == incoming.device
                and self.sdm_layer_positions == incoming.sdm_layer_positions
                and len(self.sdm_states) == len(incoming.sdm_states)
                and len(self.dense_keys) == len(incoming.dense_keys))
        if not same:
            raise ValueError("admitted faithful-SDM state is incompatible")
        for mine, theirs in zip(self.sdm_states, incoming.sdm_states):
            mine.append_banks_from(theirs)
        self.dense_keys = tuple(torch.cat((a, b)).contiguous()
                                for a, b in zip(self.dense_keys, incoming.dense_keys))
        self.dense_values = tuple(torch.cat((a, b)).contiguous()
                                  for a, b in zip(self.dense_values, incoming.dense_values))
        merged = self._position_list() + incoming._position_list()
        if merged and min(merged) == max(merged):
            self.position, self.positions = merged[0], None
        else:
            self.positions = torch.tensor(merged, device=self.device, dtype=torch.int64)
            if merged:
                self.position = max(merged)
        self.active_sequences = torch.ones(len(merged), device=self.device, dtype=torch.bool)
        return incoming.batch

    @torch.no_grad()
    def trim_sdm_pools(self, *, headroom_rows: int = 0) -> int:
        """Shrink every SDM layer's slab to its live rows plus headroom after
        a lifecycle transition (inference.py:208-215).  Returns the rows
        removed."""

        removed = 0
        for state in self.sdm_states:
            removed += state.trim_capacity(headroom_rows=headroom_rows)
        return removed

    @torch.no_grad()
    def release_and_compact(
        self,
        sequence_indices: torch.Tensor | Sequence[int] | None = None,
        *,
        trim: bool = False,
        trim_headroom_rows: int = 0,
    ) -> int:
        """``release``, ``compact`` and, with ``trim``, ``trim_sdm_pools``
        (inference.py:217-231).  Returns the rows released."""

        freed = self.release(sequence_indices)
        self.compact()
        if trim:
            self.trim_sdm_pools(headroom_rows=trim_headroom_rows)
        return freed

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
def pack_prefill_layers(
    initial_memories: Sequence[torch.Tensor],
    final_memories: Sequence[torch.Tensor],
    write_indices: Sequence[torch.Tensor],
    *,
    capacity_rows: int | None | Sequence[int | None],
    decode_capacity: int,
    growth_quantum_rows: int,
) -> list[PackedSDMCopyOnWriteState]:
    """``pack_prefill_layer`` for every SDM layer of a stack at once: the
    same states, with the host reads of the handoff made once for all
    layers (``from_dense_overlay_layers``).  No counterpart in the
    reference (which packs layer by layer, inference.py:314-366)."""

    masks, finals, templates, shapes = [], [], None, None
    for initial_memory, final_memory, indices in zip(initial_memories, final_memories,
                                                     write_indices):
        batch, time, heads, writes = indices.shape
        if initial_memory.ndim != 3 or final_memory.shape != (
                batch, heads, initial_memory.shape[1], initial_memory.shape[2]):
            raise ValueError("SDM prefill routing does not match its controller")
        slots = initial_memory.shape[1]
        active = torch.zeros(batch * heads, slots, device=indices.device, dtype=torch.bool)
        mark_written(active, indices.permute(0, 2, 1, 3).reshape(batch * heads,
                                                                 time * writes))
        masks.append(active)
        finals.append(final_memory.flatten(0, 1))
        if shapes is None:
            shapes = (batch, time, heads, writes)
            templates = torch.arange(heads, device=active.device,
                                     dtype=torch.int64).repeat(batch)
        elif shapes != (batch, time, heads, writes):
            raise ValueError("the SDM layers of one stack share batch, prefix and heads")
    if shapes is None:
        return []
    batch, time, heads, writes = shapes
    return PackedSDMCopyOnWriteState.from_dense_overlay_layers(
        list(initial_memories), finals, masks, template_indices=templates,
        capacity_rows=capacity_rows, state_dtype=torch.float32,
        maximum_future_allocations=(
            None if growth_quantum_rows else batch * heads * writes * (decode_capacity - time)),
        growth_quantum_rows=growth_quantum_rows)


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
