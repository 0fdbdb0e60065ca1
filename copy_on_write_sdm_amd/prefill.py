"""Prefill of one SDM layer on the device: the reference's
``SparseDeltaMemory`` forward over a prefix with its routing and final memory
(copy_on_write_sdm/sdm.py:1136-1262, ``return_routing=True,
include_final_memory=True``), as ``prefill_faithful_sdm_stack`` runs it for
every SDM layer (inference.py:369-456) before handing the final memory to
copy-on-write state (``_pack_prefill_layer``, inference.py:314-366;
``pack_prefill_layer`` here).

Every token of the prefix goes through the controller kernels at once
(``prepare_sdm_step`` over B*T tokens: input norm, projections, gates, the
two route selections), the routes are scattered into dense vectors
(``dense_sparse_routes``), the layer's recurrence runs over the sequence
(``gated_delta_recurrence``, csrc/recurrence.hip), and the readings go
through the controller's finish (readings norm, output gate, output
projection).  Float32; there is no CPU path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

import torch

from .controller import SDMController, finish_sdm_step, prepare_sdm_step
from .inference import FaithfulSDMDecodeState, pack_prefill_layers
from .recurrence import dense_sparse_routes, gated_delta_recurrence


@dataclass
class SDMPrefill:
    """The layer's output and routing over a prefix (the reference's
    ``SDMRouting``, sdm.py:1216-1262): routes [B, T, H, K], values
    [B, T, H, head_width], gates [B, T, H], final memory [B, H, N,
    head_width]."""

    output: torch.Tensor
    read_indices: torch.Tensor
    read_weights: torch.Tensor
    write_indices: torch.Tensor
    write_weights: torch.Tensor
    forget_log_gate: torch.Tensor
    input_gate: torch.Tensor
    values: torch.Tensor
    final_memory: torch.Tensor

    @property
    def erase_gate(self) -> torch.Tensor:
        return self.input_gate


@torch.no_grad()
def prefill_sdm_layer(controller: SDMController, initial_memory: torch.Tensor,
                      tokens: torch.Tensor) -> SDMPrefill:
    """One SDM layer over a prefix: tokens [B, T, width] and the layer's
    initial memory [H, N, head_width] (its ``initial_memory`` parameter)."""

    c = controller
    if tokens.ndim != 3 or tokens.shape[-1] != c.width:
        raise ValueError(f"SDM tokens must be [B,T,{c.width}]")
    batch, time, width = tokens.shape
    heads, head_width, slots = c.memory_heads, c.head_width, c.slots
    if time <= 0:
        raise ValueError("prefill requires at least one token")
    if initial_memory.shape != (heads, slots, head_width):
        raise ValueError("SDM initial memory must be [H,N,D] of the controller's shape")
    if initial_memory.dtype != torch.float32 or initial_memory.device != c.device:
        raise ValueError("SDM initial memory must be float32 on the controller's device")
    step = prepare_sdm_step(c, tokens.reshape(batch * time, 1, width))
    x = step.inputs            # rows (b * T + t) * H + h

    def by_bank(t: torch.Tensor) -> torch.Tensor:
        # token-major rows -> [B * H, T, ...], bank b * H + h
        rest = t.shape[1:]
        return (t.reshape(batch, time, heads, *rest).transpose(1, 2)
                .reshape(batch * heads, time, *rest).contiguous())

    write_routes = dense_sparse_routes(by_bank(x.write_weights), by_bank(x.write_indices), slots)
    read_routes = dense_sparse_routes(by_bank(x.read_weights), by_bank(x.read_indices), slots)
    start = (initial_memory.unsqueeze(0).expand(batch, -1, -1, -1)
             .reshape(batch * heads, slots, head_width).contiguous())
    readings, final = gated_delta_recurrence(start, write_routes, by_bank(x.values),
                                             by_bank(x.input_gate), by_bank(x.forget_log_gate),
                                             read_routes)
    del write_routes, read_routes
    # back to token-major rows for the controller's finish
    per_token = (readings.reshape(batch, heads, time, head_width).transpose(1, 2)
                 .reshape(batch * time * heads, head_width).contiguous())
    out = finish_sdm_step(c, step, per_token)

    def routed(t: torch.Tensor) -> torch.Tensor:
        return t.reshape(batch, time, heads, *t.shape[1:])

    return SDMPrefill(
        output=out.reshape(batch, time, width),
        read_indices=routed(x.read_indices), read_weights=routed(x.read_weights),
        write_indices=routed(x.write_indices), write_weights=routed(x.write_weights),
        forget_log_gate=routed(x.forget_log_gate), input_gate=routed(x.input_gate),
        values=routed(x.values), final_memory=final.reshape(batch, heads, slots, head_width))


def allocate_dense_cache(key: torch.Tensor, value: torch.Tensor,
                         capacity: int) -> tuple[torch.Tensor, torch.Tensor]:
    """An attention layer's K/V cache for ``capacity`` positions holding the
    prefix's keys and values [B, heads, T, head_width] in its first T
    positions (inference.py:293-306)."""

    batch, heads, time, head_width = key.shape
    if value.shape != key.shape or capacity < time:
        raise ValueError("dense prefill cache capacity is invalid")
    shape = (batch, heads, capacity, head_width)
    key_cache = torch.empty(shape, device=key.device, dtype=key.dtype)
    value_cache = torch.empty(shape, device=value.device, dtype=value.dtype)
    key_cache[:, :, :time].copy_(key)
    value_cache[:, :, :time].copy_(value)
    return key_cache, value_cache


AttentionBlock = Callable[[int, torch.Tensor], tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
SDMBlockTail = Callable[[int, torch.Tensor], torch.Tensor]


@torch.no_grad()
def prefill_faithful_sdm_stack(
    layout: str,
    sdm_layers: Sequence[tuple[SDMController, torch.Tensor]],
    tokens: torch.Tensor,
    *,
    attention_block: AttentionBlock | None = None,
    sdm_tail: SDMBlockTail | None = None,
    capacity: int | None = None,
    sdm_capacity_rows: int | Sequence[int] | None = None,
    sdm_growth_quantum_rows: int = 0,
) -> tuple[torch.Tensor, FaithfulSDMDecodeState]:
    """``prefill_faithful_sdm_stack`` (inference.py:369-456) with the SDM
    layers on the device: every "B" layer of ``layout`` runs
    ``prefill_sdm_layer`` on the tokens entering it and adds its output;
    every layer's final memory is then handed to copy-on-write state
    (``pack_prefill_layers``: the reference's per-layer handoff with the
    host reads made once for all layers); the model's other parts stay the
    caller's:

    * ``attention_block(layer, tokens) -> (tokens, key, value)`` for an "A"
      layer: the block's residual stream after it, and the prefix's keys and
      values [B, heads, T, head_width] (the reference's
      ``attention.prefill_with_cache`` plus its MLP);
    * ``sdm_tail(layer, tokens) -> tokens`` after an SDM layer's residual
      add (the reference's SDM MLP; identity when omitted).

    ``sdm_layers`` holds each "B" layer's controller and initial memory
    [H, N, head_width] in layout order.  Returns the final tokens and the
    decode state, with the attention layers' K/V caches for ``capacity``
    positions."""

    if tokens.ndim != 3:
        raise ValueError("tokens must be [B,T,width]")
    batch, time, _ = tokens.shape
    if time <= 0:
        raise ValueError("prefill requires at least one token")
    selected_capacity = time if capacity is None else capacity
    if selected_capacity < time:
        raise ValueError("prefill capacity is shorter than the prefix")
    if sdm_growth_quantum_rows < 0:
        raise ValueError("SDM growth quantum cannot be negative")
    layer_positions = tuple(i for i, kind in enumerate(layout) if kind == "B")
    if len(sdm_layers) != len(layer_positions):
        raise ValueError("one controller and initial memory per B layer")
    if isinstance(sdm_capacity_rows, Sequence) and not isinstance(sdm_capacity_rows,
                                                                   (str, bytes)):
        per_layer = tuple(int(v) for v in sdm_capacity_rows)
        if len(per_layer) != len(layer_positions):
            raise ValueError("SDM capacities must contain one value per B layer")
    else:
        per_layer = (sdm_capacity_rows,) * len(layer_positions)
    if any(kind not in "AB" for kind in layout):
        raise ValueError("layout holds A (attention) and B (SDM) layers only")
    if "A" in layout and attention_block is None:
        raise ValueError("an attention layer needs attention_block")

    keys: list[torch.Tensor] = []
    values: list[torch.Tensor] = []
    handoffs = []   # (initial memory, final memory, write routes) per SDM layer
    sdm_index = 0
    for layer, kind in enumerate(layout):
        if kind == "A":
            tokens, key, value = attention_block(layer, tokens)
            key_cache, value_cache = allocate_dense_cache(key, value, selected_capacity)
            keys.append(key_cache)
            values.append(value_cache)
            continue
        controller, initial_memory = sdm_layers[sdm_index]
        pre = prefill_sdm_layer(controller, initial_memory, tokens)
        tokens = tokens + pre.output
        if sdm_tail is not None:
            tokens = sdm_tail(layer, tokens)
        handoffs.append((initial_memory, pre.final_memory, pre.write_indices))
        del pre
        sdm_index += 1
    # every SDM layer's handoff (_pack_prefill_layer, inference.py:314-366)
    # at once: the handoff's host reads are made once for all layers
    states = pack_prefill_layers(
        [h[0] for h in handoffs], [h[1] for h in handoffs], [h[2] for h in handoffs],
        capacity_rows=list(per_layer), decode_capacity=selected_capacity,
        growth_quantum_rows=sdm_growth_quantum_rows)
    del handoffs
    return tokens, FaithfulSDMDecodeState(
        layout=layout, position=time, capacity=selected_capacity, activation_dtype=tokens.dtype,
        active_sequences=torch.ones(batch, device=tokens.device, dtype=torch.bool),
        sdm_layer_positions=layer_positions, sdm_states=tuple(states),
        dense_keys=tuple(keys), dense_values=tuple(values))
