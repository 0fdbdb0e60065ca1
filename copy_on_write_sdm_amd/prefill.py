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

import torch

from .controller import SDMController, finish_sdm_step, prepare_sdm_step
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
