"""One decode token through a stack of attention ("A") and SDM ("B") layers
over the retained serving state: ``decode_faithful_sdm_stack``
(copy_on_write_sdm/inference.py:601-669).

Every "B" layer runs the device controller step around the packed
copy-on-write step (``decode_sdm_layer_controller``: controller kernels, the
two product-key route selections, the capacity proof when the slab grows,
the fused step, the controller's finish) and adds its output to the
residual stream.  The model's other parts are the caller's, as in
``prefill_faithful_sdm_stack``:

* ``attention_decode(layer, tokens, key_cache, value_cache, position) ->
  tokens`` for an "A" layer: the block's residual stream after it (the
  reference's ``attention.decode_with_cache`` at the request positions, its
  residual add and its MLP, model.py:127-185).  It writes the token's key and
  value into that layer's cache; ``write_dense_cache`` does that write as the
  reference does;
* ``sdm_tail(layer, tokens) -> tokens`` after an SDM layer's residual add
  (the reference's SDM MLP; identity when omitted).

The reference's refusals are kept with its messages, and so is its position
bookkeeping: one shared ``position`` while every request stands at the same
token, one per request (``positions``) after admissions at other lengths.
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch

from .controller import SDMController, decode_sdm_layer_controller
from .inference import FaithfulSDMDecodeState

AttentionDecode = Callable[[int, torch.Tensor, torch.Tensor, torch.Tensor, "int | torch.Tensor"],
                           torch.Tensor]
SDMBlockTail = Callable[[int, torch.Tensor], torch.Tensor]


@torch.no_grad()
def write_dense_cache(key_cache: torch.Tensor, value_cache: torch.Tensor, key: torch.Tensor,
                      value: torch.Tensor, *, position: int | torch.Tensor) -> None:
    """The cache write of ``decode_with_cache`` (model.py:138-162): one
    token's key and value [B, heads, 1, head_width] into caches
    [B, heads, capacity, head_width], at one shared position (an int) or at
    each request's own position (a [B] tensor)."""

    if key.shape[2] != 1 or key_cache.shape != value_cache.shape or key.shape != value.shape:
        raise ValueError("dense decode cache is invalid")
    if isinstance(position, int):
        key_cache[:, :, position:position + 1].copy_(key)
        value_cache[:, :, position:position + 1].copy_(value)
        return
    positions = torch.as_tensor(position, device=key.device, dtype=torch.int64)
    if positions.shape != (key.shape[0],):
        raise ValueError("dense decode positions are invalid")
    rows = torch.arange(key.shape[0], device=key.device)
    key_cache[rows, :, positions, :] = key[:, :, 0, :]
    value_cache[rows, :, positions, :] = value[:, :, 0, :]


def _controller(entry) -> SDMController:
    # the controllers alone, or the (controller, initial memory) pairs the
    # stack prefill takes
    return entry[0] if isinstance(entry, tuple) else entry


@torch.no_grad()
def decode_faithful_sdm_stack(
    layout: str,
    sdm_layers: Sequence,
    tokens: torch.Tensor,
    state: FaithfulSDMDecodeState,
    *,
    attention_decode: AttentionDecode | None = None,
    sdm_tail: SDMBlockTail | None = None,
    backend: str = "auto",
) -> torch.Tensor:
    """``decode_faithful_sdm_stack`` (inference.py:601-669): consume one token
    [B, 1, width] through dense K/V caches and packed SDM state, advance the
    decode position(s) and return the stack's output tokens.

    ``sdm_layers`` holds each "B" layer's ``SDMController`` in layout order
    (or the (controller, initial memory) pairs given to the prefill)."""

    controllers = [_controller(entry) for entry in sdm_layers]
    width = controllers[0].width if controllers else tokens.shape[-1]
    if any(c.width != width for c in controllers):
        raise ValueError("SDM controllers of one stack share its width")
    if tokens.shape != (state.batch, 1, width):
        raise ValueError(f"decode tokens must be [{state.batch},1,{width}]")
    if state.layout != layout:
        raise ValueError("decode state layout does not match the stack")
    if tokens.device != state.device or tokens.dtype != state.dtype:
        raise ValueError("decode tokens do not match state device and dtype")
    if state.positions is None:
        if state.position >= state.capacity:
            raise ValueError("decode state has reached its fixed capacity")
        attention_position: int | torch.Tensor = int(state.position)
        furthest = int(state.position)
    else:
        positions = state.positions
        furthest = int(positions.max().item()) if positions.numel() else -1
        if furthest >= state.capacity:
            raise ValueError("decode state has reached its fixed capacity")
        attention_position = positions
    if not bool(state.active_sequences.all()):
        raise ValueError("released requests must be removed before further decode")
    expected_sdm = layout.count("B")
    expected_dense = layout.count("A")
    if (len(state.sdm_states) != expected_sdm
            or len(state.sdm_layer_positions) != expected_sdm
            or len(state.dense_keys) != expected_dense
            or len(state.dense_values) != expected_dense
            or len(controllers) != expected_sdm):
        raise ValueError("decode state does not match the stack")
    if expected_dense and attention_decode is None:
        raise ValueError("an attention layer needs attention_decode")

    dense_index = 0
    sdm_index = 0
    for layer, kind in enumerate(layout):
        if kind == "A":
            tokens = attention_decode(layer, tokens, state.dense_keys[dense_index],
                                      state.dense_values[dense_index], attention_position)
            dense_index += 1
            continue
        if state.sdm_layer_positions[sdm_index] != layer:
            raise ValueError("SDM decode layer ordering is inconsistent")
        mixed = decode_sdm_layer_controller(controllers[sdm_index], tokens,
                                            state.sdm_states[sdm_index], backend=backend)
        tokens = tokens + mixed
        if sdm_tail is not None:
            tokens = sdm_tail(layer, tokens)
        sdm_index += 1
    if state.positions is None:
        state.position += 1
    else:
        # every request moves one token on: the furthest one read above
        # bounds them all, so no second read of the positions is needed
        state.positions.add_(1)
        state.position = furthest + 1
    return tokens
