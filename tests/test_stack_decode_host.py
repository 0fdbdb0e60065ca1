"""Host-side checks of the stack decode (decode_faithful_sdm_stack,
inference.py:601-669) that run before any device work, and the dense K/V
cache write of one decode token (decode_with_cache, model.py:138-162), on
the CPU: every refusal keeps the reference's message, and a refused call
changes neither the positions nor the caches."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

import copy_on_write_sdm_amd as cow


def _state(*, layout="BAB", batch=3, position=5, capacity=8, positions=None,
           sdm=2, dense=1, layer_positions=None):
    keys = tuple(torch.zeros(batch, 2, capacity, 4) for _ in range(dense))
    return cow.FaithfulSDMDecodeState(
        layout=layout, position=position, capacity=capacity, activation_dtype=torch.float32,
        active_sequences=torch.ones(batch, dtype=torch.bool),
        sdm_layer_positions=(layer_positions if layer_positions is not None
                             else tuple(i for i, k in enumerate(layout) if k == "B")),
        sdm_states=tuple(object() for _ in range(sdm)), dense_keys=keys,
        dense_values=tuple(k.clone() for k in keys), positions=positions)


CONTROLLERS = [SimpleNamespace(width=16), SimpleNamespace(width=16)]


def _decode(state, tokens=None, layout="BAB", controllers=CONTROLLERS, **kw):
    tokens = torch.zeros(state.batch, 1, 16) if tokens is None else tokens
    kw.setdefault("attention_decode", lambda *a: a[1])
    return cow.decode_faithful_sdm_stack(layout, controllers, tokens, state, **kw)


def test_refusals_keep_the_reference_messages():
    with pytest.raises(ValueError, match=r"decode tokens must be \[3,1,16\]"):
        _decode(_state(), torch.zeros(3, 2, 16))
    with pytest.raises(ValueError, match=r"decode tokens must be \[3,1,16\]"):
        _decode(_state(), torch.zeros(2, 1, 16))
    with pytest.raises(ValueError, match="layout does not match the stack"):
        _decode(_state(layout="BBA", layer_positions=(0, 1)))
    with pytest.raises(ValueError, match="do not match state device and dtype"):
        _decode(_state(), torch.zeros(3, 1, 16, dtype=torch.float64))
    with pytest.raises(ValueError, match="reached its fixed capacity"):
        _decode(_state(position=8, capacity=8))
    with pytest.raises(ValueError, match="reached its fixed capacity"):
        _decode(_state(position=7, positions=torch.tensor([3, 8, 7])))
    released = _state()
    released.active_sequences[1] = False
    with pytest.raises(ValueError, match="released requests must be removed"):
        _decode(released)
    with pytest.raises(ValueError, match="decode state does not match the stack"):
        _decode(_state(sdm=1))
    with pytest.raises(ValueError, match="decode state does not match the stack"):
        _decode(_state(dense=0))
    with pytest.raises(ValueError, match="decode state does not match the stack"):
        _decode(_state(), controllers=CONTROLLERS[:1])
    with pytest.raises(ValueError, match="ordering is inconsistent"):
        _decode(_state(layer_positions=(2, 0)))
    with pytest.raises(ValueError, match="attention_decode"):
        _decode(_state(), attention_decode=None)
    with pytest.raises(ValueError, match="share its width"):
        _decode(_state(), controllers=[SimpleNamespace(width=16), SimpleNamespace(width=8)])


def test_refused_call_leaves_positions_alone():
    positions = torch.tensor([3, 8, 7])
    state = _state(position=8, positions=positions)
    with pytest.raises(ValueError, match="fixed capacity"):
        _decode(state)
    assert positions.tolist() == [3, 8, 7] and state.position == 8


def test_attention_only_stack_advances_positions():
    """A stack without SDM layers runs only the caller's attention and moves
    the shared position, or every request's own, one token on."""

    seen = []

    def attention(layer, tokens, key_cache, value_cache, position):
        seen.append((layer, position if isinstance(position, int) else position.tolist()))
        return tokens + 1

    state = _state(layout="AA", sdm=0, dense=2, position=2)
    out = cow.decode_faithful_sdm_stack("AA", [], torch.zeros(3, 1, 4), state,
                                        attention_decode=attention)
    assert torch.equal(out, torch.full((3, 1, 4), 2.0))
    assert seen == [(0, 2), (1, 2)] and state.position == 3 and state.positions is None
    seen.clear()
    positions = torch.tensor([1, 6, 4])
    state = _state(layout="AA", sdm=0, dense=2, position=6, positions=positions)
    cow.decode_faithful_sdm_stack("AA", [], torch.zeros(3, 1, 4), state,
                                  attention_decode=attention)
    assert seen == [(0, [1, 6, 4]), (1, [1, 6, 4])]
    assert state.positions.tolist() == [2, 7, 5] and state.position == 7


def test_dense_cache_write_at_shared_and_own_positions():
    caches = torch.zeros(3, 2, 6, 4), torch.zeros(3, 2, 6, 4)
    key = torch.arange(24, dtype=torch.float32).reshape(3, 2, 1, 4) + 1
    cow.write_dense_cache(*caches, key, -key, position=2)
    assert torch.equal(caches[0][:, :, 2:3], key) and torch.equal(caches[1][:, :, 2:3], -key)
    assert caches[0][:, :, [0, 1, 3, 4, 5]].abs().sum() == 0
    cow.write_dense_cache(*caches, 2 * key, -2 * key, position=torch.tensor([0, 5, 3]))
    for b, p in enumerate((0, 5, 3)):
        assert torch.equal(caches[0][b, :, p], 2 * key[b, :, 0])
        assert torch.equal(caches[1][b, :, p], -2 * key[b, :, 0])
    with pytest.raises(ValueError, match="positions are invalid"):
        cow.write_dense_cache(*caches, key, key, position=torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="cache is invalid"):
        cow.write_dense_cache(caches[0], caches[1][:, :, :5], key, key, position=1)
    with pytest.raises(ValueError, match="cache is invalid"):
        cow.write_dense_cache(*caches, key.expand(3, 2, 2, 4), key.expand(3, 2, 2, 4),
                              position=1)
