"""GPU parity of the stack decode over retained serving state
(decode_faithful_sdm_stack, inference.py:601-669) on a "BAB" stack, through
a lifecycle: prefill 4 requests, decode 4 tokens at one shared position,
release 2, compact, admit 2 requests prefilled with a longer prefix, decode
3 tokens at per-request positions.

Each token is checked against the reference loop composed on the host:
attention through the same caller callable on copies of the K/V caches,
every SDM layer through the controller kernels (pinned against the float64
controller oracle by test_gpu_controller.py), the reference's capacity
proof and packed step on oracle states (oracle/state.py, bit for bit) and
the controller's finish, which is also compared with the float64 oracle
finish (rtol 1e-4 / atol 2e-5).  The stack's tokens equal that composition
bit for bit, and so does the dense-table twin (the same controller around
dense_sdm_sparse_step on materialised tables); every SDM state equals its
oracle state (maps, physical rows, free stacks, growth counters, proofs);
the K/V caches hold each token's key and value at its request's position;
the positions advance as the reference's do."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from controller_cases import make_layer, params_of
from gpu_helpers import assert_state_equal
from oracle import controller as octl
from oracle import state as ref

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 2e-5
LAYOUT = "BAB"
WIDTH, SLOTS, HEADS, READS, WRITES = 64, 64, 2, 8, 4
ATT_HEADS = 4


def oracle_of(st: cow.PackedSDMCopyOnWriteState) -> ref.OracleState:
    """An oracle state holding exactly what a product state holds."""

    return ref.OracleState(
        shared_initial_memory=st.shared_initial_memory.cpu().numpy(),
        template_indices=st.template_indices.cpu().numpy().copy(),
        values=st.values.cpu().numpy().copy(),
        logical_to_physical=st.logical_to_physical.cpu().numpy().copy(),
        free_rows=st.free_rows.cpu().numpy().copy(),
        free_count=int(st.free_count.item()),
        overflow_flag=int(st.overflow_flag.item()),
        capacity_is_proven=st.capacity_is_proven,
        proven_maximum_additional_allocations=st.proven_maximum_additional_allocations,
        growth_quantum_rows=st.growth_quantum_rows,
        growth_events=st.growth_events,
        growth_rows_added=st.growth_rows_added,
        growth_rows_copied=st.growth_rows_copied)


class Attention:
    """The caller's attention block: a projection into 4 heads for queries,
    keys (and values = keys / 2), the cache write of decode_with_cache at the
    request positions, masked softmax attention over the live cache, its
    residual add and a tanh "MLP".  Every key written is recorded."""

    def __init__(self, device, seed):
        g = torch.Generator().manual_seed(seed)
        self.wq = (torch.randn(WIDTH, WIDTH, generator=g) * WIDTH ** -0.5).to(device)
        self.written = []

    def project(self, tokens):
        b, t, _ = tokens.shape
        return (tokens @ self.wq).reshape(b, t, ATT_HEADS, WIDTH // ATT_HEADS).transpose(
            1, 2).contiguous()

    def prefill(self, layer, tokens):
        key = self.project(tokens)
        return tokens + torch.tanh(tokens @ self.wq), key, key * 0.5

    def decode(self, layer, tokens, key_cache, value_cache, position, record=True):
        b = tokens.shape[0]
        key = self.project(tokens)                       # [b, heads, 1, hd]
        cow.write_dense_cache(key_cache, value_cache, key, key * 0.5, position=position)
        if record:
            self.written.append((key.clone(), position if isinstance(position, int)
                                 else position.clone()))
        if isinstance(position, int):
            live = position + 1
            visible = torch.ones(b, live, dtype=torch.bool, device=tokens.device)
        else:
            live = int(position.max()) + 1
            visible = (torch.arange(live, device=tokens.device)[None, :]
                       <= position[:, None])
        keys = torch.where(visible[:, None, :, None], key_cache[:, :, :live], 0.0)
        values = torch.where(visible[:, None, :, None], value_cache[:, :, :live], 0.0)
        scores = key @ keys.transpose(-1, -2).contiguous()
        scores = scores.masked_fill(~visible[:, None, None, :], float("-inf"))
        mixed = torch.softmax(scores, dim=-1) @ values
        mixed = mixed.transpose(1, 2).reshape(b, 1, WIDTH)
        return tokens + 0.5 * mixed + torch.tanh(tokens @ self.wq)


def tail(layer, tokens):
    return tokens * 0.9 + 0.01


def reference_token(tokens, ctrls, layers, oracles, keys, values, position, attention,
                    dense_tables):
    """The reference loop (inference.py:601-669) for one token, composed on
    the host; returns the stack output and the dense-table twin's."""

    tokens_d = tokens.clone()
    sdm = dense = 0
    for layer, kind in enumerate(LAYOUT):
        if kind == "A":
            k2, v2 = keys[dense].clone(), values[dense].clone()
            tokens = attention.decode(layer, tokens, keys[dense], values[dense], position,
                                      record=False)
            tokens_d = attention.decode(layer, tokens_d, k2, v2, position, record=False)
            dense += 1
            continue
        c, orc = ctrls[sdm], oracles[sdm]
        step = cow.prepare_sdm_step(c, tokens)
        if orc.growth_quantum_rows:
            ref.prepare_step_capacity(orc, orc.banks * c.writes)
        x = {name: getattr(step.inputs, name).cpu().numpy()
             for name in ("write_indices", "write_weights", "values", "input_gate",
                          "forget_log_gate", "read_indices", "read_weights")}
        reading, _ = ref.packed_step(orc, **x, validate_routes=False)
        out = cow.finish_sdm_step(c, step, torch.from_numpy(reading).to(tokens.device))
        want = octl.finish(params_of(layers[sdm]),
                           step.normalized.cpu().numpy().astype(np.float64),
                           reading.astype(np.float64))
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=RTOL, atol=ATOL)
        tokens = tail(layer, tokens + out)
        mixed_d = cow.decode_sdm_layer_controller_dense(c, tokens_d, dense_tables[sdm])
        tokens_d = tail(layer, tokens_d + mixed_d)
        sdm += 1
    return tokens, tokens_d


def test_stack_decode_through_lifecycle(device):
    g = torch.Generator().manual_seed(29)
    layers = [make_layer(WIDTH, slots=SLOTS, reads=READS, writes=WRITES, heads=HEADS, seed=s,
                         dtype=torch.float32) for s in (8, 9)]
    ctrls = [cow.SDMController.from_module(layer, device=device) for layer in layers]
    m0s = [(torch.randn(HEADS, SLOTS, WIDTH // HEADS, generator=g) * 0.5).to(device)
           for _ in layers]
    attention = Attention(device, 31)
    batch, time, capacity = 4, 6, 22
    quantum = batch * HEADS * WRITES * 2
    kw = dict(attention_block=attention.prefill, sdm_tail=tail, capacity=capacity,
              sdm_growth_quantum_rows=quantum)
    x = torch.randn(batch, time, WIDTH, generator=g).to(device)
    _, state = cow.prefill_faithful_sdm_stack(LAYOUT, list(zip(ctrls, m0s)), x, **kw)
    oracles = [oracle_of(st) for st in state.sdm_states]
    keys = [k.clone() for k in state.dense_keys]
    values = [v.clone() for v in state.dense_values]

    def decode_and_check(n, tag):
        for s in range(n):
            print(f"stack decode {tag} token {s} positions "
                  f"{state.position if state.positions is None else state.positions.tolist()}",
                  flush=True)
            y = torch.randn(state.batch, 1, WIDTH, generator=g).to(device)
            position = (state.position if state.positions is None
                        else state.positions.clone())
            tables = [torch.from_numpy(ref.materialize_dense(o)).to(device) for o in oracles]
            written = len(attention.written)
            got = cow.decode_faithful_sdm_stack(LAYOUT, list(zip(ctrls, m0s)), y, state,
                                                attention_decode=attention.decode,
                                                sdm_tail=tail)
            want, want_dense = reference_token(y, ctrls, layers, oracles, keys, values,
                                               position, attention, tables)
            assert torch.equal(got, want), (tag, s)
            assert torch.equal(got, want_dense), (tag, s)
            for st, orc, table in zip(state.sdm_states, oracles, tables):
                assert_state_equal(st, orc)
                assert torch.equal(st.materialize_dense(),
                                   torch.from_numpy(ref.materialize_dense(orc)).to(device))
            for got_k, want_k in zip(state.dense_keys, keys):
                assert torch.equal(got_k, want_k)
            for got_v, want_v in zip(state.dense_values, values):
                assert torch.equal(got_v, want_v)
            # the token's key sits at each request's position in the cache
            key, at = attention.written[written]
            rows = [at] * state.batch if isinstance(at, int) else at.tolist()
            for b, p in enumerate(rows):
                assert torch.equal(state.dense_keys[0][b, :, p], key[b, :, 0])
                assert torch.equal(state.dense_values[0][b, :, p], 0.5 * key[b, :, 0])
            if isinstance(position, int):
                assert state.positions is None and state.position == position + 1
            else:
                assert state.positions.tolist() == [p + 1 for p in position.tolist()]
                assert state.position == int(position.max()) + 1

    decode_and_check(4, "shared")
    assert state.position == time + 4

    # release 2 of 4, compact: rows freed per layer as the oracle frees them
    released = [1, 3]
    want_freed = 0
    for orc in oracles:
        want_freed += ref.release(orc, np.array([r * HEADS + h for r in released
                                                 for h in range(HEADS)]))
    assert state.release(released) == want_freed > 0
    kept = state.compact()
    assert kept.tolist() == [0, 2]
    for orc in oracles:
        ref.retain_banks(orc, np.array([r * HEADS + h for r in (0, 2) for h in range(HEADS)]))
    keys = [k.index_select(0, kept).contiguous() for k in keys]
    values = [v.index_select(0, kept).contiguous() for v in values]
    for st, orc in zip(state.sdm_states, oracles):
        assert_state_equal(st, orc)
        st.validate_invariants()

    # admit 2 requests with a longer prefix: per-request positions
    time2 = 13
    x2 = torch.randn(2, time2, WIDTH, generator=g).to(device)
    _, incoming = cow.prefill_faithful_sdm_stack(LAYOUT, list(zip(ctrls, m0s)), x2, **kw)
    for orc, theirs in zip(oracles, incoming.sdm_states):
        ref.append_banks_from(orc, oracle_of(theirs))
    keys = [torch.cat((a, b)).contiguous() for a, b in zip(keys, incoming.dense_keys)]
    values = [torch.cat((a, b)).contiguous() for a, b in zip(values, incoming.dense_values)]
    assert state.admit(incoming) == 2
    assert state.positions.tolist() == [time + 4, time + 4, time2, time2]
    assert state.position == time2
    for st, orc in zip(state.sdm_states, oracles):
        assert_state_equal(st, orc)

    decode_and_check(3, "mixed")
    assert state.positions.tolist() == [time + 7, time + 7, time2 + 3, time2 + 3]
    assert sum(st.growth_events for st in state.sdm_states) > 0
    for st in state.sdm_states:
        st.validate_invariants()


def test_stack_decode_refuses_at_capacity(device):
    """A request at the cache's last position decodes once more and then
    the stack refuses, with no state changed by the refused call."""

    layer = make_layer(WIDTH, slots=SLOTS, reads=READS, writes=WRITES, heads=1, seed=3,
                       dtype=torch.float32)
    ctrl = cow.SDMController.from_module(layer, device=device)
    m0 = torch.zeros(1, SLOTS, WIDTH, device=device)
    x = torch.randn(2, 3, WIDTH, generator=torch.Generator().manual_seed(4)).to(device)
    _, state = cow.prefill_faithful_sdm_stack("B", [(ctrl, m0)], x, capacity=4,
                                              sdm_growth_quantum_rows=16)
    y = torch.randn(2, 1, WIDTH, device=device)
    cow.decode_faithful_sdm_stack("B", [ctrl], y, state)
    assert state.position == 4
    before = state.sdm_states[0].materialize_dense().clone()
    with pytest.raises(ValueError, match="reached its fixed capacity"):
        cow.decode_faithful_sdm_stack("B", [ctrl], y, state)
    assert state.position == 4
    assert torch.equal(state.sdm_states[0].materialize_dense(), before)
