"""GPU parity of one SDM layer's prefill on the device (prefill.py:
SparseDeltaMemory's forward over a prefix, sdm.py:1136-1262, as
prefill_faithful_sdm_stack runs it, inference.py:369-456) and of the handoff
of its final memory (pack_prefill_layer, inference.py:314-366).

The controller kernels are pinned by test_gpu_controller.py and the
recurrence by test_gpu_recurrence.py; here the composition: the routing the
prefill returns equals the controller step's on the same tokens bit for bit,
and the layer's output and final memory equal, within rtol 1e-4 /
atol 2e-5, the float64 oracle's recurrence (oracle/serial.py) and finish
(oracle/controller.py) on that step's routes, values and gates (bank
b * H + h, tokens in order).  After the handoff the packed state
materialises to the final memory bit for bit, and decoding from it with the
controller equals the dense-table decode bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from controller_cases import make_layer, params_of
from oracle import controller as octl
from oracle import serial

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 2e-5


@pytest.mark.parametrize("heads,batch,time", [(1, 4, 12), (2, 3, 9), (4, 2, 5)])
def test_prefill_layer_matches_oracle(device, heads, batch, time):
    width, slots, reads, writes = 64, 64, 8, 4
    print(f"prefill H={heads} B={batch} T={time}", flush=True)
    layer = make_layer(width, slots=slots, reads=reads, writes=writes, heads=heads,
                       seed=40 + heads, dtype=torch.float32)
    controller = cow.SDMController.from_module(layer, device=device)
    hd = width // heads
    g = torch.Generator().manual_seed(heads)
    m0 = torch.randn(heads, slots, hd, generator=g) * 0.5
    x = torch.randn(batch, time, width, generator=g)
    pre = cow.prefill_sdm_layer(controller, m0.to(device), x.to(device))
    step = cow.prepare_sdm_step(controller, x.reshape(batch * time, 1, width).to(device))
    inp = step.inputs
    for name, k in (("write_indices", writes), ("write_weights", writes),
                    ("read_indices", reads), ("read_weights", reads)):
        assert torch.equal(getattr(pre, name).reshape(-1, k), getattr(inp, name)), name
    assert torch.equal(pre.values.reshape(-1, hd), inp.values)
    assert torch.equal(pre.input_gate.reshape(-1), inp.input_gate)
    assert torch.equal(pre.erase_gate, pre.input_gate)

    def banks(t):       # token-major rows -> [B * H, T, ...]
        a = t.cpu().numpy()
        a = a.reshape(batch, time, heads, *a.shape[1:])
        return np.swapaxes(a, 1, 2).reshape(batch * heads, time, *a.shape[3:])

    wr = serial.dense_routes(banks(inp.write_indices), banks(inp.write_weights), slots)
    rr = serial.dense_routes(banks(inp.read_indices), banks(inp.read_weights), slots)
    start = np.broadcast_to(m0.numpy()[None], (batch, heads, slots, hd)).reshape(
        batch * heads, slots, hd)
    ig = banks(inp.input_gate)
    want_r, want_m, _ = serial.serial_gated_delta_recurrence(
        start, wr, banks(inp.values), ig, banks(inp.forget_log_gate), rr, erase_gate=ig)
    per_token = np.swapaxes(want_r.reshape(batch, heads, time, hd), 1, 2).reshape(-1, hd)
    want_out = octl.finish(params_of(layer), step.normalized.cpu().numpy().astype(np.float64),
                           per_token)
    np.testing.assert_allclose(pre.output.reshape(batch * time, 1, width).cpu().numpy(),
                               want_out, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(pre.final_memory.reshape(batch * heads, slots, hd).cpu().numpy(),
                               want_m, rtol=RTOL, atol=ATOL)

    # the handoff, then decode from it: packed equals the dense table
    state = cow.pack_prefill_layer(m0.to(device), pre.final_memory, pre.write_indices,
                                   capacity_rows=None, decode_capacity=time + 8,
                                   growth_quantum_rows=batch * heads * writes * 2)
    table = pre.final_memory.reshape(batch * heads, slots, hd)
    assert torch.equal(state.materialize_dense(), table)
    dense = table.clone()
    for s in range(4):
        y = torch.randn(batch, 1, width, generator=g).to(device)
        out_p = cow.decode_sdm_layer_controller(controller, y, state)
        out_d = cow.decode_sdm_layer_controller_dense(controller, y, dense)
        assert torch.equal(out_p, out_d), s
    assert torch.equal(state.materialize_dense(), dense)
    state.validate_invariants()


def test_prefill_argument_errors(device):
    layer = make_layer(32, slots=16, reads=4, writes=2, heads=2, seed=3, dtype=torch.float32)
    controller = cow.SDMController.from_module(layer, device=device)
    m0 = torch.zeros(2, 16, 16, device=device)
    with pytest.raises(ValueError, match=r"must be \[B,T,32\]"):
        cow.prefill_sdm_layer(controller, m0, torch.zeros(2, 3, 16, device=device))
    with pytest.raises(ValueError, match="at least one token"):
        cow.prefill_sdm_layer(controller, m0, torch.zeros(2, 0, 32, device=device))
    with pytest.raises(ValueError, match="initial memory"):
        cow.prefill_sdm_layer(controller, m0[:1], torch.zeros(2, 3, 32, device=device))


def test_stack_prefill_and_admission(device):
    """prefill_faithful_sdm_stack (inference.py:369-456) over a "BAB"
    layout with the model's attention block and SDM tail supplied as
    callables: its tokens equal the same composition of prefill_sdm_layer
    calls bit for bit, every SDM layer's state materialises to that layer's
    final memory, the attention caches hold the prefix's keys and values;
    then a second prefilled cohort is admitted (inference.py:161-206): every
    SDM layer holds both cohorts' memories and the caches are stacked."""

    width, slots, heads, batch, time = 64, 64, 2, 3, 7
    g = torch.Generator().manual_seed(17)
    layers = [make_layer(width, slots=slots, reads=8, writes=4, heads=heads, seed=s,
                         dtype=torch.float32) for s in (5, 6)]
    ctrls = [cow.SDMController.from_module(layer, device=device) for layer in layers]
    m0s = [(torch.randn(heads, slots, width // heads, generator=g) * 0.5).to(device)
           for _ in layers]
    wq = (torch.randn(width, width, generator=g) * width ** -0.5).to(device)

    def attention(layer, tokens):
        b, t, _ = tokens.shape
        key = (tokens @ wq).reshape(b, t, 4, width // 4).transpose(1, 2).contiguous()
        return tokens + torch.tanh(tokens @ wq), key, key * 0.5

    def tail(layer, tokens):
        return tokens * 0.9

    quantum = batch * heads * 4 * 2
    kw = dict(attention_block=attention, sdm_tail=tail, capacity=time + 6,
              sdm_growth_quantum_rows=quantum)
    x = torch.randn(batch, time, width, generator=g).to(device)
    out, state = cow.prefill_faithful_sdm_stack("BAB", list(zip(ctrls, m0s)), x, **kw)
    pre0 = cow.prefill_sdm_layer(ctrls[0], m0s[0], x)
    t = tail(0, x + pre0.output)
    t, key, value = attention(1, t)
    pre1 = cow.prefill_sdm_layer(ctrls[1], m0s[1], t)
    t = tail(2, t + pre1.output)
    assert torch.equal(out, t)
    assert state.sdm_layer_positions == (0, 2)
    assert (state.position, state.capacity, state.batch) == (time, time + 6, batch)
    for st, pre in zip(state.sdm_states, (pre0, pre1)):
        assert torch.equal(st.materialize_dense(),
                           pre.final_memory.reshape(batch * heads, slots, width // heads))
        st.validate_invariants()
    assert state.dense_keys[0].shape == (batch, 4, time + 6, width // 4)
    assert torch.equal(state.dense_keys[0][:, :, :time], key)
    assert torch.equal(state.dense_values[0][:, :, :time], value)

    x2 = torch.randn(2, time, width, generator=g).to(device)
    _, incoming = cow.prefill_faithful_sdm_stack("BAB", list(zip(ctrls, m0s)), x2, **kw)
    expect = [torch.cat((a.materialize_dense(), b.materialize_dense()))
              for a, b in zip(state.sdm_states, incoming.sdm_states)]
    keys = torch.cat((state.dense_keys[0], incoming.dense_keys[0]))
    assert state.admit(incoming) == 2
    assert state.batch == batch + 2
    for st, want in zip(state.sdm_states, expect):
        assert torch.equal(st.materialize_dense(), want)
        st.validate_invariants()
    assert torch.equal(state.dense_keys[0], keys)

    with pytest.raises(ValueError, match="shorter than the prefix"):
        cow.prefill_faithful_sdm_stack("BAB", list(zip(ctrls, m0s)), x, **{**kw, "capacity": 3})
    with pytest.raises(ValueError, match="one value per B layer"):
        cow.prefill_faithful_sdm_stack("BAB", list(zip(ctrls, m0s)), x,
                                       **{**kw, "sdm_capacity_rows": [4096]})
    with pytest.raises(ValueError, match="attention_block"):
        cow.prefill_faithful_sdm_stack("BAB", list(zip(ctrls, m0s)), x,
                                       **{**kw, "attention_block": None})
