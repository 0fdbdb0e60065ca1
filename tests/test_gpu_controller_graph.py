"""GPU parity of the captured per-token decode with the controller on the
device (ControllerDecodeGraph): one hipGraph replay per token runs, for
every SDM layer in order, the controller's prepare kernel, the read and
write route selections, the decode loop's capacity proof and growth on the
device, the packed step and the controller's finish
(_decode_faithful_sdm_layer, inference.py:538-566), each output added to
the residual stream.

Replays equal, bit for bit, the eager per-layer loop
(decode_sdm_layer_controller with the host proof) in every token's output
and in every state (maps, physical rows, free stacks, capacities, growth
counters, proofs), with the slabs growing on the device; and they equal the
oracle composition: the same controller kernels around the reference's
capacity proof and packed step on oracle states (oracle/state.py, bit for
bit), whose finish is also compared with the float64 oracle finish (rtol
1e-4 / atol 2e-5)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from gpu_helpers import assert_state_equal, assert_states_identical
from oracle import state as ref
from test_gpu_stack_decode import oracle_of

pytestmark = pytest.mark.gpu


def _tail(layer, x):
    return x * 0.95 + 0.01 * layer


def _setup(device, *, layers, batch, heads, width, slots, reads, writes, quantum, seed):
    ctrls = [cow.SDMController.random(width, slots=slots, reads=reads, writes=writes,
                                      memory_heads=heads, seed=seed + l, spread=0.1,
                                      device=device) for l in range(layers)]
    g = torch.Generator().manual_seed(seed)
    m0 = [(torch.randn(heads, slots, width // heads, generator=g) * 0.3).to(device)
          for _ in range(layers)]

    def states():
        out = []
        for l in range(layers):
            st = cow.PackedSDMCopyOnWriteState.allocate(
                m0[l], banks=batch * heads, capacity_rows=quantum, growth_quantum_rows=quantum,
                template_indices=torch.arange(heads, device=device).repeat(batch))
            out.append(st)
        return out

    tokens = torch.randn(16, batch, 1, width, generator=g).to(device)
    return ctrls, states, tokens


@pytest.mark.parametrize("heads,batch,layers,with_tail", [
    (1, 64, 3, True), (2, 6, 2, True),
    # no tail: a layer's finish and the next layer's prepare are one launch
    (1, 64, 3, False), (2, 6, 3, False)])
def test_captured_controller_decode(device, heads, batch, layers, with_tail):
    width, slots, reads, writes = 128, 256, 16, 4
    quantum = batch * heads * writes * 2
    n = 12
    print(f"controller graph H={heads} B={batch} L={layers} tail={with_tail}", flush=True)
    tail = _tail if with_tail else (lambda layer, x: x)
    ctrls, make_states, tokens = _setup(device, layers=layers, batch=batch, heads=heads,
                                        width=width, slots=slots, reads=reads, writes=writes,
                                        quantum=quantum, seed=71 + heads)
    graphed, eager = make_states(), make_states()
    oracles = [oracle_of(st) for st in eager]
    dec = cow.ControllerDecodeGraph(ctrls, graphed, batch, tail=_tail if with_tail else None)
    dec.reserve_tokens(n)
    dec.capture()
    got = []
    for t in range(n):
        got.append(dec(tokens[t]).clone())
        if t % 5 == 2:
            torch.cuda.synchronize()    # eager work between replays
    torch.cuda.synchronize()
    dec.check()
    dec.sync()

    for t in range(n):
        x = tokens[t]
        x_ref = tokens[t]
        for l, (c, st, orc) in enumerate(zip(ctrls, eager, oracles)):
            x = tail(l, x + cow.decode_sdm_layer_controller(c, x, st))
            # the oracle composition: the same controller kernels, the
            # reference's proof and step on the oracle state
            step = cow.prepare_sdm_step(c, x_ref)
            ref.prepare_step_capacity(orc, orc.banks * c.writes)
            inputs = {k: getattr(step.inputs, k).cpu().numpy()
                      for k in ("write_indices", "write_weights", "values", "input_gate",
                                "forget_log_gate", "read_indices", "read_weights")}
            reading, _ = ref.packed_step(orc, **inputs, validate_routes=False)
            out = cow.finish_sdm_step(c, step, torch.from_numpy(reading).to(device))
            x_ref = tail(l, x_ref + out)
        assert torch.equal(got[t], x), t
        assert torch.equal(got[t], x_ref), t
    for a, b, orc in zip(graphed, eager, oracles):
        assert_states_identical(a, b)
        assert_state_equal(a, orc)
        assert a.growth_events > 0
        a.validate_invariants()


def test_captured_controller_decode_refuses_without_room(device):
    """Without reserved room the first growth past the slab's buffers
    refuses on the device and check() raises; the state is unchanged."""

    ctrls, make_states, tokens = _setup(device, layers=1, batch=4, heads=1, width=64,
                                        slots=64, reads=8, writes=4, quantum=16, seed=5)
    states = make_states()
    before = states[0].materialize_dense().clone()
    dec = cow.ControllerDecodeGraph(ctrls, states, 4)
    dec.capture()
    for t in range(3):
        dec(tokens[t])
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="stopped with status"):
        dec.check()
    dec.sync()
    # the slab of 16 rows holds one step's need (16), the second step's
    # growth passes its buffers: one step ran
    assert states[0].growth_events == 0
    assert not torch.equal(states[0].materialize_dense(), before)
    states[0].validate_invariants()
