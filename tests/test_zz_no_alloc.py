"""cowsdm_packed_step_trace_static, the decode-trace launch that allocates
nothing (its plan blocks live in the library's static device array), called
through the C-ABI and compared with cowsdm_packed_step_trace (plan blocks in
a caller-allocated buffer) bit for bit: readings, maps, physical rows, free
stacks and the control words, on two calls in a row, the second smaller."""

from __future__ import annotations

import ctypes

import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import _native as nat
from copy_on_write_sdm_amd import synthetic
from gpu_helpers import assert_states_identical

pytestmark = pytest.mark.gpu


def _case(device, *, layers, banks, slots, steps, seed, quantum):
    m0 = synthetic.make_initial_memory(layers, 1, slots, 128, seed=seed, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots, width=128,
                                  writes=4, reads=16, seed=seed + 1, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)

    def trace(static):
        states = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks, capacity_rows=64,
                                                         growth_quantum_rows=quantum)
                  for l in range(layers)]
        outputs = torch.empty(steps, layers, banks, 128, device=device)
        tr = cow.DecodeTrace(states=states, outputs=outputs, static_scan=static, **kw)
        tr.reserve_steps(steps)
        return tr

    return trace


def _launch(tr, steps, entry):
    """Upload the control words, launch `steps` device-counted steps through
    `entry` directly (ctypes), read the words back."""

    layers = tr.layer_array()
    assert tr.planned
    tr.upload()
    tr.set_step(0)
    stream = torch.cuda.current_stream().cuda_stream
    rc = entry(layers, len(tr.tables), tr.shape, ctypes.byref(tr.trace), steps, stream)
    assert rc == 0, nat.lib().cowsdm_last_error_string()
    torch.cuda.synchronize()
    tr.sync()


@pytest.mark.parametrize("order", ["large_then_small"])
def test_static_trace_matches_allocated_trace(device, order):
    lib = nat.lib()
    cases = [dict(layers=7, banks=64, slots=256, steps=48, seed=3, quantum=1024),
             dict(layers=3, banks=16, slots=64, steps=9, seed=5, quantum=64)]
    for case in cases:
        print(f"static trace {case}", flush=True)
        make = _case(device, **case)
        got, want = make(True), make(False)
        assert got.scan is None and got.trace.scan is None
        _launch(got, case["steps"], lib.cowsdm_packed_step_trace_static)
        _launch(want, case["steps"], lib.cowsdm_packed_step_trace)
        assert got.step_index.tolist() == [case["steps"]] * case["layers"]
        assert torch.equal(got.outputs, want.outputs)
        assert torch.equal(got.control, want.control)
        for a, b in zip(got.tables, want.tables):
            assert a.growth_events > 0
            assert_states_identical(a, b)
            a.validate_invariants()


def test_static_trace_refuses_past_its_array(device):
    """A call needing more plan words than the static array holds returns
    COWSDM_ELIMIT before launching anything."""

    lib = nat.lib()
    make = _case(device, layers=8, banks=256, slots=64, steps=4, seed=7, quantum=4096)
    tr = make(True)
    tr.trace.scan_steps = 512          # 8 layers x about 5 x 256 x 512 words
    layers = tr.layer_array()
    tr.upload()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.cowsdm_packed_step_trace_static(layers, 8, tr.shape, ctypes.byref(tr.trace), 4,
                                             stream)
    assert rc == -2
    assert b"static array" in lib.cowsdm_last_error_string() or \
        b"plan words" in lib.cowsdm_last_error_string()
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [0] * 8


def test_captured_static_launches_of_two_layouts(device):
    """Graphs of multi-step static launches of two layouts (64 banks over
    256 slots, 16 banks over 64 slots), replayed in turn and between eager
    static runs of a third layout, equal the allocated-plan path bit for
    bit: a replay must never take plan words another layout left in the
    shared array for its own."""

    cases = {"a": dict(layers=3, banks=64, slots=256, steps=24, seed=11, quantum=1024),
             "b": dict(layers=2, banks=16, slots=64, steps=24, seed=13, quantum=64),
             "c": dict(layers=2, banks=32, slots=128, steps=18, seed=17, quantum=256)}
    static, allocated = {}, {}
    for name, case in cases.items():
        make = _case(device, **case)
        static[name], allocated[name] = make(True), make(False)
        static[name].set_step(0)
    print("static capture: graphs of layouts a and b", flush=True)
    graphs = {name: static[name].capture(4) for name in ("a", "b")}
    for round_ in range(6):
        graphs["a"].replay()
        static["c"].run(2)          # eager static calls of a third layout
        graphs["b"].replay()
        if round_ % 2:
            torch.cuda.synchronize()
            static["c"].run(2)
    torch.cuda.synchronize()
    for name, tr in static.items():
        steps = cases[name]["steps"]
        tr.sync()
        assert tr.step_index.tolist() == [steps] * len(tr.tables), name
        assert tr.status.tolist() == [0] * len(tr.tables), name
        want = allocated[name]
        want.set_step(0)
        want.run(steps)
        torch.cuda.synchronize()
        assert torch.equal(tr.outputs, want.outputs), name
        for a, b in zip(tr.tables, want.tables):
            assert_states_identical(a, b)
            a.validate_invariants()
