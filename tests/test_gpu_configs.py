"""BASELINE configurations on the HIP path.

Config 1 (1 layer, B=1, 16-token prefill, 64 decode tokens) end to end
against the oracle, bit for bit.  The other configurations at their real
shapes, checked through properties that do not depend on size: the packed
decode (``DecodeTrace.run``) equals

* the reference's decode loop run step by step on the device
  (``decode_sdm_layer``: prepare_step_capacity(banks * W), then
  ``packed_sdm_cow_step``; inference.py:538-566) in readings, maps, physical
  rows, free stacks, capacities, growth counters and proofs;
* the dense-table decode (``decode_sdm_layer_dense`` step by step, and the
  dense persistent trace) in readings and materialised state;

and keeps the allocator invariants.

Config 2: L=7, N=256, D=128, 256-token prefill handed off, B = 1, 16, 64
(at B=64 its 512 decode steps as one persistent launch).
Config 3: B=64, 2,048-token prefill handed off, its 256 decode steps.  Config 5 (4 heads x 64
requests = 256 banks, N=65,536, Zipf(1.1) routes) decoded from an empty slab
that grows every few steps: one layer, and all 7 layers for 1,024 steps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import synthetic
from copy_on_write_sdm_amd.inference import (SDMStepInputs, decode_sdm_layer,
                                             decode_sdm_layer_dense)
from gpu_helpers import assert_state_equal, assert_states_identical, oracle_decode_loop
from oracle import state as ref

pytestmark = pytest.mark.gpu

W, R, D = 4, 16, 128


def _routes(device, *, steps, layers, banks, slots, seed, distribution="uniform", heads=1,
            **zipf):
    batch = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots, width=D,
                                 writes=W, reads=R, seed=seed, device=device,
                                 distribution=distribution, heads=heads, **zipf)
    return batch, dict(write_indices=batch.write_indices, write_weights=batch.write_weights,
                       values=batch.values, input_gate=batch.input_gate,
                       forget_log_gate=batch.forget_log_gate,
                       read_indices=batch.read_indices, read_weights=batch.read_weights)


def _handoff(device, m0, *, layers, banks, slots, prefix, quantum, seed, **routes):
    """Dense prefill of `prefix` tokens, then the copy-on-write handoff of
    every layer (inference.py:314-366).  Returns a factory of fresh states
    and the prefix routes."""

    pre, kw = _routes(device, steps=prefix, layers=layers, banks=banks, slots=slots, seed=seed,
                      **routes)
    tables = [m0[l, 0].expand(banks, -1, -1).clone(memory_format=torch.contiguous_format) for l in range(layers)]
    cow.DecodeTrace(memories=tables, **kw).launch(prefix, start=0)

    def states():
        out = []
        for l in range(layers):
            active = torch.zeros(banks, slots, dtype=torch.bool, device=device)
            cow.mark_written(active, pre.write_indices[:, l].permute(1, 0, 2).reshape(banks, -1))
            out.append(cow.PackedSDMCopyOnWriteState.from_dense_overlay(
                m0[l], tables[l], active,
                template_indices=torch.zeros(banks, dtype=torch.int64, device=device),
                growth_quantum_rows=quantum))
        return out

    return states, pre


def _reference_loop(states, batch, *, steps, layers):
    """The reference's per-layer decode call, step by step: readings
    [steps, L, B, D]."""

    outs = []
    for s in range(steps):
        outs.append(torch.stack([
            decode_sdm_layer(states[l], SDMStepInputs(**batch.step(s, l)))
            for l in range(layers)]))
    return torch.stack(outs)


def _dense_loop(tables, batch, *, steps, layers):
    outs = []
    for s in range(steps):
        outs.append(torch.stack([
            decode_sdm_layer_dense(tables[l], SDMStepInputs(**batch.step(s, l)))
            for l in range(layers)]))
    return torch.stack(outs)


def _check(states, host, dense, outputs, want, dense_out):
    assert torch.equal(outputs, want)
    assert torch.equal(dense_out, want)
    for a, b, t in zip(states, host, dense):
        assert_states_identical(a, b)
        assert torch.equal(a.materialize_dense(), t)
        a.validate_invariants()


def test_config1_end_to_end_matches_oracle(device):
    """Config 1: 1 layer, B=1, N=256, D=128, a 16-token dense prefill, the
    handoff, then 64 decode tokens with a growth quantum of 16 rows, on the
    HIP path (persistent decode and the per-step reference loop) against
    the oracle, bit for bit (readings, physical rows, counters)."""

    banks, slots, prefix, steps, quantum = 1, 256, 16, 64, 16
    m0 = synthetic.make_initial_memory(1, 1, slots, D, seed=11, device=device)
    make_states, pre = _handoff(device, m0, layers=1, banks=banks, slots=slots, prefix=prefix,
                                quantum=quantum, seed=12)
    batch, kw = _routes(device, steps=steps, layers=1, banks=banks, slots=slots, seed=13)
    # the oracle: dense prefill, handoff, decode loop
    dense = np.repeat(m0[0, 0].cpu().numpy()[None], banks, axis=0)
    for s in range(prefix):
        x = {k: v.cpu().numpy() for k, v in pre.step(s, 0).items()}
        ref.dense_step(dense, **x, validate_routes=False)
    active = np.zeros((banks, slots), dtype=bool)
    for b in range(banks):
        active[b, pre.write_indices[:, 0, b].cpu().numpy().ravel()] = True
    orc = ref.from_dense_overlay(m0[0].cpu().numpy(), dense, active,
                                 template_indices=np.zeros(banks, dtype=np.int64),
                                 growth_quantum_rows=quantum)
    traced, host = make_states(), make_states()
    assert_state_equal(traced[0], orc)
    want = oracle_decode_loop([orc], batch, steps, need=banks * W)
    outputs = torch.empty(steps, 1, banks, D, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps)
    got_host = _reference_loop(host, batch, steps=steps, layers=1)
    assert np.array_equal(outputs.cpu().numpy(), want)
    assert np.array_equal(got_host.cpu().numpy(), want)
    assert_state_equal(traced[0], orc)
    assert_state_equal(host[0], orc)
    assert traced[0].growth_events > 0
    traced[0].validate_invariants()


@pytest.mark.parametrize("batch_size,prefix,steps,split,skewed", [
    (64, 256, 512, False, False),   # config 2: its 512 decode steps as one launch
    (64, 256, 128, True, False),    # config 2, a short run then the rest
    (16, 256, 96, True, False),     # config 2, B=16
    (1, 256, 96, True, False),      # config 2, B=1
    (64, 2048, 256, True, False),   # config 3: all 256 decode steps
    (64, 2048, 256, True, True),    # config 3, bench.py --skewed's routes
])
def test_config2_and_config3_handoff_then_decode(device, batch_size, prefix, steps, split,
                                                   skewed):
    layers, banks, slots = 7, batch_size, 256
    print(f"config handoff B={banks} prefix={prefix} decode={steps} split={split} "
          f"skewed={skewed}", flush=True)
    quantum = max(16, banks * W * 4)
    # skewed: the calibrated Zipf of bench.py --skewed, one set of hot slots
    # per layer for the prefill and the decode
    routes = dict(distribution="zipf", zipf_exponent=2.42, zipf_seed=39) if skewed else {}
    m0 = synthetic.make_initial_memory(layers, 1, slots, D, seed=31, device=device)
    make_states, _ = _handoff(device, m0, layers=layers, banks=banks, slots=slots,
                              prefix=prefix, quantum=quantum, seed=32, **routes)
    batch, kw = _routes(device, steps=steps, layers=layers, banks=banks, slots=slots, seed=33,
                        **routes)
    traced, host = make_states(), make_states()
    if skewed:
        # the handoff packs about 37 % of the logical rows (the trained
        # model's occupancy the configuration quotes)
        live = sum(int(st.allocated_rows_tensor()) for st in traced) / (layers * banks * slots)
        assert 0.30 < live < 0.45, live
    dense = [st.materialize_dense() for st in traced]
    dense_steps = [t.clone() for t in dense]
    outputs = torch.empty(steps, layers, banks, D, device=device)
    tr = cow.DecodeTrace(states=traced, outputs=outputs, **kw)
    if split:
        # two runs, the first of an odd length, as a warmup then a timed run would
        tr.run(5)
        tr.run(steps - 5)
    else:
        # the bench's kernel configuration: slab buffers sized for the run,
        # then one persistent launch whose plan grows the slabs on the device
        tr.reserve_steps(steps)
        assert tr.run(steps) == {"launches": 1, "growth_rounds": 0}
    dense_out = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dense_out, **kw).launch(steps, start=0)
    want = _reference_loop(host, batch, steps=steps, layers=layers)
    dense_want = _dense_loop(dense_steps, batch, steps=steps, layers=layers)
    torch.cuda.synchronize()
    assert torch.equal(dense_want, want)
    _check(traced, host, dense, outputs, want, dense_out)
    for a, t in zip(traced, dense_steps):
        assert torch.equal(a.materialize_dense(), t)


def test_layer_groups_when_grid_exceeds_residency(device):
    """8 layers x 256 banks is more workgroups than the device holds at once:
    the persistent decode runs the layers in groups, each planned on the
    device, and matches the dense decode and the reference loop."""

    heads, requests, slots, steps, layers = 4, 64, 64, 48, 8
    banks = heads * requests
    print(f"layer groups: L={layers} banks={banks} N={slots} steps={steps}", flush=True)
    quantum = banks * W * 4
    m0 = synthetic.make_initial_memory(layers, heads, slots, D, seed=61, device=device)
    templates = torch.arange(heads, dtype=torch.int64, device=device).repeat(requests)
    batch, kw = _routes(device, steps=steps, layers=layers, banks=banks, slots=slots, seed=62,
                        heads=heads)

    def states():
        return [cow.PackedSDMCopyOnWriteState.allocate(
            m0[l], banks=banks, capacity_rows=quantum, template_indices=templates,
            growth_quantum_rows=quantum) for l in range(layers)]

    traced, host = states(), states()
    dense = [m0[l][templates].contiguous() for l in range(layers)]
    outputs = torch.empty(steps, layers, banks, D, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps)
    assert all(st.growth_events > 0 for st in traced)
    dense_out = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dense_out, **kw).launch(steps, start=0)
    want = _reference_loop(host, batch, steps=steps, layers=layers)
    torch.cuda.synchronize()
    _check(traced, host, dense, outputs, want, dense_out)


def _config5(device, *, layers, steps, seed):
    heads, requests, slots = 4, 64, 65536
    banks = heads * requests
    print(f"config 5: L={layers} banks={banks} N={slots} steps={steps}", flush=True)
    quantum = banks * W * 4
    m0 = synthetic.make_initial_memory(layers, heads, slots, D, seed=seed, device=device)
    templates = torch.arange(heads, dtype=torch.int64, device=device).repeat(requests)
    batch, kw = _routes(device, steps=steps, layers=layers, banks=banks, slots=slots,
                        seed=seed + 1, distribution="zipf", heads=heads)

    def states():
        return [cow.PackedSDMCopyOnWriteState.allocate(
            m0[l], banks=banks, capacity_rows=quantum, template_indices=templates,
            growth_quantum_rows=quantum) for l in range(layers)]

    traced, host = states(), states()
    outputs = torch.empty(steps, layers, banks, D, device=device)
    report = cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps)
    torch.cuda.synchronize()
    print(f"config 5: persistent decode done ({report})", flush=True)
    want = _reference_loop(host, batch, steps=steps, layers=layers)
    torch.cuda.synchronize()
    print("config 5: reference loop done", flush=True)
    assert torch.equal(outputs, want)
    del want
    for a, b in zip(traced, host):
        assert a.growth_events > 0
        assert_states_identical(a, b)
        a.validate_invariants()
    del host
    # the dense-table decode, one layer at a time (8 GiB per layer)
    dense_out = torch.empty(steps, 1, banks, D, device=device)
    for l in range(layers):
        table = m0[l][templates].contiguous()
        one = {k: v[:, l:l + 1].contiguous() for k, v in kw.items()}
        cow.DecodeTrace(memories=[table], outputs=dense_out, **one).launch(steps, start=0)
        assert torch.equal(dense_out[:, 0], outputs[:, l]), l
        assert torch.equal(traced[l].materialize_dense(), table), l
        print(f"config 5: dense layer {l} equal", flush=True)
        del table
    return report


def test_config5_layer_zipf_growth(device):
    _config5(device, layers=1, steps=64, seed=51)


def test_config5_full_size(device):
    """Config 5 at full size: 7 layers x 256 banks over N = 65,536 slots,
    1,024 Zipf steps with the growth quantum of 4 steps."""

    _config5(device, layers=7, steps=1024, seed=71)


@pytest.mark.parametrize("static_scan", [False, True])
def test_captured_single_step_decode_matches_reference_loop(device, static_scan):
    """Config 2's shape (L=7, B=64, N=256, D=128) after a 256-token handoff,
    decoded as one hipGraph replay per token (``DecodeTrace.capture(1)``:
    every replay is one step of all layers with the capacity proof and the
    growth decided on the device), equals the reference's per-token loop
    (``decode_sdm_layer``: prepare_step_capacity(B * W), then the step) in
    readings, maps, physical rows, free stacks, capacities, growth counters
    and proofs.  With ``static_scan`` the replays allocate nothing."""

    layers, banks, slots, prefix, steps = 7, 64, 256, 256, 40
    quantum = banks * W * 4
    print(f"captured single steps static_scan={static_scan}", flush=True)
    m0 = synthetic.make_initial_memory(layers, 1, slots, D, seed=41, device=device)
    make_states, _ = _handoff(device, m0, layers=layers, banks=banks, slots=slots,
                              prefix=prefix, quantum=quantum, seed=42)
    batch, kw = _routes(device, steps=steps, layers=layers, banks=banks, slots=slots, seed=43)
    traced, host = make_states(), make_states()
    outputs = torch.empty(steps, layers, banks, D, device=device)
    tr = cow.DecodeTrace(states=traced, outputs=outputs, max_steps_per_launch=1,
                         static_scan=static_scan, **kw)
    tr.reserve_steps(steps)
    tr.set_step(0)
    graph = tr.capture(1)
    for k in range(steps):
        graph.replay()
        if k % 7 == 3:
            torch.cuda.synchronize()   # eager work between replays
            assert tr.step_index.tolist() == [k + 1] * layers
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [steps] * layers
    assert tr.status.tolist() == [0] * layers
    tr.sync()
    want = _reference_loop(host, batch, steps=steps, layers=layers)
    torch.cuda.synchronize()
    assert torch.equal(outputs, want)
    assert sum(st.growth_events for st in host) > 0
    for a, b in zip(traced, host):
        assert_states_identical(a, b)
        a.validate_invariants()
