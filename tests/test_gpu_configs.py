"""BASELINE configurations at their real per-layer shapes, checked through
properties that do not depend on size: the packed decode equals the
dense-table decode bit for bit (readings and materialised state), equals the
host-proven per-step loop of the reference (capacities, growth counters,
private rows, free stack, readings; physical rows up to a permutation), and
keeps the allocator invariants.

Config 2: L=7, B=64, N=256, D=128, 256-token prefill handed off, decode with
the capacity proven on the device every 4 steps.  Config 3: B=64, 2,048-token
prefill handed off.  Config 5: one layer of its shape (4 heads x 64 requests
= 256 banks, N=65,536, Zipf(1.1) routes) decoded from an empty slab that
grows by one quantum every few steps.
"""

from __future__ import annotations

import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import synthetic
from gpu_helpers import assert_states_match

pytestmark = pytest.mark.gpu

W, R, D = 4, 16, 128


def _routes(device, *, steps, layers, banks, slots, seed, distribution="uniform", heads=1):
    batch = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots, width=D,
                                 writes=W, reads=R, seed=seed, device=device,
                                 distribution=distribution, heads=heads)
    return batch, dict(write_indices=batch.write_indices, write_weights=batch.write_weights,
                       values=batch.values, input_gate=batch.input_gate,
                       forget_log_gate=batch.forget_log_gate,
                       read_indices=batch.read_indices, read_weights=batch.read_weights)


def _handoff(device, m0, *, layers, banks, slots, prefix, quantum, seed):
    """Dense prefill of `prefix` tokens, then the copy-on-write handoff of
    every layer (inference.py:314-366)."""

    pre, kw = _routes(device, steps=prefix, layers=layers, banks=banks, slots=slots, seed=seed)
    tables = [m0[l, 0].expand(banks, -1, -1).contiguous() for l in range(layers)]
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

    return states


def _host_proven(states, batch, *, steps, layers, banks, proof_steps):
    """The reference's decode loop: prove capacity for a group of steps on
    the host (prepare_step_capacity), then step every layer."""

    need = banks * W * proof_steps
    outs = []
    for g in range(0, steps, proof_steps):
        for st in states:
            st.prepare_step_capacity(need)
        for s in range(g, min(g + proof_steps, steps)):
            row = []
            for l in range(layers):
                r, _ = cow.packed_sdm_cow_step(states[l], **batch.step(s, l),
                                               validate_routes=False, collect_diagnostics=False)
                row.append(r)
            outs.append(torch.stack(row))
    return torch.stack(outs)


def _check(states, host, dense, outputs, want, dense_out):
    assert torch.equal(outputs, want)
    assert torch.equal(dense_out, want)
    for a, b, t in zip(states, host, dense):
        assert a.capacity_rows == b.capacity_rows
        assert (a.growth_events, a.growth_rows_added, a.growth_rows_copied) == (
            b.growth_events, b.growth_rows_added, b.growth_rows_copied)
        assert_states_match(a, b)
        assert torch.equal(a.materialize_dense(), t)
        a.validate_invariants()


@pytest.mark.parametrize("prefix,steps", [(256, 128), (2048, 64)])
def test_config2_and_config3_handoff_then_decode(device, prefix, steps):
    layers, banks, slots, proof_steps = 7, 64, 256, 4
    print(f"config handoff prefix={prefix} decode={steps}", flush=True)
    quantum = max(16, banks * W * proof_steps)
    m0 = synthetic.make_initial_memory(layers, 1, slots, D, seed=31, device=device)
    make_states = _handoff(device, m0, layers=layers, banks=banks, slots=slots, prefix=prefix,
                           quantum=quantum, seed=32)
    batch, kw = _routes(device, steps=steps, layers=layers, banks=banks, slots=slots, seed=33)
    traced, host = make_states(), make_states()
    dense = [st.materialize_dense() for st in traced]
    outputs = torch.empty(steps, layers, banks, D, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps, proof_steps=proof_steps)
    dense_out = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dense_out, **kw).launch(steps, start=0)
    want = _host_proven(host, batch, steps=steps, layers=layers, banks=banks,
                        proof_steps=proof_steps)
    torch.cuda.synchronize()
    _check(traced, host, dense, outputs, want, dense_out)


def test_layer_groups_when_grid_exceeds_residency(device):
    """8 layers x 256 banks is twice the workgroups the device holds at once:
    the persistent decode runs the layers in groups, each still proven on the
    device, and matches the dense decode and the host-proven loop."""

    heads, requests, slots, steps, proof_steps, layers = 4, 64, 64, 48, 4, 8
    banks = heads * requests
    print(f"layer groups: L={layers} banks={banks} N={slots} steps={steps}", flush=True)
    quantum = banks * W * proof_steps
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
    report = cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps,
                                                                      proof_steps=proof_steps)
    assert report["growth_rounds"] > 0
    dense_out = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dense_out, **kw).launch(steps, start=0)
    want = _host_proven(host, batch, steps=steps, layers=layers, banks=banks,
                        proof_steps=proof_steps)
    torch.cuda.synchronize()
    _check(traced, host, dense, outputs, want, dense_out)


def test_config5_layer_zipf_growth(device):
    heads, requests, slots, steps, proof_steps = 4, 64, 65536, 64, 4
    banks = heads * requests
    print(f"config 5 layer: banks={banks} N={slots} steps={steps}", flush=True)
    quantum = banks * W * proof_steps
    m0 = synthetic.make_initial_memory(1, heads, slots, D, seed=51, device=device)
    templates = torch.arange(heads, dtype=torch.int64, device=device).repeat(requests)
    batch, kw = _routes(device, steps=steps, layers=1, banks=banks, slots=slots, seed=52,
                        distribution="zipf", heads=heads)

    def states():
        return [cow.PackedSDMCopyOnWriteState.allocate(
            m0[0], banks=banks, capacity_rows=quantum, template_indices=templates,
            growth_quantum_rows=quantum)]

    traced, host = states(), states()
    dense = [m0[0][templates].contiguous()]
    outputs = torch.empty(steps, 1, banks, D, device=device)
    report = cow.DecodeTrace(states=traced, outputs=outputs, **kw).run(steps,
                                                                      proof_steps=proof_steps)
    assert report["growth_rounds"] > 0        # the slab grew on the way
    dense_out = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dense_out, **kw).launch(steps, start=0)
    want = _host_proven(host, batch, steps=steps, layers=1, banks=banks,
                        proof_steps=proof_steps)
    torch.cuda.synchronize()
    _check(traced, host, dense, outputs, want, dense_out)
