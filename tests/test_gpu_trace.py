"""GPU parity of decode traces: the persistent multi-step kernel (many
steps per launch, forwarding rows between steps through LDS, first touches
taking the rows a plan pass listed for them) and device-counter launches
must equal single-step launches and the oracle bit for bit, physical rows
included, and the decode loop ``run`` must equal the reference's per-step
loop (prepare_step_capacity(banks * W), then the step) in capacities,
growth counters, free stacks and readings.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import _native as nat
from copy_on_write_sdm_amd import synthetic
from gpu_helpers import (assert_state_equal, assert_states_identical, assert_states_match,
                         oracle_decode_loop)
from oracle import state as ref

pytestmark = pytest.mark.gpu


def _setup(device, *, layers, banks, slots, width, writes, reads, steps, seed,
           index_dtype=torch.int32, capacity=None, sticky=False):
    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=seed, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=width, writes=writes, reads=reads, seed=seed + 1,
                                  device=device, index_dtype=index_dtype)
    if sticky:
        # steps rewrite and reread the slots written `lag` steps earlier
        # (sticky=1: the step before, forwarded from LDS; sticky=2: two steps
        # before, whose rows were popped after this step's map entries were
        # read when the slot map stays in global memory)
        lag = int(sticky)
        keep = torch.rand(steps, layers, banks, 1, device=device) < 0.7
        for s in range(lag, steps):
            routes.write_indices[s] = torch.where(keep[s], routes.write_indices[s - lag],
                                                  routes.write_indices[s])
            routes.write_indices[s] = routes.write_indices[s].sort(-1).values
            take = min(reads, writes)
            routes.read_indices[s, ..., :take] = routes.write_indices[s - lag, ..., :take]
        # reads need not be unique per bank; only writes must
    capacity = capacity or banks * slots

    def states():
        out = []
        for l in range(layers):
            st = cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks,
                                                        capacity_rows=capacity)
            st.capacity_is_proven = True
            out.append(st)
        return out

    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)
    return m0, routes, states, kw


def _per_step(states, routes, steps, layers):
    outs = []
    for s in range(steps):
        row = []
        for l in range(layers):
            r, _ = cow.packed_sdm_cow_step(states[l], **routes.step(s, l), validate_routes=False,
                                           collect_diagnostics=False)
            row.append(r)
        outs.append(torch.stack(row))
    return torch.stack(outs)


@pytest.mark.parametrize("layers,banks,slots,width,writes,reads,steps,group", [
    (7, 64, 256, 128, 4, 16, 40, 16),    # benchmark shape
    (3, 5, 64, 64, 4, 16, 20, 7),        # float per lane, partial block
    (2, 130, 64, 256, 3, 9, 12, 12),     # float4 lanes, 3 look-back windows per step
    (1, 1, 16, 8, 1, 1, 30, 30),         # one bank, one route
    (4, 33, 32, 100, 2, 5, 25, 64),      # odd width > 64 (two floats per lane)
    (2, 6, 4500, 128, 4, 16, 20, 8),     # slot map too large for LDS
    (1, 3, 4096, 64, 3, 7, 12, 5),       # largest slot map staged in LDS
    (2, 6, 64, 128, 4, 16, 200, 200),    # 200 steps in one launch: gates in 4 chunks
    (1, 4, 48, 64, 3, 5, 129, 129),      # odd launch whose last step starts a chunk
    (1, 3, 96, 64, 4, 8, 300, 300),      # one launch of more than 256 steps
])
def test_persistent_trace_matches_single_steps(device, layers, banks, slots, width, writes,
                                              reads, steps, group):
    print(f"trace L={layers} B={banks} N={slots} D={width} W={writes} R={reads} S={steps} "
          f"G={group}", flush=True)
    m0, routes, states, kw = _setup(device, layers=layers, banks=banks, slots=slots,
                                    width=width, writes=writes, reads=reads, steps=steps,
                                    seed=banks + width)
    traced, single = states(), states()
    outputs = torch.empty(steps, layers, banks, width, device=device)
    tr = cow.DecodeTrace(states=traced, outputs=outputs, max_steps_per_launch=group, **kw)
    tr.launch(steps, start=0)
    want = _per_step(single, routes, steps, layers)
    assert torch.equal(outputs, want)
    for a, b in zip(traced, single):
        assert_states_identical(a, b)
        a.validate_invariants()
    dense = [m0[l, 0].expand(banks, -1, -1).clone(memory_format=torch.contiguous_format) for l in range(layers)]
    dout = torch.empty_like(outputs)
    cow.DecodeTrace(memories=dense, outputs=dout, max_steps_per_launch=group,
                    **kw).launch(steps, start=0)
    assert torch.equal(dout, want)
    for l in range(layers):
        assert torch.equal(dense[l], traced[l].materialize_dense())


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_invalid_routes_stop_only_their_bank(device, index_dtype):
    """One launch of 100 steps (two 64-step chunks) with an out-of-range
    write slot, an out-of-range read slot, a slot written twice in one step,
    and a map entry outside the slab: each layer records exactly those
    errors, each failing bank keeps the state it had before its first failing
    step (the dense run of the steps before it) for the rest of the launch,
    and every other bank decodes as the clean routes do."""

    layers, banks, slots, width, writes, reads, steps = 2, 6, 64, 64, 4, 8, 100
    group = steps
    print(f"invalid routes {index_dtype}", flush=True)
    m0, routes, states, kw = _setup(device, layers=layers, banks=banks, slots=slots,
                                    width=width, writes=writes, reads=reads, steps=steps,
                                    seed=41, index_dtype=index_dtype)
    clean_kw = dict(kw)
    bad_w = routes.write_indices.clone()
    bad_r = routes.read_indices.clone()
    bad_w[10, 0, 2, 1] = slots                     # write slot outside [0, N)
    bad_r[70, 0, 5, 3] = -1                        # read slot outside [0, N)
    bad_w[65, 1, 4, 2] = bad_w[65, 1, 4, 0]        # one slot written twice
    kw = dict(kw, write_indices=bad_w, read_indices=bad_r)
    # layer 1, bank 1: a map entry outside the slab, first touched at step k1
    x = int(routes.read_indices[30, 1, 1, 0])
    k1 = min(s for s in range(steps)
             if x in routes.write_indices[s, 1, 1].tolist() or x in routes.read_indices[s, 1, 1].tolist())
    stops = {(0, 2): 10, (0, 5): 70, (1, 4): 65, (1, 1): k1}

    packed = states()
    packed[1].logical_to_physical[1, x] = packed[1].capacity_rows
    outputs = torch.zeros(steps, layers, banks, width, device=device)
    cow.DecodeTrace(states=packed, outputs=outputs, max_steps_per_launch=group,
                    **kw).launch(steps, start=0)
    torch.cuda.synchronize()
    errors = [int(st.scratch[nat.SCRATCH_ERRORS]) for st in packed]
    assert errors == [nat.ERR_WRITE_INDEX | nat.ERR_READ_INDEX,
                      nat.ERR_DUP_WRITE | nat.ERR_CORRUPT]
    # the failing step never ran, so the entry was never rewritten
    assert int(packed[1].logical_to_physical[1, x]) == packed[1].capacity_rows
    packed[1].logical_to_physical[1, x] = -1

    def dense_run(n):
        tables = [m0[l, 0].expand(banks, -1, -1).clone(memory_format=torch.contiguous_format) for l in range(layers)]
        out = torch.zeros(steps, layers, banks, width, device=device)
        if n:
            cow.DecodeTrace(memories=tables, outputs=out, max_steps_per_launch=group,
                            **clean_kw).launch(n, start=0)
        return tables, out

    clean_tables, clean_out = dense_run(steps)
    for l in range(layers):
        got = packed[l].materialize_dense()
        for b in range(banks):
            k = stops.get((l, b))
            if k is None:
                assert torch.equal(outputs[:, l, b], clean_out[:, l, b]), (l, b)
                assert torch.equal(got[b], clean_tables[l][b]), (l, b)
            else:
                assert torch.equal(outputs[:k, l, b], clean_out[:k, l, b]), (l, b, k)
                assert torch.equal(got[b], dense_run(k)[0][l][b]), (l, b, k)
        packed[l].scratch[nat.SCRATCH_ERRORS] = 0   # recorded above, as expected
        packed[l].validate_invariants()


def test_persistent_trace_matches_oracle(device):
    banks, slots, width, steps = 6, 32, 128, 24
    m0, routes, states, kw = _setup(device, layers=1, banks=banks, slots=slots, width=width,
                                    writes=4, reads=16, steps=steps, seed=3, sticky=True)
    traced = states()
    outputs = torch.empty(steps, 1, banks, width, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, max_steps_per_launch=10,
                    **kw).launch(steps, start=0)
    oracle = ref.allocate(m0[0].cpu().numpy(), banks=banks, capacity_rows=banks * slots)
    oracle.capacity_is_proven = True
    for s in range(steps):
        x = {k: v.cpu().numpy() for k, v in routes.step(s, 0).items()}
        want, _ = ref.packed_step(oracle, **x, validate_routes=False)
        assert np.array_equal(outputs[s, 0].cpu().numpy(), want), f"step {s}"
    assert_state_equal(traced[0], oracle)


@pytest.mark.parametrize("writes,reads,zero_values", [
    (2, 5, False), (2, 5, True), (3, 16, True), (4, 16, True)])
def test_signed_zero_sums_match_oracle_bits(device, writes, reads, zero_values):
    """Zero memory and negative weights: every term of a reading of an
    untouched slot (and, with zero values, of every reading) is -0.0, so the
    reading is -0.0.  Rows past W and R that a shape leaves out must not turn
    such a sum into +0.0.  Compared as bit patterns: torch.equal and
    np.array_equal hold -0.0 == +0.0."""

    banks, slots, width, steps = 6, 64, 128, 12
    print(f"signed zeros W={writes} R={reads} zero_values={zero_values}", flush=True)
    m0, routes, states, kw = _setup(device, layers=1, banks=banks, slots=slots, width=width,
                                    writes=writes, reads=reads, steps=steps, seed=41)
    m0.zero_()
    routes.read_weights.copy_(-routes.read_weights.abs() - 0.01)
    routes.write_weights.copy_(-routes.write_weights.abs() - 0.01)
    if zero_values:
        routes.values.zero_()
    traced, single = states(), states()
    outputs = torch.empty(steps, 1, banks, width, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, max_steps_per_launch=steps,
                    **kw).launch(steps, start=0)
    want = _per_step(single, routes, steps, 1)
    bits = outputs.view(torch.int32)
    assert torch.equal(bits, want.view(torch.int32))
    assert (bits == -2 ** 31).any()
    oracle = ref.allocate(m0[0].cpu().numpy(), banks=banks, capacity_rows=banks * slots)
    oracle.capacity_is_proven = True
    for s in range(steps):
        x = {k: v.cpu().numpy() for k, v in routes.step(s, 0).items()}
        got, _ = ref.packed_step(oracle, **x, validate_routes=False)
        assert np.array_equal(bits[s, 0].cpu().numpy(), got.view(np.int32)), f"step {s}"


@pytest.mark.parametrize("slots,reads,lag,index_dtype", [
    (48, 12, 1, torch.int32),
    (48, 12, 1, torch.int64),
    (48, 16, 1, torch.int32),      # full shape
    (48, 16, 2, torch.int32),
    (5000, 16, 1, torch.int32),    # slot map too large for LDS
    (5000, 16, 2, torch.int32),
    (5000, 12, 2, torch.int64),
])
def test_sticky_routes_forwarding(device, slots, reads, lag, index_dtype):
    """Most writes of a step hit the slots a recent step wrote (and its reads
    too): the rows must come from the forwarding paths."""

    layers, banks, steps = 2, 40, 48
    print(f"sticky N={slots} R={reads} lag={lag} idx={index_dtype}", flush=True)
    _, routes, states, kw = _setup(device, layers=layers, banks=banks, slots=slots, width=128,
                                   writes=4, reads=reads, steps=steps, seed=9, sticky=lag,
                                   index_dtype=index_dtype)
    traced, single = states(), states()
    outputs = torch.empty(steps, layers, banks, 128, device=device)
    cow.DecodeTrace(states=traced, outputs=outputs, max_steps_per_launch=48,
                    **kw).launch(steps, start=0)
    want = _per_step(single, routes, steps, layers)
    assert torch.equal(outputs, want)
    for a, b in zip(traced, single):
        assert_states_identical(a, b)


@pytest.mark.parametrize("persistent", [True, False])
def test_device_counter_graph_replay(device, persistent):
    """A captured launch of `group` device-counted steps, replayed: every
    replay runs the next group, and a replay past the recorded steps does
    nothing (packed state records COWSDM_ERR_TRACE_RANGE)."""

    layers, banks, steps, group = 3, 16, 24, 4
    _, routes, states, kw = _setup(device, layers=layers, banks=banks, slots=64, width=128,
                                   writes=4, reads=16, steps=steps, seed=17)
    traced, single = states(), states()
    outputs = torch.empty(steps, layers, banks, 128, device=device)
    tr = cow.DecodeTrace(states=traced, outputs=outputs, persistent=persistent, **kw)
    layer_array = tr.layer_array()
    tr.upload()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
        tr.launch(group, layer_array)
    tr.set_step(0)
    for k in range(steps // group):
        graph.replay()
        if k % 2:
            torch.cuda.synchronize()   # eager work between replays
            assert tr.step_index.tolist() == [(k + 1) * group] * layers
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [steps] * layers
    assert tr.status.tolist() == [0] * layers
    tr.sync()
    want = _per_step(single, routes, steps, layers)
    assert torch.equal(outputs, want)
    for a, b in zip(traced, single):
        assert_states_identical(a, b)
        a.validate_invariants()
    before = outputs.clone()
    graph.replay()                     # past the end of the recorded steps
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [steps] * layers
    assert torch.equal(outputs, before)
    assert tr.status.tolist() == [nat.TRACE_ENDED] * layers
    for a in traced:
        a.validate_invariants()


@pytest.mark.parametrize("launch_steps,capacity,quantum", [
    (64, 24, 16),    # growth every few steps, many growths per launch
    (8, 24, 16),     # launches shorter than a growth's reach
    (7, 40, 48),     # odd launch length, quantum above a step's need
    (64, 512, 16),   # never short: one proof covers the run
    (1, 24, 16),     # one step per launch (the step kernel's own proof), host growth
])
def test_decode_loop_matches_reference_loop(device, launch_steps, capacity, quantum):
    """run() against the reference's per-step loop on the oracle: the proof
    counter, the free-count reads, every growth (events, rows added and
    copied), capacities, maps, free stacks and readings are equal, with any
    step count; both growth inside the slab's buffers (on the device) and
    growth past them (on the host) occur."""

    _decode_loop_case(device, launch_steps, layers=3, banks=8, slots=64, width=128,
                      steps=37, capacity=capacity, quantum=quantum)


@pytest.mark.parametrize("launch_steps,reserve", [(64, 50), (7, 50), (64, 0)])
def test_decode_loop_banks_list_their_pops(device, launch_steps, reserve):
    """Slot maps in global memory (N above the 4,096 that fit in LDS): every
    bank lists its own pops from the launch's growth segments and the layer's
    last control wave to list rewrites the free stack.  Almost every write is
    a first touch, so a launch grows at nearly every step (growth inside the
    reserved slab buffers, or past them on the host without a reserve)."""

    _decode_loop_case(device, launch_steps, layers=2, banks=8, slots=4500, width=64,
                      steps=50, capacity=24, quantum=16, reserve=reserve)


def test_decode_loop_long_launch(device):
    """One launch of 400 steps over 4,096 slots with room for every slot."""

    states = _decode_loop_case(device, 400, layers=1, banks=4, slots=4096, width=64,
                               steps=400, capacity=4 * 4096, quantum=256)
    assert int((states[0].logical_to_physical >= 0).sum(1).min()) > 1024


def _decode_loop_case(device, launch_steps, *, layers, banks, slots, width, steps, capacity,
                      quantum, reserve=0):
    writes, reads = 4, 8
    print(f"decode loop L={layers} B={banks} N={slots} S={steps} C={capacity} q={quantum} "
          f"launch={launch_steps}", flush=True)
    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=31, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=width, writes=writes, reads=reads, seed=32, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)
    states = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks, capacity_rows=capacity,
                                                     growth_quantum_rows=quantum)
              for l in range(layers)]
    oracles = [ref.allocate(m0[l].cpu().numpy(), banks=banks, capacity_rows=capacity,
                            growth_quantum_rows=quantum) for l in range(layers)]
    outputs = torch.empty(steps, layers, banks, width, device=device)
    tr = cow.DecodeTrace(states=states, outputs=outputs, **kw)
    if reserve:
        tr.reserve_steps(reserve)
    # two runs split at an odd step: the second continues the first's proof
    first = steps // 3 + 1
    tr.run(first, launch_steps=launch_steps)
    want = oracle_decode_loop(oracles, routes, first, need=banks * writes)
    for st, orc in zip(states, oracles):
        assert_state_equal(st, orc)
    tr.run(steps - first, launch_steps=launch_steps)
    want = np.concatenate(
        [want, oracle_decode_loop(oracles, routes, steps - first, start=first,
                                  need=banks * writes)])
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [steps] * layers
    assert np.array_equal(outputs.cpu().numpy(), want)
    for st, orc in zip(states, oracles):
        assert_state_equal(st, orc)
        st.validate_invariants()
    return states


@pytest.mark.parametrize("launch_steps", [512, 1])
def test_decode_loop_grows_on_device_with_reserved_room(device, launch_steps):
    """With the slab's buffers reserved for the run, every growth happens
    inside the launches (no host round) and still equals the reference loop:
    persistent launches, and launches of one step each (the step kernel
    makes the step's proof and growth itself)."""

    layers, banks, slots, steps = 2, 16, 64, 60
    m0 = synthetic.make_initial_memory(layers, 1, slots, 128, seed=5, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=128, writes=4, reads=16, seed=6, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)
    states = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks, capacity_rows=64,
                                                     growth_quantum_rows=64)
              for l in range(layers)]
    oracles = [ref.allocate(m0[l].cpu().numpy(), banks=banks, capacity_rows=64,
                            growth_quantum_rows=64) for l in range(layers)]
    outputs = torch.empty(steps, layers, banks, 128, device=device)
    tr = cow.DecodeTrace(states=states, outputs=outputs, **kw)
    tr.reserve_steps(steps)
    report = tr.run(steps, launch_steps=launch_steps)
    assert report == {"launches": -(-steps // launch_steps), "growth_rounds": 0}
    # the live rows of the run's host report equal the device's
    assert tr.reported_live_rows() == sum(int(st.allocated_rows_tensor()) for st in states)
    want = oracle_decode_loop(oracles, routes, steps, need=banks * 4)
    assert np.array_equal(outputs.cpu().numpy(), want)
    for st, orc in zip(states, oracles):
        assert st.growth_events > 3
        assert_state_equal(st, orc)
        st.validate_invariants()
    # an assignment to a state since the run: the report no longer speaks for it
    states[0].capacity_is_proven = states[0].capacity_is_proven
    assert tr.reported_live_rows() is None


def test_graph_replay_grows_on_device(device):
    """A captured 5-step launch replayed with the decode loop's proof and
    growth on the device: after sync(), the states equal the reference loop
    and no replay needed the host."""

    layers, banks, slots, steps, group = 2, 16, 64, 40, 5
    m0 = synthetic.make_initial_memory(layers, 1, slots, 128, seed=8, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=128, writes=4, reads=16, seed=9, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)
    states = [cow.PackedSDMCopyOnWriteState.allocate(m0[l], banks=banks, capacity_rows=64,
                                                     growth_quantum_rows=128)
              for l in range(layers)]
    oracles = [ref.allocate(m0[l].cpu().numpy(), banks=banks, capacity_rows=64,
                            growth_quantum_rows=128) for l in range(layers)]
    outputs = torch.empty(steps, layers, banks, 128, device=device)
    tr = cow.DecodeTrace(states=states, outputs=outputs, **kw)
    tr.reserve_steps(steps)
    layer_array = tr.layer_array()
    assert tr.planned
    tr.upload()
    tr.set_step(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
        tr.launch(group, layer_array)
    for k in range(steps // group):
        graph.replay()
        if k % 3 == 1:
            torch.cuda.synchronize()   # eager work between replays
            assert tr.step_index.tolist() == [(k + 1) * group] * layers
    torch.cuda.synchronize()
    assert tr.step_index.tolist() == [steps] * layers
    assert tr.status.tolist() == [0] * layers
    tr.sync()
    want = oracle_decode_loop(oracles, routes, steps, need=banks * 4)
    assert np.array_equal(outputs.cpu().numpy(), want)
    for st, orc in zip(states, oracles):
        assert st.growth_events > 1
        assert_state_equal(st, orc)
        st.validate_invariants()


def test_host_offsets_past_recorded_steps_raise(device):
    _, routes, states, kw = _setup(device, layers=1, banks=4, slots=32, width=64, writes=2,
                                   reads=4, steps=6, seed=5)
    tr = cow.DecodeTrace(states=states(), **kw)
    with pytest.raises(ValueError, match="past the recorded steps"):
        tr.launch(4, start=3)


def test_persistent_overflow_sets_flag_and_keeps_partition(device):
    """A proven state whose slab is too small for the trace: the overflow
    flag latches, the launch stops committing first touches where the free
    stack runs out, and the slab stays a partition."""

    layers, banks, slots, steps = 1, 8, 64, 20
    _, routes, states, kw = _setup(device, layers=layers, banks=banks, slots=slots, width=64,
                                   writes=4, reads=8, steps=steps, seed=23, capacity=60)
    st = states()
    cow.DecodeTrace(states=st, max_steps_per_launch=steps, **kw).launch(steps, start=0)
    assert int(st[0].overflow_flag) == 1
    mapping = st[0].logical_to_physical.cpu()
    live = mapping[mapping >= 0]
    free = st[0].free_rows[: int(st[0].free_count)].cpu()
    rows = torch.cat((live, free)).sort().values
    assert torch.equal(rows, torch.arange(60, dtype=rows.dtype))


@pytest.mark.parametrize("banks,launch_steps", [(16, 20), (64, 32), (5, 3)])
def test_short_launches_plan_locally(device, banks, launch_steps):
    """Launches of at most 32 steps over at most 64 banks with slot maps in
    LDS make their plan in every control wave, with no header: while the
    slab does not grow, a launch leaves the header words of an earlier epoch
    and its pops come straight from the found stack; a launch that grows
    takes the central plan, whose header carries the launch's epoch.  Both
    equal the reference's decode loop, rows and stacks included."""

    layers, slots, width, writes, reads = 2, 64, 64, 4, 8
    steps = 3 * launch_steps + 1
    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=41, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=width, writes=writes, reads=reads, seed=42, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)

    def case(capacity, quantum):
        states = [cow.PackedSDMCopyOnWriteState.allocate(
            m0[l], banks=banks, capacity_rows=capacity, growth_quantum_rows=quantum)
            for l in range(layers)]
        oracles = [ref.allocate(m0[l].cpu().numpy(), banks=banks, capacity_rows=capacity,
                                growth_quantum_rows=quantum) for l in range(layers)]
        outputs = torch.empty(steps, layers, banks, width, device=device)
        tr = cow.DecodeTrace(states=states, outputs=outputs, **kw)
        tr.reserve_steps(steps)
        headers = []
        done = 0
        while done < steps:
            n = min(launch_steps, steps - done)
            tr.run(n, launch_steps=launch_steps)
            scan = tr.scan.cpu()
            # the launch's epoch (its last control wave stores it) against
            # the epoch of the header words
            headers.append([int(scan[l, 8]) >> 32 == int(scan[l, 0]) & 0xFFFFFFFF
                            for l in range(layers)])
            done += n
        want = oracle_decode_loop(oracles, routes, steps, need=banks * writes)
        torch.cuda.synchronize()
        assert np.array_equal(outputs.cpu().numpy(), want)
        for st, orc in zip(states, oracles):
            assert_state_equal(st, orc)
            st.validate_invariants()
        return states, headers

    # room for every slot twice over: the proof re-reads the free count every
    # few launches but never grows the slab, so every plan is local
    states, headers = case(2 * banks * slots, banks * writes)
    assert not any(any(h) for h in headers)
    assert all(st.growth_events == 0 for st in states)
    assert int(states[0].allocated_rows_tensor()) > banks * 4
    # a slab that grows in the first launch: that launch plans centrally
    states, headers = case(banks * writes, banks * writes)
    assert all(headers[0])
    assert all(st.growth_events > 0 for st in states)


def test_known_first_step_checked_against_counters(device):
    """run() hands the kernel the step every layer's counter stands at, so
    that a launch's first loads need not wait for the counter.  The kernel
    still compares the two: a first step the counters do not hold (here a
    stale host position) stops the run with a fault instead of passing
    silently, and a correct one matches the reference loop."""

    layers, banks, slots, width, writes, reads = 2, 8, 32, 64, 4, 8
    steps = 24
    m0 = synthetic.make_initial_memory(layers, 1, slots, width, seed=61, device=device)
    routes = synthetic.make_steps(steps=steps, layers=layers, banks=banks, slots=slots,
                                  width=width, writes=writes, reads=reads, seed=62, device=device)
    kw = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
              values=routes.values, input_gate=routes.input_gate,
              forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
              read_weights=routes.read_weights)
    capacity = banks * slots
    states = [cow.PackedSDMCopyOnWriteState.allocate(
        m0[l], banks=banks, capacity_rows=capacity, growth_quantum_rows=banks * writes)
        for l in range(layers)]
    oracles = [ref.allocate(m0[l].cpu().numpy(), banks=banks, capacity_rows=capacity,
                            growth_quantum_rows=banks * writes) for l in range(layers)]
    outputs = torch.empty(steps, layers, banks, width, device=device)
    tr = cow.DecodeTrace(states=states, outputs=outputs, **kw)
    tr.reserve_steps(steps)
    tr.run(8, launch_steps=8)
    tr.run(8, launch_steps=4)
    want = oracle_decode_loop(oracles, routes, 16, need=banks * writes)
    torch.cuda.synchronize()
    assert np.array_equal(outputs[:16].cpu().numpy(), want)
    for st, orc in zip(states, oracles):
        assert_state_equal(st, orc)
    assert tr.step_index.tolist() == [16] * layers
    # a stale host position: the counters stand at 16, the host says 18
    tr._positions = [18] * layers
    with pytest.raises(RuntimeError, match="fault"):
        tr.run(4, launch_steps=4)
