#!/usr/bin/env python3
"""Decode throughput of the packed copy-on-write SDM step on one MI355X.

Workload (the benchmark configuration at batch 64): L=7 SDM layers, H=1 memory head,
N=256 slots, D=128, top-4 writes / top-16 reads drawn uniformly, FP32 state.
A 256-token prefix runs through the dense-table kernel, each layer's union of
written slots is packed into a copy-on-write slab with a growth quantum of
four decode steps (max(16, B*4*4) rows), then decode runs on the packed
state.  One bench "step" is one decode token for all 7 layers and all B
requests.

Decode loop: the reference's (inference.py:538-566: prepare_step_capacity
(B*W) before every step of every layer, then the fused step), run as
persistent launches of up to 512 steps for every (layer, bank), each planned
on the device first, inside the decode kernel (first-touch counts, the
per-step capacity proof, growth within the slab's buffers, the row of every
first touch).  The slab
buffers are sized for the run before timing, so growth happens inside the
launches; the growth counters still follow the reference's formula.
--config 3 (2,048-token prefill, packed handoff timed) and --config 5
(4 heads, N = 65,536, Zipf routes, decode from an empty slab) run BASELINE's
other single-GPU configurations; --batch sets B (1/16/64).

Timing, as the reference's benchmark (5 warmup and 20 timed steps, median of
5 repetitions, experiments/benchmark_serving.py:1002-1066): W untimed warmup
steps, then 5 repetitions of exactly K steps, each between synchronisations;
the median repetition is reported (0.1 s of untimed dense-control launches
on scratch tables warm the GPU first).  Five more repetitions of the next K
steps each record HIP events at the decode kernel's own start and end for
the roofline; the wall-clock repetitions run without them (they add about
20 us of host time per launch).  The same per-token loop is also
timed as the reference's call pattern on the per-layer kernel (eager) and as
one captured graph replay per token (graph_step) and as the same launch enqueued
directly per token (launch_step).  The dense-table control runs the same
routes the same way from the same packed state; both end states must be
equal.  The CPU baseline is the torch restatement of the reference's
dense-table step on the host cores (all cores and one
thread, and a bounded sample at this workload's shape).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tokens/s at batch 64 (L=7,N=256,D=128); achieved HBM GB/s % of peak"
PEAK_HBM_GBPS = 8000.0
LAYERS, WIDTH, WRITES, READS = 7, 128, 4, 16

# BASELINE configurations on one GPU: heads, slots, dense prefill tokens,
# default warmup + timed decode steps, route distribution
CONFIGS = {
    2: dict(heads=1, slots=256, prefix=256, warmup=64, steps=512, distribution="uniform",
            text="packed copy-on-write SDM decode, prefix 256"),
    3: dict(heads=1, slots=256, prefix=2048, warmup=64, steps=192, distribution="uniform",
            text="long-prefix handoff: 2048-token dense prefill packed, then 256 decode steps"),
    5: dict(heads=4, slots=65536, prefix=0, warmup=64, steps=960, distribution="zipf",
            text="large address space: Zipf(1.1) routes, decode from an empty slab"),
}
# --skewed (config 3): Zipf routes whose exponent makes the union of a bank's
# written slots after the 2048-token prefill about 94 of 256 (measured with
# synthetic.make_steps: 2.40 -> 95.9, 2.45 -> 90.8 over 64 bank-layers), the
# trained model's occupancy the configuration quotes (about 660 private rows
# of 1,792 per request); prefill and decode share each layer's hot slots.
SKEWED_EXPONENT = 2.42


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS),
                   help="BASELINE configuration (2 is the headline metric's)")
    p.add_argument("--steps", type=int, default=None, help="timed steps (default: the config's)")
    p.add_argument("--warmup", type=int, default=None, help="warmup steps (default: the config's)")
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--launch-steps", type=int, default=512, help="decode steps per launch")
    p.add_argument("--repeats", type=int, default=5, help="timed repetitions (median reported)")
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run one 256 MiB device copy first, so that counter passes "
                        "(FETCH_SIZE, WRITE_SIZE) can be scaled by a kernel of known traffic")
    p.add_argument("--map-page-slots", type=int, default=None,
                   help="after the run, report the paged slot map with this many slots per "
                        "page (default: 16 for config 5, none otherwise)")
    p.add_argument("--eager-steps", type=int, default=None,
                   help="steps of the per-layer Python drop-in path to time (0: skip; "
                        "default 32 for config 2, else 0)")
    p.add_argument("--skewed", action="store_true",
                   help="config 3 only: calibrated Zipf routes (about 37%% of each layer's "
                        "slots written by the prefill) instead of uniform ones")
    p.add_argument("--routes", action="store_true",
                   help="time product_key_routes (the route producer) instead of the decode "
                        "step: one JSON line per shape")
    return p.parse_args()


ROUTE_SHAPES = ((64, 256, 16), (64, 256, 4), (448, 256, 16), (256, 65536, 16),
                (4096, 65536, 16), (65536, 256, 16))


def bench_routes(steps: int) -> int:
    """Kernel time of product_key_routes per call (HIP events on torch's
    current stream, the stream the kernel is launched on) at config 2's
    shapes (64 rows, N = 256; 448 = 7 layers x 64 banks in one call),
    config 5's (256 rows, N = 65,536) and two large batches.  Algorithmic
    bytes per row: 2*sqrt(N)*4 read, K*(4 + 8) written."""

    import torch

    import copy_on_write_sdm_amd as cow

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    for rows, slots, k in ROUTE_SHAPES:
        root = int(round(slots ** 0.5))
        projected = torch.randn(rows, 1, 2 * root, device=dev, generator=gen)
        w = torch.empty((rows, 1, k), device=dev)
        i = torch.empty((rows, 1, k), dtype=torch.int64, device=dev)
        lib = cow.routing.nat.lib()
        stream = torch.cuda.current_stream(dev).cuda_stream

        def call():
            rc = lib.cowsdm_product_key_routes(projected.data_ptr(), rows, slots, k,
                                               w.data_ptr(), i.data_ptr(), stream)
            assert rc == 0, rc

        for _ in range(20):
            call()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            call()
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) * 1e3 / steps
        nbytes = rows * (2 * root * 4 + k * 12)
        print(json.dumps({"kernel": "product_key_routes_kernel", "rows": rows, "slots": slots,
                          "selected": k, "calls": steps, "us_per_call": round(us, 3),
                          "algorithmic_bytes": nbytes,
                          "achieved_GBs": round(nbytes / us / 1e3, 1)}), flush=True)
    return 0


def algorithmic_bytes(banks: int, layers: int) -> int:
    """Bytes one step of one (bank, layer) must move: 2W+R rows of D floats,
    the value vector and the reading, route indices/weights/map entries
    (int32/fp32) and three gates."""

    rows = (2 * WRITES + READS) * WIDTH * 4
    vectors = 2 * WIDTH * 4
    metadata = (WRITES + READS) * (4 + 4 + 4) + 3 * 4
    return banks * layers * (rows + vectors + metadata)


def profiled_traffic(batch: int, launch_steps: float) -> dict | None:
    """HBM bytes per launch of the packed decode kernels from the committed
    counter passes (FETCH_SIZE and WRITE_SIZE, scaled by a copy of known
    size), when this run's launches ran a profiled number of steps."""

    path = ROOT / "profiles" / "traffic_packed_trace_config2_b64.json"
    if not path.exists():
        return None
    for entry in json.loads(path.read_text()).get("launches", []):
        if entry["batch"] == batch and entry["steps_per_launch"] == launch_steps:
            return entry
    return None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(batch: int, budget_s: float, seed: int) -> dict:
    """The torch restatement of the reference's dense-table CPU step
    (allocator.py:1612-1633, oracle/torch_port.py) on the host cores:

    * 1 layer, B=1, N=256, D=128, a 16-token prefill,
      then 64 decode tokens timed; median of 5, on the box's CPU share and
      on one thread;
    * this workload's shape (L=7, N=256, D=128, batch ``batch``) for a
      bounded sample of about ``budget_s`` seconds on the CPU share, the
      like-for-like point reported as ``value``."""

    import statistics

    import torch

    from copy_on_write_sdm_amd import synthetic
    from oracle import torch_port

    share = min(16, os.cpu_count() or 1)
    slots = CONFIGS[2]["slots"]

    def config1(threads: int) -> dict:
        torch.set_num_threads(threads)
        times = []
        for rep in range(5):
            m0 = synthetic.make_initial_memory(1, 1, slots, WIDTH, seed=seed + rep)
            steps = synthetic.make_steps(steps=16 + 64, layers=1, banks=1, slots=slots,
                                         width=WIDTH, writes=WRITES, reads=READS,
                                         seed=seed + 10 + rep)
            table = m0[0, 0][None].clone()
            for s in range(16):
                torch_port.dense_step(table, **steps.step(s, 0))
            t0 = time.perf_counter()
            for s in range(16, 80):
                torch_port.dense_step(table, **steps.step(s, 0))
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        return {"tokens_per_s": round(64 / t, 1), "us_per_token": round(1e6 * t / 64, 2),
                "threads": torch.get_num_threads()}

    config1_share = config1(share)
    config1_one = config1(1)

    torch.set_num_threads(share)
    steps = 48
    m0 = synthetic.make_initial_memory(LAYERS, 1, slots, WIDTH, seed=seed)
    batch_inputs = synthetic.make_steps(steps=steps, layers=LAYERS, banks=batch, slots=slots,
                                        width=WIDTH, writes=WRITES, reads=READS, seed=seed + 1)
    tables = [m0[l, 0].expand(batch, -1, -1).clone(memory_format=torch.contiguous_format)
              for l in range(LAYERS)]
    for s in range(2):
        for l in range(LAYERS):
            torch_port.dense_step(tables[l], **batch_inputs.step(s, l))
    done = 0
    t0 = time.perf_counter()
    while True:
        s = done % steps
        for l in range(LAYERS):
            torch_port.dense_step(tables[l], **batch_inputs.step(s, l))
        done += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s:
            break
    return {
        "value": round(batch * done / elapsed, 1),
        "unit": "tokens/s",
        "cores": share,
        "kind": "port",
        "sample": (f"{done} decode steps of the torch dense-table restatement "
                   f"(oracle/torch_port.py) at L={LAYERS} B={batch} N={slots} D={WIDTH} "
                   f"W={WRITES} R={READS}, {elapsed:.1f} s on {share} threads"),
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "config1": {"workload": "1 layer, B=1, N=256, D=128, 16-token prefill, 64 decode "
                                "tokens timed, median of 5",
                    "cpu_share": config1_share, "one_thread": config1_one},
    }


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(the packed SDM step has no multi-GPU path in this build)", file=sys.stderr)
        return 2
    if args.routes:
        return bench_routes(args.steps or 500)
    import statistics

    import torch

    import ctypes

    import copy_on_write_sdm_amd as cow
    from copy_on_write_sdm_amd import _native as nat
    from copy_on_write_sdm_amd import synthetic

    dev = torch.device("cuda:0")
    cfg = dict(CONFIGS[args.config])
    if args.skewed:
        if args.config != 3:
            print("--skewed applies to config 3", file=sys.stderr)
            return 2
        cfg.update(distribution="zipf", zipf_exponent=SKEWED_EXPONENT,
                   text=(f"long-prefix handoff with calibrated Zipf({SKEWED_EXPONENT}) routes "
                         "(about 37% of slots written by the prefill): 2048-token dense "
                         "prefill packed, then 256 decode steps"))
    route_kw = dict(distribution=cfg["distribution"], heads=cfg["heads"],
                    zipf_exponent=cfg.get("zipf_exponent", 1.1),
                    zipf_seed=args.seed + 7 if args.skewed else None)
    HEADS, SLOTS, PREFIX = cfg["heads"], cfg["slots"], cfg["prefix"]
    B = args.batch
    K = cfg["steps"] if args.steps is None else args.steps
    Wm = cfg["warmup"] if args.warmup is None else args.warmup
    repeats = max(1, args.repeats)
    if K <= 0 or Wm < 0:
        print("--steps must be positive and --warmup non-negative", file=sys.stderr)
        return 2
    eager_steps = (32 if args.config == 2 else 0) if args.eager_steps is None else args.eager_steps
    if args.map_page_slots is None and args.config == 5:
        args.map_page_slots = 16
    banks = B * HEADS                       # bank = request * H + head
    templates = torch.arange(HEADS, dtype=torch.int64, device=dev).repeat(B)
    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    total_steps = Wm + 2 * repeats * K      # wall-clock and kernel-timing repetitions
    quantum = max(16, banks * WRITES * 4)

    # ---- prefill (dense kernel) and copy-on-write handoff, untimed except the
    # handoff itself
    m0 = synthetic.make_initial_memory(LAYERS, HEADS, SLOTS, WIDTH, seed=args.seed, device=dev)
    handoff_ms = handoff_first_ms = None
    prefill_info = None
    if PREFIX:
        prefix = synthetic.make_steps(steps=PREFIX, layers=LAYERS, banks=banks, slots=SLOTS,
                                      width=WIDTH, writes=WRITES, reads=READS,
                                      seed=args.seed + 1, device=dev, **route_kw)
        tables = [m0[l][templates].contiguous() for l in range(LAYERS)]
        prefill = cow.DecodeTrace(memories=tables, write_indices=prefix.write_indices,
                                  write_weights=prefix.write_weights, values=prefix.values,
                                  input_gate=prefix.input_gate,
                                  forget_log_gate=prefix.forget_log_gate,
                                  read_indices=prefix.read_indices,
                                  read_weights=prefix.read_weights)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        prefill.launch(PREFIX, start=0)
        e1.record()
        torch.cuda.synchronize()
        prefill_info = {"trace_ms": round(e0.elapsed_time(e1), 3)}
        # the same prefill through the dense-route recurrence (the reference's
        # prefill kernel): route scatter and recurrence per layer, timed
        # together, and its final memory against the trace's tables
        def per_bank(t):
            return t.transpose(0, 1).contiguous()

        rec_finals, diff = [], 0.0
        e0.record()
        for l in range(LAYERS):
            wr = cow.dense_sparse_routes(per_bank(prefix.write_weights[:, l]),
                                         per_bank(prefix.write_indices[:, l]), SLOTS)
            rr = cow.dense_sparse_routes(per_bank(prefix.read_weights[:, l]),
                                         per_bank(prefix.read_indices[:, l]), SLOTS)
            rec_finals.append(cow.gated_delta_recurrence(
                m0[l][templates].contiguous(), wr, per_bank(prefix.values[:, l]),
                per_bank(prefix.input_gate[:, l]), per_bank(prefix.forget_log_gate[:, l]),
                rr)[1])
        e1.record()
        torch.cuda.synchronize()
        diff = max(float((f - t).abs().max()) for f, t in zip(rec_finals, tables))
        del rec_finals, wr, rr
        rec_ms = e0.elapsed_time(e1)
        prefill_info.update({
            "recurrence_ms": round(rec_ms, 3),
            "trace_tokens_per_s": round(B * PREFIX / (prefill_info["trace_ms"] / 1e3), 1),
            "recurrence_tokens_per_s": round(B * PREFIX / (rec_ms / 1e3), 1),
            "recurrence_vs_trace_max_abs_diff": diff,
            "what": "prefill of all layers: the sparse decode kernel (one launch over the "
                    "prefix) against dense_sparse_routes + the dense-route recurrence per layer "
                    "(different summation orders: a float tolerance, not bit equality)"})
        # the handoff twice: the first in the process also loads its kernels
        # and grows the allocator's pools (handoff_first_ms); the second is
        # the steady state of a serving process (handoff_ms), and its states
        # decode
        handoff_first_ms = None
        for _ in range(2):
            t0 = time.perf_counter()
            # every layer's written slots in one mask (a layer's rows are its
            # banks), one launch
            active = torch.zeros(LAYERS * banks, SLOTS, dtype=torch.bool, device=dev)
            cow.mark_written(active, prefix.write_indices.permute(1, 2, 0, 3).reshape(
                LAYERS * banks, -1))
            masks = list(active.view(LAYERS, banks, SLOTS))
            # every layer's handoff at once: one read of the active counts and
            # one of the invariant checks for all layers
            states = cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
                [m0[l] for l in range(LAYERS)], tables, masks, template_indices=templates,
                growth_quantum_rows=quantum)
            del masks, active
            torch.cuda.synchronize()
            handoff_ms = 1000.0 * (time.perf_counter() - t0)
            if handoff_first_ms is None:
                handoff_first_ms = handoff_ms
                del states
        del prefill, prefix, tables
    else:
        states = [cow.PackedSDMCopyOnWriteState.allocate(
            m0[l], banks=banks, capacity_rows=quantum, template_indices=templates,
            growth_quantum_rows=quantum) for l in range(LAYERS)]
    handoff_rows = [int(st.allocated_rows_tensor()) for st in states]
    handoff_capacity = [st.capacity_rows for st in states]

    # ---- decode routes
    routes = synthetic.make_steps(steps=total_steps, layers=LAYERS, banks=banks, slots=SLOTS,
                                  width=WIDTH, writes=WRITES, reads=READS, seed=args.seed + 2,
                                  device=dev, **route_kw)
    inputs = dict(write_indices=routes.write_indices, write_weights=routes.write_weights,
                  values=routes.values, input_gate=routes.input_gate,
                  forget_log_gate=routes.forget_log_gate, read_indices=routes.read_indices,
                  read_weights=routes.read_weights)
    dense_tables = [st.materialize_dense() for st in states]
    packed = cow.DecodeTrace(states=states, **inputs)
    dense = cow.DecodeTrace(memories=dense_tables, **inputs)
    # pool sizing before timing: slab buffers with room for every step of
    # the run, so that growth happens inside the launches
    packed.reserve_steps(total_steps)
    torch.cuda.synchronize()

    lib = nat.lib()

    def launch_times() -> tuple[float, float, int]:
        """Summed launch time (first kernel's start to the decode kernel's
        end), summed decode-kernel time (ms) and launches since timing was
        switched on: HIP events the library records on the launch stream."""
        span, kernel, count = ctypes.c_double(), ctypes.c_double(), ctypes.c_int32()
        nat.check(lib.cowsdm_trace_timing_read(ctypes.byref(span), ctypes.byref(kernel),
                                               ctypes.byref(count)), "trace timing")
        return span.value, kernel.value, count.value

    def live_rows(trace) -> int:
        # between repetitions from the last run's report in host memory: a
        # device read here would put copies on the stream before the next
        # timed launch
        if trace.dense:
            return 0
        rows = trace.reported_live_rows()
        return rows if rows is not None else sum(int(st.allocated_rows_tensor())
                                                 for st in trace.tables)

    def measure(trace):
        """`repeats` wall-clock repetitions of K steps with the library's
        launch events off (they cost the host about 20 us per launch), then
        `repeats` more of the next K steps each with HIP events at every
        decode kernel's own start and end on the launch stream."""

        def growths() -> int:
            return 0 if trace.dense else sum(st.growth_events for st in trace.tables)

        trace.set_step(0)
        lib.cowsdm_trace_timing(0)
        trace.run(Wm, launch_steps=args.launch_steps)   # warmup: the timed runs' host path
        torch.cuda.synchronize()
        reps = []
        for _ in range(repeats):
            rows0, grow0 = live_rows(trace), growths()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            report = trace.run(K, launch_steps=args.launch_steps)
            torch.cuda.synchronize()
            seconds = time.perf_counter() - t0
            reps.append(dict(seconds=seconds, new_rows=live_rows(trace) - rows0,
                             growths=growths() - grow0, **report))
        lib.cowsdm_trace_timing(1)
        launch_times()
        for rep in reps:
            rows0, grow0 = live_rows(trace), growths()
            torch.cuda.synchronize()
            report = trace.run(K, launch_steps=args.launch_steps)
            torch.cuda.synchronize()
            span_ms, kernel_ms, launches = launch_times()
            rep.update(span_ms=span_ms, kernel_ms=kernel_ms, timed_launches=launches,
                       kernel_new_rows=live_rows(trace) - rows0,
                       kernel_growths=growths() - grow0,
                       kernel_growth_rounds=report["growth_rounds"])
        lib.cowsdm_trace_timing(0)
        return reps

    # Warm-up before any timed run, so that the first timed repetition does
    # not pay for GPU clocks ramping up: ~0.1 s of dense-control launches on a
    # scratch copy of its tables (no trace step is consumed, and no state the
    # bench reports is touched).
    warm = cow.DecodeTrace(memories=[t.clone() for t in dense_tables], **inputs)
    warm_until = time.perf_counter() + 0.1
    while time.perf_counter() < warm_until:
        warm.launch(min(K, total_steps), start=0)
        torch.cuda.synchronize()
    del warm

    p_reps = measure(packed)
    d_reps = measure(dense)
    order = sorted(range(repeats), key=lambda r: p_reps[r]["seconds"])
    p_med = p_reps[order[(repeats - 1) // 2]]
    d_med = sorted(d_reps, key=lambda r: r["seconds"])[(repeats - 1) // 2]
    p_seconds, d_seconds = p_med["seconds"], d_med["seconds"]

    # both paths ran identical routes from identical logical state
    state_diff = max(float((st.materialize_dense() - t).abs().max())
                     for st, t in zip(states, dense_tables))
    for st in states:
        st.validate_invariants()
    if packed.step_index.tolist() != [total_steps] * LAYERS:
        raise AssertionError("packed decode did not consume the trace")
    allocator = {
        "handoff_ms": None if handoff_ms is None else round(handoff_ms, 3),
        "handoff_first_ms": None if handoff_first_ms is None else round(handoff_first_ms, 3),
        # the handoff reads every live row from the dense table and writes it
        # into the slab (2 x 4 B x D per row)
        "handoff_gbps": (None if not handoff_ms else
                         round(2 * 4 * WIDTH * sum(handoff_rows) / (handoff_ms / 1e3) / 1e9, 1)),
        "prefill": prefill_info,
        "handoff_live_rows": sum(handoff_rows),
        "handoff_capacity_rows": sum(handoff_capacity),
        "live_rows_after": sum(int(st.allocated_rows_tensor()) for st in states),
        "capacity_rows_after": sum(st.capacity_rows for st in states),
        "growth_events": sum(st.growth_events for st in states),
        "growth_rows_added": sum(st.growth_rows_added for st in states),
        "growth_rows_copied": sum(st.growth_rows_copied for st in states),
        "timed_growth_events": sum(r["growths"] for r in p_reps),
        "timed_host_growth_rounds": sum(r["growth_rounds"] for r in p_reps),
        "slab_buffer_rows": sum(packed._room(st) for st in states),
    }
    # the reference's serving-memory result (experiments/benchmark_serving.py:
    # 889-966, README.md:94-96) for the decoded state: live and allocated
    # rows over the logical rows, packed private bytes (live, and reserved
    # with this build's slab headroom) over the dense tables' bytes
    serving = cow.FaithfulSDMDecodeState(
        layout="B" * LAYERS, position=PREFIX + total_steps, capacity=PREFIX + total_steps,
        activation_dtype=torch.float32,
        active_sequences=torch.ones(B, dtype=torch.bool, device=dev),
        sdm_layer_positions=tuple(range(LAYERS)), sdm_states=tuple(states))
    packed_storage = serving.storage_bytes()
    dense_bytes = sum(4 * t.numel() for t in dense_tables)
    logical_rows = sum(st.banks * st.slots for st in states)
    memory = {
        "logical_rows": logical_rows,
        # the rows the handoff packed (private rows after the prefill)
        "handoff_live_row_fraction": round(allocator["handoff_live_rows"] / logical_rows, 4),
        "live_row_fraction": round(allocator["live_rows_after"] / logical_rows, 4),
        "physical_capacity_fraction": round(allocator["capacity_rows_after"] / logical_rows, 4),
        "packed_over_dense_live_bytes": round(
            packed_storage["per_user_live_total_excluding_shared"] / dense_bytes, 4),
        "packed_over_dense_reserved_bytes": round(
            packed_storage["total_reserved_excluding_shared"] / dense_bytes, 4),
        "slab_headroom_bytes": sum(st.storage_bytes()["slab_headroom"] for st in states),
        "dense_sdm_bytes": dense_bytes,
        "what": ("the reference's memory figures (benchmark_serving.py:889-966) after the "
                 "timed decode: packed storage_bytes() (reserved includes the slab buffers' "
                 "growth headroom that reserve_steps gave every layer) over the dense tables"),
    }

    # ---- per-layer Python drop-in path (exact reference call pattern), on
    # the decoded packed states once every check on them is done
    eager = None
    if eager_steps:
        n = min(eager_steps, total_steps)
        for s in range(2):
            for l in range(LAYERS):
                states[l].prepare_step_capacity(banks * WRITES)
                cow.packed_sdm_cow_step(states[l], **routes.step(s, l),
                                        validate_routes=False, collect_diagnostics=False)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(2, n):
            for l in range(LAYERS):
                states[l].prepare_step_capacity(banks * WRITES)
                cow.packed_sdm_cow_step(states[l], **routes.step(s, l),
                                        validate_routes=False, collect_diagnostics=False)
        torch.cuda.synchronize()
        eager = B * (n - 2) / (time.perf_counter() - t0)

    # ---- the same per-token loop as one captured graph launch per token:
    # each replay is one step of every layer with the decode loop's proof and
    # growth decided on the device (DecodeTrace.capture(1)), no host work
    graph_step = launch_step = None
    if eager_steps:
        # untimed replays first (as many as the recorded routes leave after
        # the timed ones, at most 64): the first replays of a graph run
        # slower (tens of microseconds) than the steady state
        timed = min(max(eager_steps, 2 * K), total_steps // 2)
        warm = min(64, total_steps - timed)
        n = warm + timed
        gtrace = cow.DecodeTrace(states=states, max_steps_per_launch=1, **inputs)
        gtrace.reserve_steps(n)
        gtrace.set_step(0)
        graph = gtrace.capture(1)
        for _ in range(warm):
            graph.replay()
        torch.cuda.synchronize()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        g0.record()
        for _ in range(n - warm):
            graph.replay()
        g1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gtrace.sync()
        if gtrace.step_index.tolist() != [n] * LAYERS or any(gtrace.status.tolist()):
            raise AssertionError("captured single-step decode did not run every step")
        graph_step = {
            "tokens_per_s": round(B * (n - warm) / wall, 1),
            "us_per_step": round(1e6 * wall / (n - warm), 3),
            "gpu_us_per_step": round(1000.0 * g0.elapsed_time(g1) / (n - warm), 3),
            "steps": n - warm,
            "warmup_replays": warm,
            "what": "hipGraph of one planned launch (all layers, one step) replayed per token",
        }
        del graph
        # the same launches enqueued one per token without the graph: the
        # runtime's graph launch costs about 16 us of host time per replay,
        # more than the kernel, a device-counted launch about 5 us, so the
        # stream is never empty and the rate is the kernel's
        layers_arr = gtrace.layer_array()
        gtrace.set_step(0)
        gtrace.upload()
        gtrace.status.zero_()
        for _ in range(warm):
            gtrace.launch(1, layers_arr)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g0.record()
        for _ in range(n - warm):
            gtrace.launch(1, layers_arr)
        g1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gtrace.sync()
        if gtrace.step_index.tolist() != [n] * LAYERS or any(gtrace.status.tolist()):
            raise AssertionError("per-token decode launches did not run every step")
        launch_step = {
            "tokens_per_s": round(B * (n - warm) / wall, 1),
            "us_per_step": round(1e6 * wall / (n - warm), 3),
            "gpu_us_per_step": round(1000.0 * g0.elapsed_time(g1) / (n - warm), 3),
            "steps": n - warm,
            "warmup_launches": warm,
            "what": ("the launches of graph_step enqueued directly, one per token "
                     "(DecodeTrace.launch(1): device counters, proof and growth on the "
                     "device, no host synchronisation)"),
        }

    # ---- the reference's per-token call pattern with the controller on the
    # device (decode_sdm_layer_controller: input norm, projections and gates,
    # routes, the capacity proof, the packed step, the output gate and
    # projection) for every layer, random controller weights of the
    # configuration's shape and random tokens
    controller_leg = None
    if eager_steps:
        n = min(eager_steps, 16)
        width_model = HEADS * WIDTH
        ctls = [cow.SDMController.random(width_model, slots=SLOTS, reads=READS, writes=WRITES,
                                         memory_heads=HEADS, seed=500 + l, device=dev)
                for l in range(LAYERS)]
        toks = torch.randn(n + 2, B, 1, width_model, device=dev,
                           generator=torch.Generator(device=dev).manual_seed(args.seed))

        def controller_token(s):
            for l in range(LAYERS):
                cow.decode_sdm_layer_controller(ctls[l], toks[s], states[l])

        for s in range(2):
            controller_token(s)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(2, n + 2):
            controller_token(s)
        torch.cuda.synchronize()
        controller_leg = {
            "tokens_per_s": round(B * n / (time.perf_counter() - t0), 1),
            "steps": n,
            "what": "per token and layer: controller prepare, two route selections, "
                    "prepare_step_capacity, packed step, controller finish (eager)",
        }

    # ---- the same per-token decode with the controller on the device,
    # captured once and replayed per token (ControllerDecodeGraph: per layer
    # prepare, two route selections, the proof and growth on the device, the
    # packed step, the finish, the residual add)
    controller_graph = None
    if eager_steps:
        n = max(eager_steps, 2 * K)
        warm = 16       # untimed replays, as for graph_step
        dec = cow.ControllerDecodeGraph(ctls, states, B)
        dec.reserve_tokens(n + warm)
        dec.capture()
        toks = torch.randn(n + warm, B, 1, width_model, device=dev,
                           generator=torch.Generator(device=dev).manual_seed(args.seed + 7))
        for s in range(warm):
            dec(toks[s])
        torch.cuda.synchronize()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        g0.record()
        for s in range(warm, n + warm):
            dec(toks[s])
        g1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        dec.check()
        dec.sync()
        for st in states:
            st.validate_invariants()
        controller_graph = {
            "tokens_per_s": round(B * n / wall, 1),
            "us_per_step": round(1e6 * wall / n, 3),
            "gpu_us_per_step": round(1000.0 * g0.elapsed_time(g1) / n, 3),
            "steps": n,
            "warmup_replays": warm,
            "what": "hipGraph per token of every layer's controller prepare, two route "
                    "selections, capacity proof and growth on the device, packed step, "
                    "controller finish and residual add (ControllerDecodeGraph)",
        }
        del dec

    # ---- the paged slot map (large address spaces, config 5): map bytes of
    # the decoded states, direct and paged; then fresh states of both forms
    # decoded 64 steps from an empty slab (one launch of all layers per step
    # with the host proof: paged maps have no persistent launches), outputs
    # compared, both timed, and their map bytes
    paged_leg = None
    if args.map_page_slots:
        P = args.map_page_slots
        direct_bytes = sum(st.storage_bytes()["logical_to_physical"] for st in states)
        end_paged = sum(cow.PagedSlotMap.compress(st.logical_to_physical, P).used_bytes()
                        for st in states)
        fresh_steps = 64
        fresh = synthetic.make_steps(steps=fresh_steps, layers=LAYERS, banks=banks, slots=SLOTS,
                                     width=WIDTH, writes=WRITES, reads=READS,
                                     seed=args.seed + 9, device=dev, **route_kw)
        keys = ("write_indices", "write_weights", "values", "input_gate", "forget_log_gate",
                "read_indices", "read_weights")

        def fresh_decode(page_slots):
            sts = [cow.PackedSDMCopyOnWriteState.allocate(
                m0[l], banks=banks, capacity_rows=quantum, template_indices=templates,
                growth_quantum_rows=quantum, map_page_slots=page_slots) for l in range(LAYERS)]
            outs = torch.empty(fresh_steps, LAYERS, banks, WIDTH, device=dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for s in range(fresh_steps):
                cow.PackedSDMCopyOnWriteState.prepare_step_capacity_layers(sts, banks * WRITES)
                cow.packed_sdm_cow_step_layers(sts, *[getattr(fresh, k)[s] for k in keys],
                                               outputs=list(outs[s]))
            torch.cuda.synchronize()
            return sts, outs, B * fresh_steps / (time.perf_counter() - t0)

        d_states, d_out, d_rate = fresh_decode(None)
        p_states, p_out, p_rate = fresh_decode(P)
        if not torch.equal(d_out, p_out) or not all(
                torch.equal(a.direct_map(), b.logical_to_physical)
                for a, b in zip(p_states, d_states)):
            raise AssertionError("paged and direct maps decoded differently")
        fresh_direct = sum(st.storage_bytes()["logical_to_physical"] for st in d_states)
        fresh_paged = sum(st.paged_map.used_bytes() for st in p_states)
        live = sum(int(st.allocated_rows_tensor()) for st in p_states)
        paged_leg = {
            "page_slots": P,
            "direct_map_bytes_per_layer": direct_bytes // LAYERS,
            "after_run": {
                "live_slot_fraction": memory["live_row_fraction"],
                "paged_map_bytes_per_layer": round(end_paged / LAYERS),
                "paged_over_direct_map_bytes": round(end_paged / direct_bytes, 4),
            },
            f"after_{fresh_steps}_steps": {
                "live_slot_fraction": round(live / (LAYERS * banks * SLOTS), 4),
                "paged_map_bytes_per_layer": round(fresh_paged / LAYERS),
                "paged_over_direct_map_bytes": round(fresh_paged / fresh_direct, 4),
                "stepwise_tokens_per_s_direct": round(d_rate, 1),
                "stepwise_tokens_per_s_paged": round(p_rate, 1),
                "outputs_equal": True,
            },
            "what": ("map bytes (paged: directory plus the pages in use) after the timed run, "
                     "and of fresh states after 64 steps decoded in both forms, one launch of "
                     "all layers per step with the host proof; the pages pay while few slots "
                     "of a page are live (the synthetic Zipf routes scatter hot slots over N)"),
        }
        del d_states, p_states, d_out, p_out

    # roofline of the dominant kernel, the persistent decode kernel: the
    # algorithmic bytes of the steps the timed launches ran over its mean
    # duration (HIP events at its own start and end); the count and plan
    # passes that precede it in each launch are reported beside it
    launches = sum(r["timed_launches"] for r in p_reps)
    timed_steps = repeats * K
    kernel_us = 1000.0 * sum(r["kernel_ms"] for r in p_reps) / launches
    span_us = 1000.0 * sum(r["span_ms"] for r in p_reps) / launches
    new_rows = sum(r["kernel_new_rows"] for r in p_reps)
    bytes_per_launch = (algorithmic_bytes(banks, LAYERS) * timed_steps + 8 * new_rows) / launches
    achieved = bytes_per_launch / (kernel_us * 1e-6) / 1e9
    d_launches = sum(r["timed_launches"] for r in d_reps)
    dense_kernel_us = 1000.0 * sum(r["kernel_ms"] for r in d_reps) / d_launches
    steps_per_launch = timed_steps / launches
    traffic = (profiled_traffic(B, steps_per_launch)
               if args.config == 2 and args.launch_steps == 512 else None)
    # the persistent variant that ran: full shape (W = 4, R = 16), at most 64
    # banks per layer, slot map in LDS up to 4,096 slots
    kernel = (f"sdm_trace_kernel<int, 2, false, true, {'true' if banks <= 64 else 'false'}, "
              f"{'true' if SLOTS <= 4096 else 'false'}>")

    result = {
        "metric": (METRIC if args.config == 2 and B == 64 else
                   f"decode tokens/s, config {args.config} at batch {B} (L={LAYERS},H={HEADS},"
                   f"N={SLOTS},D={WIDTH}); achieved HBM GB/s % of peak"),
        "value": round(B * K / p_seconds, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(1000.0 * p_seconds / K, 7),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "repeats": repeats,
        "repeat_tokens_per_s": [round(B * K / r["seconds"], 1) for r in p_reps],
        "repeat_kernel_us": [round(1000.0 * r["kernel_ms"] / max(1, r["timed_launches"]), 3)
                             for r in p_reps],
        "repeat_growths": [r["growths"] for r in p_reps],
        "timing": ("value and repeat_tokens_per_s: wall clock of repetitions with the "
                   "library's launch events off; kernel_us and repeat_kernel_us: HIP events "
                   "at the decode kernel's own start and end in the next repetitions of K "
                   "steps (the events add about 20 us of host time per launch)"),
        "config": {
            "workload": (f"config {args.config}: {cfg['text']}; L={LAYERS} H={HEADS} "
                         f"N={SLOTS} D={WIDTH} top-{WRITES} write / top-{READS} read "
                         f"({cfg['distribution']}), batch {B}, growth quantum 4 steps"),
            "batch": B, "heads": HEADS, "banks": banks, "layers": LAYERS, "slots": SLOTS,
            "width": WIDTH, "writes": WRITES, "reads": READS, "prefix": PREFIX,
            "distribution": cfg["distribution"],
            **({"zipf_exponent": cfg["zipf_exponent"]} if "zipf_exponent" in cfg else {}),
            "growth_quantum_rows": quantum, "max_steps_per_launch": args.launch_steps,
            "capacity_proof": ("the reference's prepare_step_capacity(B*W) before every "
                               "step, planned on the device per launch"),
            "launch": "persistent launches over all layers and banks",
            "mode": ("teacher-forced: the routes of every step are resident before the "
                     "launches (synthetic routes, as the reference's benchmark pre-generates "
                     "them), so one launch runs up to max_steps_per_launch steps; a decode "
                     "whose routes depend on the previous token runs one step per launch: "
                     "launch_step and graph_step (synthetic routes) and controller_graph "
                     "(routes from the device controller) give that per-token rate"),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": None if traffic is None else traffic["bytes_per_launch"],
            "traffic_source": None if traffic is None else traffic["source"],
            # the measured HBM bytes over the same kernel time: how busy HBM
            # actually is (rows a bank rereads and M0 hit in L2 and MALL)
            "traffic_gbps": (None if traffic is None else
                             round(traffic["bytes_per_launch"] / (kernel_us * 1e-6) / 1e9, 1)),
            "traffic_frac": (None if traffic is None else
                             round(traffic["bytes_per_launch"] / (kernel_us * 1e-6) / 1e9
                                   / PEAK_HBM_GBPS, 4)),
            "kernel": f"{kernel} (packed, {LAYERS} layers x {banks} banks)",
            "kernel_us": round(kernel_us, 3),
            "steps_per_launch": round(steps_per_launch, 3),
            "us_per_step": round(kernel_us / steps_per_launch, 4),
            "algorithmic_bytes_per_launch": int(bytes_per_launch),
            "launch_us_with_plan": round(span_us, 3),
            "frac_with_plan": round(bytes_per_launch / (span_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        },
        "dense_control": {
            "tokens_per_s": round(B * K / d_seconds, 1),
            "kernel_us": round(dense_kernel_us, 3),
            "us_per_step": round(dense_kernel_us * d_launches / timed_steps, 4),
            "packed_over_dense_latency": round(p_seconds / d_seconds, 4),
            "packed_over_dense_kernel": round(span_us * launches / (dense_kernel_us * d_launches), 4),
            "state_max_abs_diff": state_diff,
        },
        "allocator": allocator,
        "memory": memory,
        "eager_drop_in_tokens_per_s": None if eager is None else round(eager, 1),
        "graph_step": graph_step,
        "launch_step": launch_step,
        "controller_decode": controller_leg,
        "controller_graph": controller_graph,
    }
    if paged_leg is not None:
        result["paged_map"] = paged_leg
    if not args.no_cpu_baseline and args.config == 2:
        result["cpu_baseline"] = cpu_baseline(B, args.cpu_seconds, args.seed)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
