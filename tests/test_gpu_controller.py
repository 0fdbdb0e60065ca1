"""GPU parity of the controller kernels (csrc/controller.hip) against
oracle/controller.py, and of the controller-driven layer decode
(``decode_sdm_layer_controller``, inference.py:538-598) against the oracle's
step.

Tolerances (float32 kernels against a float64 oracle on the same float32
weights): the normalised tokens within rtol 1e-5 / atol 1e-5, the keys,
values, gates and outputs within rtol 1e-4 / atol 2e-5 (a projection sums
`width` products with fused multiply-adds).  Routes are compared exactly
with the oracle's routes of the kernel's own keys (a near-tie in keys that
differ by a rounding could otherwise flip a selection), and the state step
is compared bit for bit with the oracle's step on the kernel's own step
inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import controller as ctl
from controller_cases import make_layer, params_of, tokens
from gpu_helpers import assert_state_equal
from oracle import controller as octl
from oracle import routes as oroutes
from oracle import state as ref

pytestmark = pytest.mark.gpu

# (width, slots, heads, reads, writes, batch): config 2's controller, config
# 5's (4 heads of 128, N = 65,536), an odd one (batch not a multiple of the
# kernel's 4 tokens per workgroup, two heads), the widest supported
SHAPES = [(128, 256, 1, 16, 4, 64), (512, 65536, 4, 16, 4, 16), (96, 64, 2, 8, 3, 5),
          (1024, 1024, 8, 8, 2, 3)]


def _setup(device, width, slots, heads, reads, writes, batch, seed):
    layer = make_layer(width, slots=slots, reads=reads, writes=writes, heads=heads,
                       seed=seed, dtype=torch.float32)
    controller = ctl.SDMController.from_module(layer, device=device)
    x = tokens(batch, width, seed=seed + 1, dtype=torch.float32)
    return layer, controller, x


@pytest.mark.parametrize("width,slots,heads,reads,writes,batch", SHAPES)
def test_prepare_matches_oracle(device, width, slots, heads, reads, writes, batch):
    print(f"controller prepare width={width} N={slots} H={heads} B={batch}", flush=True)
    layer, controller, x = _setup(device, width, slots, heads, reads, writes, batch, seed=width)
    step = ctl.prepare_sdm_step(controller, x.to(device))
    want = octl.prepare(params_of(layer), x.numpy())
    got = step.inputs
    np.testing.assert_allclose(step.normalized.cpu().numpy(), want["normalized"],
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got.values.cpu().numpy(), want["values"], rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(got.input_gate.cpu().numpy(), want["input_gate"],
                               rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(got.forget_log_gate.cpu().numpy(), want["forget_log_gate"],
                               rtol=1e-4, atol=2e-5)
    # the keys, read back from a second launch's outputs
    keys = {}
    for name in ("read_keys", "write_keys"):
        keys[name] = torch.empty(batch * heads, 1, 2 * int(np.sqrt(slots)), device=device)
    normalized = torch.empty(batch, 1, width, device=device)
    scratch = [torch.empty(batch * heads, width // heads, device=device)] + \
              [torch.empty(batch * heads, device=device) for _ in range(2)]
    from copy_on_write_sdm_amd import _native as nat
    nat.check(nat.lib().cowsdm_controller_prepare(
        controller.c_struct(), x.to(device).data_ptr(), batch, normalized.data_ptr(),
        keys["read_keys"].data_ptr(), keys["write_keys"].data_ptr(), scratch[0].data_ptr(),
        scratch[1].data_ptr(), scratch[2].data_ptr(), nat.stream_handle(device)), "prepare")
    for name in keys:
        np.testing.assert_allclose(keys[name].cpu().numpy(), want[name], rtol=1e-4, atol=2e-5)
    # routes: exactly the oracle's routes of the kernel's keys
    for name, k, idx, w in (("read_keys", reads, got.read_indices, got.read_weights),
                            ("write_keys", writes, got.write_indices, got.write_weights)):
        ew, ei = oroutes.product_key_routes(keys[name].cpu().numpy(), slots, k)
        np.testing.assert_array_equal(idx.cpu().numpy(), ei[:, 0])
        np.testing.assert_allclose(w.cpu().numpy(), ew[:, 0], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("width,slots,heads,reads,writes,batch", SHAPES)
def test_finish_matches_oracle(device, width, slots, heads, reads, writes, batch):
    print(f"controller finish width={width} H={heads} B={batch}", flush=True)
    layer, controller, x = _setup(device, width, slots, heads, reads, writes, batch,
                                  seed=3 * width)
    step = ctl.prepare_sdm_step(controller, x.to(device))
    reading = tokens(batch * heads, width // heads, seed=77, dtype=torch.float32)[:, 0]
    out = ctl.finish_sdm_step(controller, step, reading.to(device))
    want = octl.finish(params_of(layer), step.normalized.cpu().numpy().astype(np.float64),
                       reading.numpy())
    assert out.shape == (batch, 1, width)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-4, atol=2e-5)


def test_argument_errors(device):
    layer, controller, x = _setup(device, 64, 16, 2, 4, 2, 3, seed=5)
    with pytest.raises(ValueError, match="faithful SDM decode requires one token"):
        ctl.prepare_sdm_step(controller, x.to(device)[:, 0])
    with pytest.raises(TypeError, match="float32"):
        ctl.prepare_sdm_step(controller, x.to(device).double())
    step = ctl.prepare_sdm_step(controller, x.to(device))
    with pytest.raises(ValueError, match="reading does not match"):
        ctl.finish_sdm_step(controller, step, torch.zeros(5, 32, device=device))
    with pytest.raises(ValueError, match="perfect square"):
        ctl.SDMController.random(64, slots=15, reads=2, writes=2, device=device)
    with pytest.raises(ValueError, match="divisible"):
        ctl.SDMController.random(63, slots=16, reads=2, writes=2, memory_heads=2, device=device)


@pytest.mark.parametrize("heads", [1, 2])
def test_controller_layer_decode_matches_oracle_step(device, heads):
    """Tokens through decode_sdm_layer_controller on packed state, against
    the oracle's capacity proof and step on the kernel's own step inputs
    (state bit for bit), the dense twin (readings bit for bit) and the
    oracle's finish (tolerance)."""

    width, slots, batch, steps = 128, 256, 16, 6
    print(f"controller layer decode H={heads}", flush=True)
    layer, controller, _ = _setup(device, width, slots, heads, 16, 4, batch, seed=21 + heads)
    banks = batch * heads
    m0 = torch.randn(1, slots, width // heads, generator=torch.Generator().manual_seed(3))
    state = cow.PackedSDMCopyOnWriteState.allocate(m0.to(device), banks=banks,
                                                   capacity_rows=32, growth_quantum_rows=64)
    memory = m0.expand(banks, -1, -1).clone(memory_format=torch.contiguous_format).to(device)
    orc = ref.allocate(m0.numpy(), banks=banks, capacity_rows=32, growth_quantum_rows=64)
    p = params_of(layer)
    for s in range(steps):
        x = tokens(batch, width, seed=100 + s, dtype=torch.float32).to(device)
        out = ctl.decode_sdm_layer_controller(controller, x, state)
        dense_out = ctl.decode_sdm_layer_controller_dense(controller, x, memory)
        assert torch.equal(out, dense_out)
        step = ctl.prepare_sdm_step(controller, x)     # the same inputs, again
        xi = {k: getattr(step.inputs, k).cpu().numpy()
              for k in ("write_indices", "write_weights", "values", "input_gate",
                        "forget_log_gate", "read_indices", "read_weights")}
        ref.prepare_step_capacity(orc, banks * 4)
        reading, _ = ref.packed_step(orc, **xi, validate_routes=False)
        want = octl.finish(p, step.normalized.cpu().numpy().astype(np.float64), reading)
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-4, atol=2e-5)
    assert_state_equal(state, orc)
    assert state.growth_events > 0
    state.validate_invariants()


@pytest.mark.parametrize("width,slots,heads,reads,writes,batch", SHAPES)
def test_fused_prepare_routes_and_residual_finish_equal_separate_launches(
        device, width, slots, heads, reads, writes, batch):
    """cowsdm_controller_prepare_routes (one launch for sqrt(N) <= 64, the
    separate launches above it) writes exactly what prepare and the two
    route launches write; finish_residual's out equals finish's and its sum
    is residual + out."""
    from copy_on_write_sdm_amd import _native as nat
    from copy_on_write_sdm_amd.routing import product_key_routes
    print(f"fused controller prepare width={width} N={slots} H={heads} B={batch}", flush=True)
    layer, controller, x = _setup(device, width, slots, heads, reads, writes, batch,
                                  seed=5 * width)
    x = x.to(device)
    root = int(np.sqrt(slots))
    kr, kw = min(reads, min(reads, root) ** 2), min(writes, min(writes, root) ** 2)
    rows, hw = batch * heads, width // heads
    lib, stream = nat.lib(), nat.stream_handle(device)

    def outputs():
        f = dict(device=device, dtype=torch.float32)
        return {"normalized": torch.full((batch, width), 7.0, **f),
                "read_keys": torch.full((rows, 2 * root), 7.0, **f),
                "write_keys": torch.full((rows, 2 * root), 7.0, **f),
                "values": torch.full((rows, hw), 7.0, **f),
                "input_gate": torch.full((rows,), 7.0, **f),
                "forget": torch.full((rows,), 7.0, **f),
                "read_weights": torch.full((rows, kr), 7.0, **f),
                "read_indices": torch.full((rows, kr), -7, device=device, dtype=torch.int64),
                "write_weights": torch.full((rows, kw), 7.0, **f),
                "write_indices": torch.full((rows, kw), -7, device=device, dtype=torch.int64)}

    def prepare_args(o):
        return (controller.c_struct(), x.data_ptr(), batch, o["normalized"].data_ptr(),
                o["read_keys"].data_ptr(), o["write_keys"].data_ptr(), o["values"].data_ptr(),
                o["input_gate"].data_ptr(), o["forget"].data_ptr())

    want = outputs()
    nat.check(lib.cowsdm_controller_prepare(*prepare_args(want), stream), "prepare")
    product_key_routes(want["read_keys"].view(rows, 1, -1), slots=slots, selected=reads,
                       out=(want["read_weights"].view(rows, 1, kr),
                            want["read_indices"].view(rows, 1, kr)))
    product_key_routes(want["write_keys"].view(rows, 1, -1), slots=slots, selected=writes,
                       out=(want["write_weights"].view(rows, 1, kw),
                            want["write_indices"].view(rows, 1, kw)))
    got = outputs()
    nat.check(lib.cowsdm_controller_prepare_routes(
        *prepare_args(got), reads, writes, got["read_weights"].data_ptr(),
        got["read_indices"].data_ptr(), got["write_weights"].data_ptr(),
        got["write_indices"].data_ptr(), stream), "prepare_routes")
    for name in want:
        assert torch.equal(got[name], want[name]), name

    reading = tokens(rows, hw, seed=91, dtype=torch.float32)[:, 0].to(device)
    out_want = torch.empty(batch, width, device=device)
    nat.check(lib.cowsdm_controller_finish(
        controller.c_struct(), want["normalized"].data_ptr(), reading.data_ptr(), batch,
        out_want.data_ptr(), stream), "finish")
    out, total = torch.empty_like(out_want), torch.empty_like(out_want)
    nat.check(lib.cowsdm_controller_finish_residual(
        controller.c_struct(), want["normalized"].data_ptr(), reading.data_ptr(), batch,
        out.data_ptr(), x.data_ptr(), total.data_ptr(), stream), "finish_residual")
    assert torch.equal(out, out_want)
    assert torch.equal(total, x.view(batch, width) + out_want)
    # argument checks: the route counts take product_key_routes' checks
    assert lib.cowsdm_controller_prepare_routes(
        *prepare_args(got), 0, writes, got["read_weights"].data_ptr(),
        got["read_indices"].data_ptr(), got["write_weights"].data_ptr(),
        got["write_indices"].data_ptr(), stream) != 0
    assert lib.cowsdm_controller_finish_residual(
        controller.c_struct(), want["normalized"].data_ptr(), reading.data_ptr(), batch,
        out.data_ptr(), x.data_ptr(), None, stream) != 0


@pytest.mark.parametrize("width,slots,heads,reads,writes,batch", SHAPES)
def test_finish_then_next_prepare_in_one_call_equals_two(device, width, slots, heads, reads,
                                                        writes, batch):
    """cowsdm_controller_finish_prepare_routes (one launch for sqrt(N) <= 64,
    two above) writes exactly what finish_residual then prepare_routes of
    the next layer on its sum write."""
    from copy_on_write_sdm_amd import _native as nat
    print(f"finish+prepare width={width} N={slots} H={heads} B={batch}", flush=True)
    layer, c1, x = _setup(device, width, slots, heads, reads, writes, batch, seed=7 * width)
    _, c2, _ = _setup(device, width, slots, heads, reads, writes, batch, seed=7 * width + 1)
    x = x.to(device)
    root = int(np.sqrt(slots))
    kr, kw = min(reads, min(reads, root) ** 2), min(writes, min(writes, root) ** 2)
    rows, hw = batch * heads, width // heads
    lib, stream = nat.lib(), nat.stream_handle(device)
    step = ctl.prepare_sdm_step(c1, x)
    normalized = step.normalized.contiguous()
    reading = tokens(rows, hw, seed=93, dtype=torch.float32)[:, 0].to(device)

    def outputs():
        f = dict(device=device, dtype=torch.float32)
        i64 = dict(device=device, dtype=torch.int64)
        return {"out": torch.full((batch, width), 7.0, **f),
                "sum": torch.full((batch, width), 7.0, **f),
                "normalized": torch.full((batch, width), 7.0, **f),
                "read_keys": torch.full((rows, 2 * root), 7.0, **f),
                "write_keys": torch.full((rows, 2 * root), 7.0, **f),
                "values": torch.full((rows, hw), 7.0, **f),
                "input_gate": torch.full((rows,), 7.0, **f),
                "forget": torch.full((rows,), 7.0, **f),
                "read_weights": torch.full((rows, kr), 7.0, **f),
                "read_indices": torch.full((rows, kr), -7, **i64),
                "write_weights": torch.full((rows, kw), 7.0, **f),
                "write_indices": torch.full((rows, kw), -7, **i64)}

    def prepare_args(o):
        return (o["normalized"].data_ptr(), o["read_keys"].data_ptr(),
                o["write_keys"].data_ptr(), o["values"].data_ptr(), o["input_gate"].data_ptr(),
                o["forget"].data_ptr(), reads, writes, o["read_weights"].data_ptr(),
                o["read_indices"].data_ptr(), o["write_weights"].data_ptr(),
                o["write_indices"].data_ptr())

    finish = (c1.c_struct(), normalized.data_ptr(), reading.data_ptr(), batch)
    want = outputs()
    nat.check(lib.cowsdm_controller_finish_residual(
        *finish, want["out"].data_ptr(), x.data_ptr(), want["sum"].data_ptr(), stream), "finish")
    nat.check(lib.cowsdm_controller_prepare_routes(
        c2.c_struct(), want["sum"].data_ptr(), batch, *prepare_args(want), stream), "prepare")
    got = outputs()
    nat.check(lib.cowsdm_controller_finish_prepare_routes(
        *finish, got["out"].data_ptr(), x.data_ptr(), got["sum"].data_ptr(), c2.c_struct(),
        *prepare_args(got), stream), "finish_prepare_routes")
    for name in want:
        assert torch.equal(got[name], want[name]), name
    # the residual is required
    assert lib.cowsdm_controller_finish_prepare_routes(
        *finish, got["out"].data_ptr(), None, got["sum"].data_ptr(), c2.c_struct(),
        *prepare_args(got), stream) != 0
