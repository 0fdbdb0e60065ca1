"""The SDM controller's per-token work around the copy-on-write step, on the
device (copy_on_write_sdm/inference.py:459-598).

``SDMController`` holds one layer's controller weights (the parameters of
the reference's ``SparseDeltaMemory``, sdm.py:998-1052) laid out for the
kernels: the five projections that read the normalised token as one
transposed matrix, and the output gate and projection transposed.
``prepare_sdm_step`` is ``_prepare_faithful_sdm_step`` (inference.py:459-519)
and ``finish_sdm_step`` is ``_finish_faithful_sdm_step`` (522-535), with the
same shapes and errors; ``decode_sdm_layer_controller`` and its dense twin
are ``_decode_faithful_sdm_layer`` and ``_decode_faithful_sdm_layer_dense``
(538-598).  Kernels: ``cowsdm_controller_prepare`` / ``_finish``
(csrc/controller.hip) and ``cowsdm_product_key_routes`` for the routes.
Float32 only; there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import torch

from . import _native as nat
from .allocator import PackedSDMCopyOnWriteState, dense_sdm_sparse_step, packed_sdm_cow_step
from .inference import SDMStepInputs
from .routing import product_key_routes


@dataclass
class SDMController:
    """One SDM layer's controller weights on the device (float32).

    ``proj_weight_t`` is [width, rows]: the transposed weights of
    read_projection (heads * 2*sqrt(slots) rows), write_projection (the
    same), value_projection (width), forget_projection (heads) and
    input_projection (heads), in that order; ``proj_bias`` their biases.
    ``gate_weight_t`` and ``out_weight_t`` are output_gate's and
    output_projection's weights transposed."""

    width: int
    slots: int
    reads: int
    writes: int
    memory_heads: int
    norm_weight: torch.Tensor
    norm_bias: torch.Tensor
    norm_eps: float
    proj_weight_t: torch.Tensor
    proj_bias: torch.Tensor
    a_log: torch.Tensor
    dt_bias: torch.Tensor
    gate_weight_t: torch.Tensor
    gate_bias: torch.Tensor
    out_weight_t: torch.Tensor
    out_bias: torch.Tensor
    read_norm_weight: torch.Tensor
    read_norm_bias: torch.Tensor
    read_norm_eps: float
    _struct: Any = field(default=None, repr=False, compare=False)

    @property
    def head_width(self) -> int:
        return self.width // self.memory_heads

    @property
    def key_width_per_head(self) -> int:
        return 2 * math.isqrt(self.slots)

    @property
    def device(self) -> torch.device:
        return self.proj_weight_t.device

    # --------------------------------------------------------- creation

    @classmethod
    def from_parts(cls, *, width: int, slots: int, reads: int, writes: int,
                   memory_heads: int, input_norm: tuple, read_projection: tuple,
                   write_projection: tuple, value_projection: tuple,
                   forget_projection: tuple, input_projection: tuple, a_log: torch.Tensor,
                   dt_bias: torch.Tensor, output_gate: tuple, output_projection: tuple,
                   readings_norm: tuple, device=None) -> "SDMController":
        """From the reference module's parameters: each projection as
        (weight [out, in], bias [out]) like ``nn.Linear``, each norm as
        (weight, bias, eps) like ``nn.LayerNorm``."""

        if width <= 0 or slots <= 0 or memory_heads <= 0:
            raise ValueError("width, slots, and memory_heads must be positive")
        if width % memory_heads:
            raise ValueError("width must be divisible by memory_heads")
        root = math.isqrt(slots)
        if root * root != slots:
            raise ValueError("faithful SDM slots must be a perfect square")
        if not 1 <= reads <= slots or not 1 <= writes <= slots:
            raise ValueError("read and write counts must lie within the table")
        device = torch.device(device) if device is not None else read_projection[0].device

        def put(t: torch.Tensor) -> torch.Tensor:
            return t.detach().to(device=device, dtype=torch.float32).contiguous()

        key = memory_heads * 2 * root
        projections = (read_projection, write_projection, value_projection, forget_projection,
                       input_projection)
        outs = (key, key, width, memory_heads, memory_heads)
        for (weight, bias), out in zip(projections, outs):
            if tuple(weight.shape) != (out, width) or tuple(bias.shape) != (out,):
                raise ValueError("controller projection shapes do not match the controller")
        weight = torch.cat([put(w) for w, _ in projections], dim=0)
        bias = torch.cat([put(b) for _, b in projections], dim=0)
        return cls(
            width=width, slots=slots, reads=reads, writes=writes, memory_heads=memory_heads,
            norm_weight=put(input_norm[0]), norm_bias=put(input_norm[1]),
            norm_eps=float(input_norm[2]),
            proj_weight_t=weight.t().contiguous(), proj_bias=bias,
            a_log=put(a_log), dt_bias=put(dt_bias),
            gate_weight_t=put(output_gate[0]).t().contiguous(), gate_bias=put(output_gate[1]),
            out_weight_t=put(output_projection[0]).t().contiguous(),
            out_bias=put(output_projection[1]),
            read_norm_weight=put(readings_norm[0]), read_norm_bias=put(readings_norm[1]),
            read_norm_eps=float(readings_norm[2]))

    @classmethod
    def from_module(cls, module, device=None) -> "SDMController":
        """From a module with the reference ``SparseDeltaMemory``'s
        attributes (sdm.py:1032-1052): ``input_norm``, the ``*_projection``
        linears, ``A_log``, ``dt_bias``, ``output_gate``,
        ``output_projection`` and ``readings_norm``."""

        def linear(m):
            return (m.weight, m.bias)

        def norm(m):
            return (m.weight, m.bias, m.eps)

        return cls.from_parts(
            width=module.width, slots=module.slots, reads=module.reads, writes=module.writes,
            memory_heads=module.memory_heads, input_norm=norm(module.input_norm),
            read_projection=linear(module.read_projection),
            write_projection=linear(module.write_projection),
            value_projection=linear(module.value_projection),
            forget_projection=linear(module.forget_projection),
            input_projection=linear(module.input_projection), a_log=module.A_log,
            dt_bias=module.dt_bias, output_gate=linear(module.output_gate),
            output_projection=linear(module.output_projection),
            readings_norm=norm(module.readings_norm), device=device)

    @classmethod
    def random(cls, width: int, *, slots: int, reads: int, writes: int, memory_heads: int = 1,
               norm_eps: float = 1e-6, seed: int = 0, spread: float = 0.0,
               device="cuda") -> "SDMController":
        """Weights drawn as the reference initialises them (sdm.py:1053-1085:
        truncated normal projections with std width^-0.5, A_log and dt_bias
        from their ranges); ``spread`` > 0 also draws biases and norm
        affines around their initial values (for tests of those terms)."""

        g = torch.Generator().manual_seed(seed)
        std = width ** -0.5
        root = math.isqrt(slots)
        key = memory_heads * 2 * root

        def normal(*shape, scale=std):
            return (torch.randn(*shape, generator=g) * scale).clamp(-3 * scale, 3 * scale)

        def linear(out):
            bias = normal(out, scale=spread) if spread > 0 else torch.zeros(out)
            return (normal(out, width), bias)

        def norm(n, eps):
            if spread > 0:
                return (1.0 + normal(n, scale=spread), normal(n, scale=spread), eps)
            return (torch.ones(n), torch.zeros(n), eps)

        a_log = (torch.rand(memory_heads, generator=g) * 16.0).clamp(min=1e-4).log()
        dt = torch.exp(torch.rand(memory_heads, generator=g) * (math.log(0.1) - math.log(0.001))
                       + math.log(0.001))
        dt_bias = dt + torch.log(-torch.expm1(-dt))
        return cls.from_parts(
            width=width, slots=slots, reads=reads, writes=writes, memory_heads=memory_heads,
            input_norm=norm(width, 1e-5), read_projection=linear(key),
            write_projection=linear(key), value_projection=linear(width),
            forget_projection=linear(memory_heads), input_projection=linear(memory_heads),
            a_log=a_log, dt_bias=dt_bias, output_gate=linear(width),
            output_projection=linear(width), readings_norm=norm(width // memory_heads, norm_eps),
            device=device)

    # ----------------------------------------------------------- native

    def c_struct(self) -> nat.Controller:
        if self._struct is None:
            c = nat.Controller()
            c.width, c.heads, c.slots = self.width, self.memory_heads, self.slots
            for name in ("norm_weight", "norm_bias", "proj_weight_t", "proj_bias", "a_log",
                         "dt_bias", "gate_weight_t", "gate_bias", "out_weight_t", "out_bias",
                         "read_norm_weight", "read_norm_bias"):
                setattr(c, name, getattr(self, name).data_ptr())
            c.norm_eps, c.read_norm_eps = self.norm_eps, self.read_norm_eps
            self._struct = c
        return self._struct


@dataclass
class ControllerStep:
    """One token's controller outputs for one layer (the reference's
    ``_FaithfulSDMStep``, inference.py:279-290): the normalised tokens and
    the step inputs of the layer's B * H banks (bank ``b * H + h``)."""

    normalized: torch.Tensor      # [B, 1, width]
    inputs: SDMStepInputs


def _check_tokens(controller: SDMController, tokens: torch.Tensor) -> int:
    batch = tokens.shape[0]
    if tokens.shape != (batch, 1, controller.width):
        raise ValueError("faithful SDM decode requires one token")
    if tokens.device.type != "cuda" or tokens.device != controller.device:
        raise ValueError("controller tokens must be on the controller's HIP device")
    if tokens.dtype != torch.float32:
        raise TypeError("the HIP controller takes float32 tokens")
    return batch


@torch.no_grad()
def prepare_sdm_step(controller: SDMController, tokens: torch.Tensor) -> ControllerStep:
    """``_prepare_faithful_sdm_step`` (inference.py:459-519): input norm,
    read / write keys, values and gates for one token, then the read and
    write routes (product_key_routes, sdm.py:96-159)."""

    batch = _check_tokens(controller, tokens)
    c = controller
    banks = batch * c.memory_heads
    device = tokens.device
    x = tokens.contiguous()
    normalized = torch.empty(batch, 1, c.width, device=device)
    read_keys = torch.empty(banks, 1, c.key_width_per_head, device=device)
    write_keys = torch.empty_like(read_keys)
    values = torch.empty(banks, c.head_width, device=device)
    input_gate = torch.empty(banks, device=device)
    forget = torch.empty(banks, device=device)
    nat.check(nat.lib().cowsdm_controller_prepare(
        c.c_struct(), x.data_ptr(), batch, normalized.data_ptr(), read_keys.data_ptr(),
        write_keys.data_ptr(), values.data_ptr(), input_gate.data_ptr(), forget.data_ptr(),
        nat.stream_handle(device)), "cowsdm_controller_prepare")
    read_weights, read_indices = product_key_routes(read_keys, slots=c.slots, selected=c.reads)
    write_weights, write_indices = product_key_routes(write_keys, slots=c.slots,
                                                      selected=c.writes)
    return ControllerStep(
        normalized=normalized,
        inputs=SDMStepInputs(write_indices=write_indices[:, 0], write_weights=write_weights[:, 0],
                             values=values, input_gate=input_gate, forget_log_gate=forget,
                             read_indices=read_indices[:, 0], read_weights=read_weights[:, 0]))


@torch.no_grad()
def finish_sdm_step(controller: SDMController, step: ControllerStep,
                    reading: torch.Tensor) -> torch.Tensor:
    """``_finish_faithful_sdm_step`` (inference.py:522-535): the readings
    normalised per head, gated by sigmoid(output_gate(normalized)), through
    the output projection; [B, 1, width]."""

    c = controller
    batch = step.normalized.shape[0]
    if reading.shape != (batch * c.memory_heads, c.head_width):
        raise ValueError("SDM reading does not match batch and controller")
    if reading.dtype != torch.float32 or reading.device != c.device:
        raise ValueError("SDM reading must be float32 on the controller's device")
    out = torch.empty(batch, 1, c.width, device=reading.device)
    r = reading.contiguous()
    nat.check(nat.lib().cowsdm_controller_finish(
        c.c_struct(), step.normalized.data_ptr(), r.data_ptr(), batch, out.data_ptr(),
        nat.stream_handle(reading.device)), "cowsdm_controller_finish")
    return out


@torch.no_grad()
def decode_sdm_layer_controller(controller: SDMController, tokens: torch.Tensor,
                                state: PackedSDMCopyOnWriteState, *,
                                backend: str = "auto") -> torch.Tensor:
    """``_decode_faithful_sdm_layer`` (inference.py:538-566): the controller
    step, the capacity proof when the slab grows, the packed step, the
    controller's finish."""

    step = prepare_sdm_step(controller, tokens)
    if state.banks != tokens.shape[0] * controller.memory_heads:
        raise ValueError("packed SDM banks do not match batch and memory heads")
    if state.growth_quantum_rows:
        state.prepare_step_capacity(state.banks * controller.writes)
    x = step.inputs
    reading, _ = packed_sdm_cow_step(
        state, x.write_indices, x.write_weights, x.values, x.input_gate, x.forget_log_gate,
        x.read_indices, x.read_weights, backend=backend, validate_routes=False,
        collect_diagnostics=False)
    return finish_sdm_step(controller, step, reading)


@torch.no_grad()
def decode_sdm_layer_controller_dense(controller: SDMController, tokens: torch.Tensor,
                                      memory: torch.Tensor, *,
                                      backend: str = "auto") -> torch.Tensor:
    """``_decode_faithful_sdm_layer_dense`` (inference.py:569-598): the same
    controller around the dense-table step."""

    step = prepare_sdm_step(controller, tokens)
    if memory.shape != (tokens.shape[0] * controller.memory_heads, controller.slots,
                        controller.head_width):
        raise ValueError("dense SDM memory does not match batch and controller")
    x = step.inputs
    reading = dense_sdm_sparse_step(
        memory, x.write_indices, x.write_weights, x.values, x.input_gate, x.forget_log_gate,
        x.read_indices, x.read_weights, backend=backend, validate_routes=False)
    return finish_sdm_step(controller, step, reading)


# The reference's names (inference.py:459, 522, 538, 569), taking an
# SDMController built once per layer (SDMController.from_module(module)).
_prepare_faithful_sdm_step = prepare_sdm_step
_finish_faithful_sdm_step = finish_sdm_step
_decode_faithful_sdm_layer = decode_sdm_layer_controller
_decode_faithful_sdm_layer_dense = decode_sdm_layer_controller_dense


class ControllerDecodeGraph:
    """The per-token decode of a stack of SDM layers with the controller on
    the device, captured once as a hipGraph and replayed per token.  A replay
    runs, layer after layer, what ``decode_sdm_layer_controller`` runs
    (``_decode_faithful_sdm_layer``, inference.py:538-566): the controller's
    prepare kernel (input norm, projections, gates), the read and write
    product-key route selections (sdm.py:96-159), the decode loop's capacity
    proof (prepare_step_capacity(B * H * W), allocator.py:745-773) with the
    slab's growth decided on the device, the packed step and the
    controller's finish; each layer's output joins the residual stream
    (``tokens + mixed``, then ``tail(layer, tokens)`` when given, as the
    stack decode's SDM tail).  No host work and no synchronisation per
    token.

    ``reserve_tokens(n)`` gives every slab buffer room to grow for n more
    tokens; a layer whose growth would pass its buffers refuses its step on
    the device, and ``check()`` raises then.  ``sync()`` reads the proof
    counters, capacities and growth counters back into the states before
    they are used eagerly again.  The output tensor ``__call__`` returns is
    rewritten by the next replay.  No counterpart in the reference.
    """

    def __init__(self, controllers: list[SDMController],
                 states: list[PackedSDMCopyOnWriteState], batch: int, *, tail=None):
        from .allocator import DecodeTrace

        if not controllers or len(controllers) != len(states):
            raise ValueError("one packed state per controller")
        c0 = controllers[0]
        if any(c.width != c0.width or c.device != c0.device for c in controllers):
            raise ValueError("the controllers of one stack share its width and device")
        self.controllers = list(controllers)
        self.states = list(states)
        self.batch = batch
        self.tail = tail
        self.device = c0.device
        self.tokens = torch.zeros(batch, 1, c0.width, device=self.device)
        self.output = None
        self.graph = None
        self.layers = []
        for c, st in zip(controllers, states):
            banks = batch * c.memory_heads
            if st.banks != banks or st.width != c.head_width or st.slots != c.slots:
                raise ValueError("packed SDM state does not match batch and controller")
            root = math.isqrt(c.slots)
            reads = min(c.reads, min(c.reads, root) ** 2)
            writes = min(c.writes, min(c.writes, root) ** 2)
            f32 = dict(device=self.device, dtype=torch.float32)
            i64 = dict(device=self.device, dtype=torch.int64)
            buf = {
                "normalized": torch.empty(batch, 1, c.width, **f32),
                "read_keys": torch.empty(banks, 1, c.key_width_per_head, **f32),
                "write_keys": torch.empty(banks, 1, c.key_width_per_head, **f32),
                "values": torch.empty(banks, c.head_width, **f32),
                "input_gate": torch.empty(banks, **f32),
                "forget": torch.empty(banks, **f32),
                "read_weights": torch.empty(banks, 1, reads, **f32),
                "read_indices": torch.empty(banks, 1, reads, **i64),
                "write_weights": torch.empty(banks, 1, writes, **f32),
                "write_indices": torch.empty(banks, 1, writes, **i64),
                "reading": torch.empty(1, banks, c.head_width, **f32),
                "out": torch.empty(batch, 1, c.width, **f32),
                "sum": torch.empty(batch, 1, c.width, **f32),
            }
            trace = DecodeTrace(
                states=[st], repeat=True, max_steps_per_launch=1, outputs=buf["reading"],
                write_indices=buf["write_indices"].view(1, 1, banks, writes),
                write_weights=buf["write_weights"].view(1, 1, banks, writes),
                values=buf["values"].view(1, 1, banks, c.head_width),
                input_gate=buf["input_gate"].view(1, 1, banks),
                forget_log_gate=buf["forget"].view(1, 1, banks),
                read_indices=buf["read_indices"].view(1, 1, banks, reads),
                read_weights=buf["read_weights"].view(1, 1, banks, reads))
            self.layers.append((c, buf, trace))

    def reserve_tokens(self, tokens: int) -> None:
        """Room in every slab's buffers for ``tokens`` more tokens of growth."""

        for _, _, trace in self.layers:
            trace.reserve_steps(tokens)

    @staticmethod
    def _prepare_args(c, buf) -> tuple:
        return (buf["normalized"].data_ptr(), buf["read_keys"].data_ptr(),
                buf["write_keys"].data_ptr(), buf["values"].data_ptr(),
                buf["input_gate"].data_ptr(), buf["forget"].data_ptr(), c.reads, c.writes,
                buf["read_weights"].data_ptr(), buf["read_indices"].data_ptr(),
                buf["write_weights"].data_ptr(), buf["write_indices"].data_ptr())

    def _record(self, stream: int, structs) -> torch.Tensor:
        """Per layer: prepare with the routes, the step, finish with the
        residual add.  Without a tail between layers a layer's finish and the
        next layer's prepare are one call (one launch at sqrt(N) <= 64)."""

        lib = nat.lib()
        x = self.tokens.contiguous()
        c0, buf0, _ = self.layers[0]
        nat.check(lib.cowsdm_controller_prepare_routes(
            c0.c_struct(), x.data_ptr(), self.batch, *self._prepare_args(c0, buf0), stream),
            "cowsdm_controller_prepare_routes")
        last = len(self.layers) - 1
        for index, ((c, buf, trace), layer) in enumerate(zip(self.layers, structs)):
            trace.launch(1, layer)
            finish = (c.c_struct(), buf["normalized"].data_ptr(), buf["reading"].data_ptr(),
                      self.batch, buf["out"].data_ptr(), x.data_ptr(), buf["sum"].data_ptr())
            if index < last and self.tail is None:
                cn, bufn, _ = self.layers[index + 1]
                nat.check(lib.cowsdm_controller_finish_prepare_routes(
                    *finish, cn.c_struct(), *self._prepare_args(cn, bufn), stream),
                    "cowsdm_controller_finish_prepare_routes")
                x = buf["sum"]
                continue
            nat.check(lib.cowsdm_controller_finish_residual(*finish, stream),
                      "cowsdm_controller_finish_residual")
            x = buf["sum"]
            if self.tail is not None:
                x = self.tail(index, x).contiguous()
            if index < last:
                cn, bufn, _ = self.layers[index + 1]
                nat.check(lib.cowsdm_controller_prepare_routes(
                    cn.c_struct(), x.data_ptr(), self.batch, *self._prepare_args(cn, bufn),
                    stream), "cowsdm_controller_prepare_routes")
        return x

    def capture(self) -> "torch.cuda.CUDAGraph":
        """Record the per-token decode of every layer (the control words are
        uploaded from the states first)."""

        structs = []
        for _, _, trace in self.layers:
            structs.append(trace.layer_array())
            if not trace.planned:
                raise RuntimeError("packed state needs the planned one-step kernel (W <= 4, "
                                   "R <= 16, D <= 256, banks <= 256) to prove on the device")
            trace.upload()
            trace.status.zero_()
            trace.set_step(0)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=torch.cuda.Stream(self.device)):
            self.output = self._record(nat.stream_handle(self.device), structs)
        for _, _, trace in self.layers:
            trace._positions = None
        self.graph = graph
        return graph

    @torch.no_grad()
    def __call__(self, tokens: torch.Tensor) -> torch.Tensor:
        """One token [B, 1, width] through every layer: its input copied into
        the graph's buffer, one replay."""

        if self.graph is None:
            self.capture()
        self.tokens.copy_(tokens)
        self.graph.replay()
        return self.output

    def sync(self) -> None:
        """Read the device's proof counters, capacities and growth back into
        the states."""

        for _, _, trace in self.layers:
            trace.sync()

    def check(self) -> None:
        """Raise when a replay refused a layer's step (its growth would pass
        the slab's buffers) or stopped on a fault."""

        for index, (_, _, trace) in enumerate(self.layers):
            status = int(trace.status[0])
            if status:
                raise RuntimeError(f"captured decode layer {index} stopped with status "
                                   f"{status:#x} (reserve_tokens before capturing)")
