"""The SDM recurrence over dense route vectors, on the device: the forward
recurrence the reference runs for training and prefill
(copy_on_write_sdm/sdm.py:534-607, ``_native_sdm_forward_kernel``, as
``_NativeSDMRecurrence.forward`` launches it at sdm.py:779-861, and
``gated_delta_recurrence``, sdm.py:962-995), and ``dense_sparse_routes``
(sdm.py:162-172), which scatters product-key routes into the dense vectors
the recurrence takes.

Kernels: ``cowsdm_recurrence_forward`` and ``cowsdm_dense_routes``
(csrc/recurrence.hip).  Float32 only; there is no CPU path (the reference
falls back to its serial torch loop off CUDA, this module raises).

The prefill handoff uses the recurrence's final memory: ``pack_prefill_layer``
(inference.py) packs it into copy-on-write state.
"""

from __future__ import annotations

import torch

from . import _native as nat

MAX_SLOTS = 1_024


def _device_tensor(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be on the GPU: the recurrence has no CPU path")


@torch.no_grad()
def dense_sparse_routes(weights: torch.Tensor, indices: torch.Tensor,
                        slots: int) -> torch.Tensor:
    """sdm.py:162-172: route weights [..., K] at their indices [..., K] in
    dense vectors [..., slots] (zero elsewhere; for a repeated index the
    last weight wins).  Raises ValueError for an index outside [0, slots)
    (this reads one device word back)."""

    if weights.shape != indices.shape:
        raise ValueError("route weights and indices must align")
    if slots <= 0:
        raise ValueError("slots must be positive")
    _device_tensor(weights, "route weights")
    if weights.dtype != torch.float32:
        raise TypeError("route weights must be float32")
    if indices.dtype not in (torch.int32, torch.int64):
        raise TypeError("route indices must be int32 or int64")
    if indices.device != weights.device:
        raise ValueError("route weights and indices must be on one device")
    device = weights.device
    per_row = weights.shape[-1] if weights.ndim else 1
    if per_row == 0:
        # no routes in a row: every slot of its dense vector stays zero, as
        # the reference's scatter into zeros leaves it
        return torch.zeros(*weights.shape[:-1], slots, device=device, dtype=torch.float32)
    rows = weights.numel() // per_row
    out = torch.empty(*weights.shape[:-1], slots, device=device, dtype=torch.float32)
    if out.numel() == 0:
        return out
    w = weights.contiguous()
    i = indices.contiguous()
    bad = torch.zeros(1, dtype=torch.int32, device=device)
    code = nat.INDEX_INT32 if i.dtype == torch.int32 else nat.INDEX_INT64
    nat.check(nat.lib().cowsdm_dense_routes(
        w.data_ptr(), i.data_ptr(), code, rows, per_row, slots, out.data_ptr(), bad.data_ptr(),
        nat.stream_handle(device)), "cowsdm_dense_routes")
    if int(bad.item()):
        raise ValueError("route index outside [0, slots)")
    return out


@torch.no_grad()
def sdm_recurrence(initial_memory: torch.Tensor, write_routes: torch.Tensor,
                   values: torch.Tensor, input_gate: torch.Tensor, erase_gate: torch.Tensor,
                   forget_log_gate: torch.Tensor, read_routes: torch.Tensor, *,
                   return_states: bool = False):
    """``_NativeSDMRecurrence.forward`` (sdm.py:779-861): initial memory
    [B, N, D], dense write and read routes [B, T, N], values [B, T, D],
    gates [B, T].  Returns (readings [B, T, D], final memory [B, N, D]), and
    with ``return_states`` the per-token memories [B, T, N, D] as well (the
    tensor the reference keeps for its backward pass)."""

    tensors = (initial_memory, write_routes, values, input_gate, erase_gate, forget_log_gate,
               read_routes)
    if initial_memory.ndim != 3 or values.ndim != 3:
        raise ValueError("optimized SDM recurrence inputs do not align")
    batch, slots, width = initial_memory.shape
    time = values.shape[1]
    gate_shape = (batch, time)
    if (initial_memory.dtype not in (torch.float16, torch.bfloat16, torch.float32)
            or write_routes.shape != (batch, time, slots)
            or read_routes.shape != (batch, time, slots)
            or values.shape != (batch, time, width)
            or input_gate.shape != gate_shape
            or erase_gate.shape != gate_shape
            or forget_log_gate.shape != gate_shape):
        raise ValueError("optimized SDM recurrence inputs do not align")
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError("optimized SDM recurrence inputs must be contiguous")
    if slots > MAX_SLOTS:
        raise ValueError("dense SDM training recurrence supports at most 1,024 slots")
    for t in tensors:
        _device_tensor(t, "SDM recurrence inputs")
        if t.dtype != torch.float32:
            raise TypeError("the device recurrence computes in float32: pass float32 inputs")
        if t.device != values.device:
            raise ValueError("SDM recurrence inputs must be on one device")
    device = values.device
    readings = torch.empty_like(values)
    final = torch.empty(batch, slots, width, device=device, dtype=torch.float32)
    states = (torch.empty(batch, time, slots, width, device=device, dtype=torch.float32)
              if return_states else None)
    r = nat.Recurrence()
    r.batch, r.time, r.slots, r.width = batch, time, slots, width
    r.initial_memory = initial_memory.data_ptr()
    r.write_routes = write_routes.data_ptr()
    r.values = values.data_ptr()
    r.input_gate = input_gate.data_ptr()
    r.erase_gate = erase_gate.data_ptr()
    r.forget_log_gate = forget_log_gate.data_ptr()
    r.read_routes = read_routes.data_ptr()
    r.readings = readings.data_ptr()
    r.states = states.data_ptr() if states is not None else None
    r.final_memory = final.data_ptr()
    nat.check(nat.lib().cowsdm_recurrence_forward(r, nat.stream_handle(device)),
              "cowsdm_recurrence_forward")
    if return_states:
        return readings, final, states
    return readings, final


def gated_delta_recurrence(initial_memory: torch.Tensor, write_routes: torch.Tensor,
                           values: torch.Tensor, input_gate: torch.Tensor,
                           forget_log_gate: torch.Tensor, read_routes: torch.Tensor, *,
                           erase_gate: torch.Tensor | None = None):
    """sdm.py:962-995: the recurrence with the erase gate defaulting to the
    input gate, on contiguous copies; (readings, final memory)."""

    if erase_gate is None:
        erase_gate = input_gate
    return sdm_recurrence(initial_memory.contiguous(), write_routes.contiguous(),
                          values.contiguous(), input_gate.contiguous(),
                          erase_gate.contiguous(), forget_log_gate.contiguous(),
                          read_routes.contiguous())
