"""Host-side checks of the prefill and recurrence entry points (recurrence.py,
prefill.py) that run before any device work, and the dense K/V cache
allocation (inference.py:293-306), on the CPU."""

from __future__ import annotations

import pytest
import torch

import copy_on_write_sdm_amd as cow


def _recurrence_inputs(batch=2, time=3, slots=16, width=8):
    return dict(initial_memory=torch.zeros(batch, slots, width),
                write_routes=torch.zeros(batch, time, slots), values=torch.zeros(batch, time, width),
                input_gate=torch.zeros(batch, time), erase_gate=torch.zeros(batch, time),
                forget_log_gate=torch.zeros(batch, time), read_routes=torch.zeros(batch, time, slots))


def test_recurrence_checks_follow_the_reference():
    x = _recurrence_inputs()
    with pytest.raises(ValueError, match="do not align"):
        cow.sdm_recurrence(**{**x, "read_routes": torch.zeros(2, 3, 15)})
    with pytest.raises(ValueError, match="do not align"):
        cow.sdm_recurrence(**{**x, "forget_log_gate": torch.zeros(2, 4)})
    with pytest.raises(ValueError, match="do not align"):
        cow.sdm_recurrence(**{**x, "initial_memory": torch.zeros(2, 16, 8, dtype=torch.int32)})
    with pytest.raises(ValueError, match="must be contiguous"):
        cow.sdm_recurrence(**{**x, "values": torch.zeros(3, 2, 8).transpose(0, 1)})
    with pytest.raises(ValueError, match="at most 1,024 slots"):
        cow.sdm_recurrence(**_recurrence_inputs(slots=1025))
    # a valid call off the GPU fails loudly: there is no CPU path
    with pytest.raises(RuntimeError, match="no CPU path"):
        cow.sdm_recurrence(**x)
    with pytest.raises(RuntimeError, match="no CPU path"):
        cow.gated_delta_recurrence(x["initial_memory"], x["write_routes"], x["values"],
                                   x["input_gate"], x["forget_log_gate"], x["read_routes"])


def test_dense_routes_checks():
    with pytest.raises(ValueError, match="must align"):
        cow.dense_sparse_routes(torch.zeros(2, 4), torch.zeros(2, 3, dtype=torch.int64), 16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        cow.dense_sparse_routes(torch.zeros(2, 4), torch.zeros(2, 4, dtype=torch.int64), 16)


def test_dense_cache_allocation():
    key = torch.arange(2 * 3 * 4 * 5, dtype=torch.float32).reshape(2, 3, 4, 5)
    value = -key
    k, v = cow.allocate_dense_cache(key, value, 7)
    assert k.shape == v.shape == (2, 3, 7, 5)
    assert torch.equal(k[:, :, :4], key) and torch.equal(v[:, :, :4], value)
    with pytest.raises(ValueError, match="capacity is invalid"):
        cow.allocate_dense_cache(key, value, 3)
    with pytest.raises(ValueError, match="capacity is invalid"):
        cow.allocate_dense_cache(key, value[:, :2], 7)


def test_stack_prefill_checks_before_device_work():
    tokens = torch.zeros(2, 4, 8)
    with pytest.raises(ValueError, match="shorter than the prefix"):
        cow.prefill_faithful_sdm_stack("B", [(None, None)], tokens, capacity=3)
    with pytest.raises(ValueError, match="at least one token"):
        cow.prefill_faithful_sdm_stack("B", [(None, None)], torch.zeros(2, 0, 8))
    with pytest.raises(ValueError, match="quantum cannot be negative"):
        cow.prefill_faithful_sdm_stack("B", [(None, None)], tokens, sdm_growth_quantum_rows=-1)
    with pytest.raises(ValueError, match="per B layer"):
        cow.prefill_faithful_sdm_stack("BB", [(None, None)], tokens)
    with pytest.raises(ValueError, match="one value per B layer"):
        cow.prefill_faithful_sdm_stack("B", [(None, None)], tokens, sdm_capacity_rows=[1, 2])
    with pytest.raises(ValueError, match="A .attention. and B"):
        cow.prefill_faithful_sdm_stack("BC", [(None, None)], tokens)
    with pytest.raises(ValueError, match="attention_block"):
        cow.prefill_faithful_sdm_stack("AB", [(None, None)], tokens)
