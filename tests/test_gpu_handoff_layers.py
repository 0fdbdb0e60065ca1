"""The batched handoff (from_dense_overlay_layers, pack_prefill_layers)
equals the reference's layer-by-layer handoff (from_dense_overlay,
allocator.py:587-689; _pack_prefill_layer, inference.py:314-366) bit for
bit, per-layer capacities included, and raises its errors."""

from __future__ import annotations

import pytest
import torch

import copy_on_write_sdm_amd as cow
from copy_on_write_sdm_amd import synthetic
from gpu_helpers import assert_states_identical

pytestmark = pytest.mark.gpu


def _layers(device, layers=3, banks=6, slots=64, width=32, seed=5):
    g = torch.Generator().manual_seed(seed)
    m0 = [(torch.randn(1, slots, width, generator=g) * 0.1).to(device) for _ in range(layers)]
    dense = [(torch.randn(banks, slots, width, generator=g)).to(device) for _ in range(layers)]
    masks = [(torch.rand(banks, slots, generator=g) < 0.3 + 0.1 * l).to(device)
             for l in range(layers)]
    return m0, dense, masks


@pytest.mark.parametrize("capacity", [None, [512, 600, 700]])
def test_batched_handoff_equals_per_layer(device, capacity):
    m0, dense, masks = _layers(device)
    tmpl = torch.zeros(6, dtype=torch.int64, device=device)
    kw = dict(template_indices=tmpl, growth_quantum_rows=16)
    got = cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
        m0, dense, masks, capacity_rows=capacity, **kw)
    for l, st in enumerate(got):
        want = cow.PackedSDMCopyOnWriteState.from_dense_overlay(
            m0[l], dense[l], masks[l], capacity_rows=None if capacity is None else capacity[l],
            **kw)
        assert_states_identical(st, want)
        assert torch.equal(st.materialize_dense(), want.materialize_dense())
        assert st.proven_maximum_additional_allocations == \
            want.proven_maximum_additional_allocations


def test_batched_handoff_errors(device):
    m0, dense, masks = _layers(device)
    tmpl = torch.zeros(6, dtype=torch.int64, device=device)
    with pytest.raises(ValueError, match="smaller than the prefill working set"):
        cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
            m0, dense, masks, template_indices=tmpl, capacity_rows=[512, 8, 700])
    with pytest.raises(ValueError, match="one value per layer"):
        cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
            m0, dense, masks, template_indices=tmpl, capacity_rows=[512, 600])
    with pytest.raises(ValueError, match="do not align"):
        cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
            m0, dense, [masks[0], masks[1][:, :32], masks[2]], template_indices=tmpl)
    with pytest.raises(ValueError, match="template index lies outside"):
        cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
            m0, dense, masks, template_indices=tmpl + 1)


def test_pack_prefill_layers_equals_per_layer(device):
    layers, batch, time, heads, slots, width = 3, 4, 9, 2, 64, 16
    g = torch.Generator().manual_seed(8)
    m0 = [(torch.randn(heads, slots, width, generator=g) * 0.1).to(device) for _ in range(layers)]
    finals = [torch.randn(batch, heads, slots, width, generator=g).to(device)
              for _ in range(layers)]
    routes = [torch.stack([torch.stack([torch.randperm(slots, generator=g)[:4]
                                        for _ in range(heads)]) for _ in range(batch * time)])
              .reshape(batch, time, heads, 4).to(device) for _ in range(layers)]
    kw = dict(decode_capacity=time + 6, growth_quantum_rows=0)
    got = cow.pack_prefill_layers(m0, finals, routes, capacity_rows=None, **kw)
    for l in range(layers):
        want = cow.pack_prefill_layer(m0[l], finals[l], routes[l], capacity_rows=None, **kw)
        assert_states_identical(got[l], want)
        assert got[l].capacity_is_proven and want.capacity_is_proven
