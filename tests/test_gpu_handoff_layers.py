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


def test_single_layer_entry_points_equal_batched(device):
    """The per-layer C entry points (cowsdm_count_active + cowsdm_pack_overlay
    after cowsdm_init_state), kept for C callers, leave the state the batched
    handoff leaves."""

    from copy_on_write_sdm_amd import _native as nat

    m0, dense, masks = _layers(device, layers=1, banks=6, slots=64, width=32, seed=9)
    tmpl = torch.zeros(6, dtype=torch.int64, device=device)
    got = cow.PackedSDMCopyOnWriteState.from_dense_overlay_layers(
        m0, dense, masks, template_indices=tmpl, capacity_rows=[300])[0]
    lib = nat.lib()
    stream = nat.stream_handle(device)
    banks, slots, width = dense[0].shape
    workspace = torch.empty(int(lib.cowsdm_workspace_bytes(banks * slots, 300)),
                            dtype=torch.uint8, device=device)
    total = torch.empty(1, dtype=torch.int64, device=device)
    state, result = cow.PackedSDMCopyOnWriteState._allocate_state(
        m0[0], banks=banks, capacity_rows=300, template_indices=tmpl)
    mask = masks[0].contiguous()
    nat.check(lib.cowsdm_count_active(None, banks, slots, None, banks, mask.data_ptr(),
                                      workspace.data_ptr(), total.data_ptr(), stream),
              "cowsdm_count_active")
    nat.check(lib.cowsdm_pack_overlay(dense[0].data_ptr(), mask.data_ptr(), banks, slots, width,
                                      state.logical_to_physical.data_ptr(),
                                      state.values.data_ptr(), state.free_rows.data_ptr(), 300,
                                      state.free_count.data_ptr(), workspace.data_ptr(), stream),
              "cowsdm_pack_overlay")
    torch.cuda.synchronize()
    assert int(total.item()) == int(mask.sum())
    assert int(result.item()) == 0
    live = int(total.item())
    assert torch.equal(state.logical_to_physical, got.logical_to_physical)
    assert torch.equal(state.values[:live], got.values[:live])
    assert torch.equal(state.free_rows, got.free_rows)
    assert int(state.free_count.item()) == int(got.free_count.item()) == 300 - live
