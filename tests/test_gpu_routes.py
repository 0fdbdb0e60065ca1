"""GPU parity of product_key_routes (csrc/routes.hip) against oracle/routes.py.

Indices must match exactly; weights within rtol 2e-6, atol 1e-7 (the kernel
sums the softmax in a wave tree with expf, the oracle in float64)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import copy_on_write_sdm_amd as cow
from oracle import routes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _check(projected: np.ndarray, slots: int, selected: int) -> None:
    print(f"routes {projected.shape} N={slots} k={selected}", flush=True)
    w, i = cow.product_key_routes(torch.from_numpy(projected).to(DEV), slots=slots,
                                  selected=selected)
    ew, ei = routes.product_key_routes(projected, slots, selected)
    assert i.dtype == torch.int64 and w.dtype == torch.float32
    np.testing.assert_array_equal(i.cpu().numpy(), ei)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("slots,selected,batch,steps", [
    (256, 16, 64, 1), (256, 4, 64, 1), (256, 16, 256, 1), (65536, 16, 256, 1),
    (65536, 4, 64, 3), (16, 16, 5, 2), (16, 1, 7, 1), (4, 2, 9, 1), (1, 1, 3, 1),
    (1024, 32, 33, 1), (4096, 32, 17, 2), (1 << 20, 32, 8, 1), (1 << 20, 16, 5, 1)])
def test_routes_match_oracle(slots, selected, batch, steps):
    rng = np.random.default_rng(slots * 31 + selected)
    root = int(np.sqrt(slots))
    _check(rng.standard_normal((batch, steps, 2 * root), dtype=np.float32), slots, selected)


@pytest.mark.parametrize("slots,selected", [(256, 16), (4096, 32), (16, 16), (65536, 16),
                                            (1 << 20, 32)])
def test_routes_with_many_equal_scores(slots, selected):
    rng = np.random.default_rng(selected)
    root = int(np.sqrt(slots))
    projected = rng.integers(0, 3, size=(40, 1, 2 * root)).astype(np.float32)
    _check(projected, slots, selected)


@pytest.mark.parametrize("slots,selected", [(65536, 32), (1 << 20, 16)])
def test_routes_first_stage_fallback(slots, selected):
    # entries e sit in lane e % 64; giving the first `selected` lanes every
    # large score leaves selected * sqrt(N) / 64 > 64 entries above the
    # selected-th lane maximum, so the first stage ranks every entry
    rng = np.random.default_rng(5)
    root = int(np.sqrt(slots))
    projected = rng.standard_normal((12, 1, 2 * root), dtype=np.float32)
    lanes = np.arange(2 * root) % root % 64
    projected[..., lanes < selected] += 100.0
    assert selected * (root // 64) > 64
    _check(projected, slots, selected)


def test_routes_empty_batch_and_errors():
    w, i = cow.product_key_routes(torch.zeros((0, 1, 32), device=DEV), slots=256, selected=16)
    assert w.shape == (0, 1, 16) and i.shape == (0, 1, 16)
    with pytest.raises(ValueError, match="do not match"):
        cow.product_key_routes(torch.zeros((2, 1, 30), device=DEV), slots=256, selected=16)
    with pytest.raises(RuntimeError, match="<= 32"):
        cow.product_key_routes(torch.zeros((2, 1, 128), device=DEV), slots=4096, selected=64)


def test_routes_feed_the_packed_step():
    # routes of both kinds drive a decode step exactly as in inference.py:479-512
    rng = np.random.default_rng(11)
    banks, slots, width = 8, 256, 128
    reads = rng.standard_normal((banks, 1, 32), dtype=np.float32)
    writes = rng.standard_normal((banks, 1, 32), dtype=np.float32)
    rw, ri = cow.product_key_routes(torch.from_numpy(reads).to(DEV), slots=slots, selected=16)
    ww, wi = cow.product_key_routes(torch.from_numpy(writes).to(DEV), slots=slots, selected=4)
    m0 = torch.from_numpy(rng.standard_normal((1, slots, width), dtype=np.float32)).to(DEV)
    state = cow.PackedSDMCopyOnWriteState.allocate(m0, banks=banks, capacity_rows=banks * slots)
    gate = torch.full((banks,), 0.5, device=DEV)
    values = torch.from_numpy(rng.standard_normal((banks, width), dtype=np.float32)).to(DEV)
    reading, _ = cow.packed_sdm_cow_step(
        state, write_indices=wi[:, 0], write_weights=ww[:, 0], values=values, input_gate=gate,
        forget_log_gate=-gate, read_indices=ri[:, 0], read_weights=rw[:, 0])
    from oracle import state as ref
    o = ref.allocate(m0.cpu().numpy(), banks=banks, capacity_rows=banks * slots)
    expected, _ = ref.packed_step(
        o, write_indices=wi[:, 0].cpu().numpy(), write_weights=ww[:, 0].cpu().numpy(),
        values=values.cpu().numpy(), input_gate=gate.cpu().numpy(),
        forget_log_gate=-gate.cpu().numpy(), read_indices=ri[:, 0].cpu().numpy(),
        read_weights=rw[:, 0].cpu().numpy())
    np.testing.assert_array_equal(reading.cpu().numpy(), expected)
