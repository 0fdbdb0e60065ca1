"""Host bookkeeping of FaithfulSDMDecodeState (inference.py:26-231 of the
reference) on the CPU, with stub layer states that record the bank lists
they are given: which banks each lifecycle call names and in what order,
the validation errors and their messages, and the decode positions after
compact and admit.  The GPU layer states themselves are covered by
tests/test_gpu_lifecycle.py."""

from __future__ import annotations

import pytest
import torch

from copy_on_write_sdm_amd.inference import FaithfulSDMDecodeState


class StubLayer:
    """Records the bank lists of state calls; each bank holds `rows` rows."""

    def __init__(self, banks: int, rows: int = 3):
        self.banks = banks
        self.rows = rows
        self.calls = []

    def release(self, banks):
        self.calls.append(("release", banks.tolist()))
        return torch.tensor(self.rows * banks.numel())

    def retain_banks(self, banks):
        self.calls.append(("retain", banks.tolist()))
        self.banks = banks.numel()

    def append_banks_from(self, other):
        self.calls.append(("append", other.banks))
        self.banks += other.banks
        return other.banks * other.rows

    def trim_capacity(self, *, headroom_rows=0):
        self.calls.append(("trim", headroom_rows))
        return 5


def serving(batch, heads=(1, 2), position=7, positions=None, layout="BB"):
    return FaithfulSDMDecodeState(
        layout=layout, position=position, capacity=64, activation_dtype=torch.float32,
        active_sequences=torch.ones(batch, dtype=torch.bool),
        sdm_layer_positions=tuple(range(len(heads))),
        sdm_states=tuple(StubLayer(batch * h) for h in heads),
        positions=None if positions is None else torch.tensor(positions))


def test_release_names_banks_request_major_in_the_given_order():
    s = serving(4)
    assert s.release([2, 0]) == 3 * 2 + 3 * 4
    assert s.sdm_states[0].calls == [("release", [2, 0])]
    assert s.sdm_states[1].calls == [("release", [4, 5, 0, 1])]
    assert s.active_sequences.tolist() == [False, True, False, True]
    # a tensor argument works too, and None releases every live request
    assert s.release(torch.tensor([3])) == 3 * 1 + 3 * 2
    assert s.release() == 3 * 1 + 3 * 2
    assert s.active_sequences.tolist() == [False] * 4
    assert s.release() == 0                      # nothing left to release
    assert s.release([]) == 0


@pytest.mark.parametrize("bad", [[1, 1], [4], [-1], [[0, 1]]])
def test_release_rejects_invalid_requests(bad):
    s = serving(4)
    message = ("released sequence indices must be a vector" if isinstance(bad[0], list)
               else "released sequence is invalid, duplicated, or inactive")
    with pytest.raises(ValueError, match=message):
        s.release(bad)
    assert s.active_sequences.tolist() == [True] * 4
    assert all(not layer.calls for layer in s.sdm_states)


def test_release_rejects_an_inactive_request():
    s = serving(3)
    s.release([1])
    with pytest.raises(ValueError, match="invalid, duplicated, or inactive"):
        s.release([1])


def test_compact_keeps_survivors_in_order_and_the_shared_position():
    s = serving(4, position=9)
    s.release([0, 2])
    kept = s.compact()
    assert kept.tolist() == [1, 3]
    assert s.sdm_states[1].calls[-1] == ("retain", [2, 3, 6, 7])
    assert s.batch == 2 and s.active_sequences.tolist() == [True, True]
    assert (s.position, s.positions) == (9, None)
    s.release()
    s.compact()
    assert (s.batch, s.position, s.positions) == (0, 0, None)
    # an empty batch whose layers still hold banks is inconsistent
    s.sdm_states[0].banks = 2
    with pytest.raises(AssertionError, match="empty serving batch retained SDM banks"):
        s.compact()


def test_compact_with_per_request_positions():
    s = serving(3, positions=[5, 11, 8])
    s.release([1])
    s.compact()
    assert s.positions.tolist() == [5, 8]
    assert s.position == 8


def test_banks_must_divide_by_batch():
    s = serving(4)
    s.sdm_states[0].banks = 6
    with pytest.raises(AssertionError, match="do not divide by batch"):
        s.release([0])


def test_admit_merges_positions():
    s, t = serving(2, position=18), serving(2, position=128)
    assert s.admit(t) == 2
    assert s.current_positions().tolist() == [18, 18, 128, 128]
    assert s.position == 128 and s.batch == 4
    assert s.sdm_states[1].calls[-1] == ("append", 4)
    # equal positions collapse to one shared position
    a, b = serving(1, position=3), serving(2, position=3)
    a.admit(b)
    assert (a.position, a.positions, a.batch) == (3, None, 3)


def test_admit_compacts_both_sides_first():
    s, t = serving(3, position=4), serving(3, position=4)
    s.release([1])
    t.release([0, 2])
    assert s.admit(t) == 1
    assert s.batch == 3
    assert t.batch == 1


def test_admit_rejects_incompatible_state():
    s, t = serving(2), serving(2, layout="BA")
    with pytest.raises(ValueError, match="admitted faithful-SDM state is incompatible"):
        s.admit(t)


def test_release_and_compact_trims_on_request():
    s = serving(2)
    assert s.release_and_compact([0], trim=True, trim_headroom_rows=4) == 3 + 6
    assert s.sdm_states[0].calls[-1] == ("trim", 4)
    assert s.trim_sdm_pools() == 10
