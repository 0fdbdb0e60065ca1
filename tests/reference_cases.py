"""Inputs of the reference's own allocator tests, regenerated locally.

copy_on_write_sdm's tests/test_allocator.py:14-63 seeds torch with 11, draws
M0 = randn(1, 16, 8) for 3 banks and, per step, write weights, values, gates
and read weights in a fixed order with fixed read indices.  The draws below
repeat that order with torch's CPU generator so the same inputs (and the
reference's known answers, tests/test_allocator.py:65-99) apply.
"""

from __future__ import annotations

import torch

BANKS = 3
SLOTS = 16
WIDTH = 8
READ_INDICES = [[0, 1, 2, 3], [3, 4, 5, 6], [6, 7, 8, 9]]
WRITE_INDICES = [[2, 5], [1, 7], [4, 10]]

# Known answers asserted by tests/test_allocator.py:69-70, 75-76, 77-82, 95-97.
FIRST_STEP_FIRST_TOUCHES = 6
FIRST_STEP_ALLOCATED = 6
REPEAT_STEP_FIRST_TOUCHES = 0
REPEAT_STEP_ALLOCATED = 6
UNTOUCHED_PROBE = (0, 15)
GROWTH_CAPACITY_AFTER = 8
GROWTH_ROWS_ADDED = 4
GROWTH_ROWS_COPIED = 4


def reference_case(steps: int = 2):
    """(initial [1,16,8], list of per-step input dicts) in the reference
    test's draw order; every step writes WRITE_INDICES."""

    torch.manual_seed(11)
    initial = torch.randn(1, SLOTS, WIDTH)
    out = []
    for _ in range(steps):
        write_indices = torch.tensor(WRITE_INDICES, dtype=torch.int64)
        writes = write_indices.shape[1]
        write_weights = torch.softmax(torch.randn(BANKS, writes), dim=-1)
        values = torch.randn(BANKS, WIDTH)
        input_gate = torch.sigmoid(torch.randn(BANKS))
        forget_log_gate = -torch.rand(BANKS)
        read_indices = torch.tensor(READ_INDICES, dtype=torch.int64)
        read_weights = torch.softmax(torch.randn(BANKS, 4), dim=-1)
        out.append({
            "write_indices": write_indices,
            "write_weights": write_weights,
            "values": values,
            "input_gate": input_gate,
            "forget_log_gate": forget_log_gate,
            "read_indices": read_indices,
            "read_weights": read_weights,
        })
    return initial, out
