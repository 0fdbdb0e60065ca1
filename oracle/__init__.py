"""CPU oracle for the copy-on-write SDM decode step -- TEST INFRASTRUCTURE.

Nothing in the product (the ``copy_on_write_sdm_amd`` package and its HIP
library) imports, links or calls anything here.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use these
modules, and only as the checker or as the timed CPU baseline.

Modules:

* ``oracle.state``  -- numpy restatement of the reference's packed state,
  its lifecycle operations and the packed / dense sparse steps
  (copy_on_write_sdm/allocator.py:476-1095, 1466-1525, 1612-1633).  Float
  math is float32 in the reference's operation order with sums taken
  sequentially; exp(forget_log_gate) is evaluated in float64 and rounded once.
* ``oracle.serial`` -- float64 restatements of the token-serial recurrences
  (copy_on_write_sdm/sdm.py:365-461 and 464-529) and a pure-Python loop form
  of one SDM step for tiny inputs: independent formulations used to pin
  ``oracle.state``.
* ``oracle.torch_port`` -- torch CPU restatement of the reference's torch
  branches (allocator.py:1466-1525, 1612-1633) with torch's own reductions
  and float32 exp: a second restatement for cross-checking, and the CPU
  dense-table baseline timed by bench.py.

Every function of ``oracle.state`` is pinned by at least one check that does
not restate its formula (see tests/test_oracle_pins.py): the reference's own
known answers (tests/test_allocator.py:65-99), the independent serial
recurrences, closed forms, allocator invariants and planted-mistake tests.
"""
