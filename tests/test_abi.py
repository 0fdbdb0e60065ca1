"""The C-ABI library loads and exports every symbol include/cowsdm.h
declares (CPU only: no kernel is launched)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from copy_on_write_sdm_amd import _native as nat

HEADER = Path(__file__).resolve().parent.parent / "include" / "cowsdm.h"


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int32_t|int64_t|const char\*)\s+(cowsdm_\w+)\s*\(",
                                 text, flags=re.M)))


def test_library_is_built():
    assert nat.LIBRARY.exists(), "run __graft_entry__.build() first"


def test_exports_every_header_symbol():
    lib = ctypes.CDLL(str(nat.LIBRARY))
    names = header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_header():
    assert sorted(nat.SIGNATURES) == header_functions()


def test_info_entry_points():
    lib = nat.lib()
    assert lib.cowsdm_abi_version() == nat.ABI_VERSION == 12
    # epoch and header, plan words [banks][steps], step and running totals,
    # at most banks * W pops per step and 4 words per growth segment, int64 each
    assert lib.cowsdm_trace_scan_words(64, 4, 512) == (16 + 64 * 512 + 512 + 513 + 64 * 512 * 4
                                                       + 4 * 513 + 6 * 64)
    assert lib.cowsdm_trace_scan_words(-1, 4, 512) == -1
    assert lib.cowsdm_step_scratch_words(64) == 8 + 64
    assert lib.cowsdm_step_scratch_words(-1) == -1
    assert lib.cowsdm_workspace_bytes(0, 0) == 256
    assert lib.cowsdm_workspace_bytes(4096, 100) > 256 + 2 * 4 + 2 * 400
    assert lib.cowsdm_workspace_bytes(-1, 0) == -1


def test_argument_errors_return_codes_without_launching():
    lib = nat.lib()
    assert lib.cowsdm_packed_step(None, None, None) == -1
    assert b"shape" in lib.cowsdm_last_error_string()
    shape = nat.Shape(banks=4, slots=16, width=8, writes=65, reads=4, templates=1,
                      index_dtype=0)
    layer = nat.Layer()
    assert lib.cowsdm_packed_step(ctypes.byref(layer), ctypes.byref(shape), None) == -2
    assert b"W <= 64" in lib.cowsdm_last_error_string()
    shape.writes = 4
    assert lib.cowsdm_packed_step(ctypes.byref(layer), ctypes.byref(shape), None) == -1
    assert b"null" in lib.cowsdm_last_error_string()
    assert lib.cowsdm_grow(None, 0, None, 0, 0, None, None, None, None, None) == -1
    # persistent-launch query: null arguments and shapes past the kernel's
    # limits answer 0 without touching a device
    trace = nat.Trace()
    assert lib.cowsdm_trace_persistent(None, 1, ctypes.byref(shape), ctypes.byref(trace), 0) == 0
    layer = nat.Layer()
    wide = nat.Shape(banks=4, slots=16, width=128, writes=5, reads=4, templates=1,
                     index_dtype=0)
    assert lib.cowsdm_trace_persistent(ctypes.byref(layer), 1, ctypes.byref(wide),
                                       ctypes.byref(trace), 0) == 0


def test_trace_run_argument_errors_without_launching():
    lib = nat.lib()
    shape = nat.Shape(banks=4, slots=16, width=8, writes=4, reads=4, templates=1,
                      index_dtype=0)
    layer = nat.Layer()
    trace = nat.Trace()
    # no report, no step counters: refused before any launch
    assert lib.cowsdm_trace_run(ctypes.byref(layer), 1, ctypes.byref(shape),
                                ctypes.byref(trace), 4, 4, nat.RUN_PACKED, None) == -1
    assert b"report" in lib.cowsdm_last_error_string()
    words = (ctypes.c_int64 * 64)()
    trace.step_index = trace.status = trace.report = ctypes.addressof(words)
    assert lib.cowsdm_trace_run(ctypes.byref(layer), 1, ctypes.byref(shape),
                                ctypes.byref(trace), 4, 0, nat.RUN_PACKED, None) == -1
    assert lib.cowsdm_trace_run(ctypes.byref(layer), 1, ctypes.byref(shape),
                                ctypes.byref(trace), 4, 4, 7, None) == -1
    # a report the library did not allocate
    assert lib.cowsdm_trace_run(ctypes.byref(layer), 1, ctypes.byref(shape),
                                ctypes.byref(trace), 4, 4, nat.RUN_PACKED, None) == -1
    assert b"cowsdm_host_report_alloc" in lib.cowsdm_last_error_string()
    host, device = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.cowsdm_host_report_alloc(0, ctypes.byref(host), ctypes.byref(device)) == -1
    assert lib.cowsdm_host_report_free(None) == 0


def test_trace_timing_without_launches():
    lib = nat.lib()
    assert lib.cowsdm_trace_timing(1) == 0
    span, kernel, launches = ctypes.c_double(-1.0), ctypes.c_double(-1.0), ctypes.c_int32(-1)
    assert lib.cowsdm_trace_timing_read(ctypes.byref(span), ctypes.byref(kernel),
                                        ctypes.byref(launches)) == 0
    assert (span.value, kernel.value, launches.value) == (0.0, 0.0, 0)
    assert lib.cowsdm_trace_timing(0) == 0
    assert lib.cowsdm_trace_timing_read(None, None, None) == -1


def test_structure_layout_matches_header():
    # 21 pointer-sized fields and one int64 in cowsdm_layer_t, then the
    # paged map: 3 pointers, an int64 and two int32
    assert ctypes.sizeof(nat.Layer) == 21 * 8 + 3 * 8 + 8 + 2 * 4
    assert nat.Layer.map_directory.offset == 21 * 8
    assert ctypes.sizeof(nat.Shape) == 7 * 8
    assert ctypes.sizeof(nat.Trace) == 21 * 8
    assert ctypes.sizeof(nat.Recurrence) == 14 * 8
    assert ctypes.sizeof(nat.Controller) == 15 * 8 + 2 * 4
    assert nat.REPORT_WORDS == 2 + nat.CTRL_WORDS == 14


def test_paged_map_argument_errors():
    """Rejected before any launch: page shifts outside [1, 6], slots that
    are not whole pages, null tensors."""

    lib = nat.lib()
    buf = ctypes.c_int64(0)
    p = ctypes.byref(buf)
    assert lib.cowsdm_paged_count(p, 4, 64, 0, p, p, p, None) == -1
    assert lib.cowsdm_paged_count(p, 4, 64, 7, p, p, p, None) == -1
    assert b"page shift" in lib.cowsdm_last_error_string()
    assert lib.cowsdm_paged_count(p, 4, 60, 4, p, p, p, None) == -1
    assert lib.cowsdm_paged_count(None, 4, 64, 4, p, p, p, None) == -1
    assert lib.cowsdm_paged_compress(p, 4, 60, 4, p, p, p, p, 8, p, None) == -1
    assert lib.cowsdm_paged_compress(p, 4, 64, 4, p, p, p, None, 8, p, None) == -1
    assert lib.cowsdm_paged_expand(p, p, 8, 4, 60, 4, p, None) == -1
    assert lib.cowsdm_paged_expand(None, p, 8, 4, 64, 4, p, None) == -1
    assert lib.cowsdm_paged_expand(p, p, 8, 0, 64, 4, p, None) == 0     # nothing to run


def test_recurrence_argument_errors():
    """Rejected before any launch, so no GPU is needed."""

    lib = nat.lib()
    assert lib.cowsdm_recurrence_forward(None, None) == -1
    r = nat.Recurrence()
    r.batch, r.time, r.slots, r.width = 2, 3, 1025, 8
    assert lib.cowsdm_recurrence_forward(r, None) == -2
    assert b"at most 1024 slots" in lib.cowsdm_last_error_string()
    r.slots = 0
    assert lib.cowsdm_recurrence_forward(r, None) == -1
    r.slots, r.batch = 16, 0
    assert lib.cowsdm_recurrence_forward(r, None) == 0       # nothing to run
    r.batch = 1
    assert lib.cowsdm_recurrence_forward(r, None) == -1      # null tensors
    assert lib.cowsdm_dense_routes(None, None, 0, 4, 2, 0, None, None, None) == -1
    assert lib.cowsdm_dense_routes(None, None, 7, 4, 2, 16, None, None, None) == -1
    assert lib.cowsdm_dense_routes(None, None, 0, 0, 2, 16, None, None, None) == 0
    assert lib.cowsdm_dense_routes(None, None, 0, 4, 2, 16, None, None, None) == -1


@pytest.mark.parametrize("name", ["cowsdm_packed_step", "cowsdm_dense_step",
                                  "cowsdm_release", "cowsdm_append_banks"])
def test_header_cites_reference(name):
    text = HEADER.read_text()
    block = text[:text.index(name + "(")]
    comment = block[block.rfind("/*"):]
    assert "allocator.py:" in comment


def test_fused_controller_argument_errors_without_launching():
    """The fused controller entry points check their arguments before any
    launch: the residual is required where the next layer's input is its
    sum, the layers must share their width, route counts take
    product_key_routes' checks, and a zero batch launches nothing."""
    lib = nat.lib()
    c = nat.Controller()
    c.width, c.heads, c.slots = 8, 1, 16
    other = nat.Controller()
    other.width, other.heads, other.slots = 16, 1, 16
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: every call fails first
    args = [fake] * 6
    # no residual
    assert lib.cowsdm_controller_finish_prepare_routes(
        ctypes.byref(c), fake, fake, 4, fake, None, fake, ctypes.byref(c), *args,
        4, 2, fake, fake, fake, fake, None) == -1
    assert b"residual" in lib.cowsdm_last_error_string()
    # widths differ (weights null for the finish: the pointer check comes
    # first, so give the batch 0 path the width check)
    assert lib.cowsdm_controller_finish_prepare_routes(
        ctypes.byref(c), fake, fake, 0, fake, fake, fake, ctypes.byref(other), *args,
        4, 2, fake, fake, fake, fake, None) == -1
    assert b"widths differ" in lib.cowsdm_last_error_string()
    # route counts
    assert lib.cowsdm_controller_prepare_routes(
        ctypes.byref(c), fake, 0, *args, 0, 2, fake, fake, fake, fake, None) != 0
    # a zero batch is a no-op
    assert lib.cowsdm_controller_prepare_routes(
        ctypes.byref(c), fake, 0, *args, 4, 2, fake, fake, fake, fake, None) == 0
    assert lib.cowsdm_controller_finish_residual(
        ctypes.byref(c), fake, fake, 0, fake, fake, None, None) == -1
    assert b"residual sum" in lib.cowsdm_last_error_string()
