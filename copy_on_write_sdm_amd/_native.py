"""ctypes binding of libcowsdm.so (include/cowsdm.h) and its build recipe.

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (both carry the soname libamdhip64.so.7); device pointers and
the hipStream_t handles torch hands out are then valid in the library.

There is no fallback: if the library is missing, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading
import weakref
from pathlib import Path

import numpy as np
import torch

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
# one translation unit per step-kernel family so hipcc can run in parallel
SOURCES = ("cowsdm.hip", "step_i32_packed.hip", "step_i32_dense.hip", "step_i64_packed.hip",
           "step_i64_dense.hip", "trace_plan.hip", "routes.hip", "controller.hip",
           "recurrence.hip")
INCLUDE_DIR = REPO_DIR / "include"
LIBRARY = PACKAGE_DIR / "lib" / "libcowsdm.so"
BUILD_DIR = PACKAGE_DIR / "_build"

INDEX_INT32 = 0
INDEX_INT64 = 1

ERR_WRITE_INDEX = 0x1
ERR_READ_INDEX = 0x2
ERR_DUP_WRITE = 0x4
ERR_EXHAUSTED = 0x8
ERR_TEMPLATE = 0x10
ERR_CORRUPT = 0x20
ERR_LOOKBACK = 0x40
ERR_TRACE_RANGE = 0x80

TRACE_REFUSED = 0x1   # status bit: stopped before a growth past the slab buffers
TRACE_ENDED = 0x2     # status bit: no recorded step left
TRACE_FAULT = 0x4     # status bit: a timed-out wait or corrupt state stopped the layer

# control words of a packed decode trace layer (cowsdm_trace_t.control)
CTRL_PROVEN = 0
CTRL_CAPACITY = 1
CTRL_ROOM = 2
CTRL_QUANTUM = 3
CTRL_NEED = 4
CTRL_EVENTS = 5
CTRL_ADDED = 6
CTRL_COPIED = 7
CTRL_FREE = 8
CTRL_STEPS = 9
CTRL_FIT = 10
CTRL_WORDS = 12
# a trace launch's host-mapped report per layer: step counter, status bits,
# control words (cowsdm_trace_t.report)
REPORT_STEP = 0
REPORT_STATUS = 1
REPORT_CONTROL = 2
REPORT_WORDS = 2 + CTRL_WORDS
# cowsdm_trace_run modes
RUN_PACKED = 0
RUN_PACKED_STATIC = 1
RUN_DENSE = 2

ABI_VERSION = 12
STATIC_SCAN_WORDS = 1 << 21   # COWSDM_STATIC_SCAN_WORDS

SCRATCH_EPOCH = 0
SCRATCH_ERRORS = 3
SCRATCH_SLOTS = 8

HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # every product and sum is rounded on its own, as in the reference's
    # elementwise torch ops
    "-ffp-contract=off",
    # never emit packed FP32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep each atomic as written: combining a lane-0 atomic across the wave
    # makes its result (a row claim read an iteration later) wait at once
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
)


def build_library(output: Path | None = None, *, jobs: int | None = None) -> Path:
    """Compile csrc/*.hip for gfx950 and link lib/libcowsdm.so."""

    output = Path(output) if output is not None else LIBRARY
    output.parent.mkdir(parents=True, exist_ok=True)
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    include = [f"-I{INCLUDE_DIR}", f"-I{SOURCE_DIR}"]
    objects, procs = [], []
    jobs = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1))
    pending = list(SOURCES)
    while pending or procs:
        while pending and len(procs) < jobs:
            name = pending.pop(0)
            obj = BUILD_DIR / (name.rsplit(".", 1)[0] + ".o")
            cmd = [hipcc, *HIPCC_FLAGS, *include, "-c", "-o", str(obj), str(SOURCE_DIR / name)]
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.PIPE, text=True)))
            objects.append(obj)
        cmd, proc = procs.pop(0)
        _, err = proc.communicate()
        if proc.returncode != 0:
            for _, other in procs:
                other.kill()
            raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + err)
    tmp = output.with_name(output.name + f".tmp{os.getpid()}")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + " ".join(cmd) + "\n" + proc.stderr)
    os.replace(tmp, output)
    return output


class Shape(ctypes.Structure):
    """cowsdm_shape_t."""

    _fields_ = [
        ("banks", ctypes.c_int64),
        ("slots", ctypes.c_int64),
        ("width", ctypes.c_int64),
        ("writes", ctypes.c_int64),
        ("reads", ctypes.c_int64),
        ("templates", ctypes.c_int64),
        ("index_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class Layer(ctypes.Structure):
    """cowsdm_layer_t."""

    _fields_ = [
        ("shared_initial_memory", ctypes.c_void_p),
        ("template_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("logical_to_physical", ctypes.c_void_p),
        ("free_rows", ctypes.c_void_p),
        ("free_count", ctypes.c_void_p),
        ("overflow_flag", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("capacity_rows", ctypes.c_int64),
        ("write_indices", ctypes.c_void_p),
        ("write_weights", ctypes.c_void_p),
        ("step_values", ctypes.c_void_p),
        ("input_gate", ctypes.c_void_p),
        ("erase_gate", ctypes.c_void_p),
        ("forget_log_gate", ctypes.c_void_p),
        ("read_indices", ctypes.c_void_p),
        ("read_weights", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("first_touches_out", ctypes.c_void_p),
        ("repeated_writes_out", ctypes.c_void_p),
        ("allocated_rows_out", ctypes.c_void_p),
        # paged slot map (map_page_shift > 0)
        ("map_directory", ctypes.c_void_p),
        ("map_pages", ctypes.c_void_p),
        ("map_page_count", ctypes.c_void_p),
        ("map_page_capacity", ctypes.c_int64),
        ("map_page_shift", ctypes.c_int32),
        ("map_reserved", ctypes.c_int32),
    ]


class Trace(ctypes.Structure):
    """cowsdm_trace_t."""

    _fields_ = [
        ("step_index", ctypes.c_void_p),
        ("ticket", ctypes.c_void_p),
        ("first_step", ctypes.c_int64),
        ("stride_bytes", ctypes.c_int64 * 9),
        ("scan", ctypes.c_void_p),
        ("scan_words", ctypes.c_int64),
        ("persistent", ctypes.c_int32),
        ("scan_steps", ctypes.c_int32),
        ("steps_recorded", ctypes.c_int64),
        ("status", ctypes.c_void_p),
        ("control", ctypes.c_void_p),
        ("control_stride", ctypes.c_int64),
        ("report", ctypes.c_void_p),
        ("first_known", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class Controller(ctypes.Structure):
    """cowsdm_controller_t."""

    _fields_ = [
        ("width", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("slots", ctypes.c_int64),
        ("norm_weight", ctypes.c_void_p),
        ("norm_bias", ctypes.c_void_p),
        ("proj_weight_t", ctypes.c_void_p),
        ("proj_bias", ctypes.c_void_p),
        ("a_log", ctypes.c_void_p),
        ("dt_bias", ctypes.c_void_p),
        ("gate_weight_t", ctypes.c_void_p),
        ("gate_bias", ctypes.c_void_p),
        ("out_weight_t", ctypes.c_void_p),
        ("out_bias", ctypes.c_void_p),
        ("read_norm_weight", ctypes.c_void_p),
        ("read_norm_bias", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
        ("read_norm_eps", ctypes.c_float),
    ]


class Recurrence(ctypes.Structure):
    """cowsdm_recurrence_t."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("time", ctypes.c_int64),
        ("slots", ctypes.c_int64),
        ("width", ctypes.c_int64),
        ("initial_memory", ctypes.c_void_p),
        ("write_routes", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("input_gate", ctypes.c_void_p),
        ("erase_gate", ctypes.c_void_p),
        ("forget_log_gate", ctypes.c_void_p),
        ("read_routes", ctypes.c_void_p),
        ("readings", ctypes.c_void_p),
        ("states", ctypes.c_void_p),
        ("final_memory", ctypes.c_void_p),
    ]


class HandoffLayer(ctypes.Structure):
    """cowsdm_handoff_layer_t."""

    _fields_ = [
        ("dense_memory", ctypes.c_void_p),
        ("active_mask", ctypes.c_void_p),
        ("banks", ctypes.c_int64),
        ("slots", ctypes.c_int64),
        ("width", ctypes.c_int64),
        ("workspace", ctypes.c_void_p),
        ("total", ctypes.c_void_p),
        ("template_indices", ctypes.c_void_p),
        ("templates", ctypes.c_int64),
        ("checks", ctypes.c_void_p),
        ("logical_to_physical", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("free_rows", ctypes.c_void_p),
        ("capacity_rows", ctypes.c_int64),
        ("free_count", ctypes.c_void_p),
        ("overflow_flag", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_words", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32

# name -> (restype, argtypes); the C declarations live in include/cowsdm.h
SIGNATURES: dict[str, tuple] = {
    "cowsdm_abi_version": (_I32, []),
    "cowsdm_last_error_string": (ctypes.c_char_p, []),
    "cowsdm_step_scratch_words": (_I64, [_I64]),
    "cowsdm_workspace_bytes": (_I64, [_I64, _I64]),
    "cowsdm_trace_scan_words": (_I64, [_I64, _I64, _I32]),
    "cowsdm_trace_persistent": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), ctypes.POINTER(Trace), _I32]),
    "cowsdm_controller_rows": (_I64, [_I64, _I64, _I64]),
    "cowsdm_controller_prepare": (
        _I32, [ctypes.POINTER(Controller), _P, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "cowsdm_controller_finish": (_I32, [ctypes.POINTER(Controller), _P, _P, _I64, _P, _P]),
    "cowsdm_controller_prepare_routes": (
        _I32, [ctypes.POINTER(Controller), _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P,
               _P, _P, _P]),
    "cowsdm_controller_finish_residual": (
        _I32, [ctypes.POINTER(Controller), _P, _P, _I64, _P, _P, _P, _P]),
    "cowsdm_controller_finish_prepare_routes": (
        _I32, [ctypes.POINTER(Controller), _P, _P, _I64, _P, _P, _P, ctypes.POINTER(Controller),
               _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "cowsdm_recurrence_forward": (_I32, [ctypes.POINTER(Recurrence), _P]),
    "cowsdm_dense_routes": (_I32, [_P, _P, _I32, _I64, _I64, _I64, _P, _P, _P]),
    "cowsdm_host_report_alloc": (
        _I32, [_I64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)]),
    "cowsdm_host_report_free": (_I32, [_P]),
    "cowsdm_trace_run": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), ctypes.POINTER(Trace), _I64,
               _I32, _I32, _P]),
    "cowsdm_trace_timing": (_I32, [_I32]),
    "cowsdm_trace_timing_read": (
        _I32, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
               ctypes.POINTER(_I32)]),
    "cowsdm_packed_step": (_I32, [ctypes.POINTER(Layer), ctypes.POINTER(Shape), _P]),
    "cowsdm_packed_step_layers": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), _P]),
    "cowsdm_packed_step_trace": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), ctypes.POINTER(Trace), _I32,
               _P]),
    "cowsdm_packed_step_trace_static": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), ctypes.POINTER(Trace), _I32,
               _P]),
    "cowsdm_dense_step": (_I32, [ctypes.POINTER(Layer), ctypes.POINTER(Shape), _P]),
    "cowsdm_dense_step_trace": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), ctypes.POINTER(Trace), _I32,
               _P]),
    "cowsdm_dense_step_layers": (
        _I32, [ctypes.POINTER(Layer), _I32, ctypes.POINTER(Shape), _P]),
    "cowsdm_step_precheck": (
        _I32, [ctypes.POINTER(Layer), ctypes.POINTER(Shape), _I32, _I32, _I32, _P, _P]),
    "cowsdm_init_state": (
        _I32, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P]),
    "cowsdm_grow": (_I32, [_P, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "cowsdm_count_active": (_I32, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P]),
    "cowsdm_handoff_count": (_I32, [_P, _I32, _P]),
    "cowsdm_handoff_pack": (_I32, [_P, _I32, _P]),
    "cowsdm_paged_count": (_I32, [_P, _I64, _I64, _I32, _P, _P, _P, _P]),
    "cowsdm_paged_compress": (_I32, [_P, _I64, _I64, _I32, _P, _P, _P, _P, _I64, _P, _P]),
    "cowsdm_paged_expand": (_I32, [_P, _P, _I64, _I64, _I64, _I32, _P, _P]),
    "cowsdm_pack_overlay": (
        _I32, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P]),
    "cowsdm_trim_repack": (
        _I32, [_P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P]),
    "cowsdm_append_banks": (
        _I32,
        [_P, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P,
         _P, _P]),
    "cowsdm_check_banks": (_I32, [_P, _I64, _I64, _P, _I64, _I32, _P, _P, _P]),
    "cowsdm_release": (_I32, [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _P, _P]),
    "cowsdm_retain_banks": (_I32, [_P, _P, _I64, _I64, _P, _I64, _P, _P, _P]),
    "cowsdm_materialize_dense": (
        _I32, [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "cowsdm_check_invariants": (
        _I32, [_P, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P, _P]),
    "cowsdm_mark_written": (_I32, [_P, _I64, _I64, _P, _I64, _I32, _P, _P]),
    "cowsdm_product_key_routes": (_I32, [_P, _I64, _I64, _I64, _P, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("COWSDM_LIBRARY")
    return Path(override) if override else LIBRARY


def lib() -> ctypes.CDLL:
    """The loaded HIP library; raises if it has not been built."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"libcowsdm.so not found at {path}: build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'`; the "
                    "copy-on-write SDM kernels have no CPU fallback"
                )
            handle = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if handle.cowsdm_abi_version() != ABI_VERSION:
                raise RuntimeError("libcowsdm.so ABI version mismatch")
            _lib = handle
    return _lib


def _free_host_report(host: int) -> None:
    lib().cowsdm_host_report_free(host)


class HostReport:
    """Host memory the device writes trace reports into
    (cowsdm_host_report_alloc): ``array`` is an int64 numpy view
    [layers, REPORT_WORDS] of it and ``device`` the address kernels write.
    Freed when the object is collected (left to the process's end at
    interpreter exit)."""

    def __init__(self, layers: int):
        host, device = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib().cowsdm_host_report_alloc(layers * REPORT_WORDS, ctypes.byref(host),
                                             ctypes.byref(device)), "host report")
        self.device = device.value
        words = (ctypes.c_int64 * (layers * REPORT_WORDS)).from_address(host.value)
        self.array = np.frombuffer(words, dtype=np.int64).reshape(layers, REPORT_WORDS)
        self._free = weakref.finalize(self, _free_host_report, host.value)
        self._free.atexit = False


def check(rc: int, what: str) -> None:
    """Raise RuntimeError on a nonzero C-ABI return code."""

    if rc != 0:
        message = lib().cowsdm_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {message}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (torch's raw
    getter where it has one: a tenth of the cost of building the Stream
    object)."""

    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()
