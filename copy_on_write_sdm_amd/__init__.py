"""MI355X-native copy-on-write Sparse Delta Memory decode step.

Drop-in for the decode-state path of p0rc314in/copy-on-write-sdm
(copy_on_write_sdm/allocator.py and the SDM half of inference.py): the same
class and function names, arguments and errors, backed by hand-written HIP
kernels for gfx950 in libcowsdm.so (C ABI: include/cowsdm.h).
"""

from .allocator import (
    DecodeTrace,
    PackedSDMCopyOnWriteState,
    PagedSlotMap,
    SDMCopyOnWriteStep,
    dense_sdm_sparse_step,
    dense_sdm_sparse_step_layers,
    mark_written,
    packed_sdm_cow_step,
    packed_sdm_cow_step_layers,
)
from .inference import (
    FaithfulSDMDecodeState,
    SDMStepInputs,
    decode_sdm_layer,
    decode_sdm_layer_dense,
    pack_prefill_layer,
    pack_prefill_layers,
)
from .routing import product_key_routes
from .recurrence import dense_sparse_routes, gated_delta_recurrence, sdm_recurrence
from .prefill import (
    SDMPrefill,
    allocate_dense_cache,
    prefill_faithful_sdm_stack,
    prefill_sdm_layer,
)
from .stack_decode import decode_faithful_sdm_stack, write_dense_cache
from .controller import (
    ControllerDecodeGraph,
    ControllerStep,
    SDMController,
    decode_sdm_layer_controller,
    decode_sdm_layer_controller_dense,
    finish_sdm_step,
    prepare_sdm_step,
)

__all__ = [
    "ControllerDecodeGraph",
    "ControllerStep",
    "DecodeTrace",
    "SDMController",
    "SDMPrefill",
    "FaithfulSDMDecodeState",
    "PackedSDMCopyOnWriteState",
    "PagedSlotMap",
    "SDMCopyOnWriteStep",
    "SDMStepInputs",
    "allocate_dense_cache",
    "decode_faithful_sdm_stack",
    "decode_sdm_layer",
    "decode_sdm_layer_controller",
    "decode_sdm_layer_controller_dense",
    "decode_sdm_layer_dense",
    "dense_sdm_sparse_step",
    "dense_sdm_sparse_step_layers",
    "dense_sparse_routes",
    "finish_sdm_step",
    "gated_delta_recurrence",
    "mark_written",
    "pack_prefill_layer",
    "pack_prefill_layers",
    "packed_sdm_cow_step",
    "packed_sdm_cow_step_layers",
    "prefill_faithful_sdm_stack",
    "prefill_sdm_layer",
    "prepare_sdm_step",
    "product_key_routes",
    "sdm_recurrence",
    "write_dense_cache",
]
