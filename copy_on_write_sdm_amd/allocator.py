"""Packed copy-on-write SDM state and its fused decode step on MI355X.

Drop-in for ``copy_on_write_sdm.allocator`` (p0rc314in/copy-on-write-sdm):
the same ``PackedSDMCopyOnWriteState`` fields, methods and error messages,
and the same ``packed_sdm_cow_step`` / ``dense_sdm_sparse_step`` signatures.
All state arithmetic runs in the HIP kernels of libcowsdm.so (include/
cowsdm.h); torch only allocates device memory, supplies the current stream
and reads back the few scalars the reference also synchronises on.

Differences from the reference, all deliberate:

* Physical rows for first touches are popped in bank-major order on every
  backend, so the map, slab and free stack match the reference's torch path
  (allocator.py:1471-1481) exactly instead of up to a permutation.
* ``backend`` accepts "auto", "hip" and "torch"; all three run the HIP
  kernels on device tensors (no CPU path ships, so CPU tensors raise).
  "torch" asks for the reference torch path's semantics: its results
  (bank-major pops, the same rows and counts; float sums within 1e-6 of
  torch's reduction order) and its exhaustion check before every step, which
  the reference asserts on the device (allocator.py:1474) and this build
  raises as ValueError after one synchronisation.  "triton" raises the
  reference's unavailable-backend error.
* Value state is float32 (the reference's serving path and benchmark use
  float32 state, inference.py:359); route weights, values and gates may be
  float16 or bfloat16: they compute in float32, as in both reference
  backends, and the reading comes back in the values' dtype.
* The state carries one more tensor, ``scratch`` (int64 [8 + B]), holding the
  bank-order scan slots, a ticket counter and a sticky error word.
* Route validation (``validate_routes=True``) and steps on a state without a
  capacity proof synchronise once and raise ValueError, like the reference's
  CPU path, where the reference's GPU path would device-assert.
"""

from __future__ import annotations

import ctypes
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, Sequence

import torch

from . import _native as nat


def _tensor_bytes(tensor: torch.Tensor) -> int:
    return tensor.numel() * tensor.element_size()


def _ceil_to(value: int, quantum: int) -> int:
    return ((value + quantum - 1) // quantum) * quantum


def handoff_capacity(
    active_count: int,
    banks: int,
    slots: int,
    capacity_rows: int | None,
    growth_quantum_rows: int,
    maximum_future_allocations: int | None,
) -> tuple[int, int]:
    """Slab size and proven future allocations of a prefill handoff
    (allocator.py:629-655).  Returns (capacity, proven future rows)."""

    if growth_quantum_rows < 0:
        raise ValueError("SDM growth quantum cannot be negative")
    if capacity_rows is None and growth_quantum_rows:
        selected = max(growth_quantum_rows, _ceil_to(active_count, growth_quantum_rows))
    else:
        selected = banks * slots if capacity_rows is None else capacity_rows
    if selected < active_count:
        raise ValueError("SDM physical capacity is smaller than the prefill working set")
    if maximum_future_allocations is None:
        return selected, 0
    if maximum_future_allocations < 0:
        raise ValueError("maximum future allocations cannot be negative")
    possible = min(maximum_future_allocations, banks * slots - active_count)
    if selected - active_count < possible:
        raise ValueError("SDM physical capacity cannot cover the declared decode trace")
    return selected, possible


def growth_target(minimum_capacity_rows: int, quantum: int) -> int:
    """Capacity after growth: the minimum rounded up to the quantum
    (allocator.py:706-708)."""

    return _ceil_to(minimum_capacity_rows, quantum)


def trim_target(active_count: int, headroom_rows: int, quantum: int) -> int:
    """Capacity after a trim (allocator.py:792-795)."""

    return max(quantum, _ceil_to(active_count + headroom_rows, quantum))


def _require_device(tensor: torch.Tensor, what: str) -> None:
    if tensor.device.type != "cuda":
        raise RuntimeError(
            f"{what} must live on a HIP device: the copy-on-write SDM kernels "
            "have no CPU path"
        )


def _workspace(entries: int, rows: int, device: torch.device) -> torch.Tensor:
    size = int(nat.lib().cowsdm_workspace_bytes(entries, rows))
    return torch.empty(max(size, 256), dtype=torch.uint8, device=device)


def _scratch(banks: int, device: torch.device) -> torch.Tensor:
    words = int(nat.lib().cowsdm_step_scratch_words(banks))
    return torch.zeros(words, dtype=torch.int64, device=device)


def _map_placeholder(banks: int, slots: int) -> torch.Tensor:
    """The ``logical_to_physical`` of a state whose map is paged: the direct
    map's shape on the meta device, holding no data (its pointer is null, so
    a kernel handed it fails its argument check, and reading it raises)."""

    return torch.empty((banks, slots), device="meta", dtype=torch.int32)


@dataclass
class PagedSlotMap:
    """A compressed logical-to-physical map for large address spaces: the
    direct map's entries in pages of P slots, only the pages holding a mapped
    slot stored.  The reference leaves this map as future work
    (README.md:123-130; allocator.py:485-489: "a later compressed map can
    replace it without changing SDM").

    ``directory`` int32 [B, N / P]: the page of each (bank, page of slots),
    -1 when none of its slots is mapped.  ``pages`` int32 [capacity, P]:
    rows 0 .. ``page_count`` - 1 in use; a decode step takes new pages from
    ``page_count`` up.  ``pages_bound`` is the host's upper bound on the
    pages in use (the page proof, ``prove``).  No counterpart in the
    reference."""

    directory: torch.Tensor
    pages: torch.Tensor
    page_count: torch.Tensor
    page_shift: int
    pages_bound: int = 0

    @property
    def page_slots(self) -> int:
        return 1 << self.page_shift

    @property
    def banks(self) -> int:
        return self.directory.shape[0]

    @property
    def slots(self) -> int:
        return self.directory.shape[1] << self.page_shift

    @property
    def capacity(self) -> int:
        return self.pages.shape[0]

    @staticmethod
    def _shift(page_slots: int, slots: int) -> int:
        shift = int(page_slots).bit_length() - 1
        if page_slots < 2 or page_slots > 64 or (1 << shift) != page_slots or slots % page_slots:
            raise ValueError("SDM map pages hold a power of two of 2 to 64 slots dividing N")
        return shift

    @classmethod
    def empty(cls, banks: int, slots: int, page_slots: int, device,
              capacity: int | None = None) -> "PagedSlotMap":
        """A map with no slot mapped."""

        shift = cls._shift(page_slots, slots)
        capacity = max(64, banks) if capacity is None else max(1, int(capacity))
        return cls(
            directory=torch.full((banks, slots >> shift), -1, device=device, dtype=torch.int32),
            pages=torch.empty(capacity, 1 << shift, device=device, dtype=torch.int32),
            page_count=torch.zeros((), device=device, dtype=torch.int32),
            page_shift=shift)

    @classmethod
    @torch.no_grad()
    def compress(cls, mapping: torch.Tensor, page_slots: int) -> "PagedSlotMap":
        """The paged form of a direct map [B, N]: its pages holding a mapped
        slot, numbered in row-major (bank, page) order."""

        banks, slots = mapping.shape
        shift = cls._shift(page_slots, slots)
        device = mapping.device
        per_bank = slots >> shift
        entries = banks * per_bank
        flags = torch.empty(max(entries, 1), device=device, dtype=torch.uint8)
        workspace = _workspace(entries, 0, device)
        total = torch.empty(1, device=device, dtype=torch.int64)
        stream = nat.stream_handle(device)
        direct = mapping.contiguous()
        nat.check(nat.lib().cowsdm_paged_count(
            direct.data_ptr(), banks, slots, shift, flags.data_ptr(), workspace.data_ptr(),
            total.data_ptr(), stream), "cowsdm_paged_count")
        used = int(total.item())
        out = cls.empty(banks, slots, 1 << shift, device, capacity=max(used, 64))
        nat.check(nat.lib().cowsdm_paged_compress(
            direct.data_ptr(), banks, slots, shift, flags.data_ptr(), workspace.data_ptr(),
            out.directory.data_ptr(), out.pages.data_ptr(), out.capacity,
            out.page_count.data_ptr(), stream), "cowsdm_paged_compress")
        out.pages_bound = used
        return out

    @torch.no_grad()
    def expand(self) -> torch.Tensor:
        """The direct map [B, N]."""

        mapping = torch.empty(self.banks, self.slots, device=self.directory.device,
                              dtype=torch.int32)
        nat.check(nat.lib().cowsdm_paged_expand(
            self.directory.data_ptr(), self.pages.data_ptr(), self.capacity, self.banks,
            self.slots, self.page_shift, mapping.data_ptr(),
            nat.stream_handle(self.directory.device)), "cowsdm_paged_expand")
        return mapping

    @torch.no_grad()
    def prove(self, maximum_new_pages: int) -> None:
        """Room for ``maximum_new_pages`` more pages before a step (a step
        takes at most one per write route): the page count is read only when
        the host's bound runs short, and the pool grows (doubling) when the
        pages in use leave too little room."""

        if self.pages_bound + maximum_new_pages > self.capacity:
            used = int(self.page_count.item())
            self.pages_bound = used
            if used + maximum_new_pages > self.capacity:
                grown = max(2 * self.capacity, used + maximum_new_pages)
                if grown >= 2**31:
                    raise ValueError("SDM map pages cannot pass 2^31")
                pages = torch.empty(grown, self.page_slots, device=self.pages.device,
                                    dtype=torch.int32)
                pages[:self.capacity].copy_(self.pages)
                self.pages = pages
        self.pages_bound += maximum_new_pages

    def storage_bytes(self) -> int:
        return (_tensor_bytes(self.directory) + _tensor_bytes(self.pages)
                + _tensor_bytes(self.page_count))

    def used_bytes(self) -> int:
        """Directory plus the pages in use (reads the page count)."""

        return (_tensor_bytes(self.directory)
                + int(self.page_count.item()) * self.page_slots * 4
                + _tensor_bytes(self.page_count))


@dataclass(frozen=True)
class SDMCopyOnWriteStep:
    """Diagnostics for one packed SDM decode step (allocator.py:467-473)."""

    first_touches_by_sequence: torch.Tensor
    repeated_writes_by_sequence: torch.Tensor
    allocated_rows_after_step: torch.Tensor


@dataclass
class PackedSDMCopyOnWriteState:
    """One shared slab backing several independent logical SDM tables.

    Fields as in allocator.py:476-504: ``shared_initial_memory`` [T,N,D]
    (model-shared M0), ``template_indices`` [B] int64, ``values`` [C,D] slab,
    ``logical_to_physical`` [B,N] int32 (-1 = shared M0), ``free_rows`` [C]
    int32 stack with ``free_count`` entries, ``overflow_flag``; plus
    ``scratch``, the device words of the bank-order scan.  After a growth,
    ``values`` and ``free_rows`` are the leading rows of buffers with
    headroom (``slab_buffers``), so later growths that fit move no rows.
    """

    shared_initial_memory: torch.Tensor
    template_indices: torch.Tensor
    values: torch.Tensor
    logical_to_physical: torch.Tensor
    free_rows: torch.Tensor
    free_count: torch.Tensor
    overflow_flag: torch.Tensor
    capacity_is_proven: bool = False
    proven_maximum_additional_allocations: int = 0
    growth_quantum_rows: int = 0
    growth_events: int = 0
    growth_rows_added: int = 0
    growth_rows_copied: int = 0
    scratch: torch.Tensor | None = None
    # (values buffer, free-row buffer) that values and free_rows lead, or None
    slab_buffers: Any = field(default=None, repr=False, compare=False)
    # the paged form of the map, or None; when set, logical_to_physical is a
    # data-less placeholder of the direct map's shape
    paged_map: PagedSlotMap | None = field(default=None, repr=False, compare=False)

    def __setattr__(self, name: str, value: Any) -> None:
        # every assignment counts in ``_version``: a decode trace that saw
        # the same version last time knows its device copies of the pointers
        # and proof words are current
        object.__setattr__(self, name, value)
        object.__setattr__(self, "_version", self.__dict__.get("_version", 0) + 1)

    # --------------------------------------------------------- creation

    @classmethod
    def allocate(
        cls,
        shared_initial_memory: torch.Tensor,
        *,
        banks: int,
        capacity_rows: int,
        template_indices: torch.Tensor | None = None,
        state_dtype: torch.dtype = torch.float32,
        growth_quantum_rows: int = 0,
        map_page_slots: int | None = None,
    ) -> "PackedSDMCopyOnWriteState":
        """Allocate an empty shared slab (allocator.py:506-585).  With
        ``map_page_slots`` (not in the reference) the map is paged
        (``PagedSlotMap``) with that many slots per page."""

        state, result = cls._allocate_state(
            shared_initial_memory, banks=banks, capacity_rows=capacity_rows,
            template_indices=template_indices, state_dtype=state_dtype,
            growth_quantum_rows=growth_quantum_rows, map_page_slots=map_page_slots)
        if int(result.item()) & nat.ERR_TEMPLATE:
            raise ValueError("template index lies outside shared initial memory")
        return state

    @classmethod
    def _allocate_state(cls, shared_initial_memory, *, banks, capacity_rows,
                        template_indices=None, state_dtype=torch.float32,
                        growth_quantum_rows=0, map_page_slots=None, result=None,
                        initialize=True):
        """``allocate`` with the template check's result word left on the
        device (``result``, int64, or a new one): the caller reads it.  With
        ``initialize`` False the state's tensors are left for the caller's
        kernels to fill (no template check either)."""

        if shared_initial_memory.ndim == 2:
            shared_initial_memory = shared_initial_memory.unsqueeze(0)
        if shared_initial_memory.ndim != 3:
            raise ValueError("shared initial memory must be [H,N,D] or [N,D]")
        templates, slots, width = shared_initial_memory.shape
        if banks <= 0 or capacity_rows <= 0:
            raise ValueError("banks and physical capacity must be positive")
        if growth_quantum_rows < 0:
            raise ValueError("SDM growth quantum cannot be negative")
        if state_dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("SDM COW state must use float16, bfloat16, or float32")
        if state_dtype != torch.float32:
            raise ValueError("this build keeps SDM COW state in float32")
        _require_device(shared_initial_memory, "shared initial memory")
        if shared_initial_memory.dtype != torch.float32:
            raise ValueError("shared initial memory must be float32")
        shared_initial_memory = shared_initial_memory.contiguous()
        device = shared_initial_memory.device
        if template_indices is None:
            if templates != 1:
                raise ValueError("multiple initial-memory templates require explicit mapping")
            template_indices = torch.zeros(banks, device=device, dtype=torch.int64)
        elif (
            template_indices.shape != (banks,)
            or template_indices.dtype not in (torch.int32, torch.int64)
            or template_indices.device != device
        ):
            raise ValueError("template indices must be integer [B] on the state device")
        else:
            template_indices = template_indices.to(torch.int64).contiguous()
        if capacity_rows >= 2**31 or banks * slots >= 2**31:
            raise ValueError("SDM COW state sizes must stay below 2^31 rows and entries")
        state = cls(
            shared_initial_memory=shared_initial_memory,
            template_indices=template_indices,
            values=torch.empty(capacity_rows, width, device=device, dtype=torch.float32),
            logical_to_physical=torch.empty(banks, slots, device=device, dtype=torch.int32),
            free_rows=torch.empty(capacity_rows, device=device, dtype=torch.int32),
            free_count=torch.empty((), device=device, dtype=torch.int32),
            overflow_flag=torch.empty((), device=device, dtype=torch.int32),
            growth_quantum_rows=growth_quantum_rows,
            scratch=torch.empty(
                int(nat.lib().cowsdm_step_scratch_words(banks)), device=device,
                dtype=torch.int64),
        )
        if not initialize:
            return state, None
        if result is None:
            result = torch.empty(1, device=device, dtype=torch.int64)
        nat.check(
            nat.lib().cowsdm_init_state(
                state.logical_to_physical.data_ptr(), banks, slots,
                state.free_rows.data_ptr(), capacity_rows, state.free_count.data_ptr(),
                state.overflow_flag.data_ptr(), state.scratch.data_ptr(),
                state.scratch.numel(), template_indices.data_ptr(), templates,
                result.data_ptr(), nat.stream_handle(device)),
            "cowsdm_init_state",
        )
        if map_page_slots is not None:
            state.paged_map = PagedSlotMap.empty(banks, slots, map_page_slots, device)
            state.logical_to_physical = _map_placeholder(banks, slots)
        return state, result

    @classmethod
    @torch.no_grad()
    def from_dense_overlay(
        cls,
        shared_initial_memory: torch.Tensor,
        dense_memory: torch.Tensor,
        active_slots: torch.Tensor,
        *,
        template_indices: torch.Tensor,
        capacity_rows: int | None = None,
        state_dtype: torch.dtype = torch.float32,
        maximum_future_allocations: int | None = None,
        growth_quantum_rows: int = 0,
        map_page_slots: int | None = None,
    ) -> "PackedSDMCopyOnWriteState":
        """Pack an exact full-prefix state into a first-write overlay
        (allocator.py:587-689).  With ``map_page_slots`` (not in the
        reference) the packed map is paged (``PagedSlotMap``)."""

        return cls.from_dense_overlay_layers(
            [shared_initial_memory], [dense_memory], [active_slots],
            template_indices=template_indices, capacity_rows=capacity_rows,
            state_dtype=state_dtype, maximum_future_allocations=maximum_future_allocations,
            growth_quantum_rows=growth_quantum_rows, map_page_slots=map_page_slots)[0]

    @classmethod
    @torch.no_grad()
    def from_dense_overlay_layers(
        cls,
        shared_initial_memories: Sequence[torch.Tensor],
        dense_memories: Sequence[torch.Tensor],
        active_slots: Sequence[torch.Tensor],
        *,
        template_indices: torch.Tensor,
        capacity_rows: int | None | Sequence[int | None] = None,
        state_dtype: torch.dtype = torch.float32,
        maximum_future_allocations: int | None = None,
        growth_quantum_rows: int = 0,
        map_page_slots: int | None = None,
    ) -> list["PackedSDMCopyOnWriteState"]:
        """``from_dense_overlay`` of several layers at once: the same states,
        checks and errors, with one host read of every layer's active count
        (which sizes the slabs) and one of every layer's invariant check
        (allocator.py:639, 687), instead of two reads per layer.  The
        arguments after the per-layer sequences apply to every layer
        (``capacity_rows`` may also give one per layer).  No counterpart in
        the reference."""

        layers = len(dense_memories)
        if isinstance(capacity_rows, (list, tuple)):
            if len(capacity_rows) != layers:
                raise ValueError("SDM capacities must contain one value per layer")
            capacities = list(capacity_rows)
        else:
            capacities = [capacity_rows] * layers
        if len(shared_initial_memories) != layers or len(active_slots) != layers:
            raise ValueError("one initial memory, dense memory and active mask per layer")
        prepared = []
        for m0, dense_memory, active in zip(shared_initial_memories, dense_memories,
                                           active_slots):
            if m0.ndim == 2:
                m0 = m0.unsqueeze(0)
            if m0.ndim != 3 or dense_memory.ndim != 3:
                raise ValueError("SDM handoff memory must be [H,N,D] and [B,N,D]")
            banks, slots, width = dense_memory.shape
            if (
                active.shape != (banks, slots)
                or active.dtype != torch.bool
                or active.device != dense_memory.device
                or m0.device != dense_memory.device
                or m0.shape[1:] != (slots, width)
            ):
                raise ValueError("SDM handoff state and active-slot mask do not align")
            if (
                template_indices.shape != (banks,)
                or template_indices.device != dense_memory.device
            ):
                raise ValueError("SDM handoff template indices must be [B] on device")
            _require_device(dense_memory, "SDM handoff memory")
            prepared.append((m0, dense_memory.to(torch.float32).contiguous(),
                             active.contiguous()))
        if not prepared:
            return []
        device = prepared[0][1].device
        stream = nat.stream_handle(device)
        # The count part of every layer in two launches (cowsdm_handoff_count),
        # one read of the active counts, every layer's state allocated, and
        # the pack, free stack and invariant counts of every layer in five
        # launches (cowsdm_handoff_pack), then one read of the checks.  Each
        # layer's workspace (one allocation carved for all) keeps the ranks
        # its count leaves for the pack, with room for a slab of every slot.
        lib = nat.lib()
        entries = (nat.HandoffLayer * layers)()
        rows = []
        offsets = [0]
        for (m0, dense, mask) in prepared:
            banks, slots, _ = dense.shape
            r = max(banks * slots, max((c for c in capacities if c is not None), default=0))
            rows.append(r)
            offsets.append(offsets[-1] + -(-int(lib.cowsdm_workspace_bytes(banks * slots, r)) // 256) * 256)
        workspace = torch.empty(max(offsets[-1], 256), dtype=torch.uint8, device=device)
        totals = torch.empty(layers, device=device, dtype=torch.int64)
        checks = torch.empty(layers, 9, device=device, dtype=torch.int64)
        tmpl = template_indices.to(torch.int64).contiguous()
        keep = [workspace, totals, checks, tmpl]
        for l, (m0, dense, mask) in enumerate(prepared):
            e = entries[l]
            e.dense_memory = dense.data_ptr()
            e.active_mask = mask.data_ptr()
            e.banks, e.slots, e.width = dense.shape
            e.workspace = workspace.data_ptr() + offsets[l]
            e.total = totals.data_ptr() + 8 * l
            e.template_indices = tmpl.data_ptr()
            e.templates = m0.shape[0]
            e.checks = checks.data_ptr() + 72 * l
        nat.check(lib.cowsdm_handoff_count(entries, layers, stream), "cowsdm_handoff_count")
        counts = totals.tolist()
        states = []
        for l, ((m0, dense, mask), active_count) in enumerate(zip(prepared, counts)):
            banks, slots, width = dense.shape
            selected, possible = handoff_capacity(
                active_count, banks, slots, capacities[l], growth_quantum_rows,
                maximum_future_allocations)
            state, _ = cls._allocate_state(
                m0, banks=banks, capacity_rows=selected, template_indices=template_indices,
                state_dtype=state_dtype, growth_quantum_rows=growth_quantum_rows,
                initialize=False)
            e = entries[l]
            if rows[l] < selected:
                # a slab larger than the workspace's lists: count again into one
                own = _workspace(banks * slots, selected, device)
                keep.append(own)
                e.workspace = own.data_ptr()
                nat.check(lib.cowsdm_handoff_count(ctypes.byref(e), 1, stream),
                          "cowsdm_handoff_count")
            e.logical_to_physical = state.logical_to_physical.data_ptr()
            e.values = state.values.data_ptr()
            e.free_rows = state.free_rows.data_ptr()
            e.capacity_rows = selected
            e.free_count = state.free_count.data_ptr()
            e.overflow_flag = state.overflow_flag.data_ptr()
            e.scratch = state.scratch.data_ptr()
            e.scratch_words = state.scratch.numel()
            state.capacity_is_proven = maximum_future_allocations is not None
            state.proven_maximum_additional_allocations = possible
            states.append(state)
        nat.check(lib.cowsdm_handoff_pack(entries, layers, stream), "cowsdm_handoff_pack")
        # the template checks and every layer's invariants, read once
        for state, words in zip(states, checks.tolist()):
            if words[8] & nat.ERR_TEMPLATE:
                raise ValueError("template index lies outside shared initial memory")
            state._judge_invariants(words[:8])
        del keep
        if map_page_slots is not None:
            for state in states:
                state.to_paged_map(map_page_slots)
        return states

    # ------------------------------------------------------- map forms

    @torch.no_grad()
    def to_paged_map(self, page_slots: int) -> None:
        """Keep the map paged, ``page_slots`` slots per page (a power of two
        from 2 to 64 dividing N): only pages holding a mapped slot are
        stored.  No counterpart in the reference."""

        mapping = self.direct_map()
        self.paged_map = PagedSlotMap.compress(mapping, page_slots)
        self.logical_to_physical = _map_placeholder(*mapping.shape)

    @torch.no_grad()
    def to_direct_map(self) -> None:
        """Keep the map as the direct [B, N] table again."""

        if self.paged_map is not None:
            mapping = self.paged_map.expand()
            self.paged_map = None
            self.logical_to_physical = mapping

    def direct_map(self) -> torch.Tensor:
        """The direct map [B, N] int32 (-1 = shared M0), built from the pages
        when the map is paged."""

        return self.logical_to_physical if self.paged_map is None else self.paged_map.expand()

    @contextmanager
    def _direct_form(self, *, keep: bool = True):
        """A lifecycle operation on a paged state runs on the direct map:
        expanded for it, then (``keep``: the operation changes the map)
        packed back into pages, renumbered in row-major order."""

        paged = self.paged_map
        if paged is None:
            yield
            return
        mapping = paged.expand()
        self.paged_map = None
        self.logical_to_physical = mapping
        try:
            yield
        finally:
            if keep:
                mapping = self.logical_to_physical
                self.paged_map = PagedSlotMap.compress(mapping, paged.page_slots)
            else:
                self.paged_map = paged
            self.logical_to_physical = _map_placeholder(*mapping.shape)

    # ------------------------------------------------------------ growth

    @torch.no_grad()
    def grow_capacity(self, minimum_capacity_rows: int) -> int:
        """Grow the shared value slab without changing logical state
        (allocator.py:691-743).  Row ids stay stable; new ids join the top of
        the free stack; every old row is counted as copied, as the reference
        counts them, though a slab growing within its headroom moves none."""

        if minimum_capacity_rows <= self.capacity_rows:
            return 0
        quantum = self.growth_quantum_rows
        if quantum <= 0:
            raise ValueError("SDM COW slab growth is disabled")
        selected = growth_target(minimum_capacity_rows, quantum)
        if selected >= 2**31:
            raise ValueError("SDM COW slab cannot grow past 2^31 rows")
        old_capacity = self.capacity_rows
        added = selected - old_capacity
        device = self.values.device
        buffers = self.slab_buffers
        if (buffers is not None and buffers[0].shape[0] >= selected
                and buffers[0].data_ptr() == self.values.data_ptr()
                and buffers[1].data_ptr() == self.free_rows.data_ptr()):
            # the slab leads a buffer with room: grow in place
            values, free_rows = buffers[0][:selected], buffers[1][:selected]
        else:
            # new buffers with headroom for as much growth again (at most
            # one row per logical slot beyond it), so that the growths of a
            # decode move rows a logarithmic number of times
            room = max(selected, min(growth_target(2 * selected, quantum),
                                     selected + self.banks * self.slots))
            if room >= 2**31:
                room = selected
            vbuf = torch.empty(room, self.width, device=device, dtype=self.values.dtype)
            fbuf = torch.empty(room, device=device, dtype=self.free_rows.dtype)
            self.slab_buffers = (vbuf, fbuf)
            values, free_rows = vbuf[:selected], fbuf[:selected]
        nat.check(
            nat.lib().cowsdm_grow(
                self.values.data_ptr(), old_capacity, values.data_ptr(), selected,
                self.width, self.free_rows.data_ptr(), free_rows.data_ptr(),
                self.free_count.data_ptr(), self.overflow_flag.data_ptr(),
                nat.stream_handle(device)),
            "cowsdm_grow",
        )
        self.values = values
        self.free_rows = free_rows
        self.proven_maximum_additional_allocations += added
        self.growth_events += 1
        self.growth_rows_added += added
        self.growth_rows_copied += old_capacity
        return added

    @torch.no_grad()
    def reserve_rows(self, rows: int) -> None:
        """Make ``values`` and ``free_rows`` lead buffers of at least
        ``rows`` rows, so that growth up to that capacity (on the host or
        inside a decode trace) moves no rows.  Capacity, logical state and
        growth counters are unchanged.  No counterpart in the reference."""

        rows = int(rows)
        if rows >= 2**31:
            raise ValueError("SDM COW slab cannot grow past 2^31 rows")
        buffers = self.slab_buffers
        if (buffers is not None and buffers[0].data_ptr() == self.values.data_ptr()
                and buffers[1].data_ptr() == self.free_rows.data_ptr()
                and min(buffers[0].shape[0], buffers[1].shape[0]) >= rows):
            return
        if rows <= self.capacity_rows and buffers is None:
            return
        capacity = self.capacity_rows
        rows = max(rows, capacity)
        vbuf = torch.empty(rows, self.width, device=self.values.device, dtype=self.values.dtype)
        fbuf = torch.empty(rows, device=self.values.device, dtype=self.free_rows.dtype)
        vbuf[:capacity].copy_(self.values)
        fbuf[:capacity].copy_(self.free_rows)
        self.slab_buffers = (vbuf, fbuf)
        self.values, self.free_rows = vbuf[:capacity], fbuf[:capacity]

    @torch.no_grad()
    def prepare_step_capacity(self, maximum_new_rows: int) -> int:
        """Prove one fused decode step, growing pooled headroom if short
        (allocator.py:745-773).  Host bookkeeping; reads free_count only
        when the running proof is exhausted."""

        if maximum_new_rows < 0:
            raise ValueError("maximum new SDM rows cannot be negative")
        if self.growth_quantum_rows <= 0:
            if not self.capacity_is_proven:
                raise ValueError("SDM COW capacity has no decode proof")
            return 0
        if self.proven_maximum_additional_allocations < maximum_new_rows:
            free_rows = self._read_free_count()
            if free_rows < maximum_new_rows:
                self.grow_capacity(self.capacity_rows + maximum_new_rows - free_rows)
                free_rows = int(self.free_count.item())
            self.proven_maximum_additional_allocations = free_rows
        self.proven_maximum_additional_allocations -= maximum_new_rows
        self.capacity_is_proven = True
        return self.capacity_rows

    @staticmethod
    @torch.no_grad()
    def prepare_step_capacity_layers(states: Sequence["PackedSDMCopyOnWriteState"],
                                     maximum_new_rows: int,
                                     free_counts: Sequence[int] | None = None) -> list[int]:
        """``prepare_step_capacity(maximum_new_rows)`` on every state, with
        the free counts the proofs need read in one device-to-host transfer
        (or taken from ``free_counts``, one per state, when the caller has
        just read them at the same point of the stream).

        Decisions equal separate calls made at the same point of the stream:
        each state still reads its free count only when its running proof is
        exhausted, and a grown slab's free count is known on the host (old
        free count plus the rows added)."""

        if maximum_new_rows < 0:
            raise ValueError("maximum new SDM rows cannot be negative")
        picks = [i for i, st in enumerate(states)
                 if st.growth_quantum_rows > 0
                 and st.proven_maximum_additional_allocations < maximum_new_rows]
        short = [states[i] for i in picks]
        if short:
            if free_counts is not None:
                frees = [int(free_counts[i]) for i in picks]
            else:
                # the free counts and the kernels' error words in one read
                words = torch.stack([st.free_count.to(torch.int64) for st in short]
                                    + [st.ensure_scratch()[nat.SCRATCH_ERRORS] for st in short])
                words = words.tolist()
                frees = words[:len(short)]
                for st, errors in zip(short, words[len(short):]):
                    st._raise_on_fault(errors)
            for st, free_rows in zip(short, frees):
                if free_rows < maximum_new_rows:
                    free_rows += st.grow_capacity(
                        st.capacity_rows + maximum_new_rows - free_rows)
                st.proven_maximum_additional_allocations = free_rows
        capacities = []
        for st in states:
            if st.growth_quantum_rows <= 0:
                if not st.capacity_is_proven:
                    raise ValueError("SDM COW capacity has no decode proof")
                capacities.append(0)
                continue
            st.proven_maximum_additional_allocations -= maximum_new_rows
            st.capacity_is_proven = True
            capacities.append(st.capacity_rows)
        return capacities

    def _read_free_count(self) -> int:
        """free_count, read with the kernels' sticky error word (one
        transfer); raises when a step stopped on a fault."""

        words = torch.stack([self.free_count.to(torch.int64),
                             self.ensure_scratch()[nat.SCRATCH_ERRORS]]).tolist()
        self._raise_on_fault(words[1])
        return int(words[0])

    @staticmethod
    def _raise_on_fault(errors: int) -> None:
        # a bounded wait that gave up, or state found outside the slab: the
        # step left the state inconsistent (the bits latch until cleared)
        if errors & (nat.ERR_LOOKBACK | nat.ERR_CORRUPT):
            raise RuntimeError(f"an SDM COW step stopped on a fault (error word {errors:#x}): "
                               "a bounded wait timed out or the state is corrupt")

    # -------------------------------------------------------- lifecycle

    def _count_live(self, mapping: torch.Tensor, workspace: torch.Tensor,
                    bank_list: torch.Tensor | None = None) -> torch.Tensor:
        total = torch.empty(1, device=mapping.device, dtype=torch.int64)
        nsel = mapping.shape[0] if bank_list is None else bank_list.numel()
        nat.check(
            nat.lib().cowsdm_count_active(
                mapping.data_ptr(), mapping.shape[0], mapping.shape[1], nat.ptr(bank_list),
                nsel, None,
                workspace.data_ptr(), total.data_ptr(), nat.stream_handle(mapping.device)),
            "cowsdm_count_active",
        )
        return total

    @torch.no_grad()
    def trim_capacity(self, *, headroom_rows: int = 0) -> int:
        """Repack live rows and return unused slab rows (allocator.py:775-839)."""

        if self.paged_map is not None:
            with self._direct_form():
                return self.trim_capacity(headroom_rows=headroom_rows)
        if headroom_rows < 0:
            raise ValueError("SDM trim headroom cannot be negative")
        quantum = self.growth_quantum_rows
        if quantum <= 0:
            raise ValueError("SDM COW slab trimming requires copy-on-write capacity")
        device = self.values.device
        entries = self.banks * self.slots
        workspace = _workspace(entries, self.capacity_rows, device)
        active_count = int(self._count_live(self.logical_to_physical, workspace).item())
        selected = trim_target(active_count, headroom_rows, quantum)
        if selected >= self.capacity_rows:
            return 0
        values = torch.empty(selected, self.width, device=device, dtype=self.values.dtype)
        mapping = torch.empty_like(self.logical_to_physical)
        free_rows = torch.empty(selected, device=device, dtype=self.free_rows.dtype)
        nat.check(
            nat.lib().cowsdm_trim_repack(
                self.logical_to_physical.data_ptr(), self.values.data_ptr(),
                self.capacity_rows, self.banks,
                self.slots, self.width, mapping.data_ptr(), values.data_ptr(),
                free_rows.data_ptr(), selected, self.free_count.data_ptr(),
                self.overflow_flag.data_ptr(), workspace.data_ptr(),
                nat.stream_handle(device)),
            "cowsdm_trim_repack",
        )
        removed = self.capacity_rows - selected
        self.values = values
        self.logical_to_physical = mapping
        self.free_rows = free_rows
        self.slab_buffers = None
        self.capacity_is_proven = False
        self.proven_maximum_additional_allocations = selected - active_count
        return removed

    @torch.no_grad()
    def append_banks_from(self, other: "PackedSDMCopyOnWriteState") -> int:
        """Move another cohort's banks into this pool (allocator.py:841-914).
        Only live rows are copied, into rows popped from the top of this free
        stack in the other map's row-major order."""

        if self.paged_map is not None or other.paged_map is not None:
            with self._direct_form(), other._direct_form(keep=False):
                return self.append_banks_from(other)
        if (
            other.slots != self.slots
            or other.width != self.width
            or other.values.device != self.values.device
            or other.values.dtype != self.values.dtype
            or other.shared_initial_memory.shape != self.shared_initial_memory.shape
        ):
            raise ValueError("admitted SDM banks do not match the destination pool")
        if (
            other.shared_initial_memory.data_ptr() != self.shared_initial_memory.data_ptr()
            and not torch.equal(other.shared_initial_memory, self.shared_initial_memory)
        ):
            raise ValueError("admitted SDM banks use different learned initial memory")
        device = self.values.device
        other_entries = other.banks * other.slots
        workspace = _workspace(other_entries, other.capacity_rows, device)
        active_count = int(self._count_live(other.logical_to_physical, workspace).item())
        free_count = int(self.free_count.item())
        if free_count < active_count:
            self.grow_capacity(self.capacity_rows + active_count - free_count)
        banks = self.banks + other.banks
        mapping = torch.empty(banks, self.slots, device=device, dtype=torch.int32)
        templates = torch.empty(banks, device=device, dtype=torch.int64)
        nat.check(
            nat.lib().cowsdm_append_banks(
                self.logical_to_physical.data_ptr(), self.template_indices.data_ptr(),
                self.banks, self.values.data_ptr(), self.capacity_rows,
                self.free_rows.data_ptr(), self.free_count.data_ptr(),
                other.logical_to_physical.data_ptr(), other.template_indices.data_ptr(),
                other.values.data_ptr(), other.banks, other.capacity_rows, self.slots,
                self.width, mapping.data_ptr(), templates.data_ptr(),
                workspace.data_ptr(), nat.stream_handle(device)),
            "cowsdm_append_banks",
        )
        self.logical_to_physical = mapping
        self.template_indices = templates
        self.scratch = _scratch(banks, device)
        if self.growth_quantum_rows:
            self.proven_maximum_additional_allocations = min(
                self.proven_maximum_additional_allocations, int(self.free_count.item()))
        else:
            self.capacity_is_proven = False
            self.proven_maximum_additional_allocations = 0
        return active_count

    def _bank_list(self, bank_indices: torch.Tensor, what: str) -> torch.Tensor:
        if (
            bank_indices.ndim != 1
            or bank_indices.dtype not in (torch.int32, torch.int64)
            or bank_indices.device != self.values.device
        ):
            raise ValueError(f"{what} bank indices must be integer [S] on device")
        return bank_indices.to(torch.int64).contiguous()

    def _check_banks(self, bank_list: torch.Tensor, discarded_active: bool) -> int:
        device = self.values.device
        workspace = _workspace(self.banks * self.slots, self.banks, device)
        result = torch.empty(1, device=device, dtype=torch.int64)
        nat.check(
            nat.lib().cowsdm_check_banks(
                self.logical_to_physical.data_ptr(), self.banks, self.slots,
                bank_list.data_ptr(), bank_list.numel(), int(discarded_active),
                workspace.data_ptr(), result.data_ptr(), nat.stream_handle(device)),
            "cowsdm_check_banks",
        )
        return int(result.item())

    @torch.no_grad()
    def retain_banks(self, bank_indices: torch.Tensor) -> None:
        """Compact already-released banks; values never move
        (allocator.py:916-942)."""

        if self.paged_map is not None:
            with self._direct_form():
                return self.retain_banks(bank_indices)
        bank_list = self._bank_list(bank_indices, "retained")
        flags = self._check_banks(bank_list, discarded_active=True)
        if flags & 1:
            raise ValueError("retained bank index is invalid or duplicated")
        if flags & 2:
            raise ValueError("discarded SDM banks must be released before compaction")
        device = self.values.device
        nsel = bank_list.numel()
        mapping = torch.empty(nsel, self.slots, device=device, dtype=torch.int32)
        templates = torch.empty(nsel, device=device, dtype=torch.int64)
        nat.check(
            nat.lib().cowsdm_retain_banks(
                self.logical_to_physical.data_ptr(), self.template_indices.data_ptr(),
                self.banks, self.slots, bank_list.data_ptr(), nsel, mapping.data_ptr(),
                templates.data_ptr(), nat.stream_handle(device)),
            "cowsdm_retain_banks",
        )
        self.logical_to_physical = mapping
        self.template_indices = templates
        self.scratch = _scratch(nsel, device)

    @torch.no_grad()
    def release(self, bank_indices: torch.Tensor) -> torch.Tensor:
        """Release whole banks and push their rows on the free stack
        (allocator.py:1018-1067).  Returns the released row count (0-d)."""

        if self.paged_map is not None:
            with self._direct_form():
                return self.release(bank_indices)
        bank_list = self._bank_list(bank_indices, "released")
        if bank_list.numel() == 0:
            return self.free_count.new_zeros(())
        if self._check_banks(bank_list, discarded_active=False) & 1:
            raise ValueError("released bank index is invalid or duplicated")
        device = self.values.device
        nsel = bank_list.numel()
        workspace = _workspace(nsel * self.slots, 0, device)
        self._count_live(self.logical_to_physical, workspace, bank_list)
        released = torch.empty((), device=device, dtype=torch.int64)
        nat.check(
            nat.lib().cowsdm_release(
                self.logical_to_physical.data_ptr(), self.banks, self.slots,
                bank_list.data_ptr(), nsel,
                self.free_rows.data_ptr(), self.capacity_rows, self.free_count.data_ptr(),
                workspace.data_ptr(), released.data_ptr(), nat.stream_handle(device)),
            "cowsdm_release",
        )
        return released

    # ------------------------------------------------------ properties

    @property
    def banks(self) -> int:
        return self.logical_to_physical.shape[0]

    @property
    def slots(self) -> int:
        return self.logical_to_physical.shape[1]

    @property
    def width(self) -> int:
        return self.values.shape[1]

    @property
    def capacity_rows(self) -> int:
        return self.values.shape[0]

    def allocated_rows_tensor(self) -> torch.Tensor:
        """Device-resident number of live physical rows (allocator.py:960-963)."""

        return self.free_count.new_tensor(self.capacity_rows) - self.free_count

    def storage_bytes(self) -> dict[str, int]:
        """Retained tensor storage, shared model state separate
        (allocator.py:965-982); ``step_scratch`` (allocator metadata) and
        ``slab_headroom`` (growth room beyond the capacity rows) are this
        build's extras."""

        paged = self.paged_map
        private = {
            "value_slab_reserved": _tensor_bytes(self.values),
            # a paged map: its directory and page pool
            "logical_to_physical": (_tensor_bytes(self.logical_to_physical) if paged is None
                                    else paged.storage_bytes()),
            "free_row_stack": _tensor_bytes(self.free_rows),
            "free_count": _tensor_bytes(self.free_count),
            "overflow_flag": _tensor_bytes(self.overflow_flag),
            "template_indices": _tensor_bytes(self.template_indices),
            "step_scratch": 0 if self.scratch is None else _tensor_bytes(self.scratch),
            # this build's growth headroom beyond the capacity rows
            "slab_headroom": 0 if self.slab_buffers is None else (
                _tensor_bytes(self.slab_buffers[0]) - _tensor_bytes(self.values)
                + _tensor_bytes(self.slab_buffers[1]) - _tensor_bytes(self.free_rows)),
        }
        private["private_allocator_reserved_total"] = sum(private.values())
        private["shared_initial_memory"] = _tensor_bytes(self.shared_initial_memory)
        private["including_shared_initial_memory"] = (
            private["private_allocator_reserved_total"] + private["shared_initial_memory"]
        )
        return private

    def used_bytes(self) -> dict[str, int]:
        """Live-row bytes plus resident metadata (allocator.py:984-1001)."""

        allocated = int(self.allocated_rows_tensor().item())
        live_values = allocated * self.width * self.values.element_size()
        metadata = (
            (_tensor_bytes(self.logical_to_physical) if self.paged_map is None
             else self.paged_map.used_bytes())
            + _tensor_bytes(self.free_rows)
            + _tensor_bytes(self.free_count)
            + _tensor_bytes(self.overflow_flag)
            + _tensor_bytes(self.template_indices)
            + (0 if self.scratch is None else _tensor_bytes(self.scratch))
        )
        return {
            "allocated_rows": allocated,
            "live_value_bytes": live_values,
            "allocator_metadata_bytes": metadata,
            "private_live_total": live_values + metadata,
        }

    @torch.no_grad()
    def materialize_dense(self) -> torch.Tensor:
        """Effective [B,N,D] table for validation (allocator.py:1003-1016)."""

        if self.paged_map is not None:
            with self._direct_form(keep=False):
                return self.materialize_dense()
        device = self.values.device
        dense = torch.empty(self.banks, self.slots, self.width, device=device,
                            dtype=self.values.dtype)
        nat.check(
            nat.lib().cowsdm_materialize_dense(
                self.shared_initial_memory.data_ptr(), self.shared_initial_memory.shape[0],
                self.template_indices.data_ptr(),
                self.values.data_ptr(), self.logical_to_physical.data_ptr(), self.banks,
                self.slots, self.width, self.capacity_rows, dense.data_ptr(),
                nat.stream_handle(device)),
            "cowsdm_materialize_dense",
        )
        return dense

    @torch.no_grad()
    def validate_invariants(self) -> dict[str, Any]:
        """Synchronously validate row ownership and the free-list partition
        (allocator.py:1069-1095); also surfaces the kernels' sticky error
        word."""

        stats = torch.empty(8, device=self.values.device, dtype=torch.int64)
        self._launch_invariants(stats)
        return self._judge_invariants(stats.tolist())

    @staticmethod
    @torch.no_grad()
    def validate_invariants_layers(states: Sequence["PackedSDMCopyOnWriteState"]) -> list[dict]:
        """``validate_invariants`` of every state with one device-to-host
        read for all of them.  No counterpart in the reference."""

        if not states:
            return []
        stats = torch.empty(len(states), 8, device=states[0].values.device, dtype=torch.int64)
        for st, row in zip(states, stats):
            st._launch_invariants(row)
        return [st._judge_invariants(row) for st, row in zip(states, stats.tolist())]

    def _launch_invariants(self, stats: torch.Tensor) -> None:
        """Enqueue the invariant counts (8 int64 words) into ``stats``."""

        if self.paged_map is not None:
            with self._direct_form(keep=False):
                return self._launch_invariants(stats)
        device = self.values.device
        workspace = _workspace(self.banks * self.slots, self.capacity_rows, device)
        nat.check(
            nat.lib().cowsdm_check_invariants(
                self.logical_to_physical.data_ptr(), self.banks, self.slots,
                self.free_rows.data_ptr(), self.free_count.data_ptr(),
                self.overflow_flag.data_ptr(), nat.ptr(self.scratch), self.capacity_rows,
                workspace.data_ptr(), stats.data_ptr(), nat.stream_handle(device)),
            "cowsdm_check_invariants",
        )

    def _judge_invariants(self, stats: Sequence[int]) -> dict[str, Any]:
        """The reference's assertions (allocator.py:1077-1089) on the counts."""

        (live, free, dup_live, dup_free, not_once, outside, overflow, errors) = (
            int(x) for x in stats)
        if overflow != 0:
            raise AssertionError("SDM COW allocator recorded a slab overflow")
        if errors != 0:
            raise AssertionError(f"SDM COW kernels recorded errors (flags {errors:#x})")
        if dup_live:
            raise AssertionError("one physical SDM row has multiple logical owners")
        if dup_free:
            raise AssertionError("free SDM row stack contains duplicates")
        if live + free != self.capacity_rows:
            raise AssertionError("active and free SDM rows do not cover capacity")
        if not_once or outside:
            raise AssertionError("active and free SDM rows do not partition the slab")
        return {
            "capacity_rows": self.capacity_rows,
            "allocated_rows": live,
            "free_rows": free,
            "exact_partition": True,
        }

    def ensure_scratch(self) -> torch.Tensor:
        if self.scratch is None or self.scratch.numel() != int(
                nat.lib().cowsdm_step_scratch_words(self.banks)):
            self.scratch = _scratch(self.banks, self.values.device)
        return self.scratch


# ------------------------------------------------------------- validation


def _validate_indices(indices: torch.Tensor, *, name: str, banks: int,
                      device: torch.device) -> None:
    """Host half of _validate_indices (allocator.py:1107-1126); bounds are
    checked on the device."""

    if (
        indices.ndim != 2
        or indices.shape[0] != banks
        or indices.shape[1] <= 0
        or indices.dtype not in (torch.int32, torch.int64)
        or indices.device != device
    ):
        raise ValueError(f"{name} indices must be integer [B,K] on device")


def _validate_gates(input_gate, erase_gate, forget_log_gate, *, banks: int) -> None:
    """allocator.py:1143-1155."""

    if input_gate.shape != (banks,):
        raise ValueError("native SDM input gate must be [B]")
    if erase_gate.shape != input_gate.shape or forget_log_gate.shape != input_gate.shape:
        raise ValueError("SDM input, erase, and forget gates must align")


def _select_backend(backend: str, *, tensor: torch.Tensor, writes: int, reads: int) -> bool:
    """Backend dispatch (allocator.py:1158-1176): the HIP kernels run every
    backend but "triton"; True for "torch", whose exhaustion check runs
    before every step (allocator.py:1474)."""

    if backend not in ("auto", "torch", "triton", "hip"):
        raise ValueError("allocator backend must be auto, hip, torch, or triton")
    if backend == "triton":
        raise RuntimeError("the requested Triton SDM COW backend is unavailable")
    _require_device(tensor, "SDM COW step tensors")
    if writes > 64 or reads > 256:
        raise ValueError("HIP SDM COW step supports at most 64 writes and 256 reads")
    return backend == "torch"


_NARROW_FLOATS = (torch.float16, torch.bfloat16)


def _widen(tensor: torch.Tensor) -> torch.Tensor:
    """A 16-bit float route weight, value or gate tensor widened to float32 on
    the device (exact), as both reference backends take them: the Triton
    kernels load and convert to float32 (allocator.py:74-229), the torch path
    calls .float() (allocator.py:1136-1139, 1490-1498)."""

    return tensor.float() if tensor.dtype in _NARROW_FLOATS else tensor


def _check_float_tensors(tensors: Sequence[torch.Tensor]) -> None:
    for tensor in tensors:
        if tensor.dtype != torch.float32:
            raise ValueError("HIP SDM COW step takes float32 weights, values and gates")
        if not tensor.is_contiguous():
            raise ValueError("HIP SDM COW step tensors must be contiguous")


def _index_code(write_indices: torch.Tensor, read_indices: torch.Tensor) -> int:
    if write_indices.dtype != read_indices.dtype:
        raise ValueError("write and read indices must share one integer dtype")
    if not (write_indices.is_contiguous() and read_indices.is_contiguous()):
        raise ValueError("HIP SDM COW step tensors must be contiguous")
    return nat.INDEX_INT64 if write_indices.dtype == torch.int64 else nat.INDEX_INT32


def _raise_precheck(flags: int, *, packed: bool) -> None:
    """Reference messages, in the reference's check order."""

    if flags & nat.ERR_WRITE_INDEX:
        raise ValueError("write index lies outside the logical table")
    if flags & nat.ERR_READ_INDEX:
        raise ValueError("read index lies outside the logical table")
    if flags & nat.ERR_DUP_WRITE:
        raise ValueError("one SDM step cannot write one logical slot twice")
    if flags & nat.ERR_CORRUPT:
        raise AssertionError("SDM COW logical map holds a row outside the slab")
    if packed and flags & nat.ERR_EXHAUSTED:
        raise ValueError("SDM COW physical slab is exhausted")


_precheck_buffers: dict[torch.device, torch.Tensor] = {}


def _precheck_result(device: torch.device) -> torch.Tensor:
    buf = _precheck_buffers.get(device)
    if buf is None:
        buf = torch.zeros(1, device=device, dtype=torch.int64)
        _precheck_buffers[device] = buf
    return buf


def _run_precheck(layer: nat.Layer, shape: nat.Shape, *, dense: bool, unique: bool,
                  capacity: bool, device: torch.device) -> None:
    result = _precheck_result(device)
    nat.check(
        nat.lib().cowsdm_step_precheck(
            layer, shape, int(dense), int(unique), int(capacity), result.data_ptr(),
            nat.stream_handle(device)),
        "cowsdm_step_precheck",
    )
    _raise_precheck(int(result.item()), packed=not dense)


# ------------------------------------------------------------------ steps


def _step_layer(
    state: PackedSDMCopyOnWriteState | None,
    memory: torch.Tensor | None,
    write_indices, write_weights, values, input_gate, erase_gate, forget_log_gate,
    read_indices, read_weights, output, first, repeated, allocated,
) -> nat.Layer:
    layer = nat.Layer()
    if state is not None:
        layer.shared_initial_memory = state.shared_initial_memory.data_ptr()
        layer.template_indices = state.template_indices.data_ptr()
        layer.values = state.values.data_ptr()
        paged = state.paged_map
        if paged is None:
            layer.logical_to_physical = state.logical_to_physical.data_ptr()
        else:
            layer.map_directory = paged.directory.data_ptr()
            layer.map_pages = paged.pages.data_ptr()
            layer.map_page_count = paged.page_count.data_ptr()
            layer.map_page_capacity = paged.capacity
            layer.map_page_shift = paged.page_shift
        layer.free_rows = state.free_rows.data_ptr()
        layer.free_count = state.free_count.data_ptr()
        layer.overflow_flag = state.overflow_flag.data_ptr()
        layer.scratch = state.ensure_scratch().data_ptr()
        layer.capacity_rows = state.capacity_rows
    else:
        layer.values = memory.data_ptr()
        layer.capacity_rows = 0
    layer.write_indices = write_indices.data_ptr()
    layer.write_weights = write_weights.data_ptr()
    layer.step_values = values.data_ptr()
    layer.input_gate = input_gate.data_ptr()
    layer.erase_gate = erase_gate.data_ptr()
    layer.forget_log_gate = forget_log_gate.data_ptr()
    layer.read_indices = read_indices.data_ptr()
    layer.read_weights = read_weights.data_ptr()
    layer.output = output.data_ptr()
    layer.first_touches_out = nat.ptr(first)
    layer.repeated_writes_out = nat.ptr(repeated)
    layer.allocated_rows_out = nat.ptr(allocated)
    return layer


def _check_step_inputs(banks, slots, width, device, write_indices, write_weights, values,
                       input_gate, forget_log_gate, read_indices, read_weights, erase_gate,
                       *, dense: bool):
    _validate_indices(write_indices, name="write", banks=banks, device=device)
    _validate_indices(read_indices, name="read", banks=banks, device=device)
    if (
        write_weights.shape != write_indices.shape
        or read_weights.shape != read_indices.shape
        or values.shape != (banks, width)
    ):
        raise ValueError(
            "dense SDM route weights and values do not align" if dense
            else "SDM route weights and values do not align")
    tensors = (write_weights, values, input_gate, forget_log_gate, read_weights) + (
        () if erase_gate is None else (erase_gate,))
    if any(tensor.device != device for tensor in tensors):
        raise ValueError(
            "dense SDM step tensors must share one device" if dense
            else "SDM COW step tensors must share one device")
    effective_erase = input_gate if erase_gate is None else erase_gate
    _validate_gates(input_gate, effective_erase, forget_log_gate, banks=banks)
    return effective_erase


def _shape(banks, slots, width, writes, reads, templates, index_code) -> nat.Shape:
    shape = nat.Shape()
    shape.banks = banks
    shape.slots = slots
    shape.width = width
    shape.writes = writes
    shape.reads = reads
    shape.templates = templates
    shape.index_dtype = index_code
    return shape


@torch.no_grad()
def packed_sdm_cow_step(
    state: PackedSDMCopyOnWriteState,
    write_indices: torch.Tensor,
    write_weights: torch.Tensor,
    values: torch.Tensor,
    input_gate: torch.Tensor,
    forget_log_gate: torch.Tensor,
    read_indices: torch.Tensor,
    read_weights: torch.Tensor,
    *,
    erase_gate: torch.Tensor | None = None,
    backend: str = "auto",
    validate_routes: bool = True,
    collect_diagnostics: bool = True,
) -> tuple[torch.Tensor, SDMCopyOnWriteStep | None]:
    """One exact sparse SDM write and read through the packed overlay
    (allocator.py:1381-1525), as one fused HIP launch.

    Per bank: resolve the W write routes through the map, pop free rows for
    first touches (bank-major), copy M0 rows, apply the gated-delta update in
    FP32, then the weighted read of R rows after the write.
    """

    banks, slots, width = state.banks, state.slots, state.width
    device = state.values.device
    effective_erase = _check_step_inputs(
        banks, slots, width, device, write_indices, write_weights, values, input_gate,
        forget_log_gate, read_indices, read_weights, erase_gate, dense=False)
    torch_checks = _select_backend(backend, tensor=state.values,
                                   writes=write_indices.shape[1], reads=read_indices.shape[1])
    # float16/bfloat16 weights, values and gates compute in float32; the
    # reading comes back in the values' dtype (allocator.py:1521)
    reading_dtype = values.dtype
    write_weights, values, input_gate, effective_erase, forget_log_gate, read_weights = (
        _widen(t) for t in (write_weights, values, input_gate, effective_erase,
                            forget_log_gate, read_weights))
    _check_float_tensors((write_weights, values, input_gate, effective_erase,
                          forget_log_gate, read_weights))
    index_code = _index_code(write_indices, read_indices)
    output = torch.empty_like(values)
    first = repeated = allocated = None
    if collect_diagnostics:
        first = torch.empty(banks, device=device, dtype=torch.int64)
        repeated = torch.empty(banks, device=device, dtype=torch.int64)
        allocated = torch.empty((), device=device, dtype=torch.int32)
    if state.paged_map is not None and banks:
        state.paged_map.prove(banks * write_indices.shape[1])
    layer = _step_layer(state, None, write_indices, write_weights, values, input_gate,
                        effective_erase, forget_log_gate, read_indices, read_weights, output,
                        first, repeated, allocated)
    shape = _shape(banks, slots, width, write_indices.shape[1], read_indices.shape[1],
                   state.shared_initial_memory.shape[0], index_code)
    if banks and (validate_routes or torch_checks or not state.capacity_is_proven):
        _run_precheck(layer, shape, dense=False, unique=validate_routes,
                      capacity=torch_checks or not state.capacity_is_proven, device=device)
    if banks:
        nat.check(nat.lib().cowsdm_packed_step(layer, shape, nat.stream_handle(device)),
                  "cowsdm_packed_step")
    elif allocated is not None:
        allocated = state.allocated_rows_tensor()
    if reading_dtype != output.dtype:
        output = output.to(reading_dtype)
    if not collect_diagnostics:
        return output, None
    return output, SDMCopyOnWriteStep(
        first_touches_by_sequence=first,
        repeated_writes_by_sequence=repeated,
        allocated_rows_after_step=allocated,
    )


@torch.no_grad()
def dense_sdm_sparse_step(
    memory: torch.Tensor,
    write_indices: torch.Tensor,
    write_weights: torch.Tensor,
    values: torch.Tensor,
    input_gate: torch.Tensor,
    forget_log_gate: torch.Tensor,
    read_indices: torch.Tensor,
    read_weights: torch.Tensor,
    *,
    erase_gate: torch.Tensor | None = None,
    backend: str = "auto",
    validate_routes: bool = True,
) -> torch.Tensor:
    """Dense-table control: the same sparse update and read on
    ``memory`` [B,N,D] (allocator.py:1528-1633).  Shares the packed step's
    row math, so both produce bit-identical state and readings."""

    if memory.ndim != 3:
        raise ValueError("dense SDM memory must be [B,N,D]")
    banks, slots, width = memory.shape
    device = memory.device
    effective_erase = _check_step_inputs(
        banks, slots, width, device, write_indices, write_weights, values, input_gate,
        forget_log_gate, read_indices, read_weights, erase_gate, dense=True)
    _select_backend(backend, tensor=memory, writes=write_indices.shape[1],
                    reads=read_indices.shape[1])
    reading_dtype = values.dtype
    write_weights, values, input_gate, effective_erase, forget_log_gate, read_weights = (
        _widen(t) for t in (write_weights, values, input_gate, effective_erase,
                            forget_log_gate, read_weights))
    _check_float_tensors((memory, write_weights, values, input_gate, effective_erase,
                          forget_log_gate, read_weights))
    index_code = _index_code(write_indices, read_indices)
    output = torch.empty_like(values)
    layer = _step_layer(None, memory, write_indices, write_weights, values, input_gate,
                        effective_erase, forget_log_gate, read_indices, read_weights, output,
                        None, None, None)
    shape = _shape(banks, slots, width, write_indices.shape[1], read_indices.shape[1], 1,
                   index_code)
    if banks and validate_routes:
        _run_precheck(layer, shape, dense=True, unique=True, capacity=False, device=device)
    if banks:
        nat.check(nat.lib().cowsdm_dense_step(layer, shape, nat.stream_handle(device)),
                  "cowsdm_dense_step")
    return output if reading_dtype == output.dtype else output.to(reading_dtype)


def _layer_arrays(count: int, *args):
    out = []
    for arg in args:
        if arg is None:
            out.append([None] * count)
        else:
            items = list(arg)
            if len(items) != count:
                raise ValueError("per-layer inputs must provide one entry per layer")
            out.append(items)
    return out


@torch.no_grad()
def packed_sdm_cow_step_layers(
    states: Sequence[PackedSDMCopyOnWriteState],
    write_indices, write_weights, values, input_gate, forget_log_gate,
    read_indices, read_weights,
    *,
    erase_gate=None,
    outputs: Sequence[torch.Tensor] | None = None,
    validate_routes: bool = False,
) -> list[torch.Tensor]:
    """``packed_sdm_cow_step`` for several independent layers in one launch.

    Every argument after ``states`` is a per-layer sequence (a stacked
    [L, ...] tensor works).  All layers share B, N, D, W, R and index dtype.
    Results equal L separate ``packed_sdm_cow_step`` calls.  No counterpart
    in the reference; meant for callers that hold all layers' routes, such as
    synthetic-route serving benchmarks.
    """

    count = len(states)
    if count == 0:
        return []
    (wi, ww, vv, ig, fg, ri, rw, eg, outs) = _layer_arrays(
        count, write_indices, write_weights, values, input_gate, forget_log_gate,
        read_indices, read_weights, erase_gate, outputs)
    first = states[0]
    device = first.values.device
    layers = (nat.Layer * count)()
    shape = None
    results = []
    for i, state in enumerate(states):
        if (state.banks, state.slots, state.width) != (first.banks, first.slots, first.width):
            raise ValueError("all layers of one launch must share banks, slots and width")
        effective_erase = _check_step_inputs(
            state.banks, state.slots, state.width, device, wi[i], ww[i], vv[i], ig[i], fg[i],
            ri[i], rw[i], eg[i], dense=False)
        _select_backend("auto", tensor=state.values, writes=wi[i].shape[1],
                        reads=ri[i].shape[1])
        _check_float_tensors((ww[i], vv[i], ig[i], effective_erase, fg[i], rw[i]))
        code = _index_code(wi[i], ri[i])
        out = outs[i] if outs[i] is not None else torch.empty_like(vv[i])
        results.append(out)
        if state.paged_map is not None and state.banks:
            state.paged_map.prove(state.banks * wi[i].shape[1])
        layers[i] = _step_layer(state, None, wi[i], ww[i], vv[i], ig[i], effective_erase,
                                fg[i], ri[i], rw[i], out, None, None, None)
        this_shape = _shape(state.banks, state.slots, state.width, wi[i].shape[1],
                            ri[i].shape[1], state.shared_initial_memory.shape[0], code)
        if shape is None:
            shape = this_shape
        elif (shape.writes, shape.reads, shape.index_dtype, shape.templates) != (
                this_shape.writes, this_shape.reads, this_shape.index_dtype,
                this_shape.templates):
            raise ValueError("all layers of one launch must share W, R and index dtype")
        if state.banks and (validate_routes or not state.capacity_is_proven):
            _run_precheck(layers[i], this_shape, dense=False, unique=validate_routes,
                          capacity=not state.capacity_is_proven, device=device)
    if first.banks:
        nat.check(nat.lib().cowsdm_packed_step_layers(
            layers, count, shape, nat.stream_handle(device)), "cowsdm_packed_step_layers")
    return results


@torch.no_grad()
def dense_sdm_sparse_step_layers(
    memories: Sequence[torch.Tensor],
    write_indices, write_weights, values, input_gate, forget_log_gate,
    read_indices, read_weights,
    *,
    erase_gate=None,
    outputs: Sequence[torch.Tensor] | None = None,
) -> list[torch.Tensor]:
    """``dense_sdm_sparse_step`` for several independent layers in one launch
    (the dense-table control of ``packed_sdm_cow_step_layers``)."""

    count = len(memories)
    if count == 0:
        return []
    (wi, ww, vv, ig, fg, ri, rw, eg, outs) = _layer_arrays(
        count, write_indices, write_weights, values, input_gate, forget_log_gate,
        read_indices, read_weights, erase_gate, outputs)
    device = memories[0].device
    layers = (nat.Layer * count)()
    shape = None
    results = []
    for i, memory in enumerate(memories):
        if memory.ndim != 3 or memory.shape != memories[0].shape:
            raise ValueError("all layers of one launch must share one [B,N,D] shape")
        banks, slots, width = memory.shape
        effective_erase = _check_step_inputs(
            banks, slots, width, device, wi[i], ww[i], vv[i], ig[i], fg[i], ri[i], rw[i],
            eg[i], dense=True)
        _select_backend("auto", tensor=memory, writes=wi[i].shape[1], reads=ri[i].shape[1])
        _check_float_tensors((memory, ww[i], vv[i], ig[i], effective_erase, fg[i], rw[i]))
        code = _index_code(wi[i], ri[i])
        out = outs[i] if outs[i] is not None else torch.empty_like(vv[i])
        results.append(out)
        layers[i] = _step_layer(None, memory, wi[i], ww[i], vv[i], ig[i], effective_erase,
                                fg[i], ri[i], rw[i], out, None, None, None)
        this_shape = _shape(banks, slots, width, wi[i].shape[1], ri[i].shape[1], 1, code)
        if shape is None:
            shape = this_shape
        elif (shape.writes, shape.reads, shape.index_dtype) != (
                this_shape.writes, this_shape.reads, this_shape.index_dtype):
            raise ValueError("all layers of one launch must share W, R and index dtype")
    if memories[0].shape[0]:
        nat.check(nat.lib().cowsdm_dense_step_layers(
            layers, count, shape, nat.stream_handle(device)), "cowsdm_dense_step_layers")
    return results


@torch.no_grad()
def mark_written(active: torch.Tensor, indices: torch.Tensor) -> None:
    """active[b, indices[b, k]] = True for every k (inference.py:332-347's
    union of written rows).  ``indices`` is [B, K] int32/int64."""

    if active.dtype != torch.bool or active.ndim != 2 or not active.is_contiguous():
        raise ValueError("active mask must be a contiguous bool [B,N] tensor")
    _require_device(active, "active mask")
    if indices.ndim != 2 or indices.shape[0] != active.shape[0] or indices.dtype not in (
            torch.int32, torch.int64) or indices.device != active.device:
        raise ValueError("written indices must be integer [B,K] on the mask device")
    indices = indices.contiguous()
    result = _precheck_result(active.device)
    nat.check(
        nat.lib().cowsdm_mark_written(
            active.data_ptr(), active.shape[0], active.shape[1], indices.data_ptr(),
            indices.shape[1],
            nat.INDEX_INT64 if indices.dtype == torch.int64 else nat.INDEX_INT32,
            result.data_ptr(), nat.stream_handle(active.device)),
        "cowsdm_mark_written",
    )


class DecodeTrace:
    """Routes of many decode steps for several independent layers, resident
    on the device, and the decode loop that runs them.

    Inputs are stacked [S, L, B, ...] (``values`` [S, L, B, D], gates
    [S, L, B]).  ``run(n)`` is the reference's decode loop for the next n
    steps of every layer (inference.py:538-566): before each step of a
    packed layer with a growth quantum, ``prepare_step_capacity(banks * W)``
    (allocator.py:745-773), then ``packed_sdm_cow_step``.  Readings, maps,
    slab rows, free stacks, capacities and growth counters equal that loop's
    bit for bit.

    When the shape allows it (W <= 4, R <= 16, D <= 256, banks <= 256 for
    packed state), the loop runs as persistent launches of up to
    ``max_steps_per_launch`` steps.  Each packed launch is planned on the
    device first: the capacity proof of every step, slab growth within the
    slab's buffers (``slab_buffers``) and the row of every first touch are
    decided before the steps run, from the control words (``control``: the
    proof counter, capacity, buffer rows, quantum, growth counters) that
    ``run`` uploads from the states and reads back, with the step counters,
    in one transfer.  A layer whose growth would pass its buffers stops
    there; the host then grows it exactly as ``prepare_step_capacity`` does
    and decoding goes on.  Otherwise each step is one launch after a host
    proof.

    ``launch(k)`` enqueues k steps of every layer from its device counter
    (``step_index[l]``), which the kernels advance, so a captured hipGraph of
    ``launch(k)`` replays k consecutive steps per replay without host work;
    for packed state call ``upload()`` before the first launch and ``sync()``
    after the last (and give the slabs room with ``reserve_steps``).
    ``outputs`` is [S, L, B, D] (one reading per step) or [L, B, D] (every
    step overwrites the same buffer).  ``memories`` given instead of
    ``states`` runs the dense-table control.  With ``repeat`` the inputs are
    [1, L, B, ...] buffers that the caller (or kernels captured before the
    launch) refills before every step: every launch reads them, the device
    counters count steps without bound, and only ``launch``/``capture`` of
    device-counted steps run (the decode of routes made token by token).  No
    counterpart in the reference.
    """

    _INPUTS = ("write_indices", "write_weights", "values", "input_gate", "erase_gate",
               "forget_log_gate", "read_indices", "read_weights")

    def __init__(self, *, states=None, memories=None, write_indices, write_weights, values,
                 input_gate, forget_log_gate, read_indices, read_weights, erase_gate=None,
                 outputs=None, persistent: bool = True, max_steps_per_launch: int = 512,
                 static_scan: bool = False, repeat: bool = False):
        if (states is None) == (memories is None):
            raise ValueError("give exactly one of states or memories")
        self.dense = memories is not None
        self.tables = list(memories if self.dense else states)
        layers = len(self.tables)
        if not 1 <= layers <= 8:
            raise ValueError("a decode trace drives 1 to 8 layers")
        erase_gate = input_gate if erase_gate is None else erase_gate
        self.inputs = dict(write_indices=write_indices, write_weights=write_weights,
                           values=values, input_gate=input_gate, erase_gate=erase_gate,
                           forget_log_gate=forget_log_gate, read_indices=read_indices,
                           read_weights=read_weights)
        steps = write_indices.shape[0]
        first = self.tables[0]
        banks = first.shape[0] if self.dense else first.banks
        width = first.shape[2] if self.dense else first.width
        device = first.device if self.dense else first.values.device
        for name, tensor in self.inputs.items():
            if tensor.shape[:3] != (steps, layers, banks) or not tensor.is_contiguous():
                raise ValueError(f"{name} must be a contiguous [S, L, B, ...] tensor")
            if tensor.device != device:
                raise ValueError("decode trace tensors must share one device")
        if outputs is None:
            outputs = torch.empty(layers, banks, width, device=device)
        if outputs.shape not in ((steps, layers, banks, width), (layers, banks, width)):
            raise ValueError("outputs must be [S, L, B, D] or [L, B, D]")
        self.outputs = outputs
        self.steps = steps
        self.device = device
        # one int64 report read back per round: row 0 the per-layer step
        # counters, row 1 the int32 status words, rows 2.. the control words
        # of packed layers (word k of layer l at row 2 + k)
        self._report = torch.zeros(2 + nat.CTRL_WORDS, layers, dtype=torch.int64, device=device)
        self._report_host = torch.empty(self._report.shape, dtype=torch.int64).pin_memory()
        self._report_ready = torch.cuda.Event()
        self.step_index = self._report[0]
        self.status = self._report[1].view(torch.int32)[:layers]
        self.control = self._report[2:]
        self._upload_buf = (torch.zeros(nat.CTRL_WORDS, layers, dtype=torch.int64).pin_memory()
                            if not self.dense else None)
        self._uploaded = None   # event after the last upload's copy
        # the states' versions when the device's control words and this
        # trace's layer structs last matched them, or None (dense tables
        # have no control words)
        self._synced_versions = () if self.dense else None
        self._counters_seen = [(0, 0, 0)] * layers
        self._status_clean = False      # every status word is known to be zero
        self._host_report = None        # nat.HostReport, made by the first run
        self._report_versions = None    # the states' versions the host report matches
        self._step_index_ptr = self.step_index.data_ptr()
        self.ticket = torch.zeros(1 + layers, dtype=torch.int64, device=device)
        self.banks, self.writes = banks, write_indices.shape[3]
        self.trace = nat.Trace()
        self.trace.step_index = self.step_index.data_ptr()
        self.trace.ticket = self.ticket.data_ptr()
        self.trace.status = self.status.data_ptr()
        for k, name in enumerate(self._INPUTS):
            tensor = self.inputs[name]
            self.trace.stride_bytes[k] = tensor.stride(0) * tensor.element_size()
        self.trace.stride_bytes[8] = (outputs.stride(0) * outputs.element_size()
                                      if outputs.ndim == 4 else 0)
        self.shape = _shape(banks, first.shape[1] if self.dense else first.slots, width,
                            write_indices.shape[3], read_indices.shape[3],
                            1 if self.dense else first.shared_initial_memory.shape[0],
                            _index_code(write_indices, read_indices))
        self.persistent = persistent
        self.max_steps_per_launch = max(1, min(512, int(max_steps_per_launch)))
        self.trace.persistent = int(persistent)
        self.trace.steps_recorded = steps
        self.repeat = bool(repeat)
        if self.repeat:
            if steps != 1:
                raise ValueError("a repeating decode trace takes [1, L, B, ...] input buffers")
            for k in range(9):
                self.trace.stride_bytes[k] = 0
            self.trace.steps_recorded = 1 << 62
        self.scan = None
        self.planned = False
        # static_scan: packed launches take their plan blocks from the
        # library's own device memory (cowsdm_packed_step_trace_static) and
        # this trace allocates nothing per launch
        self.static_scan = bool(static_scan) and not self.dense
        if not self.dense and persistent:
            words = int(nat.lib().cowsdm_trace_scan_words(banks, self.writes,
                                                          self.max_steps_per_launch))
            if not self.static_scan:
                self.scan = torch.zeros(layers, max(words, 1), dtype=torch.int64, device=device)
                self.trace.scan = self.scan.data_ptr()
                self.trace.scan_words = self.scan.shape[1]
            self.trace.scan_steps = self.max_steps_per_launch
            self.trace.control_stride = layers
        self._layers = None
        self._layers_versions = None     # the states' versions the layer structs match
        self._capacities = None          # the slab lengths the layer structs were built from
        self._positions = [0] * layers   # host copy of step_index, None when unknown

    # ------------------------------------------------------------ set-up

    def set_step(self, step: int) -> None:
        """Make the next device-counted launch run step ``step`` of every layer."""

        if not 0 <= step <= self.steps:
            raise ValueError("trace step outside the trace")
        self.step_index.fill_(step)
        self._positions = [step] * len(self.tables)

    def layer_array(self):
        """The per-layer C structs for the current state pointers (they
        change when a slab moves to larger buffers or is trimmed); rebuilt
        only when a pointer moved."""

        key = tuple((t.data_ptr(),) if self.dense else
                    (t.values.data_ptr(), t.free_rows.data_ptr(), t.free_count.data_ptr(),
                     t.overflow_flag.data_ptr(),
                     t.logical_to_physical.data_ptr() if t.paged_map is None else
                     (t.paged_map.directory.data_ptr(), t.paged_map.pages.data_ptr()),
                     t.template_indices.data_ptr(), t.shared_initial_memory.data_ptr(),
                     t.scratch.data_ptr() if t.scratch is not None else 0)
                    for t in self.tables)
        capacities = tuple(0 if self.dense else t.capacity_rows for t in self.tables)
        self._layers_versions = self._versions()
        self._capacities = list(capacities)
        if self._layers is not None and self._layers[0] == key:
            layers = self._layers[1]
            if self._layers[2] != capacities:
                for l, capacity in enumerate(capacities):
                    layers[l].capacity_rows = capacity
                self._layers = (key, layers, capacities)
            return layers
        count = len(self.tables)
        layers = (nat.Layer * count)()
        for l, table in enumerate(self.tables):
            x = {name: tensor[0, l] for name, tensor in self.inputs.items()}
            out = self.outputs[0, l] if self.outputs.ndim == 4 else self.outputs[l]
            layers[l] = _step_layer(
                None if self.dense else table, table if self.dense else None,
                x["write_indices"], x["write_weights"], x["values"], x["input_gate"],
                x["erase_gate"], x["forget_log_gate"], x["read_indices"], x["read_weights"],
                out, None, None, None)
        self._layers = (key, layers, capacities)
        if not self.dense:
            # planned persistent launches need the shape, the pointers'
            # alignment and the strides to allow a persistent kernel
            self.planned = self.persistent and bool(nat.lib().cowsdm_trace_persistent(
                layers, count, self.shape, self.trace, 0))
            self.trace.control = self.control.data_ptr() if self.planned else None
        return layers

    @staticmethod
    def _room(state: PackedSDMCopyOnWriteState) -> int:
        """Rows the slab can grow to without moving: its buffers' rows when
        values and free_rows lead them, else its capacity."""

        buffers = state.slab_buffers
        if (buffers is not None and buffers[0].data_ptr() == state.values.data_ptr()
                and buffers[1].data_ptr() == state.free_rows.data_ptr()):
            return min(buffers[0].shape[0], buffers[1].shape[0])
        return state.capacity_rows

    def need(self) -> int:
        """Rows the decode loop proves before each step: banks * W
        (inference.py:551-552)."""

        return self.banks * self.writes

    def _signature(self) -> list[tuple[int, int, int, int, int]]:
        """Per packed layer, the control words a launch reads from its state:
        proof counter, capacity, buffer rows, quantum and rows proven per step
        (zero for a layer without a growth quantum, whose decode makes no
        proof)."""

        need = self.need()
        return [(st.proven_maximum_additional_allocations, st.capacity_rows, self._room(st),
                 st.growth_quantum_rows, need if st.growth_quantum_rows > 0 else 0)
                for st in self.tables]

    def _versions(self) -> tuple:
        """The states' assignment counters (packed state), or () for dense
        tables, whose pointers never change."""

        return () if self.dense else tuple(st._version for st in self.tables)

    def upload(self, *, force: bool = True) -> None:
        """Write the packed layers' control words from their states and zero
        the growth counters the launches add to.  With ``force`` false the
        copy is skipped when no state changed since the device's words last
        matched them (after an upload, or a run or ``sync`` that read them
        back)."""

        if self.dense:
            return
        versions = self._versions()
        if not force and versions == self._synced_versions:
            return
        buf = self._upload_buf
        if self._uploaded is not None:
            self._uploaded.synchronize()   # the last upload has left the pinned buffer
        buf.zero_()
        for l, words in enumerate(self._signature()):
            for k, value in zip((nat.CTRL_PROVEN, nat.CTRL_CAPACITY, nat.CTRL_ROOM,
                                 nat.CTRL_QUANTUM, nat.CTRL_NEED), words):
                buf[k, l] = value
        self.control.copy_(buf, non_blocking=True)
        if self._uploaded is None:
            self._uploaded = torch.cuda.Event()
        self._uploaded.record()
        self._counters_seen = [(0, 0, 0)] * len(self.tables)
        self._synced_versions = versions

    def _absorb(self, per_layer, offset: int = 0, before: tuple | None = None) -> None:
        """Take the control words read back after launches (per layer, word
        k of layer l at per_layer[l][offset + k]) into the states: proof
        counter, capacity (grown within the buffers) and the growth the
        launches added since the last read (the device counters run from the
        last upload).  ``before``: the states' versions, when the caller has
        them."""

        tables = self.tables
        if before is None:
            before = self._versions()
        moved = False
        proven_k, capacity_k = offset + nat.CTRL_PROVEN, offset + nat.CTRL_CAPACITY
        events_k, added_k = offset + nat.CTRL_EVENTS, offset + nat.CTRL_ADDED
        copied_k = offset + nat.CTRL_COPIED
        # the slab lengths the layer structs were built from, while no state
        # changed since (a tensor's shape costs more than the whole check)
        known = self._capacities if self._layers_versions == before else None
        seen_all = self._counters_seen
        after = []
        for l, st in enumerate(tables):
            words = per_layer[l]
            d = st.__dict__
            proven = words[proven_k]
            if d["proven_maximum_additional_allocations"] != proven:
                # the assignment with its version count (__setattr__), inline
                d["proven_maximum_additional_allocations"] = proven
                d["_version"] = d["_version"] + 1
            capacity = words[capacity_k]
            if capacity != (known[l] if known is not None else st.values.shape[0]):
                vbuf, fbuf = st.slab_buffers
                st.values, st.free_rows = vbuf[:capacity], fbuf[:capacity]
                struct = self._layers[1][l] if known is not None else None
                if (struct is not None and struct.values == vbuf.data_ptr()
                        and struct.free_rows == fbuf.data_ptr()):
                    # grown within the buffers the layer struct points at:
                    # only its length changes
                    struct.capacity_rows = capacity
                    known[l] = capacity
                else:
                    moved = True
            seen = seen_all[l]
            if words[events_k] != seen[0] or words[added_k] != seen[1] or words[copied_k] != seen[2]:
                st.growth_events += words[events_k] - seen[0]
                st.growth_rows_added += words[added_k] - seen[1]
                st.growth_rows_copied += words[copied_k] - seen[2]
                seen_all[l] = (words[events_k], words[added_k], words[copied_k])
            if not d["capacity_is_proven"] and d["growth_quantum_rows"] > 0:
                st.capacity_is_proven = True
            after.append(d["_version"])
        # what matched the states before still matches them, except the
        # layer structs after a capacity grew
        after = tuple(after)
        if not moved and self._layers_versions == before:
            self._layers_versions = after
            key, structs, _ = self._layers
            self._layers = (key, structs, tuple(self._capacities))
        self._synced_versions = after if self._synced_versions == before else None

    def reported_live_rows(self) -> int | None:
        """The packed layers' live physical rows (capacity minus free count,
        allocator.py:960-963, summed) as the last ``run`` of this trace left
        them, from its report in host memory (no device read); None when
        there is no such report or this trace's states changed since.  Work
        enqueued on the states by other means (another trace's launches, a
        lifecycle call) after the run is not seen."""

        if (self.dense or self._report_versions is None or self._positions is None
                or self._report_versions != self._versions()):
            return None
        a = self._host_report.array
        base = nat.REPORT_CONTROL
        return int((a[:, base + nat.CTRL_CAPACITY] - a[:, base + nat.CTRL_FREE]).sum())

    def sync(self) -> None:
        """Read the control words back into the states after ``launch``
        calls (one synchronisation)."""

        if self.dense or not self.planned:
            return
        self._absorb([list(words) for words in zip(*self.control.tolist())])
        self._positions = None

    def reserve_steps(self, steps: int) -> None:
        """Give every packed slab buffers with room for ``steps`` more steps
        of first touches and the rounding of one growth, so that launches of
        that many steps grow on the device and never stop for the host.  No
        counterpart in the reference."""

        if self.dense:
            return
        need = self.need()
        for st in self.tables:
            q = st.growth_quantum_rows
            if q <= 0:
                continue   # a slab without a quantum never grows
            # a proof grows the slab to at most one step's need (rounded to
            # the quantum) past its live rows, and live rows never pass B * N
            want = min(st.capacity_rows + steps * need + q,
                       _ceil_to(st.banks * st.slots + need + q, q))
            st.reserve_rows(max(want, st.capacity_rows))
        self._layers = None

    # ---------------------------------------------------------- launches

    def capture(self, steps: int = 1) -> "torch.cuda.CUDAGraph":
        """A hipGraph of ``launch(steps)``: each replay runs the next
        ``steps`` steps of every layer from the device counters, the decode
        loop's proof and growth within the slab buffers included (packed
        state), with no host work and no synchronisation.  With one step per
        replay this is the reference's per-token loop (inference.py:538-566)
        as one graph launch per token.  Uploads the control words first; call
        ``sync()`` after the replays, and ``reserve_steps`` beforehand for
        room to grow (a layer whose growth would pass its buffers stops with
        COWSDM_TRACE_REFUSED in its status word).  Replays share this trace's
        plan blocks (or the library's static ones with ``static_scan``), so
        replays of graphs of one trace must not overlap.  No counterpart in
        the reference."""

        if steps < 1:
            raise ValueError("a captured launch runs at least one step")
        layers = self.layer_array()
        if not self.dense and any(t.paged_map is not None for t in self.tables):
            raise RuntimeError("a paged slot map takes its page proof on the host: decode it "
                               "with run(), not captured launches")
        if not self.dense and not self.planned:
            raise RuntimeError("packed state needs persistent launches to decide its proof "
                               "on the device")
        self.upload()
        self.status.zero_()
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=torch.cuda.Stream(self.device)):
            self.launch(steps, layers)
        self._positions = None
        return graph

    def launch(self, steps: int, layers=None, *, start: int | None = None) -> None:
        """Run ``steps`` consecutive steps of every layer: steps
        start..start+steps-1 (packed state: the decode loop ``run``), or,
        without ``start``, enqueue the next ``steps`` steps of each layer's
        device counter on the current stream."""

        if start is not None:
            if self.repeat:
                raise ValueError("a repeating decode trace runs device-counted launches only")
            if start < 0 or start + steps > self.steps:
                raise ValueError("trace launch runs past the recorded steps")
            if not self.dense:
                self.set_step(start)
                self.run(steps)
                return
            layers = self.layer_array() if layers is None else layers
            stream = nat.stream_handle(self.device)
            self._status_clean = False
            self.trace.step_index = None
            try:
                done = 0
                while done < steps:
                    n = min(steps - done, self.max_steps_per_launch) if self.persistent else steps
                    self.trace.first_step = start + done
                    self._call(layers, n, stream)
                    done += n
            finally:
                self.trace.step_index = self.step_index.data_ptr()
                self.trace.first_step = 0
            return
        if not self.dense and any(t.paged_map is not None for t in self.tables):
            raise RuntimeError("a paged slot map takes its page proof on the host: decode it "
                               "with run(), not device-counted launches")
        layers = self.layer_array() if layers is None else layers
        stream = nat.stream_handle(self.device)
        self._positions = None
        self._status_clean = False
        done = 0
        while done < steps:
            n = min(steps - done, self.max_steps_per_launch) if self.persistent else steps
            self._call(layers, n, stream)
            done += n

    def _call(self, layers, steps, stream):
        lib = nat.lib()
        fn = (lib.cowsdm_dense_step_trace if self.dense else
              lib.cowsdm_packed_step_trace_static if self.static_scan else
              lib.cowsdm_packed_step_trace)
        nat.check(fn(layers, len(self.tables), self.shape, self.trace, steps, stream),
                  "decode trace launch")

    def _read_report(self) -> list:
        """The report (step counters, status words, control words) as host
        lists, copied through pinned memory once the stream reaches it."""

        self._report_host.copy_(self._report, non_blocking=True)
        self._report_ready.record()
        self._report_ready.synchronize()
        return self._report_host.tolist()

    def _fault(self, layers_at_fault) -> None:
        errors = [int(self.tables[l].ensure_scratch()[nat.SCRATCH_ERRORS].item())
                  for l in layers_at_fault]
        raise RuntimeError(
            f"decode trace layers {layers_at_fault} stopped on a fault "
            f"(error words {[hex(e) for e in errors]}): a bounded wait timed out or the "
            "state is corrupt")

    # -------------------------------------------------------- decode loop

    def run(self, steps: int, *, launch_steps: int | None = None,
            timing: list | None = None) -> dict:
        """Decode the next ``steps`` steps of every layer from the device
        counters (which must agree): the reference's per-step loop,
        ``prepare_step_capacity(banks * W)`` then the step, for every packed
        layer with a growth quantum.  Persistent launches run
        ``launch_steps`` (default ``max_steps_per_launch``) steps each.
        With ``timing`` given, a pair of timing events brackets every launch
        on the stream and is appended to it.  Returns the number of launches
        and of host growth rounds."""

        if self.repeat:
            raise ValueError("a repeating decode trace runs device-counted launches only")
        if steps <= 0:
            return {"launches": 0, "growth_rounds": 0}
        positions = self._positions if self._positions is not None else self.step_index.tolist()
        start = positions[0]
        if positions.count(start) != len(positions):
            raise ValueError("decode trace layers stand at different steps")
        target = start + steps
        if target > self.steps:
            raise ValueError("trace run passes the recorded steps")
        launch_steps = self.max_steps_per_launch if launch_steps is None else launch_steps
        launch_steps = max(1, min(int(launch_steps), self.max_steps_per_launch))
        versions = self._versions()
        fresh = versions == self._synced_versions and versions == self._layers_versions
        layers = self._layers[1] if fresh else self.layer_array()
        if not self.dense and not self.planned:
            return self._run_stepwise(start, steps, timing)
        trace = self.trace
        saved = trace.steps_recorded
        trace.steps_recorded = target
        trace.step_index = self._step_index_ptr
        # every layer's counter stands at `start`: the first launch takes it
        # from here instead of loading the counter first
        trace.first_step = start
        trace.first_known = 1
        if not self._status_clean:
            self.status.zero_()
        self._status_clean = False
        if not fresh:
            self.upload(force=False)
            versions = self._versions()
        stream = nat.stream_handle(self.device)
        native = timing is None and (self.dense or self.planned) and self.persistent
        if native and self._host_report is None:
            self._host_report = nat.HostReport(len(self.tables))
        mode = (nat.RUN_DENSE if self.dense else
                nat.RUN_PACKED_STATIC if self.static_scan else nat.RUN_PACKED)
        launches = rounds = 0
        remaining = steps
        self._positions = None
        self._report_versions = None
        try:
            while True:
                count = -(-remaining // launch_steps)
                if native:
                    # launches, then the layers' reports straight from host
                    # memory the last wave of each layer wrote
                    trace.report = self._host_report.device
                    try:
                        rc = nat.lib().cowsdm_trace_run(
                            layers, len(self.tables), self.shape, trace, remaining,
                            launch_steps, mode, stream)
                    finally:
                        trace.report = None
                    trace.first_known = 0
                    if rc:
                        nat.check(rc, "decode trace run")
                    rows = self._host_report.array.tolist()
                    positions = [r[nat.REPORT_STEP] for r in rows]
                    status = [r[nat.REPORT_STATUS] for r in rows]
                    control = None if self.dense else rows
                    offset = nat.REPORT_CONTROL
                else:
                    for _ in range(count):
                        if timing is not None:
                            e0 = torch.cuda.Event(enable_timing=True)
                            e1 = torch.cuda.Event(enable_timing=True)
                            e0.record()
                            self._call(layers, launch_steps, stream)
                            e1.record()
                            timing.append((e0, e1))
                        else:
                            self._call(layers, launch_steps, stream)
                        trace.first_known = 0
                    rows = self._read_report()      # counters, status, control words
                    positions = rows[0]
                    words = rows[1]   # int32 status word l is half l % 2 of word l // 2
                    status = [(words[l // 2] >> (32 * (l % 2))) & 0xFFFFFFFF
                              for l in range(len(self.tables))]
                    control = None if self.dense else [list(w) for w in zip(*rows[2:])]
                    offset = 0
                launches += count
                if control is not None:
                    self._absorb(control, offset, versions if rounds == 0 else None)
                if any(status):
                    faults = [l for l, s in enumerate(status) if s & nat.TRACE_FAULT]
                    if faults:
                        self._fault(faults)
                behind = [l for l, p in enumerate(positions) if p < target]
                if not behind:
                    self._status_clean = not any(status)
                    break
                refused = [l for l in behind if status[l] & nat.TRACE_REFUSED]
                if self.dense or refused != behind:
                    raise RuntimeError(f"decode trace stopped short at steps {positions}")
                # The refused layers stand at a step whose proof reads
                # free_count and grows the slab past its buffers: the
                # reference's prepare_step_capacity at that step, on the
                # host (new buffers with headroom), except that the step's own
                # charge is left to the device, which proves it again.
                grown = [self.tables[l] for l in refused]
                PackedSDMCopyOnWriteState.prepare_step_capacity_layers(
                    grown, self.need(),
                    free_counts=[control[l][offset + nat.CTRL_FREE] for l in refused])
                for st in grown:
                    st.proven_maximum_additional_allocations += self.need()
                self.status.zero_()
                self.upload()
                layers = self.layer_array()
                remaining = target - min(positions)
                rounds += 1
        finally:
            trace.steps_recorded = saved
            trace.first_known = 0
            trace.first_step = 0
        self._positions = [target] * len(self.tables)
        if native and rounds == 0 and not self.dense:
            self._report_versions = self._synced_versions
        return {"launches": launches, "growth_rounds": rounds}

    def _run_stepwise(self, start: int, steps: int, timing: list | None) -> dict:
        """The decode loop one step at a time, for packed shapes without a
        persistent kernel: per step ``prepare_step_capacity(banks * W)`` on
        every layer with a growth quantum, then one fused launch of all
        layers (``packed_sdm_cow_step_layers``, which checks the capacity of
        unproven layers first and raises the reference's errors)."""

        need = self.need()
        x = self.inputs
        outs = self.outputs
        rounds = 0
        for t in range(start, start + steps):
            proven = [st for st in self.tables if st.growth_quantum_rows > 0]
            events = sum(st.growth_events for st in proven)
            PackedSDMCopyOnWriteState.prepare_step_capacity_layers(proven, need)
            rounds += sum(st.growth_events for st in proven) - events
            out = outs[t] if outs.ndim == 4 else outs
            if timing is not None:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
            packed_sdm_cow_step_layers(
                self.tables, x["write_indices"][t], x["write_weights"][t], x["values"][t],
                x["input_gate"][t], x["forget_log_gate"][t], x["read_indices"][t],
                x["read_weights"][t], erase_gate=x["erase_gate"][t], outputs=list(out))
            if timing is not None:
                e1.record()
                timing.append((e0, e1))
        self.step_index.fill_(start + steps)
        self._positions = [start + steps] * len(self.tables)
        return {"launches": steps, "growth_rounds": rounds}
