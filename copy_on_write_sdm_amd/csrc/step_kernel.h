// The fused copy-on-write SDM step kernels (packed and dense-table forms)
// and their launchers; each step_*.hip file instantiates one index type
// and one form.
//
// Two kernels run one decode step:
//  * sdm_step_small_kernel, for the decode shape (W <= 4, R <= 16, a row of
//    at most 64 * VEC floats, B <= 256 banks per packed layer): the route
//    metadata is spread over lanes (lane w < W holds write route w, lane
//    16 + r read route r), each lane computes its row's address, and the
//    whole step is one short straight-line path;
//  * sdm_step_kernel, for every other shape (W <= 64, R <= 256, any D, any
//    B), looping over row chunks and read batches.
// Both give bit-identical results: the same first-touch order, the same
// float operations in the same order.
#pragma once

#include "common.h"
#include "lookback.h"

namespace cowsdm_impl {

// A packed one-step launch of at most this many banks per layer with at
// most 4 writes per bank takes the bank-order prefix from a table every wave
// builds itself (lane l holds banks l, l + 64, ...: their write slots, map
// entries and templates), so no pop waits on another wave; the only wait is
// for the launch's tickets before the first-touch map entries are stored.
// Larger shapes use the decoupled look-back over scratch slots.
constexpr int kLocalTableBanks = 4 * kWave;
constexpr int kLocalTableWrites = 4;
constexpr int kTableSlots = kLocalTableBanks / kWave;
// the small kernel's read-route lanes start here
constexpr int kSmallReadLane = 16;
constexpr int kSmallReads = 16;

// OR of the error bits (COWSDM_ERR_*, bits 0-7) over the wave: one ballot
// per bit, no cross-lane data movement.
__device__ __forceinline__ int wave_or_bits(int v) {
  int r = 0;
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    if (__ballot((v >> bit) & 1) != 0) r |= 1 << bit;
  }
  return r;
}

__device__ __forceinline__ int64_t rl64(int64_t x, int lane) {
  return static_cast<int64_t>(
      (static_cast<uint64_t>(static_cast<uint32_t>(rl(static_cast<int>(x >> 32), lane))) << 32) |
      static_cast<uint32_t>(rl(static_cast<int>(x), lane)));
}

// ------------------------------------------------------------ shared parts

// A trace launch with no recorded step left for the layer: touch no input,
// leave the counter.  True when the wave must return.
template <bool DENSE>
__device__ __forceinline__ bool trace_exhausted(const StepParams& P, const cowsdm_layer_t& L,
                                                int layer_id, int bank, int lane,
                                                int64_t trace_s) {
  if (!P.trace_step || (trace_s >= 0 && trace_s < P.trace_len)) return false;
  if (lane == 0) {
    if (P.trace_status) {
      __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{2}, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    } else if (!DENSE && L.scratch) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_TRACE_RANGE), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (P.report && bank == P.banks - 1) write_report(P, layer_id, trace_s, COWSDM_TRACE_ENDED);
  return true;
}

// Planned single step of a decode trace (packed state with control words):
// the decode loop's proof for this step, prepare_step_capacity(need)
// (allocator.py:745-773), made identically by every wave from the control
// words and free_count.  A growth within the slab's buffers puts row ids
// C0 .. C0 + added - 1 on top of the found stack (grow_capacity,
// allocator.py:691-743), so pop q from the top takes C0 + added - 1 - q
// while q < added and the found stack's entry q - added after.
struct StepProof {
  int64_t capacity = 0;   // C before the step
  int64_t grown = 0;      // rows added on top of the found stack
  int64_t proven_after = 0;
  bool refused = false;   // the growth would pass the slab's buffers
};

__device__ __forceinline__ StepProof prove_step(const StepParams& P, int layer_id,
                                                int64_t capacity, int64_t old_free) {
  StepProof pr;
  pr.capacity = capacity;
  if (!P.control) return pr;
  auto word = [&](int k) __attribute__((always_inline)) -> int64_t {
    const uint64_t v = static_cast<uint64_t>(control_word(P, layer_id, k));
    return static_cast<int64_t>(
        (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32))) << 32) |
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  };
  const int64_t C = word(COWSDM_CTRL_CAPACITY);
  int64_t proven = word(COWSDM_CTRL_PROVEN);
  const int64_t room = word(COWSDM_CTRL_ROOM);
  const int64_t quantum = word(COWSDM_CTRL_QUANTUM);
  const int64_t need = word(COWSDM_CTRL_NEED);
  pr.capacity = C;
  if (need > 0 && quantum > 0) {
    if (proven < need) {
      int64_t free_rows = old_free;
      if (free_rows < need) {
        const int64_t want = C + need - free_rows;
        const int64_t selected = (want + quantum - 1) / quantum * quantum;
        if (selected > room || selected >= (int64_t{1} << 31)) {
          pr.refused = true;   // the host grows the slab into larger buffers
        } else {
          pr.grown = selected - C;
          free_rows += pr.grown;
        }
      }
      proven = free_rows;
    }
    pr.proven_after = proven - need;
  } else {
    pr.proven_after = proven;
  }
  return pr;
}

// A refused planned step: the layer takes no step; every wave of it stops
// before it takes a ticket or publishes a slot, and one bank reports the
// refusal (no other wave reads the words it writes).
__device__ __forceinline__ void report_refusal(const StepParams& P, int layer_id, int bank,
                                               int lane, int64_t trace_s, int64_t old_free) {
  if (bank != P.banks - 1) return;
  if (lane == 0) {
    atomic_store_u64(&control_word(P, layer_id, COWSDM_CTRL_FREE),
                     static_cast<uint64_t>(old_free));
    atomic_store_u64(&control_word(P, layer_id, COWSDM_CTRL_STEPS), 0);
    atomic_store_u64(&control_word(P, layer_id, COWSDM_CTRL_FIT), 0);
    if (P.trace_status) {
      __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_REFUSED},
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (P.report) write_report(P, layer_id, trace_s, COWSDM_TRACE_REFUSED);
}

// The layer's first-touch table: lane l holds banks l + 64 k.  A bank's
// count is its write slots still mapped to M0, or 0 when its write routes
// are invalid (index outside [0, N), a slot written twice, a template
// outside [0, T), a map entry outside the slab): exactly the banks that
// skip themselves.  load_slots issues the route and template loads,
// count_first the map loads once the slots are in.
struct FirstTouchTable {
  int slot[kTableSlots][kLocalTableWrites];
  int count[kTableSlots];
  bool valid[kTableSlots];

  template <typename IDX>
  __device__ __forceinline__ void load_slots(const cowsdm_layer_t& L, const void* write_indices,
                                             int B, int N, int W, int templates, int lane) {
#pragma unroll
    for (int k = 0; k < kTableSlots; ++k) {
      const int tb = lane + k * kWave;
      valid[k] = tb < B;
      count[k] = 0;
#pragma unroll
      for (int j = 0; j < kLocalTableWrites; ++j) slot[k][j] = 0;
      if (tb < B) {
        const int64_t t = L.template_indices[tb];
        if (t < 0 || t >= templates) valid[k] = false;
#pragma unroll
        for (int j = 0; j < kLocalTableWrites; ++j) {
          if (j < W) {
            const int64_t x = load_index<IDX>(write_indices, static_cast<int64_t>(tb) * W + j);
            if (x < 0 || x >= N) valid[k] = false;
            else slot[k][j] = static_cast<int>(x);
          }
        }
#pragma unroll
        for (int j = 1; j < kLocalTableWrites; ++j) {
#pragma unroll
          for (int i = 0; i < j; ++i) {
            if (j < W && slot[k][i] == slot[k][j]) valid[k] = false;
          }
        }
      }
    }
  }

  __device__ __forceinline__ void count_first(const cowsdm_layer_t& L, int B, int N, int W,
                                              int64_t C, int lane) {
#pragma unroll
    for (int k = 0; k < kTableSlots; ++k) {
      const int tb = lane + k * kWave;
      if (tb < B && valid[k]) {
        int mapped[kLocalTableWrites];
#pragma unroll
        for (int j = 0; j < kLocalTableWrites; ++j) {
          mapped[j] = j < W ? map_entry(L, tb, N, slot[k][j]) : 0;
        }
        int c = 0;
#pragma unroll
        for (int j = 0; j < kLocalTableWrites; ++j) {
          if (j < W) {
            if (mapped[j] >= C) valid[k] = false;
            c += mapped[j] < 0 ? 1 : 0;
          }
        }
        count[k] = valid[k] ? c : 0;
      }
    }
  }

  // Bank `bank`'s count, exclusive prefix and validity, and the rows the
  // step pops when the stack holds `top` rows: banks with first touches
  // whose inclusive prefix fits lead the banks with first touches, so the
  // last one's prefix is the total popped.
  __device__ __forceinline__ void prefix(int bank, int64_t top, int& own_count,
                                         int64_t& own_prefix, bool& own_valid,
                                         int64_t& served) const {
    const int own_k = bank / kWave;
    const int own_lane = bank % kWave;
    int base = 0;
    served = 0;
#pragma unroll
    for (int k = 0; k < kTableSlots; ++k) {
      const int inc = base + wave_inclusive(count[k]);
      if (k == own_k) {
        own_count = rl(count[k], own_lane);
        own_prefix = rl(inc, own_lane) - own_count;
        own_valid = rl(valid[k] ? 1 : 0, own_lane) != 0;
      }
      const uint64_t fit = __ballot(count[k] > 0 && inc <= top);
      if (fit != 0) served = rl(inc, 63 - __builtin_clzll(fit));
      base = rl(inc, kWave - 1);
    }
  }

  __device__ __forceinline__ int total() const {
    int t = 0;
#pragma unroll
    for (int k = 0; k < kTableSlots; ++k) t += count[k];
    for (int o = kWave / 2; o > 0; o >>= 1) t += __shfl_xor(t, o, kWave);
    return t;
  }
};

// Ticket of a LOCAL launch: a running count every launch adds B to (one per
// wave), taken once the wave has read the words the step rewrites
// (free_count, the control words, the step counter) and every map entry of
// its table.
__device__ __forceinline__ int64_t take_ticket(const cowsdm_layer_t& L, int lane) {
  int64_t t = -1;
  if (lane == 0) {
    t = __hip_atomic_fetch_add(&L.scratch[COWSDM_SCRATCH_TICKET], int64_t{1}, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  }
  return t;
}

// Bounded wait (lane 0 polls) until the count holds every ticket of this
// launch: then no table of the launch still reads the map, and the wave may
// store its first-touch map entries.  False (and the error bit set) when the
// wait gave up.
__device__ __forceinline__ bool wait_tickets(const cowsdm_layer_t& L, int64_t ticket, int B,
                                             int lane) {
  const int64_t mine = rl64(ticket, 0);
  const int64_t target = (mine / B + 1) * B;
  int all_in = 1;
  if (lane == 0) {
    uint64_t v = atomic_load_u64(&L.scratch[COWSDM_SCRATCH_TICKET]);
    for (int spins = 0; static_cast<int64_t>(v) < target && spins < kSpinLimit; ++spins) {
      __builtin_amdgcn_s_sleep(1);
      v = atomic_load_u64(&L.scratch[COWSDM_SCRATCH_TICKET]);
    }
    all_in = static_cast<int64_t>(v) >= target ? 1 : 0;
    if (!all_in) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  return rl(all_in, 0) != 0;
}

// The first touch of rank `rank` (bank-major, allocator.py:1471-1481) takes
// the free-stack entry prefix + rank from the top: one of the rows a growth
// put there, or the found stack's entry.  Sets *fits false (and flags the
// state corrupt) when a popped id lies outside the slab.
__device__ __forceinline__ int pop_row(const cowsdm_layer_t& L, bool take, int64_t prefix,
                                       int rank, const StepProof& pr, int64_t old_free,
                                       int lane, bool* fits) {
  const int64_t C = pr.capacity;
  const int64_t from_top = prefix + rank;        // pop position counted from the top
  const int64_t found = from_top - pr.grown;     // ... and from the found stack's top
  int row = -1;
  int bad = 0;
  if (take) {
    row = found < 0 ? static_cast<int>(C + pr.grown - 1 - from_top)
                    : L.free_rows[old_free - 1 - found];
    if (row < 0 || row >= C + pr.grown) bad = 1;
  }
  if (__ballot(bad) != 0) {
    *fits = false;
    if (lane == 0) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  return row;
}

// The wave that closes a packed layer (after every other wave has read the
// words it rewrites): free_count, the allocated-rows diagnostic, and for a
// planned step the stack entries of grown rows no pop took, the flags and
// the control words.
__device__ __forceinline__ void close_layer(const StepParams& P, const cowsdm_layer_t& L,
                                            int layer_id, int lane, const StepProof& pr,
                                            int64_t old_free, int64_t served, bool short_rows) {
  const int64_t C = pr.capacity;
  const int64_t top = old_free + pr.grown;
  const int64_t now_free = top - served;
  const bool planned = P.control != nullptr;
  if (planned && now_free > old_free) {
    // the grown rows no pop took stay on the stack, above the found ones
    int32_t* const stack = const_cast<int32_t*>(L.free_rows);
    for (int64_t p = old_free + lane; p < now_free; p += kWave) {
      stack[p] = static_cast<int32_t>(C + (p - old_free));
    }
  }
  if (lane != 0) return;
  *L.free_count = static_cast<int32_t>(now_free);
  if (L.allocated_rows_out) *L.allocated_rows_out = static_cast<int32_t>(C + pr.grown - now_free);
  if (!planned) return;
  if (pr.grown > 0) *L.overflow_flag = 0;   // grow_capacity clears it
  if (short_rows) *L.overflow_flag = 1;
  auto put = [&](int k, int64_t v) __attribute__((always_inline)) {
    atomic_store_u64(&control_word(P, layer_id, k), static_cast<uint64_t>(v));
  };
  const int64_t events = control_word(P, layer_id, COWSDM_CTRL_EVENTS);
  const int64_t added = control_word(P, layer_id, COWSDM_CTRL_ADDED);
  const int64_t copied = control_word(P, layer_id, COWSDM_CTRL_COPIED);
  put(COWSDM_CTRL_PROVEN, short_rows ? 0 : pr.proven_after);
  put(COWSDM_CTRL_CAPACITY, C + pr.grown);
  put(COWSDM_CTRL_EVENTS, events + (pr.grown > 0 ? 1 : 0));
  put(COWSDM_CTRL_ADDED, added + pr.grown);
  put(COWSDM_CTRL_COPIED, copied + (pr.grown > 0 ? C : 0));
  put(COWSDM_CTRL_FREE, now_free);
  put(COWSDM_CTRL_STEPS, 1);
  put(COWSDM_CTRL_FIT, served);
}

// End of a step on a device-counted trace: the wave that closes the layer
// moves its counter to the next step (every wave of the layer read it
// before: packed waves before their ticket or the bank-order scan, dense
// waves before their ticket), and a packed layer's report follows.
template <bool DENSE>
__device__ __forceinline__ void finish_trace(const StepParams& P, int layer_id, int lane,
                                             int64_t trace_s, bool closed_layer) {
  if (P.trace_step && lane == 0) {
    if constexpr (DENSE) {
      int64_t* layer_ticket = P.trace_ticket + 1 + layer_id;
      const int64_t done = __hip_atomic_fetch_add(layer_ticket, int64_t{1}, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      closed_layer = (done == P.banks - 1);
      if (closed_layer) atomic_store_u64(layer_ticket, 0);
    }
    if (closed_layer) {
      atomic_store_u64(&P.trace_step[layer_id], static_cast<uint64_t>(trace_s + 1));
    }
  }
  if (!DENSE && P.report && closed_layer) write_report(P, layer_id, trace_s + 1, 0);
}

__device__ __forceinline__ void record_errors(const cowsdm_layer_t& L, int lane, int err) {
  if (lane == 0 && err && L.scratch) {
    __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(err),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// First-touch map entries of one bank in a paged map (lanes w < W hold the
// write routes; `first` marks first touches, `dir` their directory entry,
// `row` their popped row).  A first touch in a page the bank already has is
// one store; the first touches in pages it lacks take one new page per
// distinct page, in lane order from the layer's page counter, and the
// wave writes each such page whole (-1 but for those first touches) and
// then its directory entry.  Called once every table of the launch is
// built (no wave reads this bank's pages after that).
__device__ __forceinline__ void store_paged(const cowsdm_layer_t& L, int64_t bank, int N,
                                            int slot, bool first, int dir, int row, int lane) {
  const int shift = L.map_page_shift;
  const int pmask = (1 << shift) - 1;
  if (first && dir >= 0) {
    L.map_pages[(static_cast<int64_t>(dir) << shift) + (slot & pmask)] = row;
  }
  const bool need = first && dir < 0;
  const int page = need ? (slot >> shift) : -1;
  // the lowest lane needing the same page takes it
  bool leads = need;
#pragma unroll
  for (int j = 0; j < kLocalTableWrites; ++j) {
    if (need && j < lane && rl(page, j) == page) leads = false;
  }
  const uint64_t leaders = __ballot(leads);
  if (leaders == 0) return;
  int base = 0;
  if (lane == 0) {
    base = __hip_atomic_fetch_add(L.map_page_count, __popcll(leaders), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  }
  base = rl(base, 0);
  if (base + __popcll(leaders) > L.map_page_capacity) {
    // the host's page proof rules this out: flag the state, write nothing
    record_errors(L, lane, COWSDM_ERR_CORRUPT);
    return;
  }
  for (uint64_t left = leaders; left != 0; left &= left - 1) {
    const int k = __ffsll(static_cast<long long>(left)) - 1;
    const int kpage = rl(page, k);
    const int id = base + __popcll(leaders & ((1ull << k) - 1));
    int entry = -1;
#pragma unroll
    for (int j = 0; j < kLocalTableWrites; ++j) {
      if (rl(page, j) == kpage && (rl(slot, j) & pmask) == lane) entry = rl(row, j);
    }
    if (lane <= pmask) L.map_pages[(static_cast<int64_t>(id) << shift) + lane] = entry;
    if (lane == 0) L.map_directory[bank * (N >> shift) + kpage] = id;
  }
}

// ------------------------------------------------- the small decode step

// One wave = one bank of one layer, for W <= 4, R <= 16 and a row that one
// wave covers in one pass (D <= 64 * VEC).  DENSE selects the dense-table
// control (allocator.py:1612-1633): rows live at values[bank, slot] and
// there is no map, free stack or table.  Packed waves build the layer's
// first-touch table (B <= kLocalTableBanks).
//
// A bank whose write routes are invalid (index outside [0, N), a slot
// written twice, a template outside [0, T), a map entry outside the slab)
// is skipped: it pops nothing and changes nothing.  A bank whose read
// routes are invalid (index outside [0, N), map entry outside the slab)
// keeps its writes and returns a zero reading.  Both set the sticky error
// word.
template <typename IDX, int VEC, bool DENSE>
__global__ __launch_bounds__(kStepThreads) void sdm_step_small_kernel(StepParams P) {
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  const int bank = __builtin_amdgcn_readfirstlane(
      (blockIdx.x % P.blocks_per_layer) * kBanksPerBlock + static_cast<int>(threadIdx.x) / kWave);
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  if (layer_id >= P.nlayers || bank >= P.banks) return;
  const cowsdm_layer_t& L = P.layer[layer_id];
  const int64_t trace_s = P.trace_step ? P.trace_step[layer_id] : P.trace_first;
  if (trace_exhausted<DENSE>(P, L, layer_id, bank, lane, trace_s)) return;
  auto step_ptr = [&](const void* base, int k) __attribute__((always_inline)) -> const char* {
    return static_cast<const char*>(base) + trace_s * P.trace_stride[k];
  };
  const void* const write_indices = step_ptr(L.write_indices, 0);
  const float* const write_weights = reinterpret_cast<const float*>(step_ptr(L.write_weights, 1));
  const float* const step_values = reinterpret_cast<const float*>(step_ptr(L.step_values, 2));
  const float* const input_gate = reinterpret_cast<const float*>(step_ptr(L.input_gate, 3));
  const float* const erase_gate = reinterpret_cast<const float*>(step_ptr(L.erase_gate, 4));
  const float* const forget_gate = reinterpret_cast<const float*>(step_ptr(L.forget_log_gate, 5));
  const void* const read_indices = step_ptr(L.read_indices, 6);
  const float* const read_weights = reinterpret_cast<const float*>(step_ptr(L.read_weights, 7));
  float* const output = const_cast<float*>(reinterpret_cast<const float*>(step_ptr(L.output, 8)));

  const int N = P.slots;
  const int D = P.width;
  const int W = P.writes;
  const int R = P.reads;
  const int B = P.banks;
  const int64_t b = bank;

  // ---- route metadata, one route per lane: write route w in lane w, read
  // route r in lane 16 + r
  const bool is_w = lane < W;
  const int r_of_lane = lane - kSmallReadLane;
  const bool is_r = r_of_lane >= 0 && r_of_lane < R;
  int slot = 0;
  float weight = 0.0f;
  int werr = 0;   // this lane's errors on the write side (skip the bank)
  int rerr = 0;   // ... on the read side (zero reading)
  if (is_w || is_r) {
    const int64_t x = is_w ? load_index<IDX>(write_indices, b * W + lane)
                           : load_index<IDX>(read_indices, b * R + r_of_lane);
    weight = is_w ? write_weights[b * W + lane] : read_weights[b * R + r_of_lane];
    if (x < 0 || x >= N) {
      if (is_w) werr |= COWSDM_ERR_WRITE_INDEX;
      else rerr |= COWSDM_ERR_READ_INDEX;
    } else {
      slot = static_cast<int>(x);
    }
  }
  const float forget = forget_gate[b];
  const float in_gate = input_gate[b];
  const float er_gate = erase_gate[b];
  float vin[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) vin[v] = 0.0f;
  const int col = lane * VEC;
  const bool col_ok = col < D;
  if (col_ok) load_row<VEC>(step_values + b * D + col, vin);

  int64_t tmpl = 0;
  int64_t old_free = 0;
  StepProof pr;
  pr.capacity = L.capacity_rows;
  FirstTouchTable table;
  if constexpr (!DENSE) {
    tmpl = L.template_indices[b];
    if (tmpl < 0 || tmpl >= P.templates) werr |= COWSDM_ERR_TEMPLATE;
    old_free = *L.free_count;
    table.template load_slots<IDX>(L, write_indices, B, N, W, P.templates, lane);
    pr = prove_step(P, layer_id, L.capacity_rows, old_free);
    if (pr.refused) {
      report_refusal(P, layer_id, bank, lane, trace_s, old_free);
      return;
    }
  }
  const int64_t C = pr.capacity;

  // ---- map lookups (packed), then the table's
  int phys = -1;
  int dir = -1;   // paged map: the slot's directory entry
  if constexpr (!DENSE) {
    if ((is_w || is_r) && !((werr | rerr) & (COWSDM_ERR_WRITE_INDEX | COWSDM_ERR_READ_INDEX))) {
      phys = map_entry(L, b, N, slot, &dir);
      if (phys >= C) {
        if (is_w) werr |= COWSDM_ERR_CORRUPT;
        else rerr |= COWSDM_ERR_CORRUPT;
      }
    }
    table.count_first(L, B, N, W, C, lane);
  }

  // ---- duplicate writes and read-after-write sources (lane order of the
  // writes: a read of a slot written this step takes the updated row)
  int src = -1;
#pragma unroll
  for (int j = 0; j < kLocalTableWrites; ++j) {
    if (j < W) {
      const int other = rl(slot, j);
      if (is_w && j < lane && other == slot) werr |= COWSDM_ERR_DUP_WRITE;
      if (is_r && other == slot) src = j;
    }
  }
  const int err_w = wave_or_bits(werr);
  const int err_r = wave_or_bits(rerr);
  const bool first = !DENSE && is_w && phys < 0;
  const uint64_t first_mask = __ballot(first);
  const int rank = __popcll(first_mask & ((1ull << lane) - 1));

  bool wok = err_w == 0;    // the bank writes
  int count = 0;
  int64_t prefix = 0;
  int64_t served = 0;
  const int64_t top = old_free + pr.grown;
  if constexpr (!DENSE) table.prefix(bank, top, count, prefix, wok, served);
  const bool rok = wok && err_r == 0;    // the bank reads

  // ---- row addresses, one per route lane: M0 row on first touch or a
  // shared read, else the slab row (dense: the table row)
  const float* row = nullptr;
  if constexpr (DENSE) {
    row = L.values + (b * N + slot) * static_cast<int64_t>(D);
  } else {
    row = phys < 0 ? L.shared_initial_memory + (tmpl * N + slot) * static_cast<int64_t>(D)
                   : L.values + static_cast<int64_t>(phys) * D;
  }
  const int64_t row_bits = static_cast<int64_t>(reinterpret_cast<uintptr_t>(row));
  // reads forwarded from this step's writes load nothing
  const uint32_t forwarded = static_cast<uint32_t>(__ballot(is_r && src >= 0) >> kSmallReadLane);

  float cur[kLocalTableWrites][VEC];
  float rv[kSmallReads][VEC];
#pragma unroll
  for (int j = 0; j < kLocalTableWrites; ++j) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) cur[j][v] = 0.0f;
  }
#pragma unroll
  for (int r = 0; r < kSmallReads; ++r) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) rv[r][v] = 0.0f;
  }
  if (wok) {
#pragma unroll
    for (int j = 0; j < kLocalTableWrites; ++j) {
      if (j < W) {
        const float* p = reinterpret_cast<const float*>(static_cast<uintptr_t>(rl64(row_bits, j)));
        if (col_ok) load_row<VEC>(p + col, cur[j]);
      }
    }
  }
  if (rok) {
#pragma unroll
    for (int r = 0; r < kSmallReads; ++r) {
      if (r < R && !((forwarded >> r) & 1u)) {
        const float* p = reinterpret_cast<const float*>(
            static_cast<uintptr_t>(rl64(row_bits, kSmallReadLane + r)));
        if (col_ok) load_row<VEC>(p + col, rv[r]);
      }
    }
  }

  // ---- pops: first touch of rank q takes stack entry prefix + q from the
  // top; their loads overlap the rows'.  Then the ticket.
  bool fits = true;
  int new_row = -1;
  int64_t ticket = -1;
  if constexpr (!DENSE) {
    fits = wok && (count == 0 || prefix + count <= top);
    new_row = pop_row(L, fits && first, prefix, rank, pr, old_free, lane, &fits);
    if (lane == 0 && !P.control && wok && !fits && count > 0) *L.overflow_flag = 1;
    const int top_lo = static_cast<int>(top);
    const int served_lo = static_cast<int>(served);
    const int proven_lo = static_cast<int>(pr.proven_after);
    asm volatile("" ::"v"(top_lo), "v"(new_row), "v"(served_lo), "v"(proven_lo) : "memory");
    ticket = take_ticket(L, lane);
  }

  // ---- gated-delta update and sparse read (the reference's operation
  // order; every product and sum rounded separately)
  const float alpha = static_cast<float>(exp(static_cast<double>(forget)));
  float acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
  if (wok) {
    // decayed = current * exp(forget); retrieved = sum_w weight_w * decayed_w
    float ret[VEC];
#pragma unroll
    for (int j = 0; j < kLocalTableWrites; ++j) {
      if (j < W) {
        const float wj = rlf(weight, j);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          cur[j][v] = cur[j][v] * alpha;
          const float term = wj * cur[j][v];
          ret[v] = (j == 0) ? term : ret[v] + term;
        }
      }
    }
    // delta = in_gate * value - erase_gate * retrieved
    // updated_w = decayed_w + weight_w * delta
    float delta[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const float a = in_gate * vin[v];
      const float e = er_gate * ret[v];
      delta[v] = a - e;
    }
#pragma unroll
    for (int j = 0; j < kLocalTableWrites; ++j) {
      if (j < W) {
        const float wj = rlf(weight, j);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float t = wj * delta[v];
          cur[j][v] = cur[j][v] + t;
        }
      }
    }
  }
  if (rok) {
    // reading = sum_r weight_r * visible_r, reads after this step's writes
#pragma unroll
    for (int r = 0; r < kSmallReads; ++r) {
      if (r < R) {
        float x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) x[v] = rv[r][v];
        if ((forwarded >> r) & 1u) {
          const int s = rl(src, kSmallReadLane + r);
#pragma unroll
          for (int j = 0; j < kLocalTableWrites; ++j) {
            if (j == s) {
#pragma unroll
              for (int v = 0; v < VEC; ++v) x[v] = cur[j][v];
            }
          }
        }
        const float wr = rlf(weight, kSmallReadLane + r);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float term = wr * x[v];
          acc[v] = (r == 0) ? term : acc[v] + term;
        }
      }
    }
  }

  // ---- stores: the reading, the updated rows (a first touch at its popped
  // row), then (packed) the map entries once the launch's tables are built
  if (col_ok) store_row<VEC>(output + b * D + col, acc);
  const bool commit = wok && fits;
  if (DENSE ? wok : commit) {
#pragma unroll
    for (int j = 0; j < kLocalTableWrites; ++j) {
      if (j < W) {
        int64_t dst_row;
        if constexpr (DENSE) {
          dst_row = b * N + rl(slot, j);
        } else {
          const int p = rl(phys, j);
          dst_row = p >= 0 ? p : rl(new_row, j);
        }
        if (col_ok) store_row<VEC>(L.values + dst_row * D + col, cur[j]);
      }
    }
  }
  bool closed_layer = false;
  if constexpr (!DENSE) {
    const bool stored_ok = wait_tickets(L, ticket, B, lane);
    if (L.map_page_shift == 0) {
      if (commit && first && stored_ok) L.logical_to_physical[b * N + slot] = new_row;
    } else if (commit && stored_ok) {
      store_paged(L, b, N, slot, first, dir, new_row, lane);
    }
    if (lane == 0) {
      if (L.first_touches_out) L.first_touches_out[b] = commit ? count : 0;
      if (L.repeated_writes_out) L.repeated_writes_out[b] = wok ? W - count : W;
    }
    record_errors(L, lane, err_w | err_r);
    closed_layer = bank == B - 1 && stored_ok;
    if (closed_layer) {
      close_layer(P, L, layer_id, lane, pr, old_free, served, served < table.total());
    }
  } else {
    record_errors(L, lane, err_w | err_r);
  }
  finish_trace<DENSE>(P, layer_id, lane, trace_s, closed_layer);
}

// --------------------------------------------------------- the fused step

// One wave = one bank of one layer, any shape: row chunks of 64 * VEC
// floats, read batches of kReadBatch rows.  DENSE selects the dense-table
// control.  LOCAL (packed, B <= kLocalTableBanks, W <= kLocalTableWrites)
// builds the layer's first-touch table in every wave instead of scanning
// with the look-back.  Error handling as in sdm_step_small_kernel.
template <typename IDX, int MAXW, int VEC, bool DENSE, bool LOCAL>
__global__ __launch_bounds__(kStepThreads) void sdm_step_kernel(StepParams P) {
  static_assert(!LOCAL || (!DENSE && MAXW <= kLocalTableWrites), "local table: packed, W <= 4");
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  const int bank = __builtin_amdgcn_readfirstlane(
      (blockIdx.x % P.blocks_per_layer) * kBanksPerBlock + static_cast<int>(threadIdx.x) / kWave);
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  if (layer_id >= P.nlayers || bank >= P.banks) return;
  const cowsdm_layer_t& L = P.layer[layer_id];
  const int64_t trace_s = P.trace_step ? P.trace_step[layer_id] : P.trace_first;
  if (trace_exhausted<DENSE>(P, L, layer_id, bank, lane, trace_s)) return;
  auto step_ptr = [&](const void* base, int k) __attribute__((always_inline)) -> const char* {
    return static_cast<const char*>(base) + trace_s * P.trace_stride[k];
  };
  const void* const write_indices = step_ptr(L.write_indices, 0);
  const float* const write_weights = reinterpret_cast<const float*>(step_ptr(L.write_weights, 1));
  const float* const step_values = reinterpret_cast<const float*>(step_ptr(L.step_values, 2));
  const float* const input_gate = reinterpret_cast<const float*>(step_ptr(L.input_gate, 3));
  const float* const erase_gate = reinterpret_cast<const float*>(step_ptr(L.erase_gate, 4));
  const float* const forget_gate = reinterpret_cast<const float*>(step_ptr(L.forget_log_gate, 5));
  const void* const read_indices = step_ptr(L.read_indices, 6);
  const float* const read_weights = reinterpret_cast<const float*>(step_ptr(L.read_weights, 7));
  float* const output = const_cast<float*>(reinterpret_cast<const float*>(step_ptr(L.output, 8)));

  const int N = P.slots;
  const int D = P.width;
  const int W = P.writes;
  const int R = P.reads;
  const int B = P.banks;
  const int64_t b = bank;

  int werr = 0;   // this lane's errors on the write side (skip the bank)
  int rerr = 0;   // ... on the read side (zero reading)

  // ---- per-bank scalars
  int64_t tmpl = 0;
  if constexpr (!DENSE) {
    tmpl = L.template_indices[b];
    if (tmpl < 0 || tmpl >= P.templates) werr |= COWSDM_ERR_TEMPLATE;
  }
  const float forget = forget_gate[b];
  const float in_gate = input_gate[b];
  const float er_gate = erase_gate[b];
  int64_t old_free = 0;
  uint32_t epoch = 0;
  StepProof pr;
  pr.capacity = L.capacity_rows;
  if constexpr (!DENSE) {
    old_free = *L.free_count;
    if constexpr (!LOCAL) epoch = static_cast<uint32_t>(L.scratch[COWSDM_SCRATCH_EPOCH]);
    pr = prove_step(P, layer_id, L.capacity_rows, old_free);
    if (pr.refused) {
      report_refusal(P, layer_id, bank, lane, trace_s, old_free);
      return;
    }
  }
  const int64_t C = pr.capacity;

  // ---- write routes: lane w < W
  int widx = 0;
  float wweight = 0.0f;
  int wphys = -1;
  if (lane < W) {
    const int64_t x = load_index<IDX>(write_indices, b * W + lane);
    wweight = write_weights[b * W + lane];
    if (x < 0 || x >= N) {
      werr |= COWSDM_ERR_WRITE_INDEX;
    } else {
      widx = static_cast<int>(x);
    }
  }
  // ---- read routes: lane l holds r = l + 64 k
  int ridx[kMaxReadSlots];
  float rweight[kMaxReadSlots];
  int rphys[kMaxReadSlots];
  int rsrc[kMaxReadSlots];
#pragma unroll
  for (int k = 0; k < kMaxReadSlots; ++k) {
    ridx[k] = 0;
    rweight[k] = 0.0f;
    rphys[k] = -1;
    rsrc[k] = -1;
    const int r = k * kWave + lane;
    if (r < R) {
      const int64_t x = load_index<IDX>(read_indices, b * R + r);
      rweight[k] = read_weights[b * R + r];
      if (x < 0 || x >= N) {
        rerr |= COWSDM_ERR_READ_INDEX;
      } else {
        ridx[k] = static_cast<int>(x);
      }
    }
  }
  FirstTouchTable table;
  if constexpr (LOCAL) table.template load_slots<IDX>(L, write_indices, B, N, W, P.templates, lane);

  // ---- map lookups (packed) for writes and reads, then the table's
  if constexpr (!DENSE) {
    if (lane < W && !(werr & COWSDM_ERR_WRITE_INDEX)) {
      wphys = L.logical_to_physical[b * N + widx];
      if (wphys >= C) werr |= COWSDM_ERR_CORRUPT;
    }
#pragma unroll
    for (int k = 0; k < kMaxReadSlots; ++k) {
      const int r = k * kWave + lane;
      if (r < R) {
        rphys[k] = L.logical_to_physical[b * N + ridx[k]];
        if (rphys[k] >= C) rerr |= COWSDM_ERR_CORRUPT;
      }
    }
  }
  if constexpr (LOCAL) table.count_first(L, B, N, W, C, lane);

  // ---- duplicate writes and read-after-write sources
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    if (j < W) {
      const int other = rl(widx, j);
      if (lane < W && j < lane && other == widx) werr |= COWSDM_ERR_DUP_WRITE;
#pragma unroll
      for (int k = 0; k < kMaxReadSlots; ++k) {
        if (k * kWave + lane < R && ridx[k] == other) rsrc[k] = j;
      }
    }
  }

  const int err_w = wave_or_bits(werr);
  const int err_r = wave_or_bits(rerr);
  const bool first = !DENSE && lane < W && wphys < 0;
  const uint64_t first_mask = __ballot(first);
  const int rank = __popcll(first_mask & ((1ull << lane) - 1));

  // ---- bank-order prefix (LOCAL): from the table
  bool wok = err_w == 0;          // the bank writes
  int count = wok ? __popcll(first_mask) : 0;
  int64_t prefix = 0;
  int64_t table_served = 0;       // rows the layer's step pops (LOCAL)
  const int64_t top = old_free + pr.grown;
  if constexpr (LOCAL) table.prefix(bank, top, count, prefix, wok, table_served);
  const bool rok = wok && err_r == 0;   // the bank reads

  // ---- row loads, issued before the pops are resolved
  const float alpha = static_cast<float>(exp(static_cast<double>(forget)));
  const float* const m0_bank =
      DENSE ? nullptr : L.shared_initial_memory + tmpl * static_cast<int64_t>(N) * D;
  float* const table_bank = DENSE ? L.values + b * N * D : nullptr;
  const int chunk_cols = kWave * VEC;
  const int nchunks = (D + chunk_cols - 1) / chunk_cols;

  float cur[MAXW][VEC];
  float rv[kReadBatch][VEC];
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) cur[j][v] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kReadBatch; ++i) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) rv[i][v] = 0.0f;
  }

  auto write_row_src = [&](int j) __attribute__((always_inline)) -> const float* {
    const int slot = rl(widx, j);
    if constexpr (DENSE) {
      return table_bank + static_cast<int64_t>(slot) * D;
    } else {
      const int p = rl(wphys, j);
      return p < 0 ? m0_bank + static_cast<int64_t>(slot) * D
                   : L.values + static_cast<int64_t>(p) * D;
    }
  };
  auto read_meta = [&](const int (&arr)[kMaxReadSlots], int r) -> int {
    const int k = r / kWave;
    const int v = k == 0 ? arr[0] : k == 1 ? arr[1] : k == 2 ? arr[2] : arr[3];
    return rl(v, r % kWave);
  };
  auto read_weight = [&](int r) __attribute__((always_inline)) -> float {
    const int k = r / kWave;
    const float v = k == 0 ? rweight[0] : k == 1 ? rweight[1]
                  : k == 2 ? rweight[2] : rweight[3];
    return rlf(v, r % kWave);
  };
  auto read_row_src = [&](int r) __attribute__((always_inline)) -> const float* {
    const int slot = read_meta(ridx, r);
    if constexpr (DENSE) {
      return table_bank + static_cast<int64_t>(slot) * D;
    } else {
      const int p = read_meta(rphys, r);
      return p < 0 ? m0_bank + static_cast<int64_t>(slot) * D
                   : L.values + static_cast<int64_t>(p) * D;
    }
  };
  auto load_writes = [&](int chunk) __attribute__((always_inline)) {
    const int col = chunk * chunk_cols + lane * VEC;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) {
      if (j < W && wok) {
        const float* src = write_row_src(j);
        if (col < D) load_row<VEC>(src + col, cur[j]);
      }
    }
  };
  auto load_read_batch = [&](int chunk, int r0) __attribute__((always_inline)) {
    const int col = chunk * chunk_cols + lane * VEC;
#pragma unroll
    for (int i = 0; i < kReadBatch; ++i) {
      const int r = r0 + i;
      if (r < R && rok && read_meta(rsrc, r) < 0) {
        const float* src = read_row_src(r);
        if (col < D) load_row<VEC>(src + col, rv[i]);
      }
    }
  };

  // ---- pops (packed): first touch of rank q takes the free-stack entry
  // prefix + q from the top (bank-major, allocator.py:1471-1481)
  bool fits = true;
  bool poisoned = false;
  int new_row = -1;
  auto pops = [&]() __attribute__((always_inline)) {
    fits = wok && !poisoned && (count == 0 || prefix + count <= top);
    new_row = pop_row(L, fits && first, prefix, rank, pr, old_free, lane, &fits);
    if (lane == 0) {
      // (planned steps: the closing wave writes the flag)
      if (!P.control && wok && !fits && count > 0 && !poisoned) *L.overflow_flag = 1;
      if (poisoned) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  };

  load_writes(0);
  load_read_batch(0, 0);

  // LOCAL: the pops are known now; their free-stack loads overlap the
  // rows'.  Then the ticket (see take_ticket).
  int64_t ticket = -1;
  bool resolved = DENSE;
  if constexpr (LOCAL) {
    pops();
    resolved = true;
    const int top_lo = static_cast<int>(top);
    const int served_lo = static_cast<int>(table_served);
    const int proven_lo = static_cast<int>(pr.proven_after);
    asm volatile("" ::"v"(top_lo), "v"(new_row), "v"(served_lo), "v"(proven_lo) : "memory");
    ticket = take_ticket(L, lane);
  }
  // look-back: bank-major pop positions from the scratch slots; the row
  // math never depends on physical row ids, so the scan waits only in front
  // of the stores of first-touch rows and map entries
  auto resolve = [&]() __attribute__((always_inline)) {
    if constexpr (!DENSE && !LOCAL) {
      int64_t* slots = L.scratch + COWSDM_SCRATCH_SLOTS;
      prefix = bank_prefix(slots, bank, epoch, count, lane, &poisoned);
      pops();
    }
    resolved = true;
  };

  // ---- gated-delta update and sparse read, chunk by chunk
  for (int chunk = 0; chunk < nchunks; ++chunk) {
    if (chunk > 0) {
      load_writes(chunk);
      load_read_batch(chunk, 0);
    }
    const int col = chunk * chunk_cols + lane * VEC;
    const bool col_ok = col < D;
    float vin[VEC];
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) { vin[v] = 0.0f; acc[v] = 0.0f; }
    if (col_ok) load_row<VEC>(step_values + b * D + col, vin);

    if (wok) {
      // decayed = current * exp(forget); retrieved = sum_w weight_w * decayed_w
      float ret[VEC];
#pragma unroll
      for (int j = 0; j < MAXW; ++j) {
        if (j < W) {
          const float wj = rlf(wweight, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            cur[j][v] = cur[j][v] * alpha;
            const float term = wj * cur[j][v];
            ret[v] = (j == 0) ? term : ret[v] + term;
          }
        }
      }
      // delta = in_gate * value - erase_gate * retrieved
      // updated_w = decayed_w + weight_w * delta
      float delta[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const float a = in_gate * vin[v];
        const float e = er_gate * ret[v];
        delta[v] = a - e;
      }
#pragma unroll
      for (int j = 0; j < MAXW; ++j) {
        if (j < W) {
          const float wj = rlf(wweight, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float t = wj * delta[v];
            cur[j][v] = cur[j][v] + t;
          }
        }
      }
    }
    if (rok) {
      // reading = sum_r weight_r * visible_r, reads after this step's writes
      for (int r0 = 0; r0 < R; r0 += kReadBatch) {
        if (r0 > 0) load_read_batch(chunk, r0);
#pragma unroll
        for (int i = 0; i < kReadBatch; ++i) {
          const int r = r0 + i;
          if (r < R) {
            const int src = read_meta(rsrc, r);
            float x[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) x[v] = rv[i][v];
            if (src >= 0) {
#pragma unroll
              for (int j = 0; j < MAXW; ++j) {
                if (j == src) {
#pragma unroll
                  for (int v = 0; v < VEC; ++v) x[v] = cur[j][v];
                }
              }
            }
            const float wr = read_weight(r);
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
              const float term = wr * x[v];
              acc[v] = (r == 0) ? term : acc[v] + term;
            }
          }
        }
      }
    }
    if (col_ok) store_row<VEC>(output + b * D + col, acc);
    if (wok) {
      // rows already private (and every dense row) need no pop
#pragma unroll
      for (int j = 0; j < MAXW; ++j) {
        if (j < W) {
          const bool is_first = DENSE ? false : (rl(wphys, j) < 0);
          if (!is_first) {
            const int row = DENSE ? rl(widx, j) : rl(wphys, j);
            float* dst = DENSE ? table_bank + static_cast<int64_t>(row) * D
                               : L.values + static_cast<int64_t>(row) * D;
            if (col_ok) store_row<VEC>(dst + col, cur[j]);
          }
        }
      }
    }
    if constexpr (!DENSE) {
      if (!resolved) resolve();
      if (wok && fits && count > 0) {
#pragma unroll
        for (int j = 0; j < MAXW; ++j) {
          if (j < W && rl(wphys, j) < 0) {
            float* dst = L.values + static_cast<int64_t>(rl(new_row, j)) * D;
            if (col_ok) store_row<VEC>(dst + col, cur[j]);
          }
        }
      }
    }
  }
  const bool commit = wok && fits;

  bool closed_layer = false;
  if constexpr (!DENSE) {
    bool stored_ok = true;
    if constexpr (LOCAL) stored_ok = wait_tickets(L, ticket, B, lane);
    if (commit && first && stored_ok) L.logical_to_physical[b * N + widx] = new_row;
    if (lane == 0) {
      if (L.first_touches_out) L.first_touches_out[b] = commit ? count : 0;
      if (L.repeated_writes_out) L.repeated_writes_out[b] = wok ? W - count : W;
    }
    record_errors(L, lane, err_w | err_r);
    // The last bank closes the layer: LOCAL, after the launch's last ticket
    // (every wave has read the words it rewrites); with the look-back, after
    // its scan, which ran once every lower bank had published (and so had
    // read them).  The rows the step popped: LOCAL, the table's last fitting
    // prefix; with the look-back, the last bank's inclusive prefix when it
    // fits, else the largest inclusive prefix that fits, read from the other
    // banks' slots.
    closed_layer = bank == B - 1 && stored_ok;
    if (closed_layer) {
      int64_t served = table_served;
      bool short_rows = false;
      if constexpr (LOCAL) {
        short_rows = served < table.total();
      } else {
        served = prefix + count;
        short_rows = poisoned || served > top;
        if (short_rows) {
          served = fitting_prefix(L.scratch + COWSDM_SCRATCH_SLOTS, B, epoch, top, lane);
        }
        if (lane == 0) {
          atomic_store_u64(&L.scratch[COWSDM_SCRATCH_EPOCH], static_cast<uint64_t>(epoch + 1u));
        }
      }
      close_layer(P, L, layer_id, lane, pr, old_free, served, short_rows);
    }
  } else {
    record_errors(L, lane, err_w | err_r);
  }
  finish_trace<DENSE>(P, layer_id, lane, trace_s, closed_layer);
}

template <typename IDX, int MAXW, int VEC, bool DENSE, bool LOCAL>
void launch_step(const StepParams& P, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((sdm_step_kernel<IDX, MAXW, VEC, DENSE, LOCAL>), dim3(blocks),
                     dim3(kStepThreads), 0, stream, P);
}

template <typename IDX, int VEC, bool DENSE>
void launch_small(const StepParams& P, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((sdm_step_small_kernel<IDX, VEC, DENSE>), dim3(blocks),
                     dim3(kStepThreads), 0, stream, P);
}

template <typename IDX, int MAXW, bool DENSE>
void launch_step_vec(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  if constexpr (MAXW <= kLocalTableWrites) {
    // the small kernel: one pass over the row, at most 16 reads, and (packed)
    // a layer the first-touch table covers
    if (P.reads <= kSmallReads && P.width <= kWave * vec &&
        (DENSE || P.banks <= kLocalTableBanks)) {
      if (vec == 4) launch_small<IDX, 4, DENSE>(P, blocks, stream);
      else if (vec == 2) launch_small<IDX, 2, DENSE>(P, blocks, stream);
      else launch_small<IDX, 1, DENSE>(P, blocks, stream);
      return;
    }
    if (!DENSE && P.banks <= kLocalTableBanks) {
      if (vec == 4) launch_step<IDX, MAXW, 4, false, true>(P, blocks, stream);
      else if (vec == 2) launch_step<IDX, MAXW, 2, false, true>(P, blocks, stream);
      else launch_step<IDX, MAXW, 1, false, true>(P, blocks, stream);
      return;
    }
  }
  if (vec == 4) launch_step<IDX, MAXW, 4, DENSE, false>(P, blocks, stream);
  else if (vec == 2) launch_step<IDX, MAXW, 2, DENSE, false>(P, blocks, stream);
  else launch_step<IDX, MAXW, 1, DENSE, false>(P, blocks, stream);
}

template <typename IDX, bool DENSE>
void launch_step_w(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  if (P.writes <= 4) launch_step_vec<IDX, 4, DENSE>(P, blocks, vec, stream);
  else if (P.writes <= 16) launch_step_vec<IDX, 16, DENSE>(P, blocks, vec, stream);
  else launch_step_vec<IDX, 64, DENSE>(P, blocks, vec, stream);
}


}  // namespace cowsdm_impl
