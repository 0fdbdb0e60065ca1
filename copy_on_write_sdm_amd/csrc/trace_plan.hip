// Plan of a packed decode-trace launch: which (step, bank) first-touches
// which slots, the capacity proof of the decode loop and the slab growth it
// triggers, and the physical row every first touch pops -- all decided
// before the persistent kernel (trace_kernel.h) runs the launch's steps.
//
// The reference's decode loop proves every step on the host before running
// it (inference.py:551-552: prepare_step_capacity(banks * W), allocator.py:
// 745-773): the proven counter drops by banks * W per step, free_count is
// read only when the counter runs short, and the slab grows by the pooled
// quantum only when free_count is below banks * W at such a read
// (grow_capacity, allocator.py:691-743: new row ids join the top of the free
// stack).  Single steps pop first-touch rows bank-major from the top of the
// stack (allocator.py:1471-1481).  Every one of those decisions depends only
// on how many first touches each (step, bank) makes, and that depends only
// on the routes and on which slots were mapped when the launch starts: slot
// x is first-touched by the first step of the launch that writes it, unless
// it was mapped already.  So two passes settle the whole launch up front:
//
//   count pass (one workgroup per (layer, bank), steps split across its four
//   waves): finds each step's first-touch write lanes and the bank's first
//   step with an invalid route (out-of-range slot, a slot written twice in
//   one step, a map entry outside the slab, an invalid template), after which
//   the bank takes no step;
//
//   plan pass (one workgroup per layer): sums the counts per step, replays
//   the decode loop's proof step by step from the control words (growing the
//   capacity within the slab's buffers, or stopping the layer before a growth
//   that would not fit), gives every (step, bank) the number of first
//   touches before it in pop order, lists the row each pop takes, and writes
//   the free stack, free_count and overflow flag the launch leaves.
//
// The persistent kernel then runs the planned steps and takes the rows of
// (step, bank) from the pop list at its offset, so maps, slabs and free
// stacks equal those of the single-step loop bit for bit.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "common.h"

namespace cowsdm_impl {

namespace {

constexpr int kCountWaves = 4;
constexpr int kCountThreads = kWave * kCountWaves;
constexpr int kCountChunks = kTraceMaxSteps / kCountThreads;   // 64-step chunks per wave
constexpr int kPlanThreads = 1024;
constexpr int kPlanBatch = 16;   // plan words a plan thread loads at once
constexpr int kIntMax = 0x7fffffff;

// Fibonacci hash of a slot into a table of 2^bits entries.
__device__ __forceinline__ uint32_t hash_slot(int x, int bits) {
  return (static_cast<uint32_t>(x) * 0x9E3779B1u) >> (32 - bits);
}

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {  // a >= 0, b > 0
  if (a < (int64_t{1} << 32) && b < (int64_t{1} << 32)) {
    return static_cast<int64_t>(static_cast<uint32_t>(a) / static_cast<uint32_t>(b));
  }
  return a / b;
}

// Exclusive prefix of v over the workgroup's threads in order; *total gets
// the sum.  Every thread of the workgroup must call it.
__device__ int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  int x = v;
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) wave_sums[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x) / kWave; ++w) {
      const int t = wave_sums[w];
      wave_sums[w] = run;
      run += t;
    }
    *total = run;
  }
  __syncthreads();
  return x - v + wave_sums[wave];
}

// ------------------------------------------------------------ count pass

// Lane = step: each lane of wave w handles steps 64 * (w + 4k) + lane.
// MAPLDS (N <= kTraceMapSlots): the bank's map row and the first step of the
// launch writing each slot sit in LDS (dynamic, 2N ints), and read slots are
// checked against the slab too.  Otherwise the first writing steps live in an
// LDS hash table of count_table entries keyed by slot (at most half full),
// and only write slots' map entries are checked (a read slot's entry outside
// the slab stops the bank in the persistent kernel alone).
template <typename IDX, bool MAPLDS>
__global__ __launch_bounds__(kCountThreads) void trace_count_kernel(StepParams P) {
  extern __shared__ int lds_dyn[];
  __shared__ int s_stop;       // the bank's first step with an invalid route
  __shared__ int s_bits;       // its COWSDM_ERR_* bits
  const int layer_id = static_cast<int>(blockIdx.x) / P.banks;
  const int bank = static_cast<int>(blockIdx.x) % P.banks;
  if (layer_id >= P.nlayers) return;
  const cowsdm_layer_t& L = P.layer[layer_id];
  int64_t first, left;
  trace_span(P, layer_id, first, left);
  const int G = static_cast<int>(left < P.plan_steps ? left : P.plan_steps);
  if (G <= 0) return;
  const int N = P.slots;
  const int W = P.writes;
  const int R = P.reads;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int64_t C = control_word(P, layer_id, COWSDM_CTRL_CAPACITY);
  const int32_t* const map_bank = L.logical_to_physical + static_cast<int64_t>(bank) * N;
  const int TS = P.count_table;
  const int bits = 31 - __builtin_clz(TS > 1 ? TS : 2);
  int* const lmap = lds_dyn;                               // MAPLDS: slot map [N]
  int* const keys = lds_dyn;                               // hash: slot of each entry
  int* const fw = lds_dyn + (MAPLDS ? N : TS);             // first writing step
  // every route index this thread checks, loaded before anything waits
  // (lane = step: each load is its own cache line, so all of them are
  // issued at once)
  IDX wv[kCountChunks][kTraceMaxWrites];
  IDX rv[kCountChunks][kTraceMaxReads];
#pragma unroll
  for (int k = 0; k < kCountChunks; ++k) {
    const int t0 = (wave + k * kCountWaves) * kWave + lane;
    const int t = t0 < G ? t0 : G - 1;
    const IDX* const w = reinterpret_cast<const IDX*>(
        static_cast<const char*>(L.write_indices) + (first + t) * P.trace_stride[0]) +
        static_cast<int64_t>(bank) * W;
    const IDX* const r = reinterpret_cast<const IDX*>(
        static_cast<const char*>(L.read_indices) + (first + t) * P.trace_stride[6]) +
        static_cast<int64_t>(bank) * R;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) wv[k][j] = w[j < W ? j : W - 1];
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) rv[k][i] = r[i < R ? i : R - 1];
  }
  if (threadIdx.x == 0) {
    const int64_t tmpl = L.template_indices[bank];
    s_stop = (tmpl < 0 || tmpl >= P.templates) ? 0 : G;
    s_bits = 0;
  }
  const int entries = MAPLDS ? N : TS;
  for (int k = static_cast<int>(threadIdx.x); k < entries; k += kCountThreads) {
    if constexpr (MAPLDS) {
      lmap[k] = map_bank[k];
    } else {
      keys[k] = -1;
    }
    fw[k] = kIntMax;
  }
  __syncthreads();

  auto find = [&](int x) __attribute__((always_inline)) -> int {
    uint32_t h = hash_slot(x, bits);
    for (int p = 0; p < TS; ++p) {
      if (keys[h] == x) break;
      h = (h + 1) & static_cast<uint32_t>(TS - 1);
    }
    return static_cast<int>(h);
  };

  // ---- phase 1: validate each step, record the first step writing each slot
  int slot[kCountChunks][kTraceMaxWrites];
  uint32_t mapped[kCountChunks];
  int err[kCountChunks];
#pragma unroll
  for (int k = 0; k < kCountChunks; ++k) {
    const int t = (wave + k * kCountWaves) * kWave + lane;
    mapped[k] = 0;
    err[k] = 0;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) slot[k][j] = -1;
    if (t >= G) continue;
    int e = 0;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W) {
        const int64_t v = static_cast<int64_t>(wv[k][j]);
        if (v < 0 || v >= N) {
          e |= COWSDM_ERR_WRITE_INDEX;
        } else {
          slot[k][j] = static_cast<int>(v);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
#pragma unroll
      for (int i = j + 1; i < kTraceMaxWrites; ++i) {
        if (slot[k][j] >= 0 && slot[k][j] == slot[k][i]) e |= COWSDM_ERR_DUP_WRITE;
      }
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      if (i < R) {
        const int64_t v = static_cast<int64_t>(rv[k][i]);
        if (v < 0 || v >= N) {
          e |= COWSDM_ERR_READ_INDEX;
        } else if (MAPLDS && lmap[v] >= C) {
          e |= COWSDM_ERR_CORRUPT;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      const int x = slot[k][j];
      if (x < 0) continue;
      const int m = MAPLDS ? lmap[x] : map_bank[x];
      if (m >= C) e |= COWSDM_ERR_CORRUPT;
      if (m >= 0) mapped[k] |= 1u << j;
    }
    err[k] = e;
    if (e != 0) atomicMin(&s_stop, t);
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      const int x = slot[k][j];
      if (x < 0) continue;
      if constexpr (MAPLDS) {
        atomicMin(&fw[x], t);
      } else {
        uint32_t h = hash_slot(x, bits);
        for (int p = 0; p < TS; ++p) {
          const int prev = atomicCAS(&keys[h], -1, x);
          if (prev == -1 || prev == x) {
            atomicMin(&fw[h], t);
            break;
          }
          h = (h + 1) & static_cast<uint32_t>(TS - 1);
        }
      }
    }
  }
  __syncthreads();
  const int stop = s_stop;
#pragma unroll
  for (int k = 0; k < kCountChunks; ++k) {
    const int t = (wave + k * kCountWaves) * kWave + lane;
    if (t == stop) atomicOr(&s_bits, err[k]);
  }

  // ---- phase 2: each step's first-touch write lanes
  int32_t* const words = plan_words(P, layer_id) + static_cast<int64_t>(bank) * P.plan_steps;
#pragma unroll
  for (int k = 0; k < kCountChunks; ++k) {
    const int t = (wave + k * kCountWaves) * kWave + lane;
    if (t >= G) continue;
    uint32_t mask = 0;
    if (t < stop) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        const int x = slot[k][j];
        if (x < 0 || ((mapped[k] >> j) & 1u)) continue;
        const int f = MAPLDS ? fw[x] : fw[find(x)];
        if (f == t) mask |= 1u << j;
      }
    }
    words[t] = static_cast<int32_t>((mask << kPlanMaskShift) |
                                    (t >= stop ? 1u << kPlanStopBit : 0u));
  }
  __syncthreads();
  if (threadIdx.x == 0 && s_bits != 0) {
    __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(s_bits),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------- plan pass

// One workgroup per layer.  Segments: segment 0 starts at the launch's first
// step with the stack as the launch found it; segment k >= 1 starts at the
// step of growth k, whose new row ids old_k .. old_k + (top_k - free_k) - 1
// sit on the stack at positions free_k .. top_k - 1 above the free_k rows
// there before it.  The stack entry at position p during segment k is the
// row the latest growth j <= k whose positions cover p put there, or the
// entry the launch found (every position below each growth's free_k was
// never popped since).
__global__ __launch_bounds__(kPlanThreads) void trace_plan_kernel(StepParams P) {
  __shared__ int s_part[kPlanThreads];           // per (part of the banks, step)
  __shared__ int s_cum[kTraceMaxSteps + 1];      // first touches before step t
  __shared__ int s_seg_step[kTraceMaxSteps + 1];
  __shared__ int s_seg_q[kTraceMaxSteps + 1];    // first touches before the segment
  __shared__ int s_seg_free[kTraceMaxSteps + 1]; // stack height before its growth
  __shared__ int s_seg_top[kTraceMaxSteps + 1];  // stack height after its growth
  __shared__ int s_seg_old[kTraceMaxSteps + 1];  // capacity before its growth
  __shared__ int s_wave_sums[kPlanThreads / kWave];
  __shared__ int s_total;
  __shared__ int s_nseg, s_stop, s_vlen, s_fit, s_over;
  __shared__ int64_t s_proven, s_capacity, s_added;
  __shared__ int64_t s_events, s_rows_added, s_rows_copied;

  const int layer_id = static_cast<int>(blockIdx.x);
  if (layer_id >= P.nlayers) return;
  const cowsdm_layer_t& L = P.layer[layer_id];
  const int tid = static_cast<int>(threadIdx.x);
  int64_t first, left;
  trace_span(P, layer_id, first, left);
  const int G = static_cast<int>(left < P.plan_steps ? left : P.plan_steps);
  if (G <= 0) {
    if (tid == 0) control_word(P, layer_id, COWSDM_CTRL_STEPS) = 0;
    return;
  }
  const int B = P.banks;
  const int S = P.plan_steps;
  int32_t* const words = plan_words(P, layer_id);
  int32_t* const pops = plan_pops(P, layer_id);
  const int64_t C0 = control_word(P, layer_id, COWSDM_CTRL_CAPACITY);
  const int F0 = *L.free_count;
  if (F0 < 0 || F0 > C0) {
    // a corrupt free count: the layer runs nothing
    if (tid == 0) {
      control_word(P, layer_id, COWSDM_CTRL_STEPS) = 0;
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
      if (P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }

  // ---- first touches per step, summed over parts of the banks
  const int Gp = (G + kWave - 1) / kWave * kWave;   // <= 512
  const int parts = kPlanThreads / Gp;               // >= 2
  const int t = tid % Gp;
  const int part = tid / Gp;
  const int b0 = part < parts ? static_cast<int>(static_cast<int64_t>(B) * part / parts) : B;
  const int b1 = part < parts ? static_cast<int>(static_cast<int64_t>(B) * (part + 1) / parts) : B;
  const bool mine = part < parts && t < G;
  // A thread's plan words are kPlanBatch independent loads at a time (a
  // loop of dependent-looking loads would wait for each one in turn).
  auto load_words = [&](int b, uint32_t (&w)[kPlanBatch]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPlanBatch; ++i) {
      const int bi = b + i < b1 ? b + i : b1 - 1;
      w[i] = static_cast<uint32_t>(words[static_cast<int64_t>(bi) * S + t]);
    }
  };
  {
    int sum = 0;
    if (mine) {
      for (int b = b0; b < b1; b += kPlanBatch) {
        uint32_t w[kPlanBatch];
        load_words(b, w);
#pragma unroll
        for (int i = 0; i < kPlanBatch; ++i) {
          if (b + i < b1) sum += __popc((w[i] >> kPlanMaskShift) & 15u);
        }
      }
    }
    s_part[tid] = sum;
  }
  __syncthreads();
  {
    // step totals (thread t < Gp), their exclusive scan over steps, and each
    // part's offset within its step
    int total = 0;
    if (tid < Gp) {
      for (int p = 0; p < parts; ++p) total += s_part[p * Gp + tid];
    }
    const int before = block_exclusive_scan(tid < Gp ? total : 0, s_wave_sums, &s_total);
    if (tid < Gp) {
      if (tid <= G) s_cum[tid] = before;
      int run = before;
      for (int p = 0; p < parts; ++p) {
        const int v = s_part[p * Gp + tid];
        s_part[p * Gp + tid] = run;
        run += v;
      }
    }
    if (tid == 0) s_cum[G] = s_total;
  }
  __syncthreads();

  // ---- the decode loop's capacity proof, step by step (one thread)
  if (tid == 0) {
    int64_t proven = control_word(P, layer_id, COWSDM_CTRL_PROVEN);
    int64_t capacity = C0;
    const int64_t room = control_word(P, layer_id, COWSDM_CTRL_ROOM);
    const int64_t quantum = control_word(P, layer_id, COWSDM_CTRL_QUANTUM);
    const int64_t need = control_word(P, layer_id, COWSDM_CTRL_NEED);
    int64_t added = 0, events = 0, rows_added = 0, rows_copied = 0;
    int nseg = 1;
    s_seg_step[0] = 0;
    s_seg_q[0] = 0;
    s_seg_free[0] = F0;
    s_seg_top[0] = F0;
    s_seg_old[0] = static_cast<int>(C0);
    int stop = G;
    bool over = false;
    if (need > 0 && quantum > 0) {
      int s = 0;
      if (proven >= need) {
        // steps still covered by the proof the launch starts with
        int64_t j = floor_div(proven, need);
        if (j > G) j = G;
        if (s_cum[j] > F0) over = true;   // the proof was not honest
        proven -= j * need;
        s = static_cast<int>(j);
      }
      // from here every step whose proof runs short re-reads free_count
      while (!over && s < G) {
        int64_t free_rows = F0 + added - s_cum[s];
        if (free_rows < need) {
          const int64_t want = capacity + need - free_rows;
          const int64_t selected = (want + quantum - 1) / quantum * quantum;
          if (selected > room || selected >= (int64_t{1} << 31)) {
            stop = s;   // the host grows the slab into a larger buffer
            break;
          }
          const int64_t a = selected - capacity;
          s_seg_step[nseg] = s;
          s_seg_q[nseg] = s_cum[s];
          s_seg_free[nseg] = static_cast<int>(free_rows);
          s_seg_top[nseg] = static_cast<int>(free_rows + a);
          s_seg_old[nseg] = static_cast<int>(capacity);
          ++nseg;
          ++events;
          rows_added += a;
          rows_copied += capacity;
          added += a;
          capacity = selected;
          free_rows += a;
        }
        int64_t j = floor_div(free_rows, need);   // >= 1
        if (j > G - s) j = G - s;
        proven = free_rows - j * need;
        s += static_cast<int>(j);
      }
    } else if (s_cum[G] > F0) {
      over = true;   // no proof: the stack runs out
    }
    s_nseg = nseg;
    s_stop = stop;
    s_over = over ? 1 : 0;
    s_vlen = static_cast<int>(over ? F0 + added : s_cum[stop]);
    s_fit = 0;
    s_proven = over ? 0 : proven;
    s_capacity = capacity;
    s_added = added;
    s_events = events;
    s_rows_added = rows_added;
    s_rows_copied = rows_copied;
  }
  __syncthreads();
  const int nseg = s_nseg;
  const int stop = s_stop;
  const int vlen = s_vlen;
  const bool over = s_over != 0;

  // ---- plan words: first touches before each (step, bank) in pop order
  if (mine) {
    int run = s_part[tid];
    for (int b = b0; b < b1; b += kPlanBatch) {
      uint32_t w[kPlanBatch];
      load_words(b, w);
#pragma unroll
      for (int i = 0; i < kPlanBatch; ++i) {
        if (b + i < b1) {
          const uint32_t v = w[i];
          const int c = __popc((v >> kPlanMaskShift) & 15u);
          words[static_cast<int64_t>(b + i) * S + t] =
              static_cast<int32_t>((v & ~kPlanBaseMask) | static_cast<uint32_t>(run));
          run += c;
          if (over && c > 0 && run <= vlen) atomicMax(&s_fit, run);
        }
      }
    }
  }

  // The stack entry at position p during segment k (see above).
  const int32_t* const found = L.free_rows;
  auto entry = [&](int p, int k) __attribute__((always_inline)) -> int {
    for (int j = k; j >= 1; --j) {
      if (p >= s_seg_free[j]) return s_seg_old[j] + (p - s_seg_free[j]);
    }
    return found[p];
  };
  // ---- the row each pop takes: segment k pops from its top down
  const int listed = vlen < s_cum[stop] ? vlen : s_cum[stop];
  for (int k = 0; k < nseg; ++k) {
    const int q0 = s_seg_q[k];
    const int q1 = k + 1 < nseg ? s_seg_q[k + 1] : listed;
    const int top = s_seg_top[k];
    for (int q = q0 + tid; q < q1; q += kPlanThreads) {
      pops[q] = entry(top - 1 - (q - q0), k);
    }
  }
  __syncthreads();   // every entry the launch found was read

  // ---- the stack the launch leaves
  const int fit = over ? s_fit : s_cum[stop];
  const int64_t height = F0 + s_added - fit;
  if (nseg > 1) {
    int lo = s_seg_free[1];
    for (int k = 2; k < nseg; ++k) lo = s_seg_free[k] < lo ? s_seg_free[k] : lo;
    // (the layer struct lists free_rows as read-only for the step kernels;
    // the plan is the one pass that rewrites it)
    int32_t* const stack = const_cast<int32_t*>(L.free_rows);
    for (int64_t p = lo + tid; p < height; p += kPlanThreads) {
      stack[p] = entry(static_cast<int>(p), nseg - 1);
    }
  }
  if (tid == 0) {
    *L.free_count = static_cast<int32_t>(height);
    if (over) {
      *L.overflow_flag = 1;
    } else if (nseg > 1) {
      *L.overflow_flag = 0;   // grow_capacity clears it
    }
    control_word(P, layer_id, COWSDM_CTRL_PROVEN) = s_proven;
    control_word(P, layer_id, COWSDM_CTRL_CAPACITY) = s_capacity;
    control_word(P, layer_id, COWSDM_CTRL_EVENTS) += s_events;
    control_word(P, layer_id, COWSDM_CTRL_ADDED) += s_rows_added;
    control_word(P, layer_id, COWSDM_CTRL_COPIED) += s_rows_copied;
    control_word(P, layer_id, COWSDM_CTRL_FREE) = height;
    control_word(P, layer_id, COWSDM_CTRL_STEPS) = stop;
    control_word(P, layer_id, COWSDM_CTRL_FIT) = vlen;
    if (stop < G && P.trace_status) {
      __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_REFUSED},
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

// Count and plan passes of one packed persistent launch (all layers of P).
// With `start` given, the count pass records it when it starts.
template <typename IDX>
int32_t launch_trace_plan(const StepParams& P, hipStream_t stream, hipEvent_t start) {
  const bool maplds = P.slots <= kTraceMapSlots;
  const size_t lds = 2 * sizeof(int) * static_cast<size_t>(maplds ? P.slots : P.count_table);
  const dim3 grid(static_cast<unsigned>(P.nlayers * P.banks));
  StepParams Q = P;
  void* args[] = {&Q};
  const void* count = maplds ? reinterpret_cast<const void*>(&trace_count_kernel<IDX, true>)
                             : reinterpret_cast<const void*>(&trace_count_kernel<IDX, false>);
  (void)hipExtLaunchKernel(count, grid, dim3(kCountThreads), args, lds, stream, start, nullptr,
                           0);
  if (int32_t e = launch_status("trace count")) return e;
  hipLaunchKernelGGL(trace_plan_kernel, dim3(static_cast<unsigned>(P.nlayers)), dim3(kPlanThreads),
                     0, stream, P);
  return launch_status("trace plan");
}

template int32_t launch_trace_plan<int32_t>(const StepParams&, hipStream_t, hipEvent_t);
template int32_t launch_trace_plan<int64_t>(const StepParams&, hipStream_t, hipEvent_t);

}  // namespace cowsdm_impl
