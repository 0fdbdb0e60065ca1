// libcowsdm: copy-on-write Sparse Delta Memory decode step for MI355X
// (gfx950), plus the slab lifecycle (growth, pack handoff, release, bank
// retention, trim, admission, invariant checks).  Exposed through the C ABI
// declared in include/cowsdm.h.
//
// Semantics follow the reference's torch path, copy_on_write_sdm/
// allocator.py:1466-1525 (packed step) and 1612-1633 (dense step), with
// first-touch rows popped from the free stack in bank-major order exactly as
// allocator.py:1471-1481 orders them.
//
// Design (one wavefront per bank):
//  * lane l < W holds write route l, lane l holds read routes l, l+64, ...;
//    route metadata is broadcast with readlane so every row address is a
//    wave-uniform base plus a lane offset: each D=128 row is one coalesced
//    512-byte access (two floats per lane).
//  * every write row and every read row that is not also written this step
//    is loaded before any cross-bank wait, so the HBM latency of the row
//    loads overlaps the free-stack resolution;
//  * a read of a slot written in the same step takes the updated row from
//    registers (read-after-write without a barrier or a reload);
//  * first touches pop rows at free_count-1-(bank prefix + rank).  The bank
//    prefix is an exclusive scan over banks computed with a decoupled
//    look-back over per-bank slots in the layer's scratch; every wave only
//    waits on lower-numbered banks of its own layer, and every wait is
//    bounded (a timed-out scan poisons the banks after it instead of
//    hanging);
//  * the last bank to finish (ticket counter) publishes the new free_count
//    and advances the scratch epoch, which retires this launch's slots.
//  * float math is the reference's operation order with every product and
//    sum rounded separately (the file is built with -ffp-contract=off);
//    exp(forget_log_gate) is evaluated in double and rounded once.

#include <hip/hip_runtime.h>
#include <stdarg.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "common.h"
#include "cowsdm.h"

namespace cowsdm_impl {

template <typename IDX, bool DENSE>
void launch_step_w(const StepParams& P, int blocks, int vec, hipStream_t stream);
extern template void launch_step_w<int32_t, false>(const StepParams&, int, int, hipStream_t);
extern template void launch_step_w<int32_t, true>(const StepParams&, int, int, hipStream_t);
extern template void launch_step_w<int64_t, false>(const StepParams&, int, int, hipStream_t);
extern template void launch_step_w<int64_t, true>(const StepParams&, int, int, hipStream_t);
template <typename IDX, bool DENSE>
int32_t launch_trace(const StepParams& P, int vec, hipStream_t stream);
extern template int32_t launch_trace<int32_t, false>(const StepParams&, int, hipStream_t);
extern template int32_t launch_trace<int32_t, true>(const StepParams&, int, hipStream_t);
extern template int32_t launch_trace<int64_t, false>(const StepParams&, int, hipStream_t);
extern template int32_t launch_trace<int64_t, true>(const StepParams&, int, hipStream_t);

namespace {
thread_local char g_error[512] = "";
}  // namespace

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int32_t launch_status(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "%s: %s", where, hipGetErrorString(e));
  }
  return 0;
}

const char* last_error() { return g_error; }

// cowsdm_trace_timing: per persistent launch, events at its first kernel's
// start, at its decode kernel's start and at the decode kernel's end
namespace {
constexpr int kTimingSlots = 1024;
bool timing_on = false;
int timing_used = 0;
int timing_made = 0;
hipEvent_t timing_first[kTimingSlots];
hipEvent_t timing_start[kTimingSlots];
hipEvent_t timing_stop[kTimingSlots];
bool timing_single[kTimingSlots];   // the decode kernel is the launch's first
}  // namespace

bool trace_timing_events(hipEvent_t* first, hipEvent_t* start, hipEvent_t* stop) {
  if (!timing_on || timing_used >= kTimingSlots) return false;
  if (timing_used == timing_made) {
    hipEvent_t e[3];
    int made = 0;
    for (; made < 3; ++made) {
      if (hipEventCreate(&e[made]) != hipSuccess) break;
    }
    if (made < 3) {
      for (int i = 0; i < made; ++i) (void)hipEventDestroy(e[i]);
      return false;
    }
    timing_first[timing_made] = e[0];
    timing_start[timing_made] = e[1];
    timing_stop[timing_made] = e[2];
    ++timing_made;
  }
  *first = timing_first[timing_used];
  *start = timing_start[timing_used];
  *stop = timing_stop[timing_used];
  timing_single[timing_used] = false;
  ++timing_used;
  return true;
}

void trace_timing_first_is_start() {
  if (timing_used > 0) timing_single[timing_used - 1] = true;
}

// Validation before a step (validate_routes=True, or a packed state whose
// capacity has no proof): bounds, duplicate writes, first touches vs the
// free stack.  One workgroup; writes its result word once.
template <typename IDX>
__global__ __launch_bounds__(1024) void precheck_kernel(
    cowsdm_layer_t L, int32_t banks, int32_t slots, int32_t writes,
    int32_t reads, int32_t dense, int32_t check_unique, int32_t check_capacity,
    int64_t* result) {
  __shared__ int s_flags;
  __shared__ unsigned long long s_first;
  if (threadIdx.x == 0) { s_flags = 0; s_first = 0; }
  __syncthreads();
  int flags = 0;
  unsigned long long first = 0;
  const int64_t nw = static_cast<int64_t>(banks) * writes;
  const int64_t C = L.capacity_rows;
  for (int64_t e = threadIdx.x; e < nw; e += blockDim.x) {
    const int64_t b = e / writes;
    const int64_t w = e % writes;
    const int64_t x = load_index<IDX>(L.write_indices, e);
    if (x < 0 || x >= slots) { flags |= COWSDM_ERR_WRITE_INDEX; continue; }
    if (check_unique) {
      for (int64_t w2 = 0; w2 < w; ++w2) {
        if (load_index<IDX>(L.write_indices, b * writes + w2) == x) {
          flags |= COWSDM_ERR_DUP_WRITE;
        }
      }
    }
    if (check_capacity && !dense) {
      const int p = map_entry(L, b, slots, static_cast<int>(x));
      if (p < 0) ++first;
      else if (p >= C) flags |= COWSDM_ERR_CORRUPT;
    }
  }
  const int64_t nr = static_cast<int64_t>(banks) * reads;
  for (int64_t e = threadIdx.x; e < nr; e += blockDim.x) {
    const int64_t x = load_index<IDX>(L.read_indices, e);
    if (x < 0 || x >= slots) flags |= COWSDM_ERR_READ_INDEX;
  }
  if (flags) atomicOr(&s_flags, flags);
  if (first) atomicAdd(&s_first, first);
  __syncthreads();
  if (threadIdx.x == 0) {
    int out = s_flags;
    if (check_capacity && !dense) {
      const int64_t f = *L.free_count;
      if (static_cast<int64_t>(s_first) > f) out |= COWSDM_ERR_EXHAUSTED;
    }
    *result = out;
  }
}

// ------------------------------------------------------------ lifecycle

__global__ void init_state_kernel(int32_t* map, int64_t map_entries,
                                  int32_t* free_rows, int64_t capacity,
                                  int32_t* free_count, int32_t* overflow,
                                  int64_t* scratch, int64_t scratch_words) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = t0; i < map_entries; i += stride) map[i] = -1;
  for (int64_t i = t0; i < capacity; i += stride) free_rows[i] = static_cast<int32_t>(i);
  for (int64_t i = t0; i < scratch_words; i += stride) scratch[i] = 0;
  if (t0 == 0) {
    *free_count = static_cast<int32_t>(capacity);
    *overflow = 0;
  }
}

__device__ __forceinline__ void check_templates_body(
    const int64_t* tmpl, int64_t banks, int64_t templates, int64_t* result) {
  __shared__ int s_bad;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();
  int bad = 0;
  for (int64_t i = threadIdx.x; i < banks; i += blockDim.x) {
    if (tmpl[i] < 0 || tmpl[i] >= templates) bad = 1;
  }
  if (bad) atomicOr(&s_bad, 1);
  __syncthreads();
  if (threadIdx.x == 0) *result = s_bad ? COWSDM_ERR_TEMPLATE : 0;
}
__global__ __launch_bounds__(256) void check_templates_kernel(
    const int64_t* tmpl, int64_t banks, int64_t templates, int64_t* result) {
  check_templates_body(tmpl, banks, templates, result);
}

// Row copy dst[dst_rows[i]] = src[src_rows[i]] for i < *count (null row
// lists mean identity); float4 when the width allows it.
__device__ __forceinline__ void copy_rows_body(float* dst, const int32_t* dst_rows,
                                 const float* src, const int32_t* src_rows,
                                 const int64_t* count_ptr, int64_t count_max,
                                 int64_t width) {
  int64_t count = count_ptr ? *count_ptr : count_max;
  if (count > count_max) count = count_max;
  const bool v4 = (width % 4) == 0;
  const int64_t per_row = v4 ? width / 4 : width;
  const int64_t total = count * per_row;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < total; i += stride) {
    const int64_t row = i / per_row;
    const int64_t c = i % per_row;
    const int64_t s = src_rows ? src_rows[row] : row;
    const int64_t d = dst_rows ? dst_rows[row] : row;
    if (s < 0 || d < 0) continue;
    if (v4) {
      reinterpret_cast<float4*>(dst + d * width)[c] =
          reinterpret_cast<const float4*>(src + s * width)[c];
    } else {
      dst[d * width + c] = src[s * width + c];
    }
  }
}
__global__ void copy_rows_kernel(float* dst, const int32_t* dst_rows,
                                 const float* src, const int32_t* src_rows,
                                 const int64_t* count_ptr, int64_t count_max,
                                 int64_t width) {
  copy_rows_body(dst, dst_rows, src, src_rows, count_ptr, count_max, width);
}

__global__ void copy_i64_kernel(int64_t* dst, const int64_t* src, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n; i += stride) {
    dst[i] = src[i];
  }
}

__global__ void grow_free_kernel(const int32_t* old_free_rows,
                                 int32_t* new_free_rows,
                                 const int32_t* free_count,
                                 int64_t old_capacity, int64_t new_capacity) {
  const int64_t f = *free_count;
  const int64_t added = new_capacity - old_capacity;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (f < 0 || f > old_capacity) return;
  for (int64_t i = t0; i < f; i += stride) new_free_rows[i] = old_free_rows[i];
  for (int64_t j = t0; j < added; j += stride) {
    new_free_rows[f + j] = static_cast<int32_t>(old_capacity + j);
  }
}

__global__ void add_counter_kernel(int32_t* counter, int64_t delta,
                                   const int64_t* delta_ptr, int32_t sign,
                                   int32_t* clear) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int64_t d = delta_ptr ? *delta_ptr : delta;
    *counter = static_cast<int32_t>(*counter + sign * d);
    if (clear) *clear = 0;
  }
}

// Workspace for ranking passes.
struct Workspace {
  int64_t* total;       // [1]
  int64_t* aux;         // [7] scratch words
  int32_t* tile_count;  // [ntiles]
  int32_t* tile_offset; // [ntiles]
  int32_t* list_a;      // [rows]
  int32_t* list_b;      // [rows]
};

int64_t num_tiles(int64_t entries) { return (entries + kTile - 1) / kTile; }

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

Workspace carve(void* base, int64_t entries, int64_t rows) {
  char* p = static_cast<char*>(base);
  Workspace w;
  w.total = reinterpret_cast<int64_t*>(p);
  w.aux = reinterpret_cast<int64_t*>(p) + 1;
  p += 256;
  const int64_t nt = num_tiles(entries);
  w.tile_count = reinterpret_cast<int32_t*>(p);
  p += align_up(nt * 4, 256);
  w.tile_offset = reinterpret_cast<int32_t*>(p);
  p += align_up(nt * 4, 256);
  w.list_a = reinterpret_cast<int32_t*>(p);
  p += align_up(rows * 4, 256);
  w.list_b = reinterpret_cast<int32_t*>(p);
  return w;
}

// Predicate source of a ranking: row `i` of the ranked order is map row
// bank_list[i] (or i), or the mask row i.
struct RankSource {
  const int32_t* map;
  const int64_t* bank_list;
  const uint8_t* mask;
  int64_t slots;
  int64_t entries;
  int64_t banks;  // rows of `map`; listed rows outside [0, banks) are empty
};

__device__ __forceinline__ int64_t rank_row(const RankSource& s, int64_t e) {
  const int64_t i = e / s.slots;
  const int64_t row = s.bank_list ? s.bank_list[i] : i;
  return (row >= 0 && row < s.banks) ? row : -1;
}

__device__ __forceinline__ bool rank_active(const RankSource& s, int64_t e) {
  if (s.mask) return s.mask[e] != 0;
  const int64_t row = rank_row(s, e);
  return row >= 0 && s.map[row * s.slots + e % s.slots] >= 0;
}

__device__ __forceinline__ void rank_count_body(
    RankSource s, int32_t* tile_count) {
  __shared__ int s_sum;
  if (threadIdx.x == 0) s_sum = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile + threadIdx.x * kPerThread;
  int c = 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t e = base + k;
    if (e < s.entries && rank_active(s, e)) ++c;
  }
  if (c) atomicAdd(&s_sum, c);
  __syncthreads();
  if (threadIdx.x == 0) tile_count[blockIdx.x] = s_sum;
}
__global__ __launch_bounds__(kTileThreads) void rank_count_kernel(
    RankSource s, int32_t* tile_count) {
  rank_count_body(s, tile_count);
}

// Exclusive scan of tile counts by one workgroup; writes the total.
__device__ __forceinline__ void rank_scan_body(
    const int32_t* tile_count, int32_t* tile_offset, int64_t ntiles,
    int64_t* total) {
  __shared__ int64_t s_part[1024];
  const int64_t per = (ntiles + blockDim.x - 1) / blockDim.x;
  const int64_t lo = threadIdx.x * per;
  const int64_t hi = lo + per < ntiles ? lo + per : ntiles;
  int64_t sum = 0;
  for (int64_t i = lo; i < hi; ++i) sum += tile_count[i];
  s_part[threadIdx.x] = sum;
  __syncthreads();
  for (int o = 1; o < static_cast<int>(blockDim.x); o <<= 1) {
    const int64_t v = threadIdx.x >= static_cast<unsigned>(o) ? s_part[threadIdx.x - o] : 0;
    __syncthreads();
    s_part[threadIdx.x] += v;
    __syncthreads();
  }
  int64_t run = s_part[threadIdx.x] - sum;
  for (int64_t i = lo; i < hi; ++i) {
    tile_offset[i] = static_cast<int32_t>(run);
    run += tile_count[i];
  }
  if (threadIdx.x == blockDim.x - 1) *total = s_part[threadIdx.x];
}
__global__ __launch_bounds__(1024) void rank_scan_kernel(
    const int32_t* tile_count, int32_t* tile_offset, int64_t ntiles,
    int64_t* total) {
  rank_scan_body(tile_count, tile_offset, ntiles, total);
}

enum RankOp : int32_t {
  kOpPack = 0,     // from_dense_overlay
  kOpTrim = 1,     // trim_capacity
  kOpAppend = 2,   // append_banks_from
  kOpRelease = 3,  // release
  kOpPages = 4,    // paged map compression: entries are (bank, page) pairs
};

struct RankApply {
  int32_t op;
  int32_t* map_out;          // pack: state map; trim/append: new map
  const int32_t* free_rows;  // append: pop source
  int32_t* free_rows_out;    // release: push target
  const int32_t* counter;    // append/release: free_count before the op
  int64_t capacity;          // rows of the slab that receives rows
  int64_t map_row_offset;    // append: first admitted bank in new map
  int32_t* list_a;           // gather source rows
  int32_t* list_b;           // scatter destination rows (append)
  int64_t list_rows;         // entries list_a / list_b can hold
  int64_t src_capacity;      // trim/append: rows of the slab read from
  int32_t* map_clear;        // release: map whose listed rows become -1
  const int32_t* page_src;   // pages: the direct map the pages copy
  int32_t* pages_out;        // pages: page rows, list_rows of them
  int32_t page_shift;        // pages: log2 of the slots per page
};

// Rank each active entry in ranked order and apply the operation.
__device__ __forceinline__ void rank_apply_body(
    RankSource s, const int32_t* tile_offset, RankApply a) {
  __shared__ int s_scan[kTileThreads];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile + threadIdx.x * kPerThread;
  bool act[kPerThread];
  int c = 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t e = base + k;
    act[k] = e < s.entries && rank_active(s, e);
    c += act[k] ? 1 : 0;
  }
  s_scan[threadIdx.x] = c;
  __syncthreads();
  for (int o = 1; o < kTileThreads; o <<= 1) {
    const int v = threadIdx.x >= static_cast<unsigned>(o) ? s_scan[threadIdx.x - o] : 0;
    __syncthreads();
    s_scan[threadIdx.x] += v;
    __syncthreads();
  }
  int64_t rank = static_cast<int64_t>(tile_offset[blockIdx.x]) + s_scan[threadIdx.x] - c;
  const int64_t counter = a.counter ? *a.counter : 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t e = base + k;
    if (e >= s.entries) break;
    const int64_t slot = e % s.slots;
    const int64_t row = s.mask ? e / s.slots : rank_row(s, e);
    const int64_t at = row * s.slots + slot;
    // live source row of a map entry, -1 when outside the source slab
    int32_t src = -1;
    if (act[k] && !s.mask) {
      src = s.map[at];
      if (src >= a.src_capacity) src = -1;
    }
    switch (a.op) {
      case kOpPack:
        a.map_out[e] = act[k] ? static_cast<int32_t>(rank) : -1;
        if (act[k] && rank < a.list_rows) a.list_a[rank] = static_cast<int32_t>(e);
        break;
      case kOpTrim:
        if (act[k]) {
          if (rank < a.list_rows) a.list_a[rank] = src;
          a.map_out[e] = static_cast<int32_t>(rank);
        } else {
          a.map_out[e] = -1;
        }
        break;
      case kOpAppend: {
        int32_t dst = -1;
        if (act[k]) {
          const int64_t pos = counter - 1 - rank;
          if (pos >= 0 && pos < a.capacity) {
            dst = a.free_rows[pos];
            if (dst < 0 || dst >= a.capacity) dst = -1;
          }
          if (rank < a.list_rows) {
            a.list_a[rank] = src;
            a.list_b[rank] = dst;
          }
        }
        a.map_out[a.map_row_offset * s.slots + e] = dst;
        break;
      }
      case kOpPages: {
        // entry e is page e % (N / P) of bank e / (N / P): its slots are the
        // direct map's entries e * P .. e * P + P - 1
        a.map_out[e] = act[k] && rank < a.list_rows ? static_cast<int32_t>(rank) : -1;
        if (act[k] && rank < a.list_rows) {
          const int64_t P = int64_t{1} << a.page_shift;
          for (int64_t i = 0; i < P; ++i) a.pages_out[rank * P + i] = a.page_src[e * P + i];
        }
        break;
      }
      case kOpRelease:
        if (row < 0) break;
        if (act[k]) {
          const int64_t pos = counter + rank;
          if (pos >= 0 && pos < a.capacity) a.free_rows_out[pos] = s.map[at];
        }
        a.map_clear[at] = -1;
        break;
      default:
        break;
    }
    if (act[k]) ++rank;
  }
}
__global__ __launch_bounds__(kTileThreads) void rank_apply_kernel(
    RankSource s, const int32_t* tile_offset, RankApply a) {
  rank_apply_body(s, tile_offset, a);
}

// Paged maps: page g of bank b holds a mapped slot (flags over [B * N / P]).
__global__ void page_flags_kernel(const int32_t* map, int64_t pages, int32_t shift,
                                  uint8_t* flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t P = int64_t{1} << shift;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < pages;
       e += stride) {
    uint8_t any = 0;
    for (int64_t i = 0; i < P; ++i) any |= map[e * P + i] >= 0 ? 1 : 0;
    flags[e] = any;
  }
}

// The direct map of a paged one: entry (b, x) through the directory.
__global__ void page_expand_kernel(const int32_t* directory, const int32_t* pages,
                                   int64_t page_capacity, int64_t entries, int32_t shift,
                                   int32_t* map) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t mask = (int64_t{1} << shift) - 1;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < entries;
       e += stride) {
    const int32_t d = directory[e >> shift];
    // (a directory entry past the pages is corrupt: an entry past every slab)
    map[e] = d < 0 ? -1 : d >= page_capacity ? 0x7fffffff : pages[(int64_t{d} << shift) + (e & mask)];
  }
}

__global__ void store_count_kernel(const int64_t* total, int32_t* count) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *count = static_cast<int32_t>(*total);
}

// free_rows[i] = A + i for i < capacity - A; free_count = capacity - A.
__global__ void fill_free_tail_kernel(int32_t* free_rows, int64_t capacity,
                                      const int64_t* live, int32_t* free_count,
                                      int32_t* overflow) {
  const int64_t a = *live;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = t0; i < capacity - a; i += stride) {
    free_rows[i] = static_cast<int32_t>(a + i);
  }
  if (t0 == 0) {
    *free_count = static_cast<int32_t>(capacity - a);
    if (overflow) *overflow = 0;
  }
}

__global__ void copy_i32_kernel(int32_t* dst, const int32_t* src, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n; i += stride) {
    dst[i] = src[i];
  }
}

__global__ void gather_banks_kernel(const int32_t* map, const int64_t* tmpl,
                                    int64_t banks, int64_t slots, const int64_t* bank_list,
                                    int64_t nsel, int32_t* new_map,
                                    int64_t* new_tmpl, const int64_t* tmpl_b,
                                    int64_t nb) {
  // new rows 0..nsel-1 gather map rows bank_list[i]; when tmpl_b is set,
  // new_tmpl = [tmpl[list] ; tmpl_b[0..nb)].
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (map) {
    for (int64_t e = t0; e < nsel * slots; e += stride) {
      const int64_t i = e / slots;
      const int64_t src = bank_list ? bank_list[i] : i;
      new_map[e] = (src >= 0 && src < banks) ? map[src * slots + e % slots] : -1;
    }
  }
  for (int64_t i = t0; i < nsel; i += stride) {
    const int64_t src = bank_list ? bank_list[i] : i;
    new_tmpl[i] = (src >= 0 && src < banks) ? tmpl[src] : 0;
  }
  if (tmpl_b) {
    for (int64_t i = t0; i < nb; i += stride) new_tmpl[nsel + i] = tmpl_b[i];
  }
}

__global__ void zero_i64_kernel(int64_t* p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n; i += stride) {
    p[i] = 0;
  }
}

__global__ void zero_i32_kernel(int32_t* p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n; i += stride) {
    p[i] = 0;
  }
}

__global__ void mark_banks_kernel(const int64_t* bank_list, int64_t nsel,
                                  int64_t banks, int32_t* marks,
                                  int64_t* result) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < nsel; i += stride) {
    const int64_t b = bank_list[i];
    if (b < 0 || b >= banks) {
      atomicOr(reinterpret_cast<unsigned long long*>(result), 1ull);
    } else if (atomicAdd(&marks[b], 1) != 0) {
      atomicOr(reinterpret_cast<unsigned long long*>(result), 1ull);
    }
  }
}

__global__ void discarded_live_kernel(const int32_t* map, int64_t banks,
                                      int64_t slots, const int32_t* marks,
                                      int64_t* result) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int found = 0;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       e < banks * slots; e += stride) {
    if (marks[e / slots] == 0 && map[e] >= 0) found = 1;
  }
  if (found) atomicOr(reinterpret_cast<unsigned long long*>(result), 2ull);
}

__global__ void materialize_kernel(const float* m0, int64_t templates, const int64_t* tmpl,
                                   const float* values, const int32_t* map,
                                   int64_t banks, int64_t slots, int64_t width,
                                   int64_t capacity, float* dense) {
  const bool v4 = (width % 4) == 0;
  const int64_t per_row = v4 ? width / 4 : width;
  const int64_t total = banks * slots * per_row;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < total; i += stride) {
    const int64_t row = i / per_row;  // b * slots + n
    const int64_t c = i % per_row;
    const int64_t b = row / slots;
    const int64_t n = row % slots;
    const int32_t p = map[row];
    int64_t t = tmpl[b];
    if (t < 0 || t >= templates) t = 0;
    const float* src = (p >= 0 && p < capacity)
                           ? values + static_cast<int64_t>(p) * width
                           : m0 + (t * slots + n) * width;
    if (v4) {
      reinterpret_cast<float4*>(dense + row * width)[c] =
          reinterpret_cast<const float4*>(src)[c];
    } else {
      dense[row * width + c] = src[c];
    }
  }
}

// Partition check: counts[row] += 1 per live owner and += 1<<16 per free
// stack entry; stats as documented in cowsdm.h.
// Adds every lane's v into *target with one atomic per wave (a wave sum
// first): counters every thread of a grid feeds would otherwise take one
// same-address atomic per thread.  Every lane of the wave calls it.
__device__ __forceinline__ void wave_add_stat(int64_t* target, unsigned long long v) {
  const int64_t sum = wave_sum64(static_cast<int64_t>(v));
  if ((threadIdx.x & (kWave - 1)) == 0 && sum != 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(target), static_cast<unsigned long long>(sum));
  }
}

__device__ __forceinline__ void own_map_body(const int32_t* map, int64_t entries,
                               int64_t capacity, int32_t* counts,
                               int64_t* stats) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  unsigned long long live = 0, outside = 0;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       e < entries; e += stride) {
    const int32_t p = map[e];
    if (p < 0) continue;
    ++live;
    if (p >= capacity) { ++outside; continue; }
    atomicAdd(&counts[p], 1);
  }
  wave_add_stat(&stats[0], live);
  wave_add_stat(&stats[5], outside);
}
__global__ void own_map_kernel(const int32_t* map, int64_t entries,
                               int64_t capacity, int32_t* counts,
                               int64_t* stats) {
  own_map_body(map, entries, capacity, counts, stats);
}

__device__ __forceinline__ void own_free_body(const int32_t* free_rows, const int32_t* free_count,
                                int64_t capacity, int32_t* counts, int64_t* stats) {
  int64_t f = *free_count;
  if (f < 0) f = 0;
  if (f > capacity) f = capacity;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  unsigned long long outside = 0;
  for (int64_t i = t0; i < f; i += stride) {
    const int32_t p = free_rows[i];
    if (p < 0 || p >= capacity) { ++outside; continue; }
    atomicAdd(&counts[p], 1 << 16);
  }
  wave_add_stat(&stats[5], outside);
  if (t0 == 0) stats[1] = f;
}
__global__ void own_free_kernel(const int32_t* free_rows, const int32_t* free_count,
                                int64_t capacity, int32_t* counts, int64_t* stats) {
  own_free_body(free_rows, free_count, capacity, counts, stats);
}

__device__ __forceinline__ void own_eval_body(const int32_t* counts, int64_t capacity,
                                const int32_t* overflow, const int64_t* scratch,
                                int64_t* stats) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  unsigned long long dup_live = 0, dup_free = 0, not_once = 0;
  for (int64_t i = t0; i < capacity; i += stride) {
    const int32_t c = counts[i];
    const int32_t owners = c & 0xffff;
    const int32_t frees = c >> 16;
    if (owners > 1) ++dup_live;
    if (frees > 1) ++dup_free;
    if (owners + frees != 1) ++not_once;
  }
  wave_add_stat(&stats[2], dup_live);
  wave_add_stat(&stats[3], dup_free);
  wave_add_stat(&stats[4], not_once);
  if (t0 == 0) {
    stats[6] = *overflow;
    stats[7] = scratch ? scratch[COWSDM_SCRATCH_ERRORS] : 0;
  }
}
__global__ void own_eval_kernel(const int32_t* counts, int64_t capacity,
                                const int32_t* overflow, const int64_t* scratch,
                                int64_t* stats) {
  own_eval_body(counts, capacity, overflow, scratch, stats);
}

template <typename IDX>
__global__ void mark_written_kernel(uint8_t* mask, int64_t banks, int64_t slots,
                                    const void* idx, int64_t per_bank,
                                    int64_t* result) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int bad = 0;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       e < banks * per_bank; e += stride) {
    const int64_t x = load_index<IDX>(idx, e);
    if (x < 0 || x >= slots) { bad = 1; continue; }
    mask[(e / per_bank) * slots + x] = 1;
  }
  if (bad && result) atomicOr(reinterpret_cast<unsigned long long*>(result), 2ull);
}

// ------------------------------------------------------------ host helpers

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int grid_for(int64_t work, int threads, int cap = 8192) {
  int64_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

int32_t check_shape(const cowsdm_shape_t* s) {
  if (!s) return fail(COWSDM_EARG, "shape is null");
  if (s->banks < 0 || s->slots <= 0 || s->width <= 0 || s->writes <= 0 ||
      s->reads <= 0) {
    return fail(COWSDM_EARG, "invalid step shape (B=%lld N=%lld D=%lld W=%lld R=%lld)",
                (long long)s->banks, (long long)s->slots, (long long)s->width,
                (long long)s->writes, (long long)s->reads);
  }
  if (s->writes > 64 || s->reads > kMaxReadSlots * kWave) {
    return fail(COWSDM_ELIMIT, "step supports W <= 64 and R <= 256 (got W=%lld R=%lld)",
                (long long)s->writes, (long long)s->reads);
  }
  if (s->slots >= (1ll << 31) || s->banks >= (1ll << 31) ||
      s->banks * s->writes >= (1ll << 30)) {
    return fail(COWSDM_ELIMIT, "step sizes exceed 32-bit index ranges");
  }
  if (s->index_dtype != COWSDM_INDEX_INT32 && s->index_dtype != COWSDM_INDEX_INT64) {
    return fail(COWSDM_EARG, "index_dtype must be COWSDM_INDEX_INT32 or _INT64");
  }
  return 0;
}

int32_t check_layer(const cowsdm_layer_t& L, bool dense) {
  if (!L.values || !L.write_indices || !L.write_weights || !L.step_values ||
      !L.input_gate || !L.erase_gate || !L.forget_log_gate ||
      !L.read_indices || !L.read_weights || !L.output) {
    return fail(COWSDM_EARG, "null tensor pointer in step layer");
  }
  if (!dense) {
    const bool paged = L.map_page_shift != 0;
    if (!L.shared_initial_memory || !L.template_indices ||
        (paged ? (!L.map_directory || !L.map_pages || !L.map_page_count)
               : !L.logical_to_physical) ||
        !L.free_rows || !L.free_count || !L.overflow_flag || !L.scratch) {
      return fail(COWSDM_EARG, "null state pointer in packed step layer");
    }
    if (paged && (L.map_page_shift < 0 || L.map_page_shift > kMaxPageShift ||
                  L.map_page_capacity <= 0 || L.map_page_capacity >= (1ll << 31))) {
      return fail(COWSDM_EARG, "paged map: page shift in [1, %d] and a positive page capacity",
                  kMaxPageShift);
    }
    if (L.capacity_rows <= 0 || L.capacity_rows >= (1ll << 31)) {
      return fail(COWSDM_EARG, "capacity_rows must be in [1, 2^31)");
    }
  }
  return 0;
}

// Float lanes per row access that the row width, the layers' pointers and a
// trace's per-step strides allow: 4, 2 or 1.
int row_vec(const cowsdm_layer_t* layers, int32_t nlayers, const cowsdm_shape_t* shape,
            bool dense, const cowsdm_trace_t* trace) {
  const int64_t D = shape->width;
  int vec = (D % 4 == 0 && D >= 4 * kWave) ? 4 : (D % 2 == 0 ? 2 : 1);
  // float2/float4 lanes need every row pointer aligned to the vector size
  for (int32_t i = 0; i < nlayers; ++i) {
    const cowsdm_layer_t& L = layers[i];
    const uintptr_t bits = reinterpret_cast<uintptr_t>(L.values) |
                           reinterpret_cast<uintptr_t>(L.step_values) |
                           reinterpret_cast<uintptr_t>(L.output) |
                           (dense ? 0 : reinterpret_cast<uintptr_t>(L.shared_initial_memory));
    while (vec > 1 && (bits % (4u * vec)) != 0) vec /= 2;
  }
  if (trace) {
    // every step's value and output rows (the only vector accesses to trace
    // inputs) must keep the vector alignment of step 0
    for (int k : {2, 8}) {
      while (vec > 1 && (trace->stride_bytes[k] % (4 * vec)) != 0) vec /= 2;
    }
  }
  return vec;
}

// Float lanes of a persistent trace launch (a row of D <= 64 floats takes
// one per lane, <= 128 two, <= 256 four), or 0 when the shape, the alignment
// or the strides rule one out.
int persistent_vec(int vec, const cowsdm_layer_t* layers, const cowsdm_shape_t* shape,
                   const cowsdm_trace_t* trace, int32_t nlayers, bool dense) {
  const int64_t D = shape->width;
  int tv = D <= kWave ? 1 : (D <= 2 * kWave ? 2 : (D <= 4 * kWave ? 4 : 0));
  if (tv && D % tv != 0) tv = 0;
  if (tv > vec) tv = 0;  // alignment of some pointer forbids it
  for (int k = 0; k < 9; ++k) {
    // the persistent kernel advances inputs by 32-bit strides
    if (trace->stride_bytes[k] < 0 || trace->stride_bytes[k] >= (1ll << 32)) tv = 0;
  }
  if (shape->writes > kTraceMaxWrites || shape->reads > kTraceMaxReads || nlayers > kMaxLayers) tv = 0;
  // (persistent launches keep the direct map)
  for (int32_t i = 0; i < nlayers && !dense; ++i) {
    if (layers[i].map_page_shift != 0) tv = 0;
  }
  if (!dense && shape->banks > kTraceMaxBanks) tv = 0;
  return tv;
}

int32_t run_step(const cowsdm_layer_t* layers, int32_t nlayers,
                 const cowsdm_shape_t* shape, bool dense, hipStream_t stream,
                 const cowsdm_trace_t* trace = nullptr, int32_t steps = 1) {
  if (int32_t e = check_shape(shape)) return e;
  if (!layers || nlayers <= 0) return fail(COWSDM_EARG, "no layers given");
  for (int32_t i = 0; i < nlayers; ++i) {
    if (int32_t e = check_layer(layers[i], dense)) return e;
  }
  if (shape->banks == 0) return 0;
  if (!dense && (shape->templates <= 0 || shape->templates >= (1ll << 31))) {
    return fail(COWSDM_EARG, "templates must be positive");
  }
  int vec = row_vec(layers, nlayers, shape, dense, trace);
  if (!dense) {
    // paged slot maps run the small one-step kernel only
    for (int32_t i = 0; i < nlayers; ++i) {
      const int shift = layers[i].map_page_shift;
      if (shift == 0) continue;
      if (shape->slots % (int64_t{1} << shift) != 0) {
        return fail(COWSDM_EARG, "paged map: %lld slots are not whole pages of %d",
                    static_cast<long long>(shape->slots), 1 << shift);
      }
      if (shape->writes > 4 || shape->reads > 16 || shape->width > kWave * vec ||
          shape->banks > 256) {
        return fail(COWSDM_ELIMIT, "paged map: steps need W <= 4, R <= 16, one row pass "
                                   "(D <= %d here) and at most 256 banks", kWave * vec);
      }
    }
  }
  if (trace) {
    if (trace->step_index && !trace->ticket) return fail(COWSDM_EARG, "trace: null ticket");
    if (trace->report && !trace->step_index) {
      return fail(COWSDM_EARG, "trace: a report needs the device step counters");
    }
    if (trace->first_step < 0) return fail(COWSDM_EARG, "trace: negative first step");
    if (trace->steps_recorded <= 0) return fail(COWSDM_EARG, "trace: no recorded steps");
    if (!trace->step_index && trace->first_step + steps > trace->steps_recorded) {
      return fail(COWSDM_EARG, "trace: steps %lld..%lld past the %lld recorded",
                  static_cast<long long>(trace->first_step),
                  static_cast<long long>(trace->first_step + steps - 1),
                  static_cast<long long>(trace->steps_recorded));
    }
    if (nlayers > kMaxLayers) {
      return fail(COWSDM_ELIMIT, "trace launches take at most %d layers", kMaxLayers);
    }
    for (int k = 0; k < 9; ++k) {
      if (trace->stride_bytes[k] % 4 != 0) return fail(COWSDM_EARG, "trace: stride not float aligned");
    }
  }
  if (steps < 0) return fail(COWSDM_EARG, "steps must be non-negative");
  // persistent multi-step launches: up to scan_steps steps per launch
  const int trace_vec = trace ? persistent_vec(vec, layers, shape, trace, nlayers, dense) : 0;
  // packed persistent launches are planned: they need the control words and
  // scan blocks of enough steps
  const bool planned = !dense && trace && trace->control;
  int32_t launch_steps = kTraceMaxSteps;
  if (planned) {
    if (trace->scan_steps <= 0 || trace->scan_steps > kTraceMaxSteps || !trace->scan ||
        trace->control_stride < nlayers ||
        trace->scan_words < cowsdm_trace_scan_words(shape->banks, shape->writes, trace->scan_steps)) {
      return fail(COWSDM_EARG, "trace: control words need scan blocks of scan_steps steps");
    }
    if (!trace->ticket) return fail(COWSDM_EARG, "trace: planned launches need the ticket words");
    launch_steps = trace->scan_steps;
  }
  const bool persistent = trace && trace->persistent && steps > 0 && trace_vec &&
                          (dense || planned);
  if (planned && !persistent && steps > 0) {
    return fail(COWSDM_ELIMIT, "trace: planned launches need a persistent launch "
                               "(W <= 4, R <= 16, D <= 256 in even lanes, banks <= 256)");
  }
  StepParams P;
  P.trace_step = trace ? trace->step_index : nullptr;
  P.trace_ticket = trace ? trace->ticket : nullptr;
  P.trace_first = trace ? trace->first_step : 0;
  P.trace_known = trace && trace->step_index && trace->first_known ? trace->first_step : -1;
  P.trace_len = trace ? trace->steps_recorded : 0;
  P.trace_status = trace ? trace->status : nullptr;
  P.scan = planned ? trace->scan : nullptr;
  P.scan_words = planned ? trace->scan_words : 0;
  P.control = planned ? trace->control : nullptr;
  P.control_stride = planned ? trace->control_stride : 0;
  P.plan_steps = planned ? trace->scan_steps : 0;
  P.report = persistent ? trace->report : nullptr;
  P.count_table = 0;
  P.steps = steps;
  for (int k = 0; k < 9; ++k) P.trace_stride[k] = trace ? trace->stride_bytes[k] : 0;
  P.banks = static_cast<int32_t>(shape->banks);
  P.slots = static_cast<int32_t>(shape->slots);
  P.width = static_cast<int32_t>(shape->width);
  P.writes = static_cast<int32_t>(shape->writes);
  P.reads = static_cast<int32_t>(shape->reads);
  P.templates = static_cast<int32_t>(dense ? 1 : shape->templates);
  P.blocks_per_layer = static_cast<int32_t>((shape->banks + kBanksPerBlock - 1) / kBanksPerBlock);
  for (int32_t start = 0; start < nlayers; start += kMaxLayers) {
    const int32_t n = (nlayers - start) < kMaxLayers ? (nlayers - start) : kMaxLayers;
    P.nlayers = n;
    for (int32_t i = 0; i < kMaxLayers; ++i) P.layer[i] = layers[start + (i < n ? i : 0)];
    const int blocks = P.blocks_per_layer * n;
    const bool i64 = shape->index_dtype == COWSDM_INDEX_INT64;
    if (persistent) {
      // launches of at most launch_steps steps each, in order
      int32_t rc = 0;
      for (int32_t done = 0; done < steps; done += launch_steps) {
        P.steps = (steps - done) < launch_steps ? (steps - done) : launch_steps;
        P.trace_first = trace->first_step + done;  // ignored when step_index is set
        // (a later launch of the call starts where the last one left each
        // layer's counter, which a refused layer leaves behind)
        P.trace_known =
            done == 0 && trace->step_index && trace->first_known ? trace->first_step : -1;
        // count pass: an LDS hash of at least twice the launch's write routes
        int table = 64;
        while (table < 2 * P.steps * P.writes) table *= 2;
        P.count_table = table;
        if (planned && P.steps == 1) {
          // one step: the step kernel makes the step's proof itself (its
          // planned mode), with no plan of many steps to wait for
          if (i64) launch_step_w<int64_t, false>(P, blocks, vec, stream);
          else launch_step_w<int32_t, false>(P, blocks, vec, stream);
          rc = 0;
        } else if (dense) {
          rc = i64 ? launch_trace<int64_t, true>(P, trace_vec, stream)
                   : launch_trace<int32_t, true>(P, trace_vec, stream);
        } else {
          rc = i64 ? launch_trace<int64_t, false>(P, trace_vec, stream)
                   : launch_trace<int32_t, false>(P, trace_vec, stream);
        }
        if (rc == 1 && (done > 0 || planned)) {
          return fail(COWSDM_ELIMIT, "trace: not even one layer's workgroups fit on the device "
                                     "at once (after %d steps)", done);
        }
        if (rc == 1) break;
        if (rc != 0) return rc;
        if (int32_t e = launch_status(dense ? "dense trace" : "packed trace")) return e;
      }
      if (rc == 0) continue;
      P.steps = steps;
      P.trace_first = trace->first_step;
    }
    for (int32_t it = 0; it < steps; ++it) {
      if (trace && !trace->step_index) P.trace_first = trace->first_step + it;
      if (dense) {
        if (i64) launch_step_w<int64_t, true>(P, blocks, vec, stream);
        else launch_step_w<int32_t, true>(P, blocks, vec, stream);
      } else {
        if (i64) launch_step_w<int64_t, false>(P, blocks, vec, stream);
        else launch_step_w<int32_t, false>(P, blocks, vec, stream);
      }
      if (int32_t e = launch_status(dense ? "dense step" : "packed step")) return e;
    }
  }
  return 0;
}

int32_t rank_count(const RankSource& src, const Workspace& ws, hipStream_t stream) {
  const int64_t nt = num_tiles(src.entries);
  if (nt == 0) {
    hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(64), 0, stream, ws.total, int64_t{1});
    return launch_status("count (empty)");
  }
  hipLaunchKernelGGL(rank_count_kernel, dim3(static_cast<unsigned>(nt)), dim3(kTileThreads),
                     0, stream, src, ws.tile_count);
  if (int32_t e = launch_status("rank count")) return e;
  hipLaunchKernelGGL(rank_scan_kernel, dim3(1), dim3(1024), 0, stream, ws.tile_count,
                     ws.tile_offset, nt, ws.total);
  return launch_status("rank scan");
}

int32_t rank_apply(const RankSource& src, const Workspace& ws, const RankApply& a,
                   hipStream_t stream) {
  const int64_t nt = num_tiles(src.entries);
  if (nt == 0) return 0;
  hipLaunchKernelGGL(rank_apply_kernel, dim3(static_cast<unsigned>(nt)), dim3(kTileThreads),
                     0, stream, src, ws.tile_offset, a);
  return launch_status("rank apply");
}

// ---- plan blocks in the library's own device memory
// (cowsdm_packed_step_trace_static, for callers that cannot allocate)

// The array's name is a host-side stand-in: host code uses the per-device
// address hipGetSymbolAddress returns for it, never the name itself.
static __device__ __align__(256) int64_t scratch[COWSDM_STATIC_SCAN_WORDS];

namespace {
constexpr int kStaticDevices = 64;
std::mutex g_static_lock;
int64_t* g_static_scan[kStaticDevices] = {};  // per device: the array's address there
// per device: the layout (banks, W, steps per launch, layers) of the last
// call, whose plan blocks the array holds
struct StaticLayout {
  int64_t banks = -1, writes = -1, steps = -1, layers = -1;
  bool operator==(const StaticLayout& o) const {
    return banks == o.banks && writes == o.writes && steps == o.steps && layers == o.layers;
  }
};
StaticLayout g_static_layout[kStaticDevices];
bool g_static_captured[kStaticDevices] = {};   // per device: a call was recorded into a graph
}  // namespace

// The array's address on the current device, looked up once per device.
// When the call's layout differs from the last call's on this device, the
// words it will use are zeroed first (a fill kernel on `stream`): words left
// by another layout could otherwise pass for this one's epoch words.
//
// Zeroed words are a valid start for every layout (epoch 0, no word tagged
// with the next epoch), so a launch whose words were all zeroed first is
// always right.  A call recorded into a hipGraph (`capturing`) runs whenever
// the graph is replayed, out of sight of this host-side record, so it always
// clears its words before its launch; and once a graph has been recorded on
// a device, the record no longer tells what the array holds (a replay may
// have written another layout's words over part of it), so from then on
// every call there clears its words first.
int32_t static_scan(int64_t** out, const StaticLayout& layout, int64_t words,
                    hipStream_t stream, bool capturing) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return fail(static_cast<int32_t>(e), "static scan: %s", hipGetErrorString(e));
  if (device < 0 || device >= kStaticDevices) {
    return fail(COWSDM_ELIMIT, "static scan: device %d past the library's %d", device,
                kStaticDevices);
  }
  std::lock_guard<std::mutex> hold(g_static_lock);
  if (!g_static_scan[device]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      return fail(e != hipSuccess ? static_cast<int32_t>(e) : COWSDM_EARG,
                  "static scan: hipGetSymbolAddress: %s", hipGetErrorString(e));
    }
    g_static_scan[device] = static_cast<int64_t*>(ptr);
  }
  *out = g_static_scan[device];
  if (capturing) g_static_captured[device] = true;
  if (g_static_captured[device] || !(g_static_layout[device] == layout)) {
    hipLaunchKernelGGL(zero_i64_kernel, dim3(grid_for(words, 256)), dim3(256), 0, stream,
                       *out, words);
    if (int32_t e = launch_status("static scan clear")) return e;
    g_static_layout[device] = layout;
  }
  return 0;
}

// True when `stream` is recording a hipGraph (see static_scan).
int32_t stream_capturing(hipStream_t stream, bool* capturing) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(stream, &status);
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "static scan: hipStreamIsCapturing: %s",
                hipGetErrorString(e));
  }
  *capturing = status == hipStreamCaptureStatusActive;
  return 0;
}

// ---- host-mapped trace reports: the device address of each allocation
// (what trace->report holds) to its host address
namespace {
std::mutex g_report_lock;
std::unordered_map<const int64_t*, int64_t*> g_report_host;
}  // namespace

int64_t* report_host(const int64_t* device) {
  std::lock_guard<std::mutex> hold(g_report_lock);
  auto it = g_report_host.find(device);
  return it == g_report_host.end() ? nullptr : it->second;
}

// ---- the handoff of several layers at once (cowsdm_handoff_count/_pack):
// blockIdx.y is the layer, and each kernel runs the per-layer bodies above
struct HandoffBatch {
  cowsdm_handoff_layer_t layer[kMaxLayers];
  Workspace ws[kMaxLayers];
  int64_t entries[kMaxLayers];   // B * N
  int64_t ntiles[kMaxLayers];
};

__global__ __launch_bounds__(kTileThreads) void handoff_count_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  if (blockIdx.x >= b.ntiles[l]) return;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  const RankSource s{nullptr, nullptr, L.active_mask, L.slots, b.entries[l], L.banks};
  rank_count_body(s, b.ws[l].tile_count);
}

// the tile offsets and total of each layer, and its template check
__global__ __launch_bounds__(1024) void handoff_scan_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  rank_scan_body(b.ws[l].tile_count, b.ws[l].tile_offset, b.ntiles[l], b.ws[l].total);
  // (the thread that wrote the workspace's total)
  if (threadIdx.x == blockDim.x - 1) *L.total = *b.ws[l].total;
  check_templates_body(L.template_indices, L.banks, L.templates, L.checks + 8);
}

// scratch, overflow flag, invariant words and the invariant counts cleared
__global__ void handoff_prep_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = t0; i < L.scratch_words; i += stride) L.scratch[i] = 0;
  for (int64_t i = t0; i < L.capacity_rows; i += stride) b.ws[l].list_b[i] = 0;
  if (t0 < 8) L.checks[t0] = 0;
  if (t0 == 0) *L.overflow_flag = 0;
}

// map entries: active pairs in row-major order get rows 0..A-1
__global__ __launch_bounds__(kTileThreads) void handoff_apply_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  if (blockIdx.x >= b.ntiles[l]) return;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  const RankSource s{nullptr, nullptr, L.active_mask, L.slots, b.entries[l], L.banks};
  RankApply a{};
  a.op = kOpPack;
  a.map_out = L.logical_to_physical;
  a.list_a = b.ws[l].list_a;
  a.list_rows = L.capacity_rows;
  a.capacity = L.capacity_rows;
  rank_apply_body(s, b.ws[l].tile_offset, a);
}

// the rows (values[r] = dense[list_a[r]] for r < A) and the free stack
// (free_rows[i] = A + i for i < C - A, i after; free_count = C - A)
__global__ void handoff_rows_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  const Workspace& w = b.ws[l];
  copy_rows_body(L.values, nullptr, L.dense_memory, w.list_a, w.total, L.capacity_rows, L.width);
  const int64_t a = *w.total;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = t0; i < L.capacity_rows; i += stride) {
    L.free_rows[i] = static_cast<int32_t>(i < L.capacity_rows - a ? a + i : i);
  }
  if (t0 == 0) *L.free_count = static_cast<int32_t>(L.capacity_rows - a);
}

// the invariant counts: each row's owners and free-stack entries ...
__global__ void handoff_own_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  own_map_body(L.logical_to_physical, b.entries[l], L.capacity_rows, b.ws[l].list_b, L.checks);
  own_free_body(L.free_rows, L.free_count, L.capacity_rows, b.ws[l].list_b, L.checks);
}

// ... and the checks on them
__global__ void handoff_eval_kernel(HandoffBatch b) {
  const int l = blockIdx.y;
  const cowsdm_handoff_layer_t& L = b.layer[l];
  own_eval_body(b.ws[l].list_b, L.capacity_rows, L.overflow_flag, L.scratch, L.checks);
}

int32_t check_handoff_layer(const cowsdm_handoff_layer_t& L, bool pack) {
  if (!L.dense_memory || !L.active_mask || !L.workspace || !L.total || !L.checks ||
      (L.banks > 0 && !L.template_indices) || L.banks < 0 || L.slots <= 0 || L.width <= 0 ||
      L.templates <= 0) {
    return fail(COWSDM_EARG, "handoff: invalid layer arguments");
  }
  if (L.banks * L.slots >= (1ll << 31)) return fail(COWSDM_ELIMIT, "handoff: too many entries");
  if (pack && (!L.logical_to_physical || !L.values || !L.free_rows || !L.free_count ||
               !L.overflow_flag || L.capacity_rows <= 0 || L.capacity_rows >= (1ll << 31) ||
               L.scratch_words < 0 || (L.scratch_words > 0 && !L.scratch))) {
    return fail(COWSDM_EARG, "handoff: invalid state arguments");
  }
  return 0;
}

// Launches of the count (pack: false) or pack part over groups of up to
// kMaxLayers layers.
int32_t run_handoff(const cowsdm_handoff_layer_t* layers, int32_t n, bool pack,
                    hipStream_t s) {
  if (!layers || n < 0) return fail(COWSDM_EARG, "handoff: no layers");
  for (int32_t i = 0; i < n; ++i) {
    if (int32_t e = check_handoff_layer(layers[i], pack)) return e;
  }
  for (int32_t start = 0; start < n; start += kMaxLayers) {
    const int32_t g = n - start < kMaxLayers ? n - start : kMaxLayers;
    HandoffBatch b{};
    int64_t tiles = 1, vecs = 1, work = 1;
    for (int32_t i = 0; i < g; ++i) {
      const cowsdm_handoff_layer_t& L = layers[start + i];
      b.layer[i] = L;
      b.entries[i] = L.banks * L.slots;
      b.ntiles[i] = num_tiles(b.entries[i]);
      // (the count carves no row lists; the pack the capacity's two)
      b.ws[i] = carve(L.workspace, b.entries[i], pack ? L.capacity_rows : 0);
      tiles = b.ntiles[i] > tiles ? b.ntiles[i] : tiles;
      if (pack) {
        // the row copy's float4s (or floats); every other pass runs over
        // the entries, the rows or the scratch words
        const int64_t v = L.capacity_rows * (L.width % 4 == 0 ? L.width / 4 : L.width);
        vecs = v > vecs ? v : vecs;
        const int64_t w = std::max({b.entries[i], L.capacity_rows, L.scratch_words});
        work = w > work ? w : work;
      }
    }
    const dim3 tile_grid(static_cast<unsigned>(tiles), static_cast<unsigned>(g));
    const dim3 grid(static_cast<unsigned>(grid_for(work, 256)), static_cast<unsigned>(g));
    const dim3 row_grid(static_cast<unsigned>(grid_for(vecs > work ? vecs : work, 256)),
                        static_cast<unsigned>(g));
    if (!pack) {
      hipLaunchKernelGGL(handoff_count_kernel, tile_grid, dim3(kTileThreads), 0, s, b);
      if (int32_t e = launch_status("handoff count")) return e;
      hipLaunchKernelGGL(handoff_scan_kernel, dim3(1, static_cast<unsigned>(g)), dim3(1024), 0, s,
                         b);
      if (int32_t e = launch_status("handoff scan")) return e;
      continue;
    }
    hipLaunchKernelGGL(handoff_prep_kernel, grid, dim3(256), 0, s, b);
    if (int32_t e = launch_status("handoff prep")) return e;
    hipLaunchKernelGGL(handoff_apply_kernel, tile_grid, dim3(kTileThreads), 0, s, b);
    if (int32_t e = launch_status("handoff apply")) return e;
    hipLaunchKernelGGL(handoff_rows_kernel, row_grid, dim3(256), 0, s, b);
    if (int32_t e = launch_status("handoff rows")) return e;
    hipLaunchKernelGGL(handoff_own_kernel, grid, dim3(256), 0, s, b);
    if (int32_t e = launch_status("handoff own")) return e;
    hipLaunchKernelGGL(handoff_eval_kernel, grid, dim3(256), 0, s, b);
    if (int32_t e = launch_status("handoff eval")) return e;
  }
  return 0;
}

}  // namespace cowsdm_impl

using namespace cowsdm_impl;

// ================================================================ C ABI

extern "C" {

int32_t cowsdm_abi_version(void) { return COWSDM_ABI_VERSION; }

const char* cowsdm_last_error_string(void) { return last_error(); }

int64_t cowsdm_step_scratch_words(int64_t banks) {
  return banks < 0 ? -1 : COWSDM_SCRATCH_SLOTS + banks;
}

int32_t cowsdm_trace_persistent(const cowsdm_layer_t* layers, int32_t nlayers,
                                const cowsdm_shape_t* shape, const cowsdm_trace_t* trace,
                                int32_t dense) {
  if (!layers || !shape || !trace || nlayers <= 0) return 0;
  if (check_shape(shape) != 0) return 0;
  const int vec = row_vec(layers, nlayers, shape, dense != 0, trace);
  return persistent_vec(vec, layers, shape, trace, nlayers, dense != 0) > 0 ? 1 : 0;
}

int64_t cowsdm_trace_scan_words(int64_t banks, int64_t writes, int32_t steps) {
  if (banks < 0 || writes < 0 || steps < 0) return -1;
  // epoch and header, plan words [banks][steps], step totals, running
  // totals, the launch's pops (at most banks * W per step), its growth
  // segments (4 words each, at most one per step and the first) and a short
  // launch's packed count words (kPlanLocalWords rows of one word per bank of
  // a wave), int64 each
  return kPlanHead + kPlanHeadWords + banks * steps + steps + (steps + 1) + banks * steps * writes +
         4 * (static_cast<int64_t>(steps) + 1) + kPlanLocalWords * kWave;
}

int32_t cowsdm_host_report_alloc(int64_t words, int64_t** host, int64_t** device) {
  if (!host || !device || words <= 0) return fail(COWSDM_EARG, "host report: bad arguments");
  void* h = nullptr;
  hipError_t e = hipHostMalloc(&h, static_cast<size_t>(words) * sizeof(int64_t),
                               hipHostMallocMapped | hipHostMallocCoherent);
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "host report: hipHostMalloc: %s", hipGetErrorString(e));
  }
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess || !d) {
    (void)hipHostFree(h);
    return fail(e != hipSuccess ? static_cast<int32_t>(e) : COWSDM_EARG,
                "host report: hipHostGetDevicePointer: %s", hipGetErrorString(e));
  }
  memset(h, 0, static_cast<size_t>(words) * sizeof(int64_t));
  {
    std::lock_guard<std::mutex> hold(g_report_lock);
    g_report_host[static_cast<int64_t*>(d)] = static_cast<int64_t*>(h);
  }
  *host = static_cast<int64_t*>(h);
  *device = static_cast<int64_t*>(d);
  return 0;
}

int32_t cowsdm_host_report_free(int64_t* host) {
  if (!host) return 0;
  {
    std::lock_guard<std::mutex> hold(g_report_lock);
    for (auto it = g_report_host.begin(); it != g_report_host.end(); ++it) {
      if (it->second == host) {
        g_report_host.erase(it);
        break;
      }
    }
  }
  const hipError_t e = hipHostFree(host);
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "host report: hipHostFree: %s", hipGetErrorString(e));
  }
  return 0;
}

int32_t cowsdm_trace_timing(int32_t enable) {
  timing_on = enable != 0;
  timing_used = 0;
  return 0;
}

int32_t cowsdm_trace_timing_read(double* launch_ms, double* kernel_ms, int32_t* launches) {
  if (!launch_ms || !kernel_ms || !launches) {
    return fail(COWSDM_EARG, "trace timing: null argument");
  }
  double span = 0.0, kernel = 0.0;
  for (int i = 0; i < timing_used; ++i) {
    float a = 0.0f, b = 0.0f;
    hipError_t e = hipEventSynchronize(timing_stop[i]);
    if (e == hipSuccess) e = hipEventElapsedTime(&b, timing_start[i], timing_stop[i]);
    if (e == hipSuccess) {
      a = b;
      if (!timing_single[i]) e = hipEventElapsedTime(&a, timing_first[i], timing_stop[i]);
    }
    if (e != hipSuccess) {
      timing_used = 0;
      return fail(static_cast<int32_t>(e), "trace timing: launch %d: %s", i, hipGetErrorString(e));
    }
    span += a;
    kernel += b;
  }
  *launch_ms = span;
  *kernel_ms = kernel;
  *launches = timing_used;
  timing_used = 0;
  return 0;
}

int64_t cowsdm_workspace_bytes(int64_t entries, int64_t capacity_rows) {
  if (entries < 0 || capacity_rows < 0) return -1;
  const int64_t nt = num_tiles(entries);
  return 256 + 2 * align_up(nt * 4, 256) + 2 * align_up(capacity_rows * 4, 256);
}

int32_t cowsdm_packed_step(const cowsdm_layer_t* layer, const cowsdm_shape_t* shape,
                           void* stream) {
  return run_step(layer, 1, shape, false, as_stream(stream));
}

int32_t cowsdm_packed_step_layers(const cowsdm_layer_t* layers, int32_t nlayers,
                                  const cowsdm_shape_t* shape, void* stream) {
  return run_step(layers, nlayers, shape, false, as_stream(stream));
}

int32_t cowsdm_dense_step(const cowsdm_layer_t* layer, const cowsdm_shape_t* shape,
                          void* stream) {
  return run_step(layer, 1, shape, true, as_stream(stream));
}

int32_t cowsdm_dense_step_layers(const cowsdm_layer_t* layers, int32_t nlayers,
                                 const cowsdm_shape_t* shape, void* stream) {
  return run_step(layers, nlayers, shape, true, as_stream(stream));
}

int32_t cowsdm_packed_step_trace(const cowsdm_layer_t* layers, int32_t nlayers,
                                 const cowsdm_shape_t* shape, const cowsdm_trace_t* trace,
                                 int32_t steps, void* stream) {
  if (!trace) return fail(COWSDM_EARG, "trace is null");
  return run_step(layers, nlayers, shape, false, as_stream(stream), trace, steps);
}

int32_t cowsdm_packed_step_trace_static(const cowsdm_layer_t* layers, int32_t nlayers,
                                        const cowsdm_shape_t* shape,
                                        const cowsdm_trace_t* trace, int32_t steps,
                                        void* stream) {
  if (!trace || !shape) return fail(COWSDM_EARG, "trace or shape is null");
  if (trace->scan) {
    return fail(COWSDM_EARG, "static trace: scan must be null (the library supplies it)");
  }
  cowsdm_trace_t t = *trace;
  if (t.control) {
    const int64_t per_layer = cowsdm_trace_scan_words(shape->banks, shape->writes, t.scan_steps);
    if (per_layer < 0 || nlayers < 0 || t.scan_steps <= 0 ||
        per_layer * nlayers > COWSDM_STATIC_SCAN_WORDS) {
      return fail(COWSDM_ELIMIT,
                  "static trace: %d layers of %lld plan words pass the library's %lld "
                  "(fewer steps per launch or fewer layers per call)",
                  nlayers, static_cast<long long>(per_layer),
                  static_cast<long long>(COWSDM_STATIC_SCAN_WORDS));
    }
    StaticLayout layout;
    layout.banks = shape->banks;
    layout.writes = shape->writes;
    layout.steps = t.scan_steps;
    layout.layers = nlayers;
    bool capturing = false;
    if (int32_t e = stream_capturing(as_stream(stream), &capturing)) return e;
    if (int32_t e = static_scan(&t.scan, layout, per_layer * nlayers, as_stream(stream),
                                capturing)) {
      return e;
    }
    t.scan_words = per_layer;
  }
  return run_step(layers, nlayers, shape, false, as_stream(stream), &t, steps);
}

int32_t cowsdm_trace_run(const cowsdm_layer_t* layers, int32_t nlayers,
                         const cowsdm_shape_t* shape, const cowsdm_trace_t* trace,
                         int64_t steps, int32_t launch_steps, int32_t mode, void* stream) {
  if (!trace || !trace->report || !trace->step_index || !trace->status) {
    return fail(COWSDM_EARG, "trace run: needs the step counters, status words and a report");
  }
  if (mode < 0 || mode > 2 || launch_steps <= 0 || steps < 0 || nlayers <= 0 ||
      nlayers > kMaxLayers) {
    return fail(COWSDM_EARG, "trace run: bad mode, layer count or step counts");
  }
  int64_t* const host = report_host(trace->report);
  if (!host) return fail(COWSDM_EARG, "trace run: the report is not from cowsdm_host_report_alloc");
  // not written yet: no word of a report takes this value (counters,
  // status bits and control words are never below -1)
  constexpr int64_t kUnwritten = INT64_MIN + 1;
  const int64_t words = static_cast<int64_t>(nlayers) * COWSDM_REPORT_WORDS;
  for (int64_t k = 0; k < words; ++k) __atomic_store_n(&host[k], kUnwritten, __ATOMIC_RELAXED);
  hipStream_t s = as_stream(stream);
  // launches after the first read the counters the one before left
  cowsdm_trace_t later = *trace;
  later.first_known = 0;
  for (int64_t done = 0; done < steps; done += launch_steps) {
    const int32_t n = static_cast<int32_t>(steps - done < launch_steps ? steps - done : launch_steps);
    const cowsdm_trace_t* const t = done == 0 ? trace : &later;
    const int32_t rc =
        mode == 0 ? cowsdm_packed_step_trace(layers, nlayers, shape, t, n, stream)
        : mode == 1 ? cowsdm_packed_step_trace_static(layers, nlayers, shape, t, n, stream)
                    : cowsdm_dense_step_trace(layers, nlayers, shape, t, n, stream);
    if (rc != 0) return rc;
  }
  if (steps > 0 && steps <= launch_steps) {
    // One launch: its layers' last waves write every report word into host
    // memory before the kernel's remaining waves exit, so return as soon as
    // all words are in (each is one 8-byte store: a word that is not
    // kUnwritten is this launch's).  The caller's work after the return
    // overlaps the kernel's exit; later work on the stream still waits for
    // it.  A launch that writes no report (one-step kernels) or fails is
    // found done by the stream query and takes the path below.
    for (uint32_t spin = 0;; ++spin) {
      bool all = true;
      for (int64_t k = 0; k < words && all; ++k) {
        all = __atomic_load_n(&host[k], __ATOMIC_ACQUIRE) != kUnwritten;
      }
      if (all) return 0;
      if ((spin & 63u) == 63u && hipStreamQuery(s) != hipErrorNotReady) break;
    }
  }
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "trace run: %s", hipGetErrorString(e));
  }
  bool written = true;
  for (int64_t k = 0; k < words; ++k) written = written && host[k] != kUnwritten;
  if (written) return 0;
  // launches of one step each (no persistent kernel fits) write no report:
  // read the words from the device
  int64_t counters[kMaxLayers];
  int32_t status[kMaxLayers];
  e = hipMemcpy(counters, trace->step_index, sizeof(int64_t) * nlayers, hipMemcpyDeviceToHost);
  if (e == hipSuccess) {
    e = hipMemcpy(status, trace->status, sizeof(int32_t) * nlayers, hipMemcpyDeviceToHost);
  }
  if (e != hipSuccess) {
    return fail(static_cast<int32_t>(e), "trace run: report: %s", hipGetErrorString(e));
  }
  for (int32_t l = 0; l < nlayers; ++l) {
    int64_t* const col = host + l * COWSDM_REPORT_WORDS;
    col[0] = counters[l];
    col[1] = static_cast<uint32_t>(status[l]);
    for (int k = 0; k < COWSDM_CTRL_WORDS; ++k) {
      col[2 + k] = 0;
      if (trace->control && mode != 2) {
        e = hipMemcpy(&col[2 + k], trace->control + k * trace->control_stride + l,
                      sizeof(int64_t), hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
          return fail(static_cast<int32_t>(e), "trace run: report: %s", hipGetErrorString(e));
        }
      }
    }
  }
  return 0;
}

int32_t cowsdm_dense_step_trace(const cowsdm_layer_t* layers, int32_t nlayers,
                                const cowsdm_shape_t* shape, const cowsdm_trace_t* trace,
                                int32_t steps, void* stream) {
  if (!trace) return fail(COWSDM_EARG, "trace is null");
  return run_step(layers, nlayers, shape, true, as_stream(stream), trace, steps);
}

int32_t cowsdm_step_precheck(const cowsdm_layer_t* layer, const cowsdm_shape_t* shape,
                             int32_t dense, int32_t check_unique,
                             int32_t check_capacity, int64_t* result, void* stream) {
  if (int32_t e = check_shape(shape)) return e;
  if (!layer || !result) return fail(COWSDM_EARG, "precheck: null argument");
  if (!layer->write_indices || !layer->read_indices) {
    return fail(COWSDM_EARG, "precheck: null route indices");
  }
  if (check_capacity && !dense &&
      ((layer->map_page_shift == 0 ? !layer->logical_to_physical : !layer->map_directory) ||
       !layer->free_count)) {
    return fail(COWSDM_EARG, "precheck: capacity check needs map and free_count");
  }
  const hipStream_t s = as_stream(stream);
  const int32_t B = static_cast<int32_t>(shape->banks);
  const int32_t N = static_cast<int32_t>(shape->slots);
  const int32_t W = static_cast<int32_t>(shape->writes);
  const int32_t R = static_cast<int32_t>(shape->reads);
  if (shape->index_dtype == COWSDM_INDEX_INT64) {
    hipLaunchKernelGGL(precheck_kernel<int64_t>, dim3(1), dim3(1024), 0, s, *layer, B, N,
                       W, R, dense, check_unique, check_capacity, result);
  } else {
    hipLaunchKernelGGL(precheck_kernel<int32_t>, dim3(1), dim3(1024), 0, s, *layer, B, N,
                       W, R, dense, check_unique, check_capacity, result);
  }
  return launch_status("step precheck");
}

int32_t cowsdm_init_state(int32_t* map, int64_t banks, int64_t slots, int32_t* free_rows,
                          int64_t capacity_rows, int32_t* free_count, int32_t* overflow_flag,
                          int64_t* scratch, int64_t scratch_words,
                          const int64_t* template_indices, int64_t templates,
                          int64_t* result, void* stream) {
  if (banks < 0 || slots <= 0 || capacity_rows <= 0 || scratch_words < 0) {
    return fail(COWSDM_EARG, "init_state: invalid sizes");
  }
  if ((banks > 0 && !map) || !free_rows || !free_count || !overflow_flag ||
      (scratch_words > 0 && !scratch)) {
    return fail(COWSDM_EARG, "init_state: null pointer");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t work = banks * slots > capacity_rows ? banks * slots : capacity_rows;
  hipLaunchKernelGGL(init_state_kernel, dim3(grid_for(work, 256)), dim3(256), 0, s, map,
                     banks * slots, free_rows, capacity_rows, free_count, overflow_flag,
                     scratch, scratch_words);
  if (int32_t e = launch_status("init_state")) return e;
  if (result) {
    if (banks > 0 && !template_indices) return fail(COWSDM_EARG, "init_state: null templates");
    hipLaunchKernelGGL(check_templates_kernel, dim3(1), dim3(256), 0, s, template_indices,
                       banks, templates, result);
    return launch_status("check templates");
  }
  return 0;
}

int32_t cowsdm_grow(const float* old_values, int64_t old_capacity, float* new_values,
                    int64_t new_capacity, int64_t width, const int32_t* old_free_rows,
                    int32_t* new_free_rows, int32_t* free_count, int32_t* overflow_flag,
                    void* stream) {
  if (!old_values || !new_values || !old_free_rows || !new_free_rows || !free_count ||
      !overflow_flag || old_capacity <= 0 || new_capacity < old_capacity || width <= 0) {
    return fail(COWSDM_EARG, "grow: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  if (new_values != old_values) {
    // (a slab with headroom grows in place: its rows stay where they are)
    const int64_t vecs = old_capacity * (width % 4 == 0 ? width / 4 : width);
    hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, s,
                       new_values, static_cast<const int32_t*>(nullptr), old_values,
                       static_cast<const int32_t*>(nullptr), static_cast<const int64_t*>(nullptr),
                       old_capacity, width);
    if (int32_t e = launch_status("grow copy")) return e;
  }
  hipLaunchKernelGGL(grow_free_kernel, dim3(grid_for(new_capacity, 256)), dim3(256), 0, s,
                     old_free_rows, new_free_rows, free_count, old_capacity, new_capacity);
  if (int32_t e = launch_status("grow free")) return e;
  hipLaunchKernelGGL(add_counter_kernel, dim3(1), dim3(64), 0, s, free_count,
                     new_capacity - old_capacity, static_cast<const int64_t*>(nullptr), 1,
                     overflow_flag);
  return launch_status("grow counter");
}

int32_t cowsdm_count_active(const int32_t* map, int64_t banks, int64_t slots,
                            const int64_t* bank_list, int64_t nsel,
                            const uint8_t* active_mask, void* workspace, int64_t* total,
                            void* stream) {
  if (!workspace || !total || slots <= 0 || nsel < 0 || banks < 0 ||
      (!map && !active_mask)) {
    return fail(COWSDM_EARG, "count_active: invalid arguments");
  }
  const int64_t entries = nsel * slots;
  if (entries >= (1ll << 31)) return fail(COWSDM_ELIMIT, "count_active: too many entries");
  const hipStream_t s = as_stream(stream);
  Workspace ws = carve(workspace, entries, 0);
  RankSource src{map, bank_list, active_mask, slots, entries, banks};
  if (int32_t e = rank_count(src, ws, s)) return e;
  hipLaunchKernelGGL(copy_i64_kernel, dim3(1), dim3(64), 0, s, total,
                     static_cast<const int64_t*>(ws.total), int64_t{1});
  return launch_status("count copy");
}

int32_t cowsdm_pack_overlay(const float* dense_memory, const uint8_t* active_mask,
                            int64_t banks, int64_t slots, int64_t width, int32_t* map,
                            float* values, int32_t* free_rows, int64_t capacity_rows,
                            int32_t* free_count, void* workspace, void* stream) {
  if (!dense_memory || !active_mask || !map || !values || !free_rows || !free_count ||
      !workspace || banks < 0 || slots <= 0 || width <= 0 || capacity_rows <= 0) {
    return fail(COWSDM_EARG, "pack_overlay: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t entries = banks * slots;
  Workspace ws = carve(workspace, entries, capacity_rows);
  RankSource src{nullptr, nullptr, active_mask, slots, entries, banks};
  RankApply a{};
  a.op = kOpPack;
  a.map_out = map;
  a.list_a = ws.list_a;
  a.list_rows = capacity_rows;
  a.capacity = capacity_rows;
  if (int32_t e = rank_apply(src, ws, a, s)) return e;
  const int64_t vecs = capacity_rows * (width % 4 == 0 ? width / 4 : width);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, s, values,
                     static_cast<const int32_t*>(nullptr), dense_memory, ws.list_a,
                     static_cast<const int64_t*>(ws.total), capacity_rows, width);
  if (int32_t e = launch_status("pack copy")) return e;
  hipLaunchKernelGGL(fill_free_tail_kernel, dim3(grid_for(capacity_rows, 256)), dim3(256), 0,
                     s, free_rows, capacity_rows, static_cast<const int64_t*>(ws.total),
                     free_count, static_cast<int32_t*>(nullptr));
  return launch_status("pack free");
}

int32_t cowsdm_trim_repack(const int32_t* map, const float* values, int64_t capacity_rows,
                           int64_t banks, int64_t slots, int64_t width, int32_t* new_map,
                           float* new_values,
                           int32_t* new_free_rows, int64_t new_capacity, int32_t* free_count,
                           int32_t* overflow_flag, void* workspace, void* stream) {
  if (!map || !values || !new_map || !new_values || !new_free_rows || !free_count ||
      !overflow_flag || !workspace || banks < 0 || slots <= 0 || width <= 0 ||
      new_capacity <= 0 || capacity_rows <= 0) {
    return fail(COWSDM_EARG, "trim_repack: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t entries = banks * slots;
  Workspace ws = carve(workspace, entries, new_capacity);
  RankSource src{map, nullptr, nullptr, slots, entries, banks};
  RankApply a{};
  a.op = kOpTrim;
  a.map_out = new_map;
  a.list_a = ws.list_a;
  a.list_rows = new_capacity;
  a.capacity = new_capacity;
  a.src_capacity = capacity_rows;
  if (int32_t e = rank_apply(src, ws, a, s)) return e;
  const int64_t vecs = new_capacity * (width % 4 == 0 ? width / 4 : width);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, s,
                     new_values, static_cast<const int32_t*>(nullptr), values, ws.list_a,
                     static_cast<const int64_t*>(ws.total), new_capacity, width);
  if (int32_t e = launch_status("trim copy")) return e;
  hipLaunchKernelGGL(fill_free_tail_kernel, dim3(grid_for(new_capacity, 256)), dim3(256), 0,
                     s, new_free_rows, new_capacity, static_cast<const int64_t*>(ws.total),
                     free_count, overflow_flag);
  return launch_status("trim free");
}

int32_t cowsdm_append_banks(const int32_t* map, const int64_t* tmpl, int64_t banks,
                            float* values, int64_t capacity_rows, const int32_t* free_rows,
                            int32_t* free_count, const int32_t* other_map,
                            const int64_t* other_tmpl, const float* other_values,
                            int64_t other_banks, int64_t other_capacity_rows, int64_t slots,
                            int64_t width, int32_t* new_map, int64_t* new_tmpl,
                            void* workspace, void* stream) {
  if ((banks > 0 && (!map || !tmpl)) || (other_banks > 0 && (!other_map || !other_tmpl)) ||
      !other_values || !values || !free_rows || !free_count || !new_map || !new_tmpl ||
      !workspace || banks < 0 || other_banks < 0 || slots <= 0 || width <= 0 ||
      capacity_rows <= 0 || other_capacity_rows < 0) {
    return fail(COWSDM_EARG, "append_banks: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t entries = other_banks * slots;
  Workspace ws = carve(workspace, entries, other_capacity_rows);
  if (banks > 0) {
    hipLaunchKernelGGL(copy_i32_kernel, dim3(grid_for(banks * slots, 256)), dim3(256), 0, s,
                       new_map, map, banks * slots);
    if (int32_t e = launch_status("append copy map")) return e;
  }
  hipLaunchKernelGGL(gather_banks_kernel, dim3(grid_for(banks + other_banks, 256)),
                     dim3(256), 0, s, static_cast<const int32_t*>(nullptr), tmpl, banks, slots,
                     static_cast<const int64_t*>(nullptr), banks,
                     static_cast<int32_t*>(nullptr), new_tmpl, other_tmpl, other_banks);
  if (int32_t e = launch_status("append templates")) return e;
  if (entries == 0) return 0;
  RankSource src{other_map, nullptr, nullptr, slots, entries, other_banks};
  RankApply a{};
  a.op = kOpAppend;
  a.map_out = new_map;
  a.free_rows = free_rows;
  a.counter = free_count;
  a.capacity = capacity_rows;
  a.map_row_offset = banks;
  a.list_a = ws.list_a;
  a.list_b = ws.list_b;
  a.list_rows = other_capacity_rows;
  a.src_capacity = other_capacity_rows;
  if (int32_t e = rank_apply(src, ws, a, s)) return e;
  const int64_t vecs = other_capacity_rows * (width % 4 == 0 ? width / 4 : width);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, s, values,
                     ws.list_b, other_values, ws.list_a, static_cast<const int64_t*>(ws.total),
                     other_capacity_rows, width);
  if (int32_t e = launch_status("append copy")) return e;
  hipLaunchKernelGGL(add_counter_kernel, dim3(1), dim3(64), 0, s, free_count, int64_t{0},
                     static_cast<const int64_t*>(ws.total), -1, static_cast<int32_t*>(nullptr));
  return launch_status("append counter");
}

int32_t cowsdm_check_banks(const int32_t* map, int64_t banks, int64_t slots,
                           const int64_t* bank_list, int64_t nsel, int32_t discarded_active,
                           void* workspace, int64_t* result, void* stream) {
  if (!workspace || !result || banks < 0 || slots <= 0 || nsel < 0 ||
      (nsel > 0 && !bank_list) || (discarded_active && banks > 0 && !map)) {
    return fail(COWSDM_EARG, "check_banks: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  Workspace ws = carve(workspace, banks * slots, banks);
  hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(64), 0, s, result, int64_t{1});
  if (int32_t e = launch_status("check_banks zero")) return e;
  if (banks > 0) {
    hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_for(banks, 256)), dim3(256), 0, s,
                       ws.list_a, banks);
    if (int32_t e = launch_status("check_banks marks")) return e;
  }
  if (nsel > 0) {
    hipLaunchKernelGGL(mark_banks_kernel, dim3(grid_for(nsel, 256)), dim3(256), 0, s,
                       bank_list, nsel, banks, ws.list_a, result);
    if (int32_t e = launch_status("check_banks mark")) return e;
  }
  if (discarded_active && banks > 0) {
    hipLaunchKernelGGL(discarded_live_kernel, dim3(grid_for(banks * slots, 256)), dim3(256),
                       0, s, map, banks, slots, static_cast<const int32_t*>(ws.list_a),
                       result);
    return launch_status("check_banks discarded");
  }
  return 0;
}

int32_t cowsdm_release(int32_t* map, int64_t banks, int64_t slots, const int64_t* bank_list,
                       int64_t nsel, int32_t* free_rows, int64_t capacity_rows,
                       int32_t* free_count, void* workspace, int64_t* released,
                       void* stream) {
  if (!map || !bank_list || !free_rows || !free_count || !workspace || !released ||
      slots <= 0 || nsel < 0 || banks < 0 || capacity_rows <= 0) {
    return fail(COWSDM_EARG, "release: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t entries = nsel * slots;
  Workspace ws = carve(workspace, entries, 0);
  RankSource src{map, bank_list, nullptr, slots, entries, banks};
  RankApply a{};
  a.op = kOpRelease;
  a.free_rows_out = free_rows;
  a.counter = free_count;
  a.capacity = capacity_rows;
  a.map_clear = map;
  if (int32_t e = rank_apply(src, ws, a, s)) return e;
  hipLaunchKernelGGL(add_counter_kernel, dim3(1), dim3(64), 0, s, free_count, int64_t{0},
                     static_cast<const int64_t*>(ws.total), 1, static_cast<int32_t*>(nullptr));
  if (int32_t e = launch_status("release counter")) return e;
  hipLaunchKernelGGL(copy_i64_kernel, dim3(1), dim3(64), 0, s, released,
                     static_cast<const int64_t*>(ws.total), int64_t{1});
  return launch_status("release count");
}

int32_t cowsdm_retain_banks(const int32_t* map, const int64_t* tmpl, int64_t banks,
                            int64_t slots, const int64_t* bank_list, int64_t nsel,
                            int32_t* new_map, int64_t* new_tmpl, void* stream) {
  if (slots <= 0 || nsel < 0 || banks < 0 ||
      (nsel > 0 && (!map || !tmpl || !bank_list || !new_map || !new_tmpl))) {
    return fail(COWSDM_EARG, "retain_banks: invalid arguments");
  }
  if (nsel == 0) return 0;
  const hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(gather_banks_kernel, dim3(grid_for(nsel * slots, 256)), dim3(256), 0, s,
                     map, tmpl, banks, slots, bank_list, nsel, new_map, new_tmpl,
                     static_cast<const int64_t*>(nullptr), int64_t{0});
  return launch_status("retain_banks");
}

int32_t cowsdm_paged_count(const int32_t* map, int64_t banks, int64_t slots, int32_t page_shift,
                           uint8_t* flags, void* workspace, int64_t* total, void* stream) {
  if (!map || !flags || !workspace || !total || banks < 0 || slots <= 0 ||
      page_shift < 1 || page_shift > kMaxPageShift || slots % (int64_t{1} << page_shift) != 0) {
    return fail(COWSDM_EARG, "paged_count: invalid arguments (page shift in [1, %d], whole pages)",
                kMaxPageShift);
  }
  const int64_t pages = banks * (slots >> page_shift);
  if (pages >= (1ll << 31)) return fail(COWSDM_ELIMIT, "paged_count: too many pages");
  const hipStream_t s = as_stream(stream);
  if (pages > 0) {
    hipLaunchKernelGGL(page_flags_kernel, dim3(grid_for(pages, 256)), dim3(256), 0, s, map,
                       pages, page_shift, flags);
    if (int32_t e = launch_status("page flags")) return e;
  }
  return cowsdm_count_active(nullptr, banks, slots >> page_shift, nullptr, banks, flags,
                             workspace, total, stream);
}

int32_t cowsdm_paged_compress(const int32_t* map, int64_t banks, int64_t slots,
                              int32_t page_shift, const uint8_t* flags, void* workspace,
                              int32_t* directory, int32_t* pages, int64_t page_capacity,
                              int32_t* page_count, void* stream) {
  if (!map || !flags || !workspace || !directory || !page_count || banks < 0 || slots <= 0 ||
      page_shift < 1 || page_shift > kMaxPageShift || slots % (int64_t{1} << page_shift) != 0 ||
      page_capacity < 0 || (page_capacity > 0 && !pages)) {
    return fail(COWSDM_EARG, "paged_compress: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  const int64_t per_bank = slots >> page_shift;
  const int64_t entries = banks * per_bank;
  Workspace ws = carve(workspace, entries, 0);
  RankSource src{nullptr, nullptr, flags, per_bank, entries, banks};
  RankApply a{};
  a.op = kOpPages;
  a.map_out = directory;
  a.list_rows = page_capacity;
  a.page_src = map;
  a.pages_out = pages;
  a.page_shift = page_shift;
  if (int32_t e = rank_apply(src, ws, a, s)) return e;
  hipLaunchKernelGGL(store_count_kernel, dim3(1), dim3(64), 0, s,
                     static_cast<const int64_t*>(ws.total), page_count);
  return launch_status("paged compress");
}

int32_t cowsdm_paged_expand(const int32_t* directory, const int32_t* pages,
                            int64_t page_capacity, int64_t banks, int64_t slots,
                            int32_t page_shift, int32_t* map, void* stream) {
  if (!directory || !map || banks < 0 || slots <= 0 || page_shift < 1 ||
      page_shift > kMaxPageShift || slots % (int64_t{1} << page_shift) != 0 ||
      page_capacity < 0 || (page_capacity > 0 && !pages)) {
    return fail(COWSDM_EARG, "paged_expand: invalid arguments");
  }
  const int64_t entries = banks * slots;
  if (entries == 0) return 0;
  hipLaunchKernelGGL(page_expand_kernel, dim3(grid_for(entries, 256)), dim3(256), 0,
                     as_stream(stream), directory, pages, page_capacity, entries, page_shift, map);
  return launch_status("paged expand");
}

int32_t cowsdm_materialize_dense(const float* m0, int64_t templates, const int64_t* tmpl,
                                 const float* values, const int32_t* map, int64_t banks,
                                 int64_t slots, int64_t width, int64_t capacity_rows,
                                 float* dense, void* stream) {
  if (banks < 0 || slots <= 0 || width <= 0 || templates <= 0 ||
      (banks > 0 && (!m0 || !tmpl || !values || !map || !dense))) {
    return fail(COWSDM_EARG, "materialize_dense: invalid arguments");
  }
  if (banks == 0) return 0;
  const hipStream_t s = as_stream(stream);
  const int64_t vecs = banks * slots * (width % 4 == 0 ? width / 4 : width);
  hipLaunchKernelGGL(materialize_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, s, m0,
                     templates, tmpl, values, map, banks, slots, width, capacity_rows, dense);
  return launch_status("materialize_dense");
}

int32_t cowsdm_check_invariants(const int32_t* map, int64_t banks, int64_t slots,
                                const int32_t* free_rows, const int32_t* free_count,
                                const int32_t* overflow_flag, const int64_t* scratch,
                                int64_t capacity_rows, void* workspace, int64_t* stats,
                                void* stream) {
  if (!free_rows || !free_count || !overflow_flag || !workspace || !stats || banks < 0 ||
      slots <= 0 || capacity_rows <= 0 || (banks > 0 && !map)) {
    return fail(COWSDM_EARG, "check_invariants: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  Workspace ws = carve(workspace, banks * slots, capacity_rows);
  hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(64), 0, s, stats, int64_t{8});
  if (int32_t e = launch_status("invariants zero stats")) return e;
  hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_for(capacity_rows, 256)), dim3(256), 0, s,
                     ws.list_a, capacity_rows);
  if (int32_t e = launch_status("invariants zero counts")) return e;
  if (banks > 0) {
    hipLaunchKernelGGL(own_map_kernel, dim3(grid_for(banks * slots, 256)), dim3(256), 0, s,
                       map, banks * slots, capacity_rows, ws.list_a, stats);
    if (int32_t e = launch_status("invariants map")) return e;
  }
  hipLaunchKernelGGL(own_free_kernel, dim3(grid_for(capacity_rows, 256)), dim3(256), 0, s,
                     free_rows, free_count, capacity_rows, ws.list_a, stats);
  if (int32_t e = launch_status("invariants free")) return e;
  hipLaunchKernelGGL(own_eval_kernel, dim3(grid_for(capacity_rows, 256)), dim3(256), 0, s,
                     static_cast<const int32_t*>(ws.list_a), capacity_rows, overflow_flag,
                     scratch, stats);
  return launch_status("invariants eval");
}

int32_t cowsdm_handoff_count(const cowsdm_handoff_layer_t* layers, int32_t nlayers,
                             void* stream) {
  return run_handoff(layers, nlayers, false, as_stream(stream));
}

int32_t cowsdm_handoff_pack(const cowsdm_handoff_layer_t* layers, int32_t nlayers,
                            void* stream) {
  return run_handoff(layers, nlayers, true, as_stream(stream));
}

int32_t cowsdm_mark_written(uint8_t* active_mask, int64_t banks, int64_t slots,
                            const void* indices, int64_t per_bank, int32_t index_dtype,
                            int64_t* result, void* stream) {
  if (!active_mask || banks < 0 || slots <= 0 || per_bank < 0 ||
      (banks * per_bank > 0 && !indices) ||
      (index_dtype != COWSDM_INDEX_INT32 && index_dtype != COWSDM_INDEX_INT64)) {
    return fail(COWSDM_EARG, "mark_written: invalid arguments");
  }
  const hipStream_t s = as_stream(stream);
  if (result) {
    hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(64), 0, s, result, int64_t{1});
    if (int32_t e = launch_status("mark_written zero")) return e;
  }
  if (banks * per_bank == 0) return 0;
  if (index_dtype == COWSDM_INDEX_INT64) {
    hipLaunchKernelGGL(mark_written_kernel<int64_t>, dim3(grid_for(banks * per_bank, 256)),
                       dim3(256), 0, s, active_mask, banks, slots, indices, per_bank, result);
  } else {
    hipLaunchKernelGGL(mark_written_kernel<int32_t>, dim3(grid_for(banks * per_bank, 256)),
                       dim3(256), 0, s, active_mask, banks, slots, indices, per_bank, result);
  }
  return launch_status("mark_written");
}

}  // extern "C"
