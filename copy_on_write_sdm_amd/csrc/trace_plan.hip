// Count part of a packed decode-trace launch's plan for slot maps too large
// for LDS (N > kTraceMapSlots): which write lanes of every (step, bank)
// first-touch a slot, and each bank's first step with an invalid route
// (out-of-range slot, a slot written twice in one step, a write slot's map
// entry outside the slab, an invalid template), after which the bank takes no
// step.  It runs just before the persistent kernel, which makes the rest of
// the plan (trace_plan.h) and counts for itself when the map fits in LDS.
// A slot is first-touched by the launch's first step that writes it, unless
// it was mapped already; the first writing steps of a bank live in an LDS
// hash table keyed by slot.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "common.h"

namespace cowsdm_impl {

namespace {

constexpr int kCountWaves = 4;
constexpr int kCountThreads = kWave * kCountWaves;
constexpr int kCountChunks = kTraceMaxSteps / kCountThreads;   // 64-step chunks per wave
constexpr int kIntMax = 0x7fffffff;

// Fibonacci hash of a slot into a table of 2^bits entries.
__device__ __forceinline__ uint32_t hash_slot(int x, int bits) {
  return (static_cast<uint32_t>(x) * 0x9E3779B1u) >> (32 - bits);
}

// ------------------------------------------------------------ count pass

// One workgroup per (layer, bank); lane = step: each lane of wave w handles
// steps 64 * (w + 4k) + lane.  The first writing steps live in an LDS hash
// table of count_table entries keyed by slot (at most half full).  Only write
// slots' map entries are checked (a read slot's entry outside the slab stops
// the bank in the persistent kernel alone).  Writes the bank's count words,
// tagged with the launch's epoch.
template <typename IDX>
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
  int* const keys = lds_dyn;        // slot of each hash entry
  int* const fw = lds_dyn + TS;      // its first writing step
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
  for (int k = static_cast<int>(threadIdx.x); k < TS; k += kCountThreads) {
    keys[k] = -1;
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
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      const int x = slot[k][j];
      if (x < 0) continue;
      const int m = map_bank[x];
      if (m >= C) e |= COWSDM_ERR_CORRUPT;
      if (m >= 0) mapped[k] |= 1u << j;
    }
    err[k] = e;
    if (e != 0) atomicMin(&s_stop, t);
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      const int x = slot[k][j];
      if (x < 0) continue;
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
  __syncthreads();
  const int stop = s_stop;
#pragma unroll
  for (int k = 0; k < kCountChunks; ++k) {
    const int t = (wave + k * kCountWaves) * kWave + lane;
    if (t == stop) atomicOr(&s_bits, err[k]);
  }

  // ---- phase 2: each step's first-touch write lanes, as tagged count words
  const PlanBlock pb = plan_block(P, layer_id);
  const uint32_t epoch = launch_epoch(pb);
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
        if (fw[find(x)] == t) mask |= 1u << j;
      }
    }
    atomic_store_u64(pb.word(bank, t),
                     tagged(epoch, mask | (t >= stop ? kCountStop : 0u)));
  }
  __syncthreads();
  if (threadIdx.x == 0 && s_bits != 0) {
    __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(s_bits),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

// Count part of one packed persistent launch with a slot map in HBM (all
// layers of P); with `start` given, the kernel records it when it starts.
template <typename IDX>
int32_t launch_trace_count(const StepParams& P, hipStream_t stream, hipEvent_t start) {
  const size_t lds = 2 * sizeof(int) * static_cast<size_t>(P.count_table);
  const dim3 grid(static_cast<unsigned>(P.nlayers * P.banks));
  StepParams Q = P;
  void* args[] = {&Q};
  (void)hipExtLaunchKernel(reinterpret_cast<const void*>(&trace_count_kernel<IDX>), grid,
                           dim3(kCountThreads), args, lds, stream, start, nullptr, 0);
  return launch_status("trace count");
}

template int32_t launch_trace_count<int32_t>(const StepParams&, hipStream_t, hipEvent_t);
template int32_t launch_trace_count<int64_t>(const StepParams&, hipStream_t, hipEvent_t);

}  // namespace cowsdm_impl
