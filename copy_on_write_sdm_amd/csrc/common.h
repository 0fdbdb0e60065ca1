// Shared declarations of libcowsdm's translation units: constants,
// launch parameters and wave-level device helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "cowsdm.h"

namespace cowsdm_impl {

constexpr int kWave = 64;
constexpr int kBanksPerBlock = 4;           // waves (banks) per workgroup
constexpr int kStepThreads = kWave * kBanksPerBlock;
constexpr int kMaxLayers = 8;               // layers per step launch
constexpr int kReadBatch = 16;              // read rows in flight per batch
constexpr int kMaxReadSlots = 4;            // R <= 256 = 4 * 64
constexpr int kSpinLimit = 1 << 16;         // bounded look-back wait
constexpr int kFreeWindow = 256;            // prefetched free-stack entries
constexpr int kTile = 2048;                 // ranking tile (entries)
constexpr int kTileThreads = 256;
constexpr int kPerThread = kTile / kTileThreads;
// persistent multi-step launches
constexpr int kTraceMaxWrites = 4;
constexpr int kTraceMaxReads = 16;
constexpr int kTraceMaxSteps = 512;         // steps per persistent launch
constexpr int kTraceScanWindows = 4;        // up to 256 banks per layer
constexpr int kTraceFreeWindow = 1024;      // top of the free stack staged in LDS
constexpr int kTraceMapSlots = 4096;        // largest N whose slot maps are staged in LDS
constexpr int kTraceBanksPerBlock = 2;      // banks per persistent workgroup
constexpr int kTraceThreads = 2 * kWave * kTraceBanksPerBlock;  // a control and a data wave per bank
constexpr int kTraceRing = 16;              // steps handed from control to data wave in flight
// packed layers of at most 64 banks: a fifth wave sums the capacity proofs
constexpr int kTraceProofThreads = kTraceThreads + kWave;
// claim counters of the runs of one launch (runs of at least 2 steps), at the
// end of a layer's scan words
constexpr int kTraceRunCounters = kTraceMaxSteps / 2 + 1;
constexpr int64_t kClaimFailBase = int64_t{1} << 40;  // failed claim p recorded as base - p

constexpr uint32_t kStatusEmpty = 0;
constexpr uint32_t kStatusAggregate = 1;
constexpr uint32_t kStatusInclusive = 2;
constexpr uint32_t kStatusPoison = 3;
constexpr uint64_t kValueMask = (1ull << 30) - 1;

// Record a message for cowsdm_last_error_string() and return `code`.
int32_t fail(int32_t code, const char* fmt, ...);
// 0, or the pending hipError_t of the last launch (recorded by fail()).
int32_t launch_status(const char* where);
// cowsdm_trace_timing: the start/stop events to record around the next
// trace kernel launch, or false when timing is off (or its slots are full).
bool trace_timing_events(hipEvent_t* start, hipEvent_t* stop);
const char* last_error();

struct StepParams {
  cowsdm_layer_t layer[kMaxLayers];
  int64_t* trace_step;           // per-layer device step counters, or null
  int64_t* trace_ticket;         // [1 + layer]: waves of a layer done with the launch
  int64_t trace_first;           // step of this launch when trace_step is null
  int64_t trace_len;             // steps the trace inputs hold
  int64_t trace_proof_rows;      // device capacity proof per run of proof steps, or 0
  int32_t* trace_status;         // per-layer status bits, or null
  int64_t* trace_free_out;       // per-layer free_count after a launch, or null
  int32_t trace_proof_steps;
  int64_t trace_stride[9];
  int64_t* scan;                 // persistent launches: per-layer scan words
  int64_t scan_words;            // words per layer in `scan`
  int32_t steps;                 // persistent launches: steps per launch
  int32_t nlayers;
  int32_t banks;
  int32_t slots;
  int32_t width;
  int32_t writes;
  int32_t reads;
  int32_t templates;
  int32_t blocks_per_layer;
};

// ------------------------------------------------------------ wave helpers

__device__ __forceinline__ int rl(int x, int lane) {
  return __builtin_amdgcn_readlane(x, lane);
}

__device__ __forceinline__ float rlf(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_or(int v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v |= __shfl_xor(v, o, kWave);
  return v;
}

template <typename IDX>
__device__ __forceinline__ int64_t load_index(const void* base, int64_t i) {
  return static_cast<int64_t>(static_cast<const IDX*>(base)[i]);
}

template <int VEC>
__device__ __forceinline__ void load_row(const float* p, float (&x)[VEC]) {
  if constexpr (VEC == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
  } else if constexpr (VEC == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    x[0] = t.x; x[1] = t.y;
  } else {
    x[0] = *p;
  }
}

template <int VEC>
__device__ __forceinline__ void store_row(float* p, const float (&x)[VEC]) {
  if constexpr (VEC == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  } else if constexpr (VEC == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
  } else {
    *p = x[0];
  }
}

__device__ __forceinline__ uint64_t atomic_load_u64(const int64_t* p) {
  return static_cast<uint64_t>(__hip_atomic_load(
      const_cast<int64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ void atomic_store_u64(int64_t* p, uint64_t v) {
  __hip_atomic_store(p, static_cast<int64_t>(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t slot_word(uint32_t epoch, uint32_t status,
                                              uint64_t value) {
  return (static_cast<uint64_t>(epoch) << 32) |
         (static_cast<uint64_t>(status) << 30) | (value & kValueMask);
}


}  // namespace cowsdm_impl
