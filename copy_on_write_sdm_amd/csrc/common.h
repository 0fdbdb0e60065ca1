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
constexpr int kMaxPageShift = 6;            // paged slot maps: at most 64 slots per page
constexpr int kTile = 2048;                 // ranking tile (entries)
constexpr int kTileThreads = 256;
constexpr int kPerThread = kTile / kTileThreads;
// persistent multi-step launches
constexpr int kTraceMaxWrites = 4;
constexpr int kTraceMaxReads = 16;
constexpr int kTraceMaxSteps = 512;         // steps per persistent launch
constexpr int kTraceMaxBanks = 256;         // banks per packed layer of a persistent launch
constexpr int kTraceMapSlots = 4096;        // largest N whose slot maps are staged in LDS
constexpr int kTraceBanksPerBlock = 2;      // banks per persistent workgroup
constexpr int kTraceThreads = 2 * kWave * kTraceBanksPerBlock;  // a control and a data wave per bank
constexpr int kTraceRing = 16;              // steps handed from control to data wave in flight
// Plan word of a (step, bank) as the control wave stages it for its steps:
// bits 0-23 the first touches of the launch before it (step-major,
// bank-major within a step), bits 24-27 its first-touch write lanes, bit 28
// set from the bank's first step with an invalid route on.
constexpr uint32_t kPlanBaseMask = (1u << 24) - 1;
constexpr int kPlanMaskShift = 24;
constexpr int kPlanStopBit = 28;
// Words a packed launch's plan exchanges between workgroups are 64-bit, the
// launch's epoch in the high half and the value in the low half: a reader
// polls a word until it carries the current epoch, so no fence orders one
// word against another.  Count words (value: bits 0-3 the first-touch write
// lanes, bit 4 the stop bit) become prefix words once the first touches of
// lower banks at the same step are known (bits 5-28, bit 31 set).
constexpr uint32_t kCountStop = 1u << 4;
constexpr int kPrefixShift = 5;
constexpr uint32_t kPrefixDone = 1u << 31;
constexpr int kPlanHead = 8;        // header words (tagged): steps, fit, capacity
constexpr int kPlanHeadWords = 8;
constexpr int kPlanSegments = kTraceMaxSteps + 1;   // growth segments of one launch
constexpr int kPlanLocalWords = 6;  // a short launch's packed count words per bank
constexpr uint32_t kPlanReady = 1u << 31;            // the plan's steps are in a sync word
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
bool trace_timing_events(hipEvent_t* first, hipEvent_t* start, hipEvent_t* stop);
// the launch whose events trace_timing_events just gave out has no kernel
// before its decode kernel: its launch time is the decode kernel's
void trace_timing_first_is_start();
const char* last_error();

struct StepParams {
  cowsdm_layer_t layer[kMaxLayers];
  int64_t* trace_step;           // per-layer device step counters, or null
  int64_t* trace_ticket;         // [1 + layer]: waves of a layer done with the launch
  int64_t trace_first;           // step of this launch when trace_step is null
  int64_t trace_known;           // every layer's trace_step value when the caller knows it, or -1
  int64_t trace_len;             // steps the trace inputs hold
  int32_t* trace_status;         // per-layer status bits, or null
  int64_t trace_stride[9];
  int64_t* scan;                 // packed persistent launches: per-layer plan blocks
  int64_t scan_words;            // words per layer in `scan`
  int64_t* control;              // packed persistent launches: COWSDM_CTRL_* words
  int64_t control_stride;        // word k of layer l at control[k * stride + l]
  int64_t* report;               // host-mapped COWSDM_REPORT_WORDS per layer, or null
  int32_t plan_steps;            // steps per launch a plan block holds
  int32_t count_table;           // count pass: LDS hash entries per bank (N > kTraceMapSlots)
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

// Wave-inclusive sum over lanes (lane order), in DPP moves: shifts by 1, 2,
// 4 and 8 lanes within each row of 16, then row 0's and row 1's last lanes
// broadcast into the rows after them (a lane shifted in from outside its
// row, or a row the mask leaves out, adds the identity 0).
__device__ __forceinline__ int wave_inclusive(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31, rows 2 and 3
  return v;
}

// OR of v over the wave, in every lane (DPP OR scan, lane 63's result)
__device__ __forceinline__ uint32_t wave_or_all(uint32_t v) {
  int x = static_cast<int>(v);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
  x |= __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
  x |= __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
  x |= __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
  x |= __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15
  x |= __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(x, kWave - 1));
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_or(int v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v |= __shfl_xor(v, o, kWave);
  return v;
}

// Map entry of bank `bank`'s slot `slot` (N slots per bank): the direct
// map's, or through the paged map's directory (*dir_out: the directory
// entry, -1 when the page does not exist; the direct map gives 0).
__device__ __forceinline__ int map_entry(const cowsdm_layer_t& L, int64_t bank, int N, int slot,
                                         int* dir_out = nullptr) {
  const int shift = L.map_page_shift;
  if (shift == 0) {
    if (dir_out) *dir_out = 0;
    return L.logical_to_physical[bank * N + slot];
  }
  const int d = L.map_directory[bank * (N >> shift) + (slot >> shift)];
  if (dir_out) *dir_out = d;
  if (d < 0) return -1;
  // a directory entry past the pages is corrupt: an entry past every slab
  if (d >= L.map_page_capacity) return 0x7fffffff;
  return L.map_pages[(static_cast<int64_t>(d) << shift) + (slot & ((1 << shift) - 1))];
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

// A packed decode trace layer's plan block (int64 words; S = plan_steps,
// B = banks, W = writes): the epoch, the header, the plan words [B][S]
// (bank-major: a bank's words of consecutive steps are contiguous), the step
// totals [S], the running totals [S + 1], the pops [S * B * W] and the
// growth segments [S + 1][4].
struct PlanBlock {
  int64_t* epoch;
  int64_t* head;
  int64_t* words;
  int64_t* totals;
  int64_t* cum;
  int64_t* pops;
  int64_t* segs;   // [S + 1][4]: the growth segments (plan_layer)
  int64_t* local;  // [kPlanLocalWords][kWave]: short launches' packed count words (k-major)
  int64_t steps;   // S
  __device__ int64_t* word(int bank, int t) const {
    return words + static_cast<int64_t>(bank) * steps + t;
  }
};
__device__ __forceinline__ PlanBlock plan_block(const StepParams& P, int layer) {
  int64_t* const b = P.scan + static_cast<int64_t>(layer) * P.scan_words;
  const int64_t S = P.plan_steps;
  PlanBlock pb;
  pb.epoch = b;
  pb.head = b + kPlanHead;
  pb.words = pb.head + kPlanHeadWords;
  pb.totals = pb.words + S * P.banks;
  pb.cum = pb.totals + S;
  pb.pops = pb.cum + S + 1;
  pb.segs = pb.pops + S * P.banks * P.writes;
  pb.local = pb.segs + 4 * (S + 1);
  pb.steps = S;
  return pb;
}
// The tag of a layer's words in the launch now starting: one past the epoch
// word, which the layer's last control wave sets to it when the launch ends.
// Never 0, so that zeroed memory carries no valid word.
// the launch's epoch from the layer's epoch word (the last launch's epoch,
// stored zero-extended: its low half, read on its own, is all of it)
__device__ __forceinline__ uint32_t epoch_after(uint32_t word) {
  const uint32_t e = word + 1u;
  return e == 0 ? 1u : e;
}
__device__ __forceinline__ uint32_t epoch_word(const PlanBlock& pb) {
  return __hip_atomic_load(reinterpret_cast<uint32_t*>(pb.epoch), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t launch_epoch(const PlanBlock& pb) {
  return epoch_after(epoch_word(pb));
}
__device__ __forceinline__ uint64_t tagged(uint32_t epoch, uint32_t value) {
  return (static_cast<uint64_t>(epoch) << 32) | value;
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t epoch) {
  return static_cast<uint32_t>(w >> 32) == epoch;
}
__device__ __forceinline__ int64_t& control_word(const StepParams& P, int layer, int k) {
  return P.control[static_cast<int64_t>(k) * P.control_stride + layer];
}

// A layer's report in host memory, lane k of the calling wave writing word
// k: the step counter `step`, the status bits (with `extra` set) and the
// control words.  Called by one wave once no other wave of the layer
// changes them.
__device__ __forceinline__ void write_report(const StepParams& P, int layer, int64_t step,
                                             int32_t extra) {
  const int k = static_cast<int>(threadIdx.x) & (kWave - 1);
  if (k >= COWSDM_REPORT_WORDS) return;
  int64_t v = 0;
  if (k == 0) {
    v = step;
  } else if (k == 1) {
    const int32_t status = P.trace_status ? __hip_atomic_load(&P.trace_status[layer],
                                                              __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT)
                                          : 0;
    v = static_cast<uint32_t>(status | extra);
  } else if (P.control) {
    v = static_cast<int64_t>(atomic_load_u64(&control_word(P, layer, k - 2)));
  }
  __hip_atomic_store(P.report + static_cast<int64_t>(layer) * COWSDM_REPORT_WORDS + k, v,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The steps a trace launch runs for a layer: its first step (from the
// device counter when there is one) and how many, never past the recorded
// steps.  Every thread reading it gets the same value: a counter changes only
// after every wave of its layer is done with the launch.
__device__ __forceinline__ void trace_span(const StepParams& P, int layer, int64_t& first,
                                           int64_t& left) {
  first = P.trace_first;
  left = P.steps;
  if (P.trace_step) {
    first = P.trace_step[layer];
    const int64_t recorded = P.trace_len - first;
    left = first < 0 ? 0 : (recorded < left ? recorded : left);
  }
}


}  // namespace cowsdm_impl
