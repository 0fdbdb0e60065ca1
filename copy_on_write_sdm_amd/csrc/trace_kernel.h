// Persistent multi-step form of the copy-on-write SDM step: one launch runs
// G <= 512 consecutive decode steps of device-resident routes for every
// (layer, bank), with the results of G single-step launches.
//
// Each (layer, bank) has two waves in one workgroup, which hand steps over
// through a ring of kTraceRing slots in LDS:
//
//   the control wave loads the step's slots and map entries, classifies the
//   step (first touches, slots written by the step before, read-after-write),
//   fetches the rows its first touches pop from the launch's plan, and
//   publishes the addresses of the rows the step loads, two steps ahead of
//   the data wave's loads; two steps later it takes the popped rows, stores
//   them in the map and publishes the rows the step's updates are stored to
//   and the step's masks;
//
//   the data wave loads the rows of step s+1 from the published addresses
//   while it computes step s (gated-delta update, sparse read) from rows
//   loaded one iteration earlier, stores the reading and the updated rows,
//   and keeps the updated rows in LDS for the step after.
//
// Only the data wave reads or writes rows, in program order: a step's rows
// were stored by earlier steps of the same wave, except the rows of the step
// just before, which it takes from LDS.  The control wave runs up to
// kTraceRing - 3 steps ahead, so the map lookups and pop-list loads it waits
// on stay off the data wave's path.  It classifies step t after resolving
// step t-2, but before step t-1 has its rows: slots written at t-1 take their
// rows from that step's result.  When a bank's map fits (N <=
// kTraceMapSlots), the control wave keeps it in LDS for the launch (it is the
// only writer of its bank's entries) and the global map is written
// alongside; otherwise step t's entries are loaded from the global map an
// iteration early, before step t-2's pops, and slots written at t-2 take the
// rows popped for them.  Values in flight live in even/odd homes (both loops
// are unrolled by two) and are only read one iteration after their load was
// issued, so no register copy waits on memory.
//
// Rows (packed state): the count and plan passes (trace_plan.hip) ran before
// the launch.  They fixed how many steps each layer runs (the decode loop's
// capacity proof may stop a layer before a growth its slab buffers cannot
// hold), the capacity the launch grows to, each (step, bank)'s first-touch
// lanes and its offset in pop order (step-major, bank-major within a step,
// as single steps pop), and the row of every pop; they also wrote the free
// stack and free_count the launch leaves.  A (step, bank) with c first
// touches at offset e takes pops e .. e+c-1 if e + c fits the rows the plan
// could give out (the launch's FIT word; every step fits unless a capacity
// proof was missing or dishonest), else it overflows and the bank stops for
// the rest of the launch.  Banks never wait on one another.
#pragma once

#include <hip/hip_ext.h>

#include <atomic>

#include "common.h"
#include "trace_plan.h"

namespace cowsdm_impl {

typedef float vf4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef uint64_t u64x2_t __attribute__((ext_vector_type(2)));

// A row of zeros, read (never written) by the read lanes past R: with a
// weight of -0.0 each of their terms is -0.0, which leaves any sum unchanged.
static __device__ __align__(16) const float kTraceZeroRow[kWave * 4] = {};

template <int VEC>
struct TraceRows {                  // operands of one step, loaded one step ahead
  float w[kTraceMaxWrites][VEC];    // rows of the write slots, before the decay
  float r[kTraceMaxReads][VEC];     // rows of the read slots, before this step
  float vin[VEC];                   // the step's value
};

struct TraceIdx {                   // lane j: write slot j / read slot j
  int widx, ridx, err;
  int k0, k1;                       // staged slots: the step's class words 0 and 1 (in
                                    // every lane, made scalar when the step is classified)
};

struct TraceRoute {                 // a classified step
  int widx, ridx;
  int base;       // wave-uniform (packed): first touches before it in pop order
  int wrow;       // write lane: physical row (-1: M0, or a first touch not yet popped)
  int wsrc;       // write lane: written by step t-1 lane j (j), else -1
  int rsrc;       // read lane: the same
  int rraw;       // read lane: write lane of step t itself with this slot, else -1
  int rank;       // write lane: rank among the bank's first touches
  uint32_t u;     // wave-uniform: bits 0-3 first-touch write lanes, 4-7 their count,
                  // 8 the step runs (routes valid, every earlier step ran)
  uint32_t fwd;   // wave-uniform: rows from step t-1, bits 0-3 writes, 4-19 reads
  uint32_t rawm;  // wave-uniform: reads that see a write of step t itself
};

__device__ __forceinline__ uint32_t route_fmask(uint32_t u) { return u & 15u; }
__device__ __forceinline__ int route_count(uint32_t u) { return static_cast<int>((u >> 4) & 15u); }
__device__ __forceinline__ bool route_ok(uint32_t u) { return (u >> 8) & 1u; }

// One step handed from the control wave to the data wave.
// The per-lane arrays have kTraceMaxReads entries (writes use the first
// kTraceMaxWrites), so that lanes 0-15 write all three in one store pass.
struct TraceSlot {
  uint64_t wptr[kTraceMaxReads];    // address of write j's row before the step
  uint64_t rptr[kTraceMaxReads];    // address of read i's row (a zero row past R)
  int32_t drow[kTraceMaxReads];     // row write j's update is stored to
  // ctl[0]: bits 0-19 rows forwarded from the step before (0-3 writes, 4-19
  //         reads), bit 20 the step runs, bits 24-27 write rows to store;
  // ctl[1]: bits 0-15 reads of the step's own writes, bits 16-19 and 20-23
  //         the low and high bits of each forwarded write's source row;
  // ctl[2]: bits 0-15 and 16-31, the same for forwarded reads;
  // ctl[3]: the same for reads of the step's own writes.
  uint32_t ctl[4];
};

typedef __attribute__((address_space(1))) float gfloat;
typedef float vf2 __attribute__((ext_vector_type(2)));
typedef float vf4 __attribute__((ext_vector_type(4)));

// Row accesses at a wave-uniform base plus this lane's 32-bit byte offset,
// through global-address-space pointers: global_load/store with a scalar
// base, no per-lane 64-bit address arithmetic.
template <int VEC>
__device__ __forceinline__ void gload_row(const float* base, uint32_t off, float (&x)[VEC]) {
  const __attribute__((address_space(1))) char* p =
      (const __attribute__((address_space(1))) char*)(base) + off;
  if constexpr (VEC == 4) {
    const vf4 t = *(const __attribute__((address_space(1))) vf4*)(p);
    x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
  } else if constexpr (VEC == 2) {
    const vf2 t = *(const __attribute__((address_space(1))) vf2*)(p);
    x[0] = t.x; x[1] = t.y;
  } else {
    x[0] = *(const gfloat*)(p);
  }
}

template <int VEC>
__device__ __forceinline__ void gstore_row(float* base, uint32_t off, const float (&x)[VEC]) {
  __attribute__((address_space(1))) char* p = (__attribute__((address_space(1))) char*)(base) + off;
  if constexpr (VEC == 4) {
    vf4 t;
    t.x = x[0]; t.y = x[1]; t.z = x[2]; t.w = x[3];
    *(__attribute__((address_space(1))) vf4*)(p) = t;
  } else if constexpr (VEC == 2) {
    vf2 t;
    t.x = x[0]; t.y = x[1];
    *(__attribute__((address_space(1))) vf2*)(p) = t;
  } else {
    *(gfloat*)(p) = x[0];
  }
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// A wave-uniform value the loop keeps in a register: values read from the
// kernel arguments would otherwise be reloaded, and waited on, inside it.
template <typename T>
__device__ __forceinline__ T pin(T x) {
  asm volatile("" : "+s"(x));
  return x;
}

// The lane's column offset as a fresh 32-bit value: the compiler then pairs
// it with a wave-uniform row base as global_load/store's scalar base plus
// vector offset, instead of materialising a 64-bit address per row.
__device__ __forceinline__ uint32_t fresh(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Hand-over words between the two waves of a bank (LDS, workgroup scope):
// a release store orders the ring writes before it, an acquire load the
// ring reads after it.
__device__ __forceinline__ uint32_t sync_load(uint32_t* p) {
  return __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
}
__device__ __forceinline__ void sync_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Sum over the wave of per-lane counts of one launch's first touches (at
// most kTraceMaxWrites * kTraceMaxSteps per bank), by bit planes: ballots
// and scalar adds, no LDS round trip.
constexpr int kLaunchCountBits = 32 - __builtin_clz(kTraceMaxWrites * kTraceMaxSteps);
__device__ __forceinline__ int wave_sum_launch(int v) {
  int sum = 0;
#pragma unroll
  for (int b = 0; b < kLaunchCountBits; ++b) sum += __popcll(__ballot((v >> b) & 1)) << b;
  return sum;
}

// Source row (0..3) of entry i from two bit planes of a control word.
__device__ __forceinline__ int plane_code(uint32_t w, int lo, int hi) {
  return static_cast<int>(((w >> lo) & 1u) | (((w >> hi) & 1u) << 1));
}

// Every step handles kTraceMaxWrites write rows and kTraceMaxReads read rows
// without a branch on W or R; FULL (W and R at those maxima) drops the
// selects and the zero rows that leave the others out.
// FEW: at most 64 banks per layer (the compiler may then give a wave every
// register; a grid of more banks needs two workgroups per CU).
// MAPLDS: packed, the bank's slot map staged in dynamic LDS (N ints per bank).
// A bank's pops when its launch's plan is in: the row of every first touch
// of its steps (plan words in LDS, `plan`) into the plan's pop list, from the
// launch's growth segments when it grows, else the found stack's entry
// found - 1 - pop.  Lane = step, 64 steps a round; every round's stack
// entries are loaded before the first is used, so the listing waits for one
// load's latency, not one per round.  False when a segment never arrives.
__device__ __forceinline__ bool list_bank_pops(const PlanBlock& pb, uint32_t epoch, int segments,
                                               int found, int G, int fit, const int* plan,
                                               int* seg, const int32_t* stack) {
  constexpr int kRounds = kTraceMaxSteps / kWave;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  bool ok = true;
  if (segments > 1) ok = plan_segments(pb, epoch, segments, seg);
  // row[c][r]: the row of pop r of step c * 64 + lane, or -2 - p for the
  // found stack's entry at position p
  int row[kRounds][kTraceMaxWrites];
  int base[kRounds], n[kRounds];
#pragma unroll
  for (int c = 0; c < kRounds; ++c) {
    const int t = c * kWave + lane;
    const uint32_t w = t < G ? static_cast<uint32_t>(plan[t]) : 0u;
    base[c] = static_cast<int>(w & kPlanBaseMask);
    n[c] = __popc((w >> kPlanMaskShift) & 15u);
#pragma unroll
    for (int r = 0; r < kTraceMaxWrites; ++r) {
      const int q = base[c] + r;
      row[c][r] = 0;
      if (r < n[c] && q < fit) {
        if (segments > 1) {
          const int k = segment_of(seg, segments, q);
          const int pos = seg[2 * kPlanSegments + k] - 1 - (q - seg[k]);
          const int v = segment_entry(seg, pos, k);
          row[c][r] = v >= 0 ? v : -2 - pos;
        } else {
          row[c][r] = -2 - (found - 1 - q);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < kRounds; ++c) {
#pragma unroll
    for (int r = 0; r < kTraceMaxWrites; ++r) {
      if (row[c][r] <= -2) row[c][r] = stack[-2 - row[c][r]];
    }
  }
#pragma unroll
  for (int c = 0; c < kRounds; ++c) {
#pragma unroll
    for (int r = 0; r < kTraceMaxWrites; ++r) {
      if (r < n[c] && base[c] + r < fit) {
        atomic_store_u64(pb.pops + base[c] + r, tagged(epoch, static_cast<uint32_t>(row[c][r])));
      }
    }
  }
  return ok;
}

// The free stack a growing launch leaves (segments staged in `seg`, the
// capacity it grows to, the pops that fit), by one wave once every control
// wave of the layer has listed its pops: every position above the lowest
// growth that a growth covers holds the row the latest such growth put
// there.
__device__ __forceinline__ void rewrite_stack(const int* seg, int segments, int capacity, int fit,
                                              int32_t* stack) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  int lo = seg[kPlanSegments + 1];
  for (int k = 2; k < segments; ++k) {
    lo = seg[kPlanSegments + k] < lo ? seg[kPlanSegments + k] : lo;
  }
  // segment 0 holds the stack height and the capacity the launch found
  const int top = seg[kPlanSegments] + (capacity - seg[3 * kPlanSegments]) - fit;
  for (int p = lo + lane; p < top; p += kWave) {
    const int v = segment_entry(seg, p, segments - 1);
    if (v >= 0) stack[p] = v;
  }
}

template <typename IDX, int VEC, bool DENSE, bool FULL, bool FEW, bool MAPLDS>
__global__ __launch_bounds__(kTraceThreads)
__attribute__((amdgpu_waves_per_eu(1, FEW ? 1 : 2)))
void sdm_trace_kernel(StepParams P) {
  constexpr int kRow = kWave * VEC;  // floats of one LDS row
  constexpr int NB = kTraceBanksPerBlock;
  constexpr uint32_t kNoStop = 0xFFFFu;
  // data wave: the last computed step's updated rows
  __shared__ float lds_rows[NB][kTraceMaxWrites][kRow];
  // data wave: the next step's weights, written per lane at the end of an
  // iteration, read back as broadcasts by the step's compute
  __shared__ vf4_t lds_weights[NB][2][kWave / 4];
  __shared__ TraceSlot lds_ring[NB][kTraceRing];
  // [0]: control -> data, (stop step << 16) | steps whose row addresses are
  // published (the masks and store rows of all but the last of them);
  // [1]: data -> control, steps computed; [2]: control -> data, packed:
  // kPlanReady | the steps the launch's plan lets the bank run; [3]: data ->
  // control, packed short launch: 2 + the local plan's result (plan_local)
  __shared__ uint32_t lds_sync[NB][4];
  // data -> control: the local plan's pops, found stack height and proof
  __shared__ int64_t lds_local[NB][3];
  // the workgroup's control waves done with the launch (the last of them
  // takes the layer's tickets for all)
  __shared__ uint32_t lds_done;
  // control wave: the slots of two 64-step chunks, per step W write slots
  // then R read slots (-1: outside [0, N)) and the step's four class words,
  // staged from registers a chunk ahead (map in LDS, or dense)
  constexpr int kIdxRow = kTraceMaxWrites + kTraceMaxReads;
  constexpr int kIdxLds = kIdxRow + 4;
  __shared__ __align__(16) int lds_idx[(DENSE || MAPLDS) ? NB : 1][2][kWave][kIdxLds];
  // control wave (packed): the plan words of two 64-step chunks, staged from
  // registers a chunk ahead
  __shared__ int lds_plan[DENSE ? 1 : NB][DENSE ? 1 : kTraceMaxSteps];
  // packed, slot maps in global memory: the launch's growth segments (the
  // planner's, then every bank's copy when it lists its pops; the same values
  // in every workgroup)
  __shared__ int lds_seg[DENSE || MAPLDS ? 1 : 4 * kPlanSegments];
  // map in LDS (dynamic, 2 banks x 2 x N ints): each bank's slot map, then
  // each bank's first step of the launch writing each slot (the count part
  // of the launch's plan)
  extern __shared__ int lds_map_all[];

  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int pair = wave >> 1;
  const bool data_wave = (wave & 1) != 0;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  if (layer_id >= P.nlayers) return;  // whole workgroup
  const int bank = (blockIdx.x % P.blocks_per_layer) * NB + pair;
  const cowsdm_layer_t& L = P.layer[layer_id];
  // Device-counted launches read the layer's first step from its counter
  // (every thread reads the same value: it changes only after all waves of
  // the layer are done), or take it from the caller when it knows where the
  // counters stand (the control wave of bank 0 then compares the counter
  // with it once its steps are out, off the critical path), and run at most
  // the steps recorded after it.
  const bool known_first = P.trace_step && P.trace_known >= 0;
  int64_t first = P.trace_first;
  int64_t left = P.steps;
  if (P.trace_step) {
    const uint64_t f = known_first ? static_cast<uint64_t>(P.trace_known)
                                   : static_cast<uint64_t>(P.trace_step[layer_id]);
    first = static_cast<int64_t>(
        (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(f >> 32))) << 32) |
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(f)));
    const int64_t recorded = P.trace_len - first;
    left = first < 0 ? 0 : (recorded < left ? recorded : left);
  }
  if (left <= 0) {
    // no recorded step left for this layer: touch no input, leave the counter
    if (threadIdx.x == 0 && blockIdx.x % P.blocks_per_layer == 0) {
      if (P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_ENDED},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else if (!DENSE) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_TRACE_RANGE), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (P.report && threadIdx.x < kWave && blockIdx.x % P.blocks_per_layer == 0) {
      write_report(P, layer_id, first, COWSDM_TRACE_ENDED);
    }
    return;  // whole workgroup
  }
  const int N = P.slots;
  const int D = P.width;
  const int W = FULL ? kTraceMaxWrites : P.writes;
  const int R = FULL ? kTraceMaxReads : P.reads;
  const int B = P.banks;
  // steps of this launch: G0 before the plan; the plan may stop a packed
  // layer earlier (before a growth its slab buffers cannot hold), G
  const int G0 = static_cast<int>(left);
  int G = G0;
  // slab capacity (rows are int32): at launch start, then the capacity the
  // launch's plan grows the slab to
  const int C0 = DENSE ? 0 : pin(__builtin_amdgcn_readfirstlane(
                                 static_cast<int>(control_word(P, layer_id, COWSDM_CTRL_CAPACITY))));
  int C = C0;
  // lanes past the row width repeat the last columns: they load, compute and
  // store exactly what the last full lane does, so no access needs a lane mask
  const int col = lane * VEC < D ? lane * VEC : D - VEC;
  const uint32_t coff = static_cast<uint32_t>(col) * 4u;
  const uint32_t row_bytes = static_cast<uint32_t>(D) * 4u;

  int base_err = 0;
  if (lane == 0 && !data_wave) {
    lds_sync[pair][0] = kNoStop << 16;
    lds_sync[pair][1] = 0;
    lds_sync[pair][2] = 0;
    lds_sync[pair][3] = 0;
  }
  if (threadIdx.x == 0) lds_done = 0;
  __syncthreads();
  if (bank >= B) return;  // both waves of the bank

  uint32_t* const sync = lds_sync[pair];
  TraceSlot* const ring = lds_ring[pair];
  auto slot_of = [&](int t) __attribute__((always_inline)) -> TraceSlot& {
    return ring[static_cast<uint32_t>(t) % kTraceRing];
  };
  const uint64_t wlanes = W >= kWave ? ~0ull : ((1ull << W) - 1);
  const uint64_t rlanes = R >= kWave ? ~0ull : ((1ull << R) - 1);
  float* const slab = DENSE ? nullptr : pin(L.values);
  float* const table_bank = DENSE ? L.values + static_cast<int64_t>(bank) * N * D : nullptr;
  auto first_step = [&](const void* base, int k) __attribute__((always_inline)) -> const char* {
    return static_cast<const char*>(base) + first * P.trace_stride[k];
  };
  auto at = [](const char* p, uint32_t stride, int t) __attribute__((always_inline)) -> const char* {
    return p + static_cast<uint64_t>(static_cast<uint32_t>(t)) * stride;
  };
  const int wl = lane < W ? lane : 0;
  const int rl_ = lane < R ? lane : 0;

  if (data_wave) {
    // ======================= data wave =======================
    float* const lds_wave = &lds_rows[pair][0][0];
    float* const store_base = DENSE ? table_bank : slab;
    const char* const ww_l = first_step(L.write_weights, 1) + (static_cast<int64_t>(bank) * W + wl) * 4;
    const char* const v_l = first_step(L.step_values, 2) + (static_cast<int64_t>(bank) * D + col) * 4;
    const char* const rw_l = first_step(L.read_weights, 7) + (static_cast<int64_t>(bank) * R + rl_) * 4;
    const char* const out_l = first_step(L.output, 8) + (static_cast<int64_t>(bank) * D + col) * 4;
    const uint32_t st_ww = pin(static_cast<uint32_t>(P.trace_stride[1]));
    const uint32_t st_v = pin(static_cast<uint32_t>(P.trace_stride[2]));
    const uint32_t st_rw = pin(static_cast<uint32_t>(P.trace_stride[7]));
    const uint32_t st_out = pin(static_cast<uint32_t>(P.trace_stride[8]));

    // gates in chunks of 64 steps, lane k holding step 64c + k of chunk c;
    // the next chunk is loaded one chunk ahead
    auto load_gates = [&](int c, float& fg, float& ig, float& eg) __attribute__((always_inline)) {
      const int t = c * kWave + lane;
      fg = 0.0f;
      ig = 0.0f;
      eg = 0.0f;
      if (t < G) {
        fg = reinterpret_cast<const float*>(first_step(L.forget_log_gate, 5) +
                                            static_cast<int64_t>(t) * P.trace_stride[5])[bank];
        ig = reinterpret_cast<const float*>(first_step(L.input_gate, 3) +
                                            static_cast<int64_t>(t) * P.trace_stride[3])[bank];
        eg = reinterpret_cast<const float*>(first_step(L.erase_gate, 4) +
                                            static_cast<int64_t>(t) * P.trace_stride[4])[bank];
      }
    };
    float alpha_l, in_l, er_l, fg_n, in_n, er_n;
    {
      float fg0;
      load_gates(0, fg0, in_l, er_l);
      alpha_l = static_cast<float>(exp(static_cast<double>(fg0)));
      load_gates(1, fg_n, in_n, er_n);
    }
    // before step s (s even): the step's chunk in the lane registers
    auto gates_for = [&](int s) __attribute__((always_inline)) {
      if (s > 0 && (s & (kWave - 1)) == 0) {
        alpha_l = static_cast<float>(exp(static_cast<double>(fg_n)));
        in_l = in_n;
        er_l = er_n;
        if (s + kWave < G) load_gates(s / kWave + 1, fg_n, in_n, er_n);
      }
    };

    // lane j's write and read weight of step t, loaded two iterations ahead
    // and handed to LDS at the end of the iteration before
    auto load_weights = [&](int t, float& ww, float& rw) __attribute__((always_inline)) {
      const int tc = t < G ? t : G - 1;
      ww = *(const gfloat*)(at(ww_l, st_ww, tc));
      rw = *(const gfloat*)(at(rw_l, st_rw, tc));
    };
    auto put_weights = [&](float ww, float rw) __attribute__((always_inline)) {
      float* const wv = reinterpret_cast<float*>(&lds_weights[pair][0][0]);
      wv[lane] = ww;
      wv[kWave + lane] = FULL || lane < R ? rw : -0.0f;
    };

    // What the data wave reads from LDS for a step: step t+1's row addresses
    // (a broadcast read gives every lane two of them), and, one iteration
    // before it needs them, step t's masks, store rows and weights.
    constexpr int kPtrPairs = (kTraceMaxWrites + kTraceMaxReads) / 2;
    struct Handed {
      u64x2_t ptr[kPtrPairs];  // the W write addresses, then the R read addresses
      u32x4_t cw;
      i32x4_t dr;
      vf4_t wwv;
      vf4_t rwv[kTraceMaxReads / 4];
    };
    auto read_ptrs = [&](int t, Handed& h) __attribute__((always_inline)) {
      const TraceSlot& sl = slot_of(t);
      const u64x2_t* const pw = reinterpret_cast<const u64x2_t*>(sl.wptr);
      const u64x2_t* const pr = reinterpret_cast<const u64x2_t*>(sl.rptr);
#pragma unroll
      for (int k = 0; k < kTraceMaxWrites / 2; ++k) h.ptr[k] = pw[k];
#pragma unroll
      for (int k = 0; k < kTraceMaxReads / 2; ++k) h.ptr[kTraceMaxWrites / 2 + k] = pr[k];
    };
    // lane j put weight j there: every lane reads all of them as vectors,
    // instead of a readlane per weight
    auto read_step = [&](int t, Handed& h) __attribute__((always_inline)) {
      const TraceSlot& sl = slot_of(t);
      h.cw = *reinterpret_cast<const u32x4_t*>(sl.ctl);
      h.dr = *reinterpret_cast<const i32x4_t*>(sl.drow);
      h.wwv = lds_weights[pair][0][0];
#pragma unroll
      for (int k = 0; k < kTraceMaxReads / 4; ++k) h.rwv[k] = lds_weights[pair][1][k];
    };

    // Step t's rows from the published addresses: each row load takes its
    // own 64-bit vector address (no scalar base, whose write by a readlane a
    // load could not follow at once).  Every row is loaded: write lanes past
    // W point at a row of slot 0, read lanes past R at the zero row, and the
    // step leaves both out.
    auto issue_rows = [&](int t, const Handed& h, TraceRows<VEC>& buf) __attribute__((always_inline)) {
      const int tc = t < G ? t : G - 1;
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; j += 2) {
        const u64x2_t two = h.ptr[j / 2];
        gload_row<VEC>(reinterpret_cast<const float*>(two.x), coff, buf.w[j]);
        gload_row<VEC>(reinterpret_cast<const float*>(two.y), coff, buf.w[j + 1]);
      }
#pragma unroll
      for (int i = 0; i < kTraceMaxReads; i += 2) {
        const u64x2_t two = h.ptr[(kTraceMaxWrites + i) / 2];
        gload_row<VEC>(reinterpret_cast<const float*>(two.x), coff, buf.r[i]);
        gload_row<VEC>(reinterpret_cast<const float*>(two.y), coff, buf.r[i + 1]);
      }
      gload_row<VEC>(reinterpret_cast<const float*>(at(v_l, st_v, tc)), 0u, buf.vin);
    };

    auto lds_get = [&](int row, float (&x)[VEC]) __attribute__((always_inline)) {
      const float* p = lds_wave + row * kRow + col;
      if constexpr (VEC == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
      } else if constexpr (VEC == 2) {
        const float2 t = *reinterpret_cast<const float2*>(p);
        x[0] = t.x; x[1] = t.y;
      } else {
        x[0] = *p;
      }
    };
    auto lds_put = [&](int row, const float (&x)[VEC]) __attribute__((always_inline)) {
      float* p = lds_wave + row * kRow + col;
      if constexpr (VEC == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
      } else if constexpr (VEC == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
      } else {
        *p = x[0];
      }
    };

    // updated rows of the last computed step
    float cur[kTraceMaxWrites][VEC];
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) cur[j][v] = 0.0f;
    }

    // Step t: LDS row j holds write j of step t-1 until this step replaces it.
    auto compute = [&](int t, const Handed& h, TraceRows<VEC>& buf)
        __attribute__((always_inline)) {
      const u32x4_t cw = h.cw;
      const i32x4_t dr = h.dr;
      const uint32_t c0 = __builtin_amdgcn_readfirstlane(cw.x);
      const bool run = ((c0 >> 20) & 1u) != 0;
      float acc[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
      if (run) {
        const uint32_t c1 = __builtin_amdgcn_readfirstlane(cw.y);
        const uint32_t fwd = c0 & 0xFFFFFu;
        if (fwd != 0) {
          const uint32_t c2 = __builtin_amdgcn_readfirstlane(cw.z);
#pragma unroll
          for (int j = 0; j < kTraceMaxWrites; ++j) {
            if ((fwd >> j) & 1u) lds_get(plane_code(c1, 16 + j, 20 + j), buf.w[j]);
          }
#pragma unroll
          for (int i = 0; i < kTraceMaxReads; ++i) {
            if ((fwd >> (kTraceMaxWrites + i)) & 1u) lds_get(plane_code(c2, i, 16 + i), buf.r[i]);
          }
        }
        const vf4_t wwv = h.wwv;
        const float alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha_l), t & (kWave - 1)));
        const float in_gate = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(in_l), t & (kWave - 1)));
        const float er_gate = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(er_l), t & (kWave - 1)));
        float ret[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) ret[v] = 0.0f;
        // rows past W are computed and left out of the sum by a select on the
        // wave-uniform row count (a decayed row can be infinite or NaN, so no
        // term of theirs is exactly neutral); rows past R add -0.0
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          const float wj = wwv[j];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float d = buf.w[j][v] * alpha;
            cur[j][v] = d;
            const float term = wj * d;
            ret[v] = (j == 0) ? term : (j < W ? ret[v] + term : ret[v]);
          }
        }
        float delta[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float a = in_gate * buf.vin[v];
          const float e = er_gate * ret[v];
          delta[v] = a - e;
        }
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          const float wj = wwv[j];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float u = wj * delta[v];
            cur[j][v] = cur[j][v] + u;
          }
          lds_put(j, cur[j]);
        }
        const uint32_t rawm = c1 & 0xFFFFu;
        if (rawm != 0) {
          const uint32_t c3 = __builtin_amdgcn_readfirstlane(cw.w);
#pragma unroll
          for (int i = 0; i < kTraceMaxReads; ++i) {
            if ((rawm >> i) & 1u) lds_get(plane_code(c3, i, 16 + i), buf.r[i]);
          }
        }
#pragma unroll
        for (int i = 0; i < kTraceMaxReads; ++i) {
          const float wr = h.rwv[i / 4][i % 4];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float term = wr * buf.r[i][v];
            acc[v] = (i == 0) ? term : acc[v] + term;
          }
        }
      }
      gstore_row<VEC>(reinterpret_cast<float*>(const_cast<char*>(at(out_l, st_out, t))), 0u, acc);
      if (run) {
        const uint32_t smask = (c0 >> 24) & 15u;
        const uint32_t co = fresh(coff);
        const int32_t rows[kTraceMaxWrites] = {dr.x, dr.y, dr.z, dr.w};
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          if ((smask >> j) & 1u) {
            const uint32_t r = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rows[j]));
            float* const dst = reinterpret_cast<float*>(reinterpret_cast<char*>(store_base) +
                                                        static_cast<uint64_t>(r) * row_bytes);
            gstore_row<VEC>(dst, co, cur[j]);
          }
        }
      }
    };

    // the control wave has published `need` steps' row addresses (and the
    // masks of all but the last); false if it never does
    uint32_t seen = 0, stop = kNoStop;
    auto await = [&](uint32_t need) __attribute__((always_inline)) -> bool {
      if (seen >= need) return true;
      for (int spins = 0; spins < 4 * kSpinLimit; ++spins) {
        const uint32_t w = sync_load(&sync[0]);
        seen = w & 0xFFFFu;
        stop = w >> 16;
        if (seen >= need) return true;
        __builtin_amdgcn_s_sleep(1);
      }
      return false;
    };

    TraceRows<VEC> bufA, bufB;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) { bufA.w[j][v] = 0.0f; bufB.w[j][v] = 0.0f; }
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) { bufA.r[i][v] = 0.0f; bufB.r[i][v] = 0.0f; }
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) { bufA.vin[v] = 0.0f; bufB.vin[v] = 0.0f; }
    float wwA = 0.0f, rwA = 0.0f, wwB = 0.0f, rwB = 0.0f;  // weights in flight
    {
      float ww0 = 0.0f, rw0 = 0.0f;
      load_weights(0, ww0, rw0);
      put_weights(ww0, rw0);
      load_weights(1, wwB, rwB);     // handed over at the end of iteration 0
    }

    // Iteration t: loads step t+1's rows, computes step t, then reads step
    // t+1's masks, store rows and weights from LDS.  The progress word goes
    // out after this step's LDS writes and before those reads, so its release
    // waits for no read in flight.  (The row addresses are read just before
    // their loads: held across an iteration they would cost 40 registers.)
    Handed hd;
    auto iteration = [&](int t, TraceRows<VEC>& rows_t, TraceRows<VEC>& rows_next,
                         float& ww_self, float& rw_self, float ww_other, float rw_other)
        __attribute__((always_inline)) {
      load_weights(t + 2, ww_self, rw_self);
      read_ptrs(t + 1, hd);
      issue_rows(t + 1, hd, rows_next);
      compute(t, hd, rows_t);
      put_weights(ww_other, rw_other);   // step t+1's
      if (lane == 0) sync_store(&sync[1], static_cast<uint32_t>(t + 1));
      read_step(t + 1, hd);
    };

    // the published steps the reads of iteration t+1 need (capped at what
    // the control wave publishes in all: addresses up to step G+1)
    auto need = [&](int t) __attribute__((always_inline)) -> uint32_t {
      return static_cast<uint32_t>(t + 3 < G + 1 ? t + 3 : G + 1);
    };
    // packed short launch, slot map in LDS: the local plan (trace_plan.h)
    // is made here while the control wave classifies the launch's first
    // chunk; the control wave takes the result from LDS
    if constexpr (!DENSE && MAPLDS) {
      const PlanBlock pbd = plan_block(P, layer_id);
      if (local_plan_fits(G0, B, pbd)) {
        const uint32_t ep = static_cast<uint32_t>(
            __builtin_amdgcn_readfirstlane(static_cast<int>(launch_epoch(pbd))));
        const PlanControl pcd = plan_control(P, layer_id);
        LocalPlan lp{};
        const int r = plan_local(pbd, B, G0, ep, bank, pcd, &lds_plan[pair][0], lp);
        if (lane == 0) {
          lds_local[pair][0] = lp.fit;
          lds_local[pair][1] = lp.found;
          lds_local[pair][2] = lp.proven;
          sync_store(&sync[3], static_cast<uint32_t>(2 + r));
        }
      }
    }
    // packed: the steps the launch's plan lets this bank run, from the
    // control wave before it publishes any step (bounded wait)
    bool go = true;
    if constexpr (!DENSE) {
      uint32_t w = 0;
      for (int spins = 0; spins < 64 * kSpinLimit; ++spins) {
        w = sync_load(&sync[2]);
        if (w & kPlanReady) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (w & kPlanReady) {
        const int planned = static_cast<int>(w & ~kPlanReady);
        G = planned < G ? planned : G;
        if (G <= 0) {
          if (lane == 0) sync_store(&sync[1], kNoStop);   // finished (see below)
          return;
        }
      } else {
        go = false;
      }
    }
    go = go && await(need(-1));
    bool lost = !go;
    if (go) {
      read_ptrs(0, hd);
      issue_rows(0, hd, bufA);
      read_step(0, hd);
    }
    // Drain the prologue's loads: the loop head then has one state of loads
    // in flight (the back edge's), and the waits the compiler places there
    // stay as loose as the steady state allows.
    __builtin_amdgcn_s_waitcnt(0);
    // Pairs of steps, then an odd last step; the control wave stops early
    // only before an even step (when this wave stopped taking steps), so the
    // loop's only exit is at its head.
    int s = 0;
    for (; go && s + 1 < G; s += 2) {
      if (!await(need(s + 1))) {
        lost = true;
        go = false;
        break;
      }
      if (static_cast<uint32_t>(s) >= stop) {
        go = false;
        break;
      }
      gates_for(s);
      iteration(s, bufA, bufB, wwA, rwA, wwB, rwB);
      iteration(s + 1, bufB, bufA, wwB, rwB, wwA, rwA);
    }
    if (go && s < G) {
      if (!await(need(s))) {
        lost = true;
      } else if (static_cast<uint32_t>(s) < stop) {
        gates_for(s);
        iteration(s, bufA, bufB, wwA, rwA, wwB, rwB);
      }
    }
    if (lost && lane == 0) {
      // the control wave never published (a bounded wait): record it, and
      // never hold the control wave back
      if constexpr (!DENSE) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
      if (P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);   // the bits have reached the coherent point
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    // finished: the control wave waits for this before it reports the layer
    // (and no later step of the launch waits on this wave)
    if (lane == 0) sync_store(&sync[1], kNoStop);
    return;
  }

  // ======================= control wave =======================
  int64_t tmpl = 0;
  if constexpr (!DENSE) {
    tmpl = L.template_indices[bank];
    if (tmpl < 0 || tmpl >= P.templates) {
      base_err |= COWSDM_ERR_TEMPLATE;
      tmpl = 0;
    }
  }
  const float* const m0_bank =
      DENSE ? nullptr : L.shared_initial_memory + tmpl * static_cast<int64_t>(N) * D;
  int32_t* const map_bank = DENSE ? nullptr : L.logical_to_physical + static_cast<int64_t>(bank) * N;
  int* const lds_map = MAPLDS ? lds_map_all + pair * N : nullptr;
  const char* const wi_l = first_step(L.write_indices, 0) + (static_cast<int64_t>(bank) * W + wl) * sizeof(IDX);
  const char* const ri_l = first_step(L.read_indices, 6) + (static_cast<int64_t>(bank) * R + rl_) * sizeof(IDX);
  const uint32_t st_wi = pin(static_cast<uint32_t>(P.trace_stride[0]));
  const uint32_t st_ri = pin(static_cast<uint32_t>(P.trace_stride[6]));
  const char* const wbase = first_step(L.write_indices, 0) + static_cast<int64_t>(bank) * W * sizeof(IDX);
  const char* const rbase = first_step(L.read_indices, 6) + static_cast<int64_t>(bank) * R * sizeof(IDX);
  // packed, slot map in LDS: the slots of the launch's first chunks, for the
  // plan's count part, are loaded before anything else (their round trip
  // overlaps the slot map's); chunk 0's then serve the steps too.  The
  // slots of chunks c + 1 .. c + kAhead load while chunk c is counted.
  constexpr int kAhead = sizeof(IDX) == 4 ? 2 : 1;
  IDX sbuf[kAhead + 1][kIdxRow];
  auto load_slots = [&](int c, IDX (&dst)[kIdxRow]) __attribute__((always_inline)) {
    const int t = c * kWave + lane;
    const int tc = t < G0 ? t : G0 - 1;
    const char* const w = at(wbase, st_wi, tc);
    const char* const r = at(rbase, st_ri, tc);
    if constexpr (FULL && sizeof(IDX) == 4) {
      // a step's 4 write and 16 read slots are 16 and 64 contiguous,
      // 16-byte aligned bytes: five vector loads per lane
      const i32x4_t a = *(const __attribute__((address_space(1))) i32x4_t*)(w);
      dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
#pragma unroll
      for (int k = 0; k < kTraceMaxReads / 4; ++k) {
        const i32x4_t b = *(const __attribute__((address_space(1))) i32x4_t*)(r + 16 * k);
        dst[kTraceMaxWrites + 4 * k] = b.x;
        dst[kTraceMaxWrites + 4 * k + 1] = b.y;
        dst[kTraceMaxWrites + 4 * k + 2] = b.z;
        dst[kTraceMaxWrites + 4 * k + 3] = b.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        dst[j] = *(const __attribute__((address_space(1))) IDX*)(w + (j < W ? j : W - 1) * sizeof(IDX));
      }
#pragma unroll
      for (int i = 0; i < kTraceMaxReads; ++i) {
        dst[kTraceMaxWrites + i] =
            *(const __attribute__((address_space(1))) IDX*)(r + (i < R ? i : R - 1) * sizeof(IDX));
      }
    }
  };
  if constexpr (!DENSE && MAPLDS) {
#pragma unroll
    for (int c = 0; c < kAhead; ++c) {
      if (c * kWave < G0) load_slots(c, sbuf[c]);
    }
  }
  bool any_bad = false;  // a map entry outside the slab (checked per chunk only then)
  if constexpr (MAPLDS) {
    // the bank's slot map into LDS, 4 loads in flight per lane (one memory
    // round trip for N <= 256)
    constexpr int kStage = 4;
    uint64_t bad = 0;
    for (int b = 0; b < N; b += kStage * kWave) {
      int v[kStage];
#pragma unroll
      for (int i = 0; i < kStage; ++i) {
        const int x = b + i * kWave + lane;
        v[i] = x < N ? map_bank[x] : -1;
      }
#pragma unroll
      for (int i = 0; i < kStage; ++i) {
        const int x = b + i * kWave + lane;
        if (x < N) lds_map[x] = v[i];
        bad |= __ballot(v[i] >= C);
      }
    }
    any_bad = bad != 0;
  }
  // ---- the launch's plan (packed): block, epoch, the pops that fit
  PlanBlock pb{};
  uint32_t epoch = 0;
  int fit_rows = 0;
  int found_top = 0;      // the stack height the launch found
  int plan_segs = 1;      // growth segments of the launch (1: none)
  // the launch's plan was made by this wave alone (plan_local): its plan
  // words are in LDS, its pops come straight from the found stack, and the
  // layer's last control wave writes what the launch leaves
  bool local_plan = false;
  int64_t local_proven = 0;
  bool chunk0_classified = false;   // chunk 0's class words are in LDS
  if constexpr (!DENSE) {
    pb = plan_block(P, layer_id);
    // the epoch word changes only when the layer's last control wave ends
    epoch = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(launch_epoch(pb))));
  }
  // ---- plan words (packed): every step's word of this bank, from its prefix
  // word and the step's running total, staged into LDS once the plan's header
  // is in (composed as: first touches before it | first-touch lanes << 24 |
  // stop bit 28); false when a word never arrives
  auto stage_plan = [&]() __attribute__((always_inline)) -> bool {
    bool ok = true;
    if constexpr (!DENSE) {
      if (local_plan) return true;   // staged by the local plan
      constexpr int KC = kTraceMaxSteps / kWave;
      uint64_t w[KC], c[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int t = k * kWave + lane;
        const int tc = t < G ? t : G - 1;
        if (k * kWave < G) {
          w[k] = atomic_load_u64(pb.word(bank, tc));
          c[k] = atomic_load_u64(pb.cum + tc);
        }
      }
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int t = k * kWave + lane;
        const int tc = t < G ? t : G - 1;
        if (k * kWave >= G) break;
        if (__ballot(!tag_is(w[k], epoch) || !(w[k] & kPrefixDone)) != 0) {
          ok = poll_tagged(pb.word(bank, tc), true, epoch, w[k], true) && ok;
        }
        if (__ballot(!tag_is(c[k], epoch)) != 0) {
          ok = poll_tagged(pb.cum + tc, true, epoch, c[k]) && ok;
        }
        const uint32_t v = static_cast<uint32_t>(w[k]);
        const uint32_t base = static_cast<uint32_t>(c[k]) + ((v & ~kPrefixDone) >> kPrefixShift);
        if (t < G) {
          lds_plan[pair][t] = static_cast<int>((base & kPlanBaseMask) | ((v & 15u) << kPlanMaskShift) |
                                               ((v & kCountStop) ? 1u << kPlanStopBit : 0u));
        }
      }
    }
    return ok;
  };
  auto plan_of = [&](int t) __attribute__((always_inline)) -> uint32_t {
    if constexpr (DENSE) return 0u;
    const int tc = t < G ? t : G - 1;
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lds_plan[DENSE ? 0 : pair][tc]));
  };
  // chunk c's first-touch lanes, lane l for step 64c + l
  auto chunk_fm = [&](int c) __attribute__((always_inline)) -> uint32_t {
    if constexpr (DENSE) return 0u;
    const int t = c * kWave + lane;
    return (static_cast<uint32_t>(lds_plan[DENSE ? 0 : pair][t < G ? t : G - 1]) >> kPlanMaskShift) & 15u;
  };

  // ---- this bank's pops, before its first step.  In a launch that grows,
  // the layer's last control wave to list its pops then rewrites the free
  // stack above the lowest growth: every entry the launch found there has
  // been read by then (each wave's stack loads have returned before its
  // ticket, which the high half of the layer's ticket word counts; the
  // launch's last wave to finish clears the word).
  auto list_pops = [&](bool ok) __attribute__((always_inline)) -> bool {
    if constexpr (DENSE || MAPLDS) {
      return ok;   // dense, or the planner listed them
    } else {
      if (ok) {
        ok = list_bank_pops(pb, epoch, plan_segs, found_top, G, fit_rows, &lds_plan[pair][0],
                            lds_seg, L.free_rows);
      }
      if (plan_segs > 1) {
        int64_t listed = 0;
        if (lane == 0) {
          listed = __hip_atomic_fetch_add(P.trace_ticket + 1 + layer_id, int64_t{1} << 32,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (__builtin_amdgcn_readfirstlane(static_cast<int>(listed >> 32)) == B - 1 && ok) {
          rewrite_stack(lds_seg, plan_segs, C, fit_rows, const_cast<int32_t*>(L.free_rows));
        }
      }
      return ok;
    }
  };

  // ---- this lane's slots at the launch's first step; step t adds t * stride

  // ---- stages
  auto load_idx = [&](int t, TraceIdx& m) __attribute__((always_inline)) {
    const int tc = t < G ? t : G - 1;
    const int64_t xw = static_cast<int64_t>(*(const __attribute__((address_space(1))) IDX*)(at(wi_l, st_wi, tc)));
    const int64_t xr = static_cast<int64_t>(*(const __attribute__((address_space(1))) IDX*)(at(ri_l, st_ri, tc)));
    const bool bw = xw < 0 || xw >= N;
    const bool br = xr < 0 || xr >= N;
    m.err = (lane < W && bw ? COWSDM_ERR_WRITE_INDEX : 0) | (lane < R && br ? COWSDM_ERR_READ_INDEX : 0);
    m.widx = (lane < W && !bw) ? static_cast<int>(xw) : 0;
    m.ridx = (lane < R && !br) ? static_cast<int>(xr) : 0;
  };

  // Map in LDS (or dense): the slots reach the wave through LDS, 64 steps at
  // a time.  Lane l loads step 64c + l of chunk c into registers a chunk
  // ahead and writes it to LDS when the chunk before starts being used, so
  // vector memory is waited on once per 64 steps instead of every step (it
  // completes in order, so a per-step wait would also wait for every claim
  // and device-scope store issued before it).
  IDX chunk[kIdxRow];
#pragma unroll
  for (int k = 0; k < kIdxRow; ++k) chunk[k] = 0;
  auto load_chunk = [&](int c) __attribute__((always_inline)) {
    const int st = c * kWave + lane < G ? c * kWave + lane : G - 1;
    const char* const w = at(wbase, st_wi, st);
    const char* const r = at(rbase, st_ri, st);
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      chunk[j] = *(const __attribute__((address_space(1))) IDX*)(w + (j < W ? j : 0) * sizeof(IDX));
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      chunk[kTraceMaxWrites + i] =
          *(const __attribute__((address_space(1))) IDX*)(r + (i < R ? i : 0) * sizeof(IDX));
    }
  };
  // Chunk c's slots and class words, lane l for step t = 64c + l: the step's
  // classification, done here for 64 steps at once with plain per-lane
  // compares instead of per step with cross-lane reads (slot values past W
  // or R take no part; an invalid slot compares as slot 0, as the per-step
  // path reads it):
  //   word 0: bits 0-19 rows from step t-1 (write lanes 0-3, read lanes
  //           4-19), 20-23 first touches (fm: lane l's first-touch mask from
  //           the launch's plan), 24-31 the COWSDM_ERR_* bits of its routes
  //   word 1: bits 0-15 reads of a slot step t writes, 16-19 and 20-23 the
  //           two bit planes of each write lane's source lane in step t-1
  //   words 2, 3: the planes of each read lane's source lane in step t-1 and
  //           in step t (read-after-write)
  // (Source planes are zero when the step forwards nothing; lanes without a
  // source have both plane bits set.)
  auto write_chunk = [&](int c, uint32_t fm) __attribute__((always_inline)) {
    int v[kIdxRow];
#pragma unroll
    for (int k = 0; k < kIdxRow; ++k) {
      const int64_t x = static_cast<int64_t>(chunk[k]);
      v[k] = x >= 0 && x < N ? static_cast<int>(x) : -1;
    }
    int (*const buf)[kWave][kIdxLds] = lds_idx[(DENSE || MAPLDS) ? pair : 0];
    // write slots: this step's and step t-1's (lane 0: the last step of
    // chunk c-1, or none before step 0), invalid ones as slot 0, -1 past W
    int w[kTraceMaxWrites], pw[kTraceMaxWrites];
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      w[j] = j < W ? (v[j] < 0 ? 0 : v[j]) : -1;
      int up = __shfl_up(w[j], 1, kWave);
      if (lane == 0) {
        const int last = c > 0 ? buf[(c - 1) & 1][kWave - 1][j] : -2;
        up = c > 0 && j < W ? (last < 0 ? 0 : last) : -2;
      }
      pw[j] = up;
    }
    int err = 0;
    bool dup = false;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W && v[j] < 0) err |= COWSDM_ERR_WRITE_INDEX;
#pragma unroll
      for (int k = j + 1; k < kTraceMaxWrites; ++k) dup |= k < W && w[k] == w[j];
    }
    uint32_t fwd = 0, w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      int src = -1;
#pragma unroll
      for (int k = 0; k < kTraceMaxWrites; ++k) src = w[j] >= 0 && w[j] == pw[k] ? k : src;
      fwd |= (src >= 0 ? 1u : 0u) << j;
      w0 |= static_cast<uint32_t>(src & 1) << j;
      w1 |= static_cast<uint32_t>((src >> 1) & 1) << j;
    }
    uint32_t rawm = 0, f0 = 0, f1 = 0, a0 = 0, a1 = 0;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      const int x = i < R ? (v[kTraceMaxWrites + i] < 0 ? 0 : v[kTraceMaxWrites + i]) : -3;
      if (i < R && v[kTraceMaxWrites + i] < 0) err |= COWSDM_ERR_READ_INDEX;
      int raw = -1, src = -1;
#pragma unroll
      for (int k = 0; k < kTraceMaxWrites; ++k) {
        raw = x == w[k] ? k : raw;
        src = x == pw[k] ? k : src;
      }
      if (raw >= 0) src = -1;
      rawm |= (raw >= 0 ? 1u : 0u) << i;
      fwd |= (src >= 0 ? 1u : 0u) << (kTraceMaxWrites + i);
      f0 |= static_cast<uint32_t>(src & 1) << i;
      f1 |= static_cast<uint32_t>((src >> 1) & 1) << i;
      a0 |= static_cast<uint32_t>(raw & 1) << i;
      a1 |= static_cast<uint32_t>((raw >> 1) & 1) << i;
      if constexpr (MAPLDS) {
        // a map entry outside the slab (only one present at launch start can be)
        if (any_bad && i < R) bad |= lds_map[x] >= C;
      }
    }
    if constexpr (MAPLDS) {
      if (any_bad) {
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          if (j < W) bad |= lds_map[w[j]] >= C;
        }
      }
    }
    if (dup) err |= COWSDM_ERR_DUP_WRITE;
    if (bad) err |= COWSDM_ERR_CORRUPT;
    const bool planes = (fwd | rawm) != 0;
    i32x4_t q[kIdxLds / 4];
#pragma unroll
    for (int k = 0; k < kIdxRow / 4; ++k) {
      q[k].x = v[4 * k]; q[k].y = v[4 * k + 1]; q[k].z = v[4 * k + 2]; q[k].w = v[4 * k + 3];
    }
    q[kIdxRow / 4].x = static_cast<int>(fwd | (fm << 20) | (static_cast<uint32_t>(err) << 24));
    q[kIdxRow / 4].y = static_cast<int>(rawm | (planes ? (w0 << 16) | (w1 << 20) : 0u));
    q[kIdxRow / 4].z = static_cast<int>(planes ? f0 | (f1 << 16) : 0u);
    q[kIdxRow / 4].w = static_cast<int>(planes ? a0 | (a1 << 16) : 0u);
    i32x4_t* const row = reinterpret_cast<i32x4_t*>(&buf[c & 1][lane][0]);
#pragma unroll
    for (int k = 0; k < kIdxLds / 4; ++k) row[k] = q[k];
  };
  auto idx_row = [&](int t) __attribute__((always_inline)) -> const int* {
    const int tc = t < G ? t : G - 1;
    return &lds_idx[(DENSE || MAPLDS) ? pair : 0][(tc >> 6) & 1][tc & (kWave - 1)][0];
  };
  auto read_idx = [&](int t, TraceIdx& m) __attribute__((always_inline)) {
    const int* const row = idx_row(t);
    const int xw = row[lane < kTraceMaxWrites ? lane : 0];
    const int xr = row[kTraceMaxWrites + (lane < kTraceMaxReads ? lane : 0)];
    const u32x4_t k = *reinterpret_cast<const u32x4_t*>(row + kIdxRow);
    m.err = (lane < W && xw < 0 ? COWSDM_ERR_WRITE_INDEX : 0) | (lane < R && xr < 0 ? COWSDM_ERR_READ_INDEX : 0);
    m.widx = lane < W && xw >= 0 ? xw : 0;
    m.ridx = lane < R && xr >= 0 ? xr : 0;
    m.k0 = static_cast<int>(k.x);
    m.k1 = static_cast<int>(k.y);
  };

  auto issue_map = [&](const TraceIdx& m, int& wraw, int& rraw) __attribute__((always_inline)) {
    wraw = -1;
    rraw = -1;
    if constexpr (!DENSE) {
      const __attribute__((address_space(1))) int32_t* map_g =
          (const __attribute__((address_space(1))) int32_t*)(map_bank);
      const int a = map_g[m.widx];
      const int c = map_g[m.ridx];
      wraw = lane < W ? a : -1;
      rraw = lane < R ? c : -1;
    }
  };

  // Step t from its slots and map entries.  r1: step t-1 (classified), r2:
  // step t-2 (its first touches popped).  Returns the read lane's row.
  // Lanes past W (R) hold slot 0 as their write (read) slot: they compute
  // along, and their results are masked once at the end.
  auto classify = [&](int t, const TraceIdx& m, int wraw, int rraw, TraceRoute& rt,
                      const TraceRoute& r1, const TraceRoute& r2, bool ok_prev)
      __attribute__((always_inline)) -> int {
    if constexpr (MAPLDS) {
      // every step up to t-2 has stored its pops here; read first, so that
      // the matching below covers the LDS latency
      wraw = lds_map[m.widx];
      rraw = lds_map[m.ridx];
    }
    if constexpr (DENSE || MAPLDS) {
      // staged slots: the chunk's pass classified the step (class words)
      const uint32_t k0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(m.k0));
      const uint32_t k1 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(m.k1));
      const int e = static_cast<int>(k0 >> 24) | base_err;
      if (!DENSE && e != 0 && t < G) {
        if (lane == 0) {
          __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(e),
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if constexpr (!DENSE) {
        // an entry outside the slab (reported above) reads as shared
        wraw = wraw >= C ? -1 : wraw;
        rraw = rraw >= C ? -1 : rraw;
      }
      // the plan stops the bank from its first step with an invalid route
      const uint32_t pw = plan_of(t);
      const bool ok = ok_prev && e == 0 && ((pw >> kPlanStopBit) & 1u) == 0;
      const uint32_t fwd = k0 & 0xFFFFFu;
      const uint32_t fm = DENSE || !ok ? 0u : (k0 >> 20) & 15u;
      rt.u = fm | (static_cast<uint32_t>(__popc(fm)) << 4) | (ok ? 1u << 8 : 0u);
      rt.base = static_cast<int>(pw & kPlanBaseMask);
      rt.fwd = fwd;
      rt.rawm = k1 & 0xFFFFu;
      rt.rank = lanes_below(fm);
      rt.widx = m.widx;
      rt.ridx = m.ridx;
      rt.wrow = lane < W ? wraw : -1;
      rt.wsrc = lane < W && ((fwd >> (lane & 3)) & 1u) != 0
                    ? plane_code(k1, 16 + (lane & 3), 20 + (lane & 3)) : -1;
      rt.rsrc = -1;   // (the read lanes' sources reach the data wave as class words)
      rt.rraw = -1;
      return lane < R ? rraw : -1;
    }
    int wsrc = -1, rsrc = -1, rraw_lane = -1;
    uint64_t dup = 0;
    // write j's slot, or -1 (no slot) past W: every row runs without a branch
    auto wslot = [&](int x, int j) __attribute__((always_inline)) -> int {
      return j < W ? rl(x, j) : -1;
    };
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      const int sj = wslot(m.widx, j);
      // a write lane above j with the same slot
      dup |= __ballot(m.widx == sj) & wlanes & ~((2ull << j) - 1);
      if (m.ridx == sj) rraw_lane = j;
    }
    if (t >= 1) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        const int sj = wslot(r1.widx, j);
        if (m.widx == sj) wsrc = j;
        if (m.ridx == sj) rsrc = j;
      }
    }
    if (rraw_lane >= 0) rsrc = -1;
    uint64_t bad = 0;  // map entries outside the slab
    if constexpr (!DENSE) {
      bad = (__ballot(wraw >= C) & wlanes) | (__ballot(rraw >= C) & rlanes);
      if (bad != 0) {
        // rare: report, and treat the entry as shared
        wraw = wraw >= C ? -1 : wraw;
        rraw = rraw >= C ? -1 : rraw;
      }
    }
    if (!DENSE && !MAPLDS && t >= 2) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        const int sj = wslot(r2.widx, j);
        const int row = rl(r2.wrow, j);
        if (wsrc < 0 && m.widx == sj) wraw = row;
        if (rsrc < 0 && m.ridx == sj) rraw = row;
      }
    }
    const bool any_err = (__ballot((m.err | base_err) != 0) | dup | bad) != 0;
    if (!DENSE && any_err && t < G) {
      int lerr = m.err | base_err;
      if (lane == 0) {
        lerr |= (dup != 0 ? COWSDM_ERR_DUP_WRITE : 0) | (bad != 0 ? COWSDM_ERR_CORRUPT : 0);
      }
      const int e = wave_or(lerr);
      if (lane == 0) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(e),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    const uint32_t pw = plan_of(t);
    bool ok = ok_prev && !any_err && ((pw >> kPlanStopBit) & 1u) == 0;
    uint64_t fm = DENSE || !ok ? 0ull : __ballot(wsrc < 0 && wraw < 0) & wlanes;
    if (!DENSE && ok && static_cast<uint32_t>(fm) != ((pw >> kPlanMaskShift) & 15u)) {
      // the plan counted other first touches: the state changed under the
      // launch; stop the bank rather than pop rows meant for others
      if (lane == 0 && t < G) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
      ok = false;
      fm = 0;
    }
    rt.u = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(fm & 15u) | (static_cast<uint32_t>(__popcll(fm)) << 4) |
        (ok ? 1u << 8 : 0u));
    rt.base = static_cast<int>(pw & kPlanBaseMask);
    rt.fwd = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(__ballot(wsrc >= 0) & wlanes) |
        (static_cast<uint32_t>(__ballot(rsrc >= 0) & rlanes) << kTraceMaxWrites));
    rt.rawm = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(__ballot(rraw_lane >= 0) & rlanes));
    rt.rank = lanes_below(fm);
    rt.widx = m.widx;
    rt.ridx = m.ridx;
    rt.wrow = lane < W ? wraw : -1;
    rt.wsrc = lane < W ? wsrc : -1;
    rt.rsrc = lane < R ? rsrc : -1;
    rt.rraw = lane < R ? rraw_lane : -1;
    // past R the lane loads the zero row, never a slab row that the
    // bad-entry check above did not cover
    return lane < R ? rraw : -1;
  };

  // Publish step t's row addresses: lane j's write row and read row.
  // Lane j's write row and read row of a step (M0 row or slab row).
  auto row_addrs = [&](const TraceRoute& rt, int rrow, const float*& wp, const float*& rp)
      __attribute__((always_inline)) {
    // row r of a base: base + r * D floats, r non-negative
    auto row_at = [&](const float* base, int r) __attribute__((always_inline)) -> const float* {
      return reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) +
                                            static_cast<uint64_t>(static_cast<uint32_t>(r)) * row_bytes);
    };
    if constexpr (DENSE) {
      wp = row_at(table_bank, rt.widx);
      rp = row_at(table_bank, rt.ridx);
    } else {
      wp = rt.wrow < 0 ? row_at(m0_bank, rt.widx) : row_at(slab, rt.wrow);
      rp = rrow < 0 ? row_at(m0_bank, rt.ridx) : row_at(slab, rrow);
    }
    if constexpr (!FULL) {
      if (lane >= R) rp = kTraceZeroRow;
    }
  };
  // Publish step t's row addresses (the prologue's steps).
  auto publish_rows = [&](int t, const TraceRoute& rt, int rrow) __attribute__((always_inline)) {
    const float* wp;
    const float* rp;
    row_addrs(rt, rrow, wp, rp);
    TraceSlot& sl = slot_of(t);
    if (lane < kTraceMaxReads) {
      sl.wptr[lane] = reinterpret_cast<uint64_t>(wp);
      sl.rptr[lane] = reinterpret_cast<uint64_t>(rp);
    }
  };

  // End of iteration s: publish step s+2's row addresses (rc, rrow), step
  // s's store rows and masks (rt; run: it runs, fitted: its first touches
  // got rows) and the progress word, in one store pass of lanes 0-15 and one
  // of lane 0.  The source-row planes of forwarded rows are only built for a
  // step that forwards some.
  // kq: step s's class words (map in LDS, or dense), read at the start of
  // the iteration: the release store below waits for every LDS access anyway
  auto publish = [&](int s, const TraceRoute& rt, bool run, bool fitted, const TraceRoute& rc,
                     int rrow, const u32x4_t& kq) __attribute__((always_inline)) {
    const float* wp;
    const float* rp;
    row_addrs(rc, rrow, wp, rp);
    const uint32_t fm = route_fmask(rt.u);
    const uint32_t smask = run ? ((static_cast<uint32_t>(wlanes) & ~fm) | (fitted ? fm : 0u)) : 0u;
    const int drow = DENSE ? rt.widx : (rt.wrow < 0 ? 0 : rt.wrow);
    u32x4_t c;
    c.x = rt.fwd | (run ? 1u << 20 : 0u) | (smask << 24);
    c.y = rt.rawm;
    c.z = 0;
    c.w = 0;
    if constexpr (DENSE || MAPLDS) {
      // the source planes were built with the chunk (class words 1-3)
      c.y = kq.y;
      c.z = kq.z;
      c.w = kq.w;
    } else if ((rt.fwd | rt.rawm) != 0) {
      const uint32_t w0 = static_cast<uint32_t>(__ballot((rt.wsrc & 1) != 0)) & 15u;
      const uint32_t w1 = static_cast<uint32_t>(__ballot((rt.wsrc & 2) != 0)) & 15u;
      const uint32_t f0 = static_cast<uint32_t>(__ballot((rt.rsrc & 1) != 0)) & 0xFFFFu;
      const uint32_t f1 = static_cast<uint32_t>(__ballot((rt.rsrc & 2) != 0)) & 0xFFFFu;
      const uint32_t a0 = static_cast<uint32_t>(__ballot((rt.rraw & 1) != 0)) & 0xFFFFu;
      const uint32_t a1 = static_cast<uint32_t>(__ballot((rt.rraw & 2) != 0)) & 0xFFFFu;
      c.y |= (w0 << 16) | (w1 << 20);
      c.z = f0 | (f1 << 16);
      c.w = a0 | (a1 << 16);
    }
    TraceSlot& ahead = slot_of(s + 2);
    TraceSlot& now = slot_of(s);
    if (lane < kTraceMaxReads) {
      ahead.wptr[lane] = reinterpret_cast<uint64_t>(wp);
      ahead.rptr[lane] = reinterpret_cast<uint64_t>(rp);
      now.drow[lane] = drow;
    }
    if (lane == 0) {
      *reinterpret_cast<u32x4_t*>(now.ctl) = c;
      sync_store(&sync[0], (kNoStop << 16) | static_cast<uint32_t>(s + 2));
    }
  };

  // ---- pops (packed)
  bool alive = true;  // every step of this bank so far got its rows

  // Step t's first touches take their rows from the plan's pop list: write
  // lane j, of rank k among the step's first touches, loads pop base + k when
  // the step is classified, and the row is used two iterations later, when
  // the step resolves.  A step whose pops reach past the rows the plan could
  // give out (a capacity proof that was missing or not honest) overflows: it
  // takes none, and the bank stops.  After a local plan (no growth) pop q is
  // the found stack's entry found_top - 1 - q, loaded from the stack itself.
  auto claim = [&](const TraceRoute& rt, uint64_t& home) __attribute__((always_inline)) {
    if constexpr (!DENSE) {
      const int count = route_count(rt.u);
      if (count > 0 && route_ok(rt.u) && rt.base + count <= fit_rows) {
        const bool first = lane < kTraceMaxWrites && ((route_fmask(rt.u) >> lane) & 1u);
        if (first) {
          home = local_plan
                     ? static_cast<uint64_t>(static_cast<uint32_t>(
                           L.free_rows[found_top - 1 - (rt.base + rt.rank)]))
                     : atomic_load_u64(pb.pops + rt.base + rt.rank);
        }
      }
    }
  };

  // Step t's first touches, from the rows loaded for them (home: lane j holds
  // write j's pop word, tagged with the epoch once the plan wrote it).  r1:
  // step t+1, whose rewrites of step t's slots take its physical rows.
  auto resolve = [&](int t, TraceRoute& rt, TraceRoute& r1, uint64_t home)
      __attribute__((always_inline)) {
    const int count = route_count(rt.u);
    if (count > 0 && route_ok(rt.u) && alive) {
      const uint32_t fmask = route_fmask(rt.u);
      bool fits = rt.base + count <= fit_rows;
      if (fits) {
        const bool first = lane < kTraceMaxWrites && ((fmask >> lane) & 1u);
        if (!local_plan && __ballot(first && !tag_is(home, epoch)) != 0) {
          // rare: the pop was loaded before it arrived
          if (!poll_tagged(pb.pops + rt.base + rt.rank, first, epoch, home)) {
            if (lane == 0) {
              __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                                    static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
            }
            home = tagged(epoch, 0xFFFFFFFFu);
          }
        }
        const int new_row = first ? static_cast<int>(static_cast<uint32_t>(home)) : -1;
        if (__ballot(first && (new_row < 0 || new_row >= C)) != 0) {
          fits = false;
          if (lane == 0) {
            __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                                  static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
          }
        } else if (first) {
          rt.wrow = new_row;
          map_bank[rt.widx] = new_row;
          if constexpr (MAPLDS) lds_map[rt.widx] = new_row;
        }
      }
      // an overflow stops the bank (the plan set the overflow flag)
      alive = fits;
    }
    // step t+1 rewrites some of step t's slots in the rows just found
    if ((r1.fwd & ((1u << kTraceMaxWrites) - 1)) != 0) {
      const int s1 = r1.wsrc;
      const int v1 = __shfl(rt.wrow, s1 >= 0 ? s1 : 0, kWave);
      if (s1 >= 0) r1.wrow = v1;
    }
  };

  // After classifying step t: load the rows its first touches pop.
  auto after_classify = [&](int t, const TraceRoute& rt, uint64_t& home) __attribute__((always_inline)) {
    if constexpr (!DENSE) {
      if (t < G) claim(rt, home);
    }
  };

  // the data wave has finished `need` steps, so the ring slots the next
  // steps reuse are free; false if it never does.  Iteration u overwrites
  // the addresses of step u+2-K and the masks of step u-K, which the data
  // wave has read once it finished step u+2-K (it reads step 0's addresses
  // before its first step): iteration u needs u+3-K steps finished.
  uint32_t dseen = 0;
  auto room = [&](int need) __attribute__((always_inline)) -> bool {
    if (need <= 0 || dseen >= static_cast<uint32_t>(need)) return true;
    for (int spins = 0; spins < kSpinLimit; ++spins) {
      dseen = sync_load(&sync[1]);
      if (dseen >= static_cast<uint32_t>(need)) return true;
      __builtin_amdgcn_s_sleep(1);
    }
    return false;
  };

  // ---- the launch's plan (packed; trace_plan.h), before any step
  if constexpr (!DENSE) {
    bool ok = true;
    PlanControl pc{};
    // a short launch tries the local plan first (the data wave makes it)
    const bool local_try = MAPLDS && local_plan_fits(G0, B, pb);
    if (bank == 0) pc = plan_control(P, layer_id);
    if constexpr (MAPLDS) {
      // count part: this bank's first touches, step by step.  A slot is
      // first-touched by the launch's first step that writes it, unless it
      // was mapped at launch start: one LDS minimum per write slot over all
      // steps (lane = step, 64 steps a round) gives that step.  A step with
      // an invalid route stops the bank from there on.
      int* const first_write = lds_map_all + NB * N + pair * N;
      for (int k = lane; k < N; k += kWave) first_write[k] = 0x7fffffff;
      constexpr int KC = kTraceMaxSteps / kWave;
      int wsl[KC][kTraceMaxWrites];   // write slots (-1: none) of step 64c + lane
      uint32_t mapped[KC];
      int err_step = (base_err & COWSDM_ERR_TEMPLATE) ? 0 : G0;
      int err_bits[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int t = c * kWave + lane;
        mapped[c] = 0;
        err_bits[c] = 0;
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) wsl[c][j] = -1;
        if (c * kWave >= G0) continue;
        if ((c + kAhead) * kWave < G0) load_slots(c + kAhead, sbuf[(c + kAhead) % (kAhead + 1)]);
        const IDX (&cur)[kIdxRow] = sbuf[c % (kAhead + 1)];
        int e = 0;
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          if (j < W) {
            const int64_t v = static_cast<int64_t>(cur[j]);
            if (v < 0 || v >= N) {
              e |= COWSDM_ERR_WRITE_INDEX;
            } else {
              wsl[c][j] = static_cast<int>(v);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < kTraceMaxReads; ++i) {
          if (i < R) {
            const int64_t v = static_cast<int64_t>(cur[kTraceMaxWrites + i]);
            if (v < 0 || v >= N) {
              e |= COWSDM_ERR_READ_INDEX;
            } else if (any_bad && lds_map[v] >= C0) {
              e |= COWSDM_ERR_CORRUPT;
            }
          }
        }
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
#pragma unroll
          for (int i = j + 1; i < kTraceMaxWrites; ++i) {
            if (wsl[c][j] >= 0 && wsl[c][j] == wsl[c][i]) e |= COWSDM_ERR_DUP_WRITE;
          }
          const int x = wsl[c][j];
          if (x >= 0) {
            const int m = lds_map[x];
            if (m >= C0) e |= COWSDM_ERR_CORRUPT;
            if (m >= 0) mapped[c] |= 1u << j;
            if (t < G0) {
              __hip_atomic_fetch_min(&first_write[x], t, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP);
            }
          }
        }
        if (t < G0 && e != 0) {
          err_bits[c] = e;
          err_step = t < err_step ? t : err_step;
        }
        if (c == 0) {
          // chunk 0's slots serve the steps too (the prologue's chunk)
#pragma unroll
          for (int k = 0; k < kIdxRow; ++k) chunk[k] = cur[k];
        }
      }
      // the bank's first invalid step (a ballot per chunk: lane = step) and
      // its errors
      {
        int first_bad = (base_err & COWSDM_ERR_TEMPLATE) ? 0 : G0;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          if (c * kWave < G0) {
            const uint64_t m = __ballot(err_bits[c] != 0);
            if (m != 0) {
              const int t = c * kWave + static_cast<int>(__builtin_ctzll(m));
              first_bad = t < first_bad ? t : first_bad;
            }
          }
        }
        err_step = first_bad;
      }
      int bits = 0;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        if (c * kWave < G0 && err_step < G0 && (err_step >> 6) == c) {
          bits = __builtin_amdgcn_readlane(err_bits[c], err_step & (kWave - 1));
        }
      }
      // one wave's LDS accesses apply in issue order: keep the reads after
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      uint32_t count0 = 0;   // lane t < 64: step t's count word
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int t = c * kWave + lane;
        if (c * kWave >= G0 || t >= G0) continue;
        uint32_t mask = 0;
        if (t < err_step) {
#pragma unroll
          for (int j = 0; j < kTraceMaxWrites; ++j) {
            const int x = wsl[c][j];
            if (x >= 0 && !((mapped[c] >> j) & 1u) && first_write[x] == t) mask |= 1u << j;
          }
        }
        const uint32_t word = mask | (t >= err_step ? kCountStop : 0u);
        if (c == 0) count0 = word;
        atomic_store_u64(pb.word(bank, t), tagged(epoch, word));
      }
      if (local_try) {
        // the same words packed for the local plan, kLocalStepsPerWord steps
        // per word, into the plan block's local rows
        uint32_t packed = 0;
#pragma unroll
        for (int k = 0; k < kLocalWords; ++k) {
          uint32_t v = 0;
#pragma unroll
          for (int i = 0; i < kLocalStepsPerWord; ++i) {
            const int t = k * kLocalStepsPerWord + i;
            if (t < kLocalPlanSteps && t < G0) {
              v |= static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(count0), t))
                   << (kLocalBits * i);
            }
          }
          if (lane == k) packed = v;
        }
        if (lane < local_words(G0)) {
          atomic_store_u64(local_word(pb, bank, lane), tagged(epoch, packed));
        }
        // chunk 0's class words while the data wave makes the local plan:
        // the first-touch lanes are this bank's own count words' (the plan
        // adds only where the rows come from)
        write_chunk(0, count0 & 15u);
        chunk0_classified = true;
      }
      if (lane == 0 && bits != 0) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(bits),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    PlanHeader head{0, 0, C0, 0, 1};
    int local = 0;
    if constexpr (MAPLDS) {
      if (local_try) {
        // the data wave's local plan (bounded wait)
        uint32_t r = 0;
        for (int spins = 0; spins < 64 * kSpinLimit && r == 0; ++spins) {
          r = sync_load(&sync[3]);
          if (r == 0) __builtin_amdgcn_s_sleep(1);
        }
        local = r == 0 ? -1 : static_cast<int>(r) - 2;
        if (local > 0) {
          head.steps = G0;
          head.fit = static_cast<int>(lds_local[pair][0]);
          head.found = static_cast<int>(lds_local[pair][1]);
          local_plan = true;
          local_proven = lds_local[pair][2];
        } else if (local < 0) {
          ok = false;
        }
      }
    }
    if (local == 0) {
      // the central plan: prefix part (a contiguous share of the steps per
      // bank), the layer part (bank 0), the header
      {
        const int per = (G0 + B - 1) / B;
        const int t0 = bank * per < G0 ? bank * per : G0;
        ok = plan_prefix(pb, B, epoch, t0, t0 + per < G0 ? t0 + per : G0);
      }
      if (bank == 0) {
        // slot maps in LDS: the planner lists the pops (its segments in the
        // chunk slots' LDS, unused until the steps start); else every bank
        // lists its own
        ok = plan_layer<!MAPLDS>(P, layer_id, pb, B, G0, epoch,
                                 MAPLDS ? &lds_idx[0][0][0][0] : &lds_seg[0], &lds_plan[pair][0],
                                 pc) && ok;
      }
      ok = plan_header<!MAPLDS>(pb, epoch, head) && ok;
    }
    int steps = head.steps, fit = head.fit, capacity = head.capacity;
    if (!ok) {
      if (lane == 0) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
        if (P.trace_status) {
          __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      steps = 0;
    }
    G = steps < G0 ? steps : G0;
    fit_rows = fit;
    plan_segs = ok ? head.segments : 1;
    found_top = head.found;   // BANKS_LIST, or a local plan
    C = pin(capacity);
    if (lane == 0) sync_store(&sync[2], kPlanReady | static_cast<uint32_t>(G));
  }

  int done_steps = G;
  if (G > 0) {
  // ---- prologue: steps 0 and 1 classified, their pops loaded and their rows
  // published
  TraceIdx idxA, idxB, ready1, ready2;
  int mwA = -1, mrA = -1, mwB = -1, mrB = -1;
  uint64_t popA = 0, popB = 0;     // pops in flight, homed by the parity of their step
  TraceRoute q, rA, rB;            // steps s and s+1 at the start of iteration s
  q.widx = 0; q.ridx = 0; q.base = 0; q.wrow = -1; q.wsrc = -1; q.rsrc = -1; q.rraw = -1;
  q.rank = 0; q.u = 0; q.fwd = 0; q.rawm = 0;
  // (packed with the map in LDS: chunk 0 was loaded for the plan's count,
  // and for a short launch classified beside the local plan: again here
  // after a central plan whose planner used this LDS, or whose growth
  // changed the capacity the class words check map entries against)
  if constexpr (DENSE) load_chunk(0);
  bool plan_ok = list_pops(stage_plan());
  if constexpr (DENSE || MAPLDS) {
    if (!chunk0_classified || (!local_plan && (bank == 0 || C != C0))) {
      write_chunk(0, chunk_fm(0));
    }
    if (G > kWave) load_chunk(1);  // written before step 64 is read
  }
  {
    TraceIdx i0, i1;
    if constexpr (DENSE || MAPLDS) {
      read_idx(0, i0);
      read_idx(1, i1);
    } else {
      load_idx(0, i0);
      load_idx(1, i1);
    }
    int mw0, mr0, mw1, mr1;
    issue_map(i0, mw0, mr0);
    issue_map(i1, mw1, mr1);
    const int rrow0 = classify(0, i0, mw0, mr0, rA, q, q, true);
    after_classify(0, rA, popA);
    publish_rows(0, rA, rrow0);
    const int rrow1 = classify(1, i1, mw1, mr1, rB, rA, q, route_ok(rA.u));
    after_classify(1, rB, popB);
    publish_rows(1, rB, rrow1);
  }
  if (lane == 0) sync_store(&sync[0], (kNoStop << 16) | 1u);
  if constexpr (DENSE || MAPLDS) {
    read_idx(2, idxB);             // classified in iteration 0
  } else {
    load_idx(2, ready1);           // its map entries, classified in iteration 0
    issue_map(ready1, mwB, mrB);
    load_idx(3, idxB);             // its map entries are loaded in iteration 0
  }

  // Iteration s: resolves step s (claimed two iterations before), classifies
  // and claims step s+2 and publishes its rows, publishes step s's masks.
  // Step s+2's map lookups see every pop up to step s (in LDS; the global
  // map's entries, loaded earlier, take step s's pops from its route), and
  // its slots written at step s+1 take their rows from that step.  `self`
  // homes are written now and read in iteration s+1 (claims: s+2), `other`
  // homes were written in iteration s-1 and are read now.
  auto iteration = [&](int s, TraceIdx& idx_self, TraceIdx& idx_other, int& mw_self, int& mr_self,
                       int& mw_other, int& mr_other, uint64_t& pop)
      __attribute__((always_inline)) {
    u32x4_t kq = {0u, 0u, 0u, 0u};
    if constexpr (DENSE || MAPLDS) kq = *reinterpret_cast<const u32x4_t*>(idx_row(s) + kIdxRow);
    const bool run = route_ok(rA.u) && alive;
    if constexpr (!DENSE) resolve(s, rA, rB, pop);
    TraceRoute rC;
    int rrow;
    if constexpr (DENSE || MAPLDS) {
      read_idx(s + 3, idx_self);
      rrow = classify(s + 2, idx_other, -1, -1, rC, rB, rA, route_ok(rB.u));
      after_classify(s + 2, rC, pop);
    } else {
      load_idx(s + 4, idx_self);
      issue_map(idx_other, mw_self, mr_self);   // step s+3
      ready2 = idx_other;
      rrow = classify(s + 2, ready1, mw_other, mr_other, rC, rB, rA, route_ok(rB.u));
      after_classify(s + 2, rC, pop);
      ready1 = ready2;
    }
    publish(s, rA, run, alive, rC, rrow, kq);
    rA = rB;
    rB = rC;
  };
  // Drain the prologue's loads (see the data wave).
  __builtin_amdgcn_s_waitcnt(0);

  int s = 0;
  bool stopped = false;
  // the data wave stopped taking steps (a bounded wait ran out): record it
  auto lost = [&]() __attribute__((always_inline)) {
    if (lane == 0) {
      if constexpr (!DENSE) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
      if (P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  };
  for (; s + 1 < G; s += 2) {
    if (!room(s + 4 - kTraceRing)) {
      lost();
      done_steps = s;
      stopped = true;
      break;
    }
    // chunk c's first slots are read in iteration 64c - 2; the buffer they
    // replace held chunk c - 2, whose last step was read long before
    if constexpr (DENSE || MAPLDS) {
      if (((s + 4) & (kWave - 1)) == 0 && s + 4 < G) {
        const int c = (s + 4) >> 6;
        write_chunk(c, chunk_fm(c));
        if ((c + 1) * kWave < G) load_chunk(c + 1);
      }
    }
    iteration(s, idxA, idxB, mwA, mrA, mwB, mrB, popA);
    iteration(s + 1, idxB, idxA, mwB, mrB, mwA, mrA, popB);
  }
  if (!stopped && s < G) {
    if (!room(s + 3 - kTraceRing)) {
      lost();
      done_steps = s;
      stopped = true;
    } else {
      iteration(s, idxA, idxB, mwA, mrA, mwB, mrB, popA);
    }
  }
  // the data wave computes the steps before done_steps, and no more
  if (stopped && lane == 0) {
    sync_store(&sync[0], (static_cast<uint32_t>(done_steps) << 16) | kNoStop);
  }
  if (!plan_ok) lost();   // a plan word never arrived: its steps took no rows
  } else {
    list_pops(true);        // no steps: the count of control waves that listed
  }

  // ---- the layer's last control wave to finish advances the layer's device
  // counter and (packed) the plan's epoch.  Every wave of the layer read both
  // before taking its ticket.  The data waves' row stores need no ordering
  // here: the next launch on the stream starts after this one has ended.
  // With a report to write, each control wave first waits for its data wave
  // to finish, so that the last ticket follows every status bit of the layer.
  if (!DENSE || P.trace_step) {
    // a first step the caller gave that the counter does not hold: the
    // launch ran the wrong steps (the counter is still the launch's: only
    // the layer's last wave advances it, after every ticket)
    if (known_first && bank == 0 && lane == 0 &&
        __hip_atomic_load(P.trace_step + layer_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
            P.trace_known) {
      if (P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if constexpr (!DENSE) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_TRACE_RANGE), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (P.report) {
      bool finished = false;
      for (int spins = 0; spins < 64 * kSpinLimit && !finished; ++spins) {
        finished = sync_load(&sync[1]) == kNoStop;
        if (!finished) __builtin_amdgcn_s_sleep(1);
      }
      if (!finished && lane == 0 && P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{COWSDM_TRACE_FAULT},
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // The status bits and control words are device-scope atomics, which
    // every wave performs at the same coherent point: once this wave's have
    // completed (the wait), a wave that takes a later ticket and then loads
    // them sees them.  No release fence: on this chip it writes back the
    // whole L2 of the wave's XCD.
    if (P.report) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    // The workgroup's control waves combine their tickets in LDS: the last
    // of them to finish takes one for each (fewer atomics on the layer's
    // word, which serialise), the others are done.  Their status bits have
    // completed before their LDS add (the wait above), and so before it.
    const int members = __builtin_amdgcn_readfirstlane(
        B - (bank - pair) < NB ? B - (bank - pair) : NB);
    int take = 1;
    bool last_here = true;
    if (members > 1) {
      uint32_t before = 0;
      if (lane == 0) {
        before = __hip_atomic_fetch_add(&lds_done, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      last_here = __builtin_amdgcn_readfirstlane(static_cast<int>(before)) + 1 == members;
      take = members;
    }
    int64_t done = -1;
    if (last_here && lane == 0) {
      int64_t* const ticket = P.trace_ticket + 1 + layer_id;
      done = __hip_atomic_fetch_add(ticket, int64_t{take}, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
    // the low half counts the waves done with the launch
    if (last_here && __builtin_amdgcn_readfirstlane(static_cast<int>(done)) + take == B) {
      if constexpr (!DENSE) {
        if (local_plan) {
          // what a local plan leaves (the central plan's layer part writes
          // these before the steps; here every wave has read the free count
          // and control words by now): the stack's new height and the proof
          if (lane == 0) *L.free_count = static_cast<int32_t>(found_top - fit_rows);
          if (lane < 4) {
            int k = COWSDM_CTRL_PROVEN;
            int64_t v = local_proven;
            if (lane == 1) { k = COWSDM_CTRL_FREE; v = found_top - fit_rows; }
            if (lane == 2) { k = COWSDM_CTRL_STEPS; v = G0; }
            if (lane == 3) { k = COWSDM_CTRL_FIT; v = fit_rows; }
            atomic_store_u64(&control_word(P, layer_id, k), static_cast<uint64_t>(v));
          }
          // the report below reads the control words back
          __builtin_amdgcn_s_waitcnt(0);
        }
      }
      if (lane == 0) {
        atomic_store_u64(P.trace_ticket + 1 + layer_id, 0);
        if (P.trace_step) {
          atomic_store_u64(&P.trace_step[layer_id], static_cast<uint64_t>(first + done_steps));
        }
        if constexpr (!DENSE) atomic_store_u64(pb.epoch, static_cast<uint64_t>(epoch));
      }
      if (P.report) write_report(P, layer_id, first + done_steps, 0);
    }
  }
}

// Count part of a packed persistent launch whose slot maps do not fit in LDS
// (trace_plan.hip).
template <typename IDX>
int32_t launch_trace_count(const StepParams& P, hipStream_t stream, hipEvent_t start);
extern template int32_t launch_trace_count<int32_t>(const StepParams&, hipStream_t, hipEvent_t);
extern template int32_t launch_trace_count<int64_t>(const StepParams&, hipStream_t, hipEvent_t);

// Residency of one persistent kernel variant: how many of its workgroups a
// device holds at once for a given slot-map size, cached as one word
// (device + 1 in bits 48-63, the slot-map key in bits 24-47, the workgroups
// in bits 0-23; 0: nothing cached) so that a reader never pairs one query's
// key with another's count.
__host__ inline uint64_t residency_word(int device, int key, int blocks) {
  return (static_cast<uint64_t>(device + 1) << 48) |
         ((static_cast<uint64_t>(key) & 0xFFFFFFu) << 24) |
         (static_cast<uint64_t>(blocks) & 0xFFFFFFu);
}

// Workgroups of a persistent launch wait on one another, so every one of them
// must be resident at once.  Returns 0 when launched, 1 (nothing launched)
// when the grid exceeds what the device can hold for this kernel (the caller
// then falls back to one launch per step), else an error code.  The residency check assumes the launch has
// the device's compute units to itself: another process's kernels holding
// CUs meanwhile could delay the launch's last workgroups until the bounded
// waits of the first ones run out (the launch then reports
// COWSDM_TRACE_FAULT, it does not hang).
template <typename IDX, bool DENSE, bool MAPLDS>
int32_t launch_trace_kernels(const StepParams& P0, int vec, hipStream_t stream) {
  StepParams P = P0;
  P.blocks_per_layer = (P.banks + kTraceBanksPerBlock - 1) / kTraceBanksPerBlock;
  const int blocks = P.blocks_per_layer * P.nlayers;
  // the full shape folds every row count; other shapes select per row
  bool full = P.writes == kTraceMaxWrites && P.reads == kTraceMaxReads;
  if (full && sizeof(IDX) == 4) {
    // the full variant loads a step's int32 slots as 16-byte vectors
    uintptr_t bits = static_cast<uintptr_t>(P.trace_stride[0] | P.trace_stride[6]);
    for (int l = 0; l < P.nlayers; ++l) {
      bits |= reinterpret_cast<uintptr_t>(P.layer[l].write_indices) |
              reinterpret_cast<uintptr_t>(P.layer[l].read_indices);
    }
    full = (bits % 16) == 0;
  }
  const bool few = P.banks <= kWave;
  const int variant = (full ? 1 : 0) + (few ? 2 : 0);
  const void* kernels[4][3] = {
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, false, false, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, false, false, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, false, false, MAPLDS>)},
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, true, false, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, true, false, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, true, false, MAPLDS>)},
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, false, true, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, false, true, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, false, true, MAPLDS>)},
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, true, true, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, true, true, MAPLDS>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, true, true, MAPLDS>)}};
  // Residency depends on the device and on the LDS map's size: cached per
  // kernel variant for the last (device, slot count) it was asked for.  The
  // cache is process-wide and each entry one atomic word; host threads
  // calling at once may each query the occupancy, which is harmless.
  static std::atomic<uint64_t> resident[4][3];
  const int which = vec == 4 ? 2 : (vec == 2 ? 1 : 0);
  const void* kernel = kernels[variant][which];
  // map in LDS: per bank the slot map
  // map in LDS: per bank the slot map and each slot's first writing step
  const size_t lds_bytes =
      MAPLDS ? 2 * sizeof(int) * kTraceBanksPerBlock * static_cast<size_t>(P.slots) : 0;
  const int key = MAPLDS ? P.slots : 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    (void)hipGetLastError();
    return 1;
  }
  int resident_blocks = 0;
  const uint64_t cached = resident[variant][which].load(std::memory_order_relaxed);
  if (cached != 0 && (cached >> 24) == (residency_word(device, key, 0) >> 24)) {
    resident_blocks = static_cast<int>(cached & 0xFFFFFFu);
  } else {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kTraceThreads, lds_bytes) !=
            hipSuccess) {
      (void)hipGetLastError();
      resident_blocks = 0;
    } else {
      resident_blocks = cus * per_cu;
    }
    resident[variant][which].store(residency_word(device, key, resident_blocks),
                                   std::memory_order_relaxed);
  }
  // Layers are independent within a launch: when the whole grid cannot be
  // resident, launch groups of layers that can, one after another on the
  // stream, each with its per-layer words offset to its first layer.
  const int per_launch = resident_blocks / P.blocks_per_layer;
  if (per_launch <= 0) return 1;
  // With timing on, events at the launch's first kernel's start (the count
  // pass of packed state), at the decode kernel's start and at its end.
  hipEvent_t first = nullptr, start = nullptr, stop = nullptr;
  if (!trace_timing_events(&first, &start, &stop)) first = start = stop = nullptr;
  if (!DENSE && !MAPLDS) {
    // the count part of every layer's plan, before the decode kernel
    if (int32_t e = launch_trace_count<IDX>(P, stream, first)) return e;
  } else if (first) {
    trace_timing_first_is_start();   // the decode kernel is the launch's first
  }
  auto launch = [&](StepParams* q, int grid, bool last) {
    void* args[] = {q};
    (void)hipExtLaunchKernel(kernel, dim3(grid), dim3(kTraceThreads), args, lds_bytes, stream,
                             start, last ? stop : nullptr, 0);
    start = nullptr;
  };
  if (blocks <= resident_blocks) {
    launch(&P, blocks, true);
    return 0;  // a failed launch is reported by the caller's launch_status()
  }
  for (int l0 = 0; l0 < P0.nlayers; l0 += per_launch) {
    StepParams Q = P;
    Q.nlayers = P0.nlayers - l0 < per_launch ? P0.nlayers - l0 : per_launch;
    for (int i = 0; i < kMaxLayers; ++i) Q.layer[i] = P0.layer[l0 + i < P0.nlayers ? l0 + i : l0];
    if (P0.trace_step) Q.trace_step = P0.trace_step + l0;
    if (P0.trace_ticket) Q.trace_ticket = P0.trace_ticket + l0;  // word 1 + layer
    if (P0.trace_status) Q.trace_status = P0.trace_status + l0;
    if (P0.control) Q.control = P0.control + l0;
    if (P0.report) Q.report = P0.report + static_cast<int64_t>(l0) * COWSDM_REPORT_WORDS;
    if (P0.scan) Q.scan = P0.scan + static_cast<int64_t>(l0) * P0.scan_words;
    launch(&Q, Q.blocks_per_layer * Q.nlayers, l0 + per_launch >= P0.nlayers);
  }
  return 0;
}

template <typename IDX, bool DENSE>
int32_t launch_trace(const StepParams& P, int vec, hipStream_t stream) {
  // packed layers whose slot map fits keep it in LDS
  if (!DENSE && P.slots <= kTraceMapSlots) {
    return launch_trace_kernels<IDX, DENSE, true>(P, vec, stream);
  }
  return launch_trace_kernels<IDX, DENSE, false>(P, vec, stream);
}

}  // namespace cowsdm_impl
