// Persistent multi-step form of the copy-on-write SDM step: one launch runs
// G consecutive decode steps of device-resident routes for every (layer,
// bank), with results identical to G single-step launches.
//
// Each wave owns one (layer, bank) for all G steps and software-pipelines
// them so that every memory access has about one iteration to land before
// its value is used.  Iteration s
//   1. loads every bank's first-touch count of step s (published one
//      iteration earlier), the slots of step s+3 (s+2 for dense tables) and
//      the map entries of step s+2;
//   2. classifies step s+1 (first touches, slots written by steps s and s-1,
//      read-after-write), publishes its first-touch count and loads its rows;
//   3. computes step s (gated-delta update, sparse read) from rows loaded one
//      iteration earlier; stores its reading and the rows already private;
//   4. pops the free rows of step s's first touches and stores them and their
//      map entries.
// Step t's map entries are read before steps t-2 and t-1 have stored their
// first touches: slots written at t-1 take their rows from that step's
// result, kept in LDS, and slots written at t-2 take the physical rows popped
// for them.  Every other row step t needs was stored earlier by the same
// wave, in program order.  Values in flight live in even/odd homes (the loop
// is unrolled by two) and are only read one iteration after their load was
// issued, so no register copy waits on memory; per-row values picked by
// run-time lanes are read from LDS, never selected out of registers.
//
// First touches of (step t, bank b) pop free_rows[F - 1 - Q(t, b) - rank],
// where F is free_count at launch and Q the exclusive prefix of first-touch
// counts over (step, bank) pairs in step-major, bank-minor order: exactly the
// rows G single-step launches would pop.  Each wave publishes one count per
// step and reads the counts of every bank of the layer, so it knows both its
// own prefix and the running total without waiting on another wave's prefix.
// The wave of bank B-1 closes the launch: it writes free_count and advances
// the scan epoch.
#pragma once

#include "common.h"

namespace cowsdm_impl {

typedef float vf4_t __attribute__((ext_vector_type(4)));

template <int VEC>
struct TraceRows {                  // operands of one step, loaded one step ahead
  float w[kTraceMaxWrites][VEC];    // rows of the write slots, before the decay
  float r[kTraceMaxReads][VEC];     // rows of the read slots, before this step
  float vin[VEC];                   // the step's value
  float ww, rw;                     // lane j: weight of write j / read j
};

struct TraceIdx {                   // lane j: write slot j / read slot j
  int widx, ridx, err;
};

struct TraceRoute {                 // a classified step
  int widx, ridx;
  int wrow;       // write lane: physical row (-1: M0, or a first touch not yet popped)
  int wsrc;       // write lane: written by step t-1 lane j (j), else -1
  int rsrc;       // read lane: the same
  int rraw;       // read lane: write lane of step t itself with this slot, else -1
  int rank;       // write lane: rank among the bank's first touches
  uint32_t u;     // wave-uniform: bits 0-3 first-touch write lanes, 4-7 their count,
                  // 8 the step runs (routes valid, every earlier step ran),
                  // 9 a row comes from step t-1, 10 a read sees a write of step t
};

__device__ __forceinline__ uint32_t route_fmask(uint32_t u) { return u & 15u; }
__device__ __forceinline__ int route_count(uint32_t u) { return static_cast<int>((u >> 4) & 15u); }
__device__ __forceinline__ bool route_ok(uint32_t u) { return (u >> 8) & 1u; }
__device__ __forceinline__ bool route_fix(uint32_t u) { return (u >> 9) & 1u; }
__device__ __forceinline__ bool route_raw(uint32_t u) { return (u >> 10) & 1u; }

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

__device__ __forceinline__ const float* rl_ptr(const float* p, int lane) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(v >> 32), lane);
  return reinterpret_cast<const float*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// Weighted population count of per-lane values 0..7 held as three bit masks.
__device__ __forceinline__ int64_t sum3(uint64_t b0, uint64_t b1, uint64_t b2, uint64_t m) {
  return __popcll(b0 & m) + 2 * __popcll(b1 & m) + 4 * __popcll(b2 & m);
}

// FULL: W == kTraceMaxWrites and R == kTraceMaxReads, every row guard folds away.
// SCANW: 64-bank windows of the count scan (1: at most 64 banks per layer).
template <typename IDX, int VEC, bool DENSE, bool FULL, int SCANW>
__global__ __launch_bounds__(kStepThreads)
__attribute__((amdgpu_waves_per_eu(1, SCANW == 1 ? 1 : 2)))
void sdm_trace_kernel(StepParams P) {
  constexpr int kRow = kWave * VEC;  // floats of one LDS row
  __shared__ float lds_rows[kBanksPerBlock][kTraceMaxWrites][kRow];
  // full shape: the step's weights, written per lane, read back broadcast
  __shared__ vf4_t lds_weights[kBanksPerBlock][2][kWave / 4];
  __shared__ int lds_free[DENSE ? 1 : kTraceFreeWindow];

  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  if (layer_id >= P.nlayers) return;  // whole workgroup
  const int bank = (blockIdx.x % P.blocks_per_layer) * kBanksPerBlock + wave;
  const cowsdm_layer_t& L = P.layer[layer_id];
  // Device-counted launches read the layer's first step from its counter
  // (every thread reads the same value: it changes only after all waves of
  // the layer are done) and run at most the steps recorded after it.
  int64_t first = P.trace_first;
  int64_t left = P.steps;
  if (P.trace_step) {
    const uint64_t f = static_cast<uint64_t>(P.trace_step[layer_id]);
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
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{2}, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      } else if (!DENSE) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_TRACE_RANGE), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;  // whole workgroup
  }

  const int N = P.slots;
  const int D = P.width;
  const int W = FULL ? kTraceMaxWrites : P.writes;
  const int R = FULL ? kTraceMaxReads : P.reads;
  const int B = P.banks;
  const int G = static_cast<int>(left);
  const int C = static_cast<int>(L.capacity_rows);  // rows are int32
  // lanes past the row width repeat the last columns: they load, compute and
  // store exactly what the last full lane does, so no access needs a lane mask
  const int col = lane * VEC < D ? lane * VEC : D - VEC;
  const uint32_t coff = static_cast<uint32_t>(col) * 4u;

  // ---- launch constants
  int base_err = 0;
  int old_free = 0;
  int window = 0;
  if constexpr (!DENSE) {
    old_free = __builtin_amdgcn_readfirstlane(*L.free_count);
    if (old_free < 0 || old_free > C) {
      base_err |= COWSDM_ERR_CORRUPT;
    } else {
      window = old_free < kTraceFreeWindow ? old_free : kTraceFreeWindow;
    }
    for (int k = static_cast<int>(threadIdx.x); k < window; k += kStepThreads) {
      lds_free[k] = L.free_rows[old_free - 1 - k];
    }
    __syncthreads();
  }
  if (bank >= B) return;
  int64_t tmpl = 0;
  uint32_t epoch = 0;
  int64_t* slots = nullptr;
  if constexpr (!DENSE) {
    tmpl = L.template_indices[bank];
    if (tmpl < 0 || tmpl >= P.templates) {
      base_err |= COWSDM_ERR_TEMPLATE;
      tmpl = 0;
    }
    int64_t* const scan = P.scan + static_cast<int64_t>(layer_id) * P.scan_words;
    epoch = static_cast<uint32_t>(scan[COWSDM_SCRATCH_EPOCH]);
    slots = scan + COWSDM_SCRATCH_SLOTS + bank;  // + t * B: this bank's word of step t
  }
  const float* const m0_bank =
      DENSE ? nullptr : L.shared_initial_memory + tmpl * static_cast<int64_t>(N) * D;
  float* const table_bank = DENSE ? L.values + static_cast<int64_t>(bank) * N * D : nullptr;
  int32_t* const map_bank = DENSE ? nullptr : L.logical_to_physical + static_cast<int64_t>(bank) * N;
  float* const lds_wave = &lds_rows[wave][0][0];

  // ---- this lane's inputs at the launch's first step; step t adds t * stride
  const int wl = lane < W ? lane : 0;
  const int rl_ = lane < R ? lane : 0;
  auto first_step = [&](const void* base, int k) __attribute__((always_inline)) -> const char* {
    return static_cast<const char*>(base) + first * P.trace_stride[k];
  };
  const char* const wi_l = first_step(L.write_indices, 0) + (static_cast<int64_t>(bank) * W + wl) * sizeof(IDX);
  const char* const ww_l = first_step(L.write_weights, 1) + (static_cast<int64_t>(bank) * W + wl) * 4;
  const char* const v_l = first_step(L.step_values, 2) + (static_cast<int64_t>(bank) * D + col) * 4;
  const char* const ri_l = first_step(L.read_indices, 6) + (static_cast<int64_t>(bank) * R + rl_) * sizeof(IDX);
  const char* const rw_l = first_step(L.read_weights, 7) + (static_cast<int64_t>(bank) * R + rl_) * 4;
  const char* const out_l = first_step(L.output, 8) + (static_cast<int64_t>(bank) * D + col) * 4;
  const uint32_t st_wi = static_cast<uint32_t>(P.trace_stride[0]);
  const uint32_t st_ww = static_cast<uint32_t>(P.trace_stride[1]);
  const uint32_t st_v = static_cast<uint32_t>(P.trace_stride[2]);
  const uint32_t st_ri = static_cast<uint32_t>(P.trace_stride[6]);
  const uint32_t st_rw = static_cast<uint32_t>(P.trace_stride[7]);
  const uint32_t st_out = static_cast<uint32_t>(P.trace_stride[8]);
  auto at = [](const char* p, uint32_t stride, int t) __attribute__((always_inline)) -> const char* {
    return p + static_cast<uint64_t>(static_cast<uint32_t>(t)) * stride;
  };

  // ---- gates of every step, lane t holding step t's
  float alpha_l = 0.0f, in_l = 0.0f, er_l = 0.0f;
  if (lane < G) {
    const float fg = reinterpret_cast<const float*>(first_step(L.forget_log_gate, 5) +
                                                    static_cast<int64_t>(lane) * P.trace_stride[5])[bank];
    in_l = reinterpret_cast<const float*>(first_step(L.input_gate, 3) +
                                          static_cast<int64_t>(lane) * P.trace_stride[3])[bank];
    er_l = reinterpret_cast<const float*>(first_step(L.erase_gate, 4) +
                                          static_cast<int64_t>(lane) * P.trace_stride[4])[bank];
    alpha_l = static_cast<float>(exp(static_cast<double>(fg)));
  }

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
  auto classify = [&](int t, const TraceIdx& m, int wraw, int rraw, TraceRoute& rt,
                      const TraceRoute& r1, const TraceRoute& r2, bool ok_prev)
      __attribute__((always_inline)) -> int {
    int lerr = m.err | base_err;
    if constexpr (!DENSE) {
      if (lane < W && wraw >= C) { lerr |= COWSDM_ERR_CORRUPT; wraw = -1; }
      if (lane < R && rraw >= C) { lerr |= COWSDM_ERR_CORRUPT; rraw = -1; }
    }
    int wsrc = -1, rsrc = -1, rraw_lane = -1;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W) {
        const int sj = rl(m.widx, j);
        if (lane < W && lane > j && m.widx == sj) lerr |= COWSDM_ERR_DUP_WRITE;
        if (lane < R && m.ridx == sj) rraw_lane = j;
      }
    }
    if (t >= 1) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const int sj = rl(r1.widx, j);
          if (lane < W && m.widx == sj) wsrc = j;
          if (lane < R && m.ridx == sj) rsrc = j;
        }
      }
    }
    if (!DENSE && t >= 2) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const int sj = rl(r2.widx, j);
          const int row = rl(r2.wrow, j);
          if (lane < W && wsrc < 0 && m.widx == sj) wraw = row;
          if (lane < R && rsrc < 0 && m.ridx == sj) rraw = row;
        }
      }
    }
    if (rraw_lane >= 0) rsrc = -1;
    const bool any_err = __ballot(lerr != 0) != 0;
    if (!DENSE && any_err && t < G) {
      const int e = wave_or(lerr);
      if (lane == 0) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(e),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    const bool ok = ok_prev && !any_err;
    const bool first = !DENSE && ok && lane < W && wsrc < 0 && wraw < 0;
    const uint64_t fm = __ballot(first);
    const bool fix = __ballot((lane < W && wsrc >= 0) || (lane < R && rsrc >= 0)) != 0;
    const bool raw = __ballot(lane < R && rraw_lane >= 0) != 0;
    rt.u = static_cast<uint32_t>(fm & 15u) | (static_cast<uint32_t>(__popcll(fm)) << 4) |
           (ok ? 1u << 8 : 0u) | (fix ? 1u << 9 : 0u) | (raw ? 1u << 10 : 0u);
    rt.rank = lanes_below(fm);
    rt.widx = m.widx;
    rt.ridx = m.ridx;
    rt.wrow = lane < W ? wraw : -1;
    rt.wsrc = lane < W ? wsrc : -1;
    rt.rsrc = lane < R ? rsrc : -1;
    rt.rraw = lane < R ? rraw_lane : -1;
    return rraw;
  };

  auto publish = [&](int t, const TraceRoute& rt) __attribute__((always_inline)) {
    if constexpr (!DENSE) {
      if (lane == 0 && t < G) {
        atomic_store_u64(&slots[static_cast<int64_t>(t) * B],
                         slot_word(epoch, kStatusAggregate, static_cast<uint64_t>(route_count(rt.u))));
      }
    }
  };

  auto issue_rows = [&](int t, const TraceRoute& rt, int rrow, TraceRows<VEC>& buf)
      __attribute__((always_inline)) {
    const int tc = t < G ? t : G - 1;
    const float* wp;
    const float* rp;
    if constexpr (DENSE) {
      wp = table_bank + static_cast<int64_t>(rt.widx) * D;
      rp = table_bank + static_cast<int64_t>(rt.ridx) * D;
    } else {
      wp = rt.wrow < 0 ? m0_bank + static_cast<int64_t>(rt.widx) * D
                       : L.values + static_cast<int64_t>(rt.wrow) * D;
      rp = rrow < 0 ? m0_bank + static_cast<int64_t>(rt.ridx) * D
                    : L.values + static_cast<int64_t>(rrow) * D;
    }
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W) {
        const float* p = rl_ptr(wp, j);
        gload_row<VEC>(p, coff, buf.w[j]);
      }
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      if (i < R) {
        const float* p = rl_ptr(rp, i);
        gload_row<VEC>(p, coff, buf.r[i]);
      }
    }
    gload_row<VEC>(reinterpret_cast<const float*>(at(v_l, st_v, tc)), 0u, buf.vin);
    buf.ww = *(const gfloat*)(at(ww_l, st_ww, tc));
    buf.rw = *(const gfloat*)(at(rw_l, st_rw, tc));
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
  bool alive = true;

  // Step t: LDS row j holds write j of step t-1 until this step replaces it.
  auto compute = [&](int t, const TraceRoute& rt, TraceRows<VEC>& buf)
      __attribute__((always_inline)) {
    const bool run = route_ok(rt.u) && alive;
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
    if (run) {
      if (route_fix(rt.u)) {
#pragma unroll
        for (int j = 0; j < kTraceMaxWrites; ++j) {
          if (j < W) {
            const int src = rl(rt.wsrc, j);
            if (src >= 0) lds_get(src, buf.w[j]);
          }
        }
#pragma unroll
        for (int i = 0; i < kTraceMaxReads; ++i) {
          if (i < R) {
            const int src = rl(rt.rsrc, i);
            if (src >= 0) lds_get(src, buf.r[i]);
          }
        }
      }
      vf4_t wwv = 0.0f, rwv[kTraceMaxReads / 4];
      if constexpr (FULL) {
        // lane j holds weight j; one LDS round trip gives every lane all of
        // them as vectors, instead of a readlane per weight
        float* const wl = reinterpret_cast<float*>(&lds_weights[wave][0][0]);
        wl[lane] = buf.ww;
        wl[kWave + lane] = buf.rw;
        wwv = lds_weights[wave][0][0];
#pragma unroll
        for (int k = 0; k < kTraceMaxReads / 4; ++k) rwv[k] = lds_weights[wave][1][k];
      }
      const float alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha_l), t));
      const float in_gate = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(in_l), t));
      const float er_gate = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(er_l), t));
      float ret[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) ret[v] = 0.0f;
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const float wj = FULL ? wwv[j] : rlf(buf.ww, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float d = buf.w[j][v] * alpha;
            cur[j][v] = d;
            const float term = wj * d;
            ret[v] = (j == 0) ? term : ret[v] + term;
          }
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
        if (j < W) {
          const float wj = FULL ? wwv[j] : rlf(buf.ww, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float u = wj * delta[v];
            cur[j][v] = cur[j][v] + u;
          }
          lds_put(j, cur[j]);
        }
      }
      if (route_raw(rt.u)) {
#pragma unroll
        for (int i = 0; i < kTraceMaxReads; ++i) {
          if (i < R) {
            const int src = rl(rt.rraw, i);
            if (src >= 0) lds_get(src, buf.r[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kTraceMaxReads; ++i) {
        if (i < R) {
          const float wr = FULL ? rwv[i / 4][i % 4] : rlf(buf.rw, i);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float term = wr * buf.r[i][v];
            acc[v] = (i == 0) ? term : acc[v] + term;
          }
        }
      }
    }
    gstore_row<VEC>(reinterpret_cast<float*>(const_cast<char*>(at(out_l, st_out, t))), 0u, acc);
    if (run) {
      float* const dst = DENSE ? table_bank + static_cast<int64_t>(rt.widx) * D
                               : L.values + static_cast<int64_t>(rt.wrow < 0 ? 0 : rt.wrow) * D;
      const uint32_t fmask = route_fmask(rt.u);
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W && !((fmask >> j) & 1u)) {
          float* p = const_cast<float*>(rl_ptr(dst, j));
          gstore_row<VEC>(p, coff, cur[j]);
        }
      }
    }
  };

  // ---- pops (packed)
  int base = 0;     // first touches of the launch's earlier steps, all banks
  int served = 0;   // largest inclusive prefix that fits the free stack
  bool over = false;
  uint64_t sw[SCANW];
#pragma unroll
  for (int k = 0; k < SCANW; ++k) sw[k] = 0;
  const int64_t* const step_words = DENSE ? nullptr : slots - bank;  // word of (t, b): t*B + b

  auto issue_scan = [&](int t) __attribute__((always_inline)) {
    if constexpr (!DENSE) {
      const int64_t tc = t < G ? t : G - 1;
#pragma unroll
      for (int k = 0; k < SCANW; ++k) {
        if (k * kWave < B) {
          const int bk = k * kWave + lane < B ? k * kWave + lane : B - 1;
          sw[k] = atomic_load_u64(&step_words[tc * B + bk]);
        }
      }
    }
  };

  // Step t's first touches, after its counts (sw) have been loaded.  r1: step
  // t+1, whose rewrites of step t's slots take its physical rows.
  auto resolve = [&](int t, TraceRoute& rt, TraceRoute& r1)
      __attribute__((always_inline)) {
    int partial = 0, total = 0;
    bool poisoned = false;
    auto word_ready = [&](uint64_t w) __attribute__((always_inline)) -> bool {
      return static_cast<uint32_t>(w >> 32) == epoch && ((w >> 30) & 3u) == kStatusAggregate;
    };
#pragma unroll
    for (int k = 0; k < SCANW; ++k) {
      if (k * kWave < B) {
        const bool in = k * kWave + lane < B;
        uint64_t w = sw[k];
        bool ready = !in || word_ready(w);
        if (__ballot(!ready) != 0) {
          // a bank has not published step t yet: bounded wait
          int spins = 0;
          while (!ready && spins < kSpinLimit) {
            __builtin_amdgcn_s_sleep(1);
            w = atomic_load_u64(&step_words[static_cast<int64_t>(t) * B + k * kWave + lane]);
            ready = word_ready(w);
            ++spins;
          }
          if (__ballot(!ready) != 0) poisoned = true;
          sw[k] = ready ? w : 0;
        }
        const int v = (in && ready) ? static_cast<int>(w & 7u) : 0;
        const uint64_t b0 = __ballot(v & 1), b1 = __ballot(v & 2), b2 = __ballot(v & 4);
        const int below = bank - k * kWave;
        const uint64_t m = below <= 0 ? 0ull : (below >= kWave ? ~0ull : ((1ull << below) - 1));
        partial += static_cast<int>(sum3(b0, b1, b2, m));
        total += static_cast<int>(sum3(b0, b1, b2, ~0ull));
      }
    }
    if (!over) {
      if (base + total <= old_free) {
        served = base + total;
      } else {
        // largest inclusive prefix of this step's banks that still fits
        over = true;
        int carry = base;
        bool done = false;
#pragma unroll
        for (int k = 0; k < SCANW; ++k) {
          if (k * kWave < B && !done) {
            const bool in = k * kWave + lane < B;
            const int v = (in && word_ready(sw[k])) ? static_cast<int>(sw[k] & 7u) : 0;
            const uint64_t b0 = __ballot(v & 1), b1 = __ballot(v & 2), b2 = __ballot(v & 4);
            const int incl = carry + lanes_below(b0) + 2 * lanes_below(b1) + 4 * lanes_below(b2) + v;
            const uint64_t fit = __ballot(in && incl <= old_free);
            if (fit != 0) served = __shfl(incl, 63 - __clzll(static_cast<long long>(fit)), kWave);
            if (fit != __ballot(in)) done = true;
            carry += static_cast<int>(sum3(b0, b1, b2, ~0ull));
          }
        }
      }
    }
    const int prefix = base + partial;
    base += total;

    const int count = route_count(rt.u);
    const uint32_t fmask = route_fmask(rt.u);
    const bool first = lane < kTraceMaxWrites && ((fmask >> lane) & 1u);
    bool fits = route_ok(rt.u) && alive && !poisoned && (count == 0 || prefix + count <= old_free);
    int new_row = -1;
    if (fits && count > 0) {
      const int k = prefix + rt.rank;
      if (first && k < window) new_row = lds_free[k];
      if (__ballot(first && k >= window) != 0) {
        if (first && k >= window) new_row = L.free_rows[old_free - 1 - k];
        // wait for it here, on this rare path, so that no later use of the
        // popped rows has to drain every load in flight
        asm volatile("" ::"v"(new_row));
      }
      if (__ballot(first && (new_row < 0 || new_row >= C)) != 0) {
        fits = false;
        if (lane == 0) {
          __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                                static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    if (lane == 0) {
      if (route_ok(rt.u) && alive && !poisoned && !fits && count > 0) *L.overflow_flag = 1;
      if (poisoned) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (fits && count > 0) {
      if (first) {
        rt.wrow = new_row;
        map_bank[rt.widx] = new_row;
      }
      float* const dst = L.values + static_cast<int64_t>(rt.wrow < 0 ? 0 : rt.wrow) * D;
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W && ((fmask >> j) & 1u)) {
          float* p = const_cast<float*>(rl_ptr(dst, j));
          gstore_row<VEC>(p, coff, cur[j]);
        }
      }
    }
    alive = alive && fits;
    // step t+1 rewrites some of step t's slots in the rows just found
    const int s1 = r1.wsrc;
    const int v1 = __shfl(rt.wrow, s1 >= 0 ? s1 : 0, kWave);
    if (s1 >= 0) r1.wrow = v1;
  };

  // ---- prologue: step 0 classified with its rows in flight
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
  // slots and map entries in flight, homed by the parity of the iteration
  // that issued them
  TraceIdx idxA, idxB, ready1, ready2;
  int mwA = -1, mrA = -1, mwB = -1, mrB = -1;
  TraceRoute q, r0;
  q.widx = 0; q.ridx = 0; q.wrow = -1; q.wsrc = -1; q.rsrc = -1; q.rraw = -1; q.rank = 0; q.u = 0;
  {
    TraceIdx i0;
    load_idx(0, i0);
    int mw0, mr0;
    issue_map(i0, mw0, mr0);
    const int rrow = classify(0, i0, mw0, mr0, r0, q, q, true);
    publish(0, r0);
    issue_rows(0, r0, rrow, bufA);
  }
  if constexpr (DENSE) {
    load_idx(1, idxB);             // classified in iteration 0
  } else {
    load_idx(1, ready1);           // its map entries, classified in iteration 0
    issue_map(ready1, mwB, mrB);
    load_idx(2, idxB);             // its map entries are loaded in iteration 0
  }

  // Iteration s.  `self` homes are written now and read in iteration s+1,
  // `other` homes were written in iteration s-1 and are read now.
  // device capacity proof: before each run of proof_steps steps the layer
  // needs proof_rows free rows; every wave of the layer sees the same pops
  // (base), so all of them stop at the same step
  const int64_t proof_rows = DENSE ? 0 : P.trace_proof_rows;
  const int proof_steps = P.trace_proof_steps > 0 ? P.trace_proof_steps : 1;
  int done_steps = G;
  // does the capacity proof stop the layer before step s?  Wave-uniform by
  // construction; readfirstlane lets the compiler see it, so the loop exit
  // stays a scalar branch.
  auto proof_stops = [&](int s) __attribute__((always_inline)) -> bool {
    if (__builtin_amdgcn_readfirstlane(
            (proof_rows > 0 && s % proof_steps == 0 && old_free - base < proof_rows) ? 1 : 0)) {
      done_steps = s;
      return true;
    }
    return false;
  };
  auto iteration = [&](int s, TraceRows<VEC>& rows_s, TraceRows<VEC>& rows_next,
                       TraceIdx& idx_self, TraceIdx& idx_other, int& mw_self, int& mr_self,
                       int& mw_other, int& mr_other) __attribute__((always_inline)) {
    issue_scan(s);
    TraceRoute r1;
    if constexpr (DENSE) {
      load_idx(s + 2, idx_self);
      const int rrow = classify(s + 1, idx_other, -1, -1, r1, r0, q, route_ok(r0.u));
      publish(s + 1, r1);
      issue_rows(s + 1, r1, rrow, rows_next);
      compute(s, r0, rows_s);
    } else {
      load_idx(s + 3, idx_self);
      issue_map(idx_other, mw_self, mr_self);   // step s+2
      ready2 = idx_other;
      const int rrow = classify(s + 1, ready1, mw_other, mr_other, r1, r0, q, route_ok(r0.u));
      publish(s + 1, r1);
      issue_rows(s + 1, r1, rrow, rows_next);
      compute(s, r0, rows_s);
      resolve(s, r0, r1);
      ready1 = ready2;
    }
    q = r0;
    r0 = r1;
  };
  // Drain the prologue's loads: the loop head then has one state of loads in
  // flight (the back edge's), and the waits the compiler places there stay
  // as loose as the steady state allows.
  __builtin_amdgcn_s_waitcnt(0);

  // Pairs of steps, then an odd last step outside the loop.  Capacity proofs
  // come in runs of an even number of steps (the host checks), so the only
  // exit from the loop body is at its head: the compiler then sees one state
  // of the loads in flight there and waits on none of them early.
  int s = 0;
  bool stopped = false;
  for (; s + 1 < G; s += 2) {
    if (proof_stops(s)) {
      stopped = true;
      break;
    }
    iteration(s, bufA, bufB, idxA, idxB, mwA, mrA, mwB, mrB);
    iteration(s + 1, bufB, bufA, idxB, idxA, mwB, mrB, mwA, mrA);
  }
  if (!stopped && s < G && !proof_stops(s)) {
    iteration(s, bufA, bufB, idxA, idxB, mwA, mrA, mwB, mrB);
  }

  // ---- the last bank closes the launch
  if constexpr (!DENSE) {
    if (bank == B - 1 && lane == 0) {
      *L.free_count = old_free - served;
      int64_t* const scan = P.scan + static_cast<int64_t>(layer_id) * P.scan_words;
      atomic_store_u64(&scan[COWSDM_SCRATCH_EPOCH], static_cast<uint64_t>(epoch + 1u));
      if (done_steps < G && P.trace_status) {
        __hip_atomic_fetch_or(&P.trace_status[layer_id], int32_t{1}, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // ---- device counters: the layer's last wave to finish (every wave of the
  // layer read the counter before taking its ticket) moves the counter past
  // the steps the layer ran
  if (P.trace_step && lane == 0) {
    int64_t* const ticket = P.trace_ticket + 1 + layer_id;
    const int64_t done = __hip_atomic_fetch_add(ticket, int64_t{1}, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (done == B - 1) {
      atomic_store_u64(ticket, 0);
      atomic_store_u64(&P.trace_step[layer_id], static_cast<uint64_t>(first + done_steps));
    }
  }
}

// Workgroups of a persistent launch wait on one another, so every one of them
// must be resident at once.  Returns false (nothing launched) when the grid
// exceeds what the device can hold for this kernel; the caller then falls
// back to one launch per step.
template <typename IDX, bool DENSE>
bool launch_trace(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  // the full-shape variant loads each bank's weights as 16-byte vectors
  bool full = P.writes == kTraceMaxWrites && P.reads == kTraceMaxReads &&
              P.trace_stride[1] % 16 == 0 && P.trace_stride[7] % 16 == 0;
  for (int l = 0; l < P.nlayers && full; ++l) {
    if ((reinterpret_cast<uintptr_t>(P.layer[l].write_weights) |
         reinterpret_cast<uintptr_t>(P.layer[l].read_weights)) % 16 != 0) {
      full = false;
    }
  }
  // one scan window when a layer has at most 64 banks (full shape only)
  const int variant = !full ? 0 : (!DENSE && P.banks <= kWave ? 2 : 1);
  const void* kernels[3][3] = {
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, false, kTraceScanWindows>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, false, kTraceScanWindows>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, false, kTraceScanWindows>)},
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, true, kTraceScanWindows>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, true, kTraceScanWindows>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, true, kTraceScanWindows>)},
      {reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE, true, DENSE ? kTraceScanWindows : 1>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE, true, DENSE ? kTraceScanWindows : 1>),
       reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE, true, DENSE ? kTraceScanWindows : 1>)}};
  static int resident[3][3] = {{-1, -1, -1}, {-1, -1, -1}, {-1, -1, -1}};
  const int which = vec == 4 ? 2 : (vec == 2 ? 1 : 0);
  const void* kernel = kernels[variant][which];
  if (resident[variant][which] < 0) {
    int device = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kStepThreads, 0) !=
            hipSuccess) {
      (void)hipGetLastError();
      resident[variant][which] = 0;
    } else {
      resident[variant][which] = cus * per_cu;
    }
  }
  if (blocks > resident[variant][which]) return false;
  void* args[] = {const_cast<StepParams*>(&P)};
  (void)hipLaunchKernel(kernel, dim3(blocks), dim3(kStepThreads), args, 0, stream);
  return true;  // a failed launch is reported by the caller's launch_status()
}

}  // namespace cowsdm_impl
