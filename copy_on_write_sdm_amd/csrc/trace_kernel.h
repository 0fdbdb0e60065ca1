// Persistent multi-step form of the copy-on-write SDM step: one launch runs
// G consecutive decode steps of device-resident routes for every (layer,
// bank), with results identical to G single-step launches.
//
// Each wave owns one (layer, bank) for all G steps and software-pipelines
// them.  In iteration s it
//   0. issues the map lookups of step s+1;
//   1. resolves step s-1's pops (bank-order prefix over the (step, bank)
//      sequence) and stores s-1's first-touch rows and map entries;
//   2. classifies step s+1 (first touches, read-after-write), publishes its
//      first-touch count and issues its row loads;
//   3. computes step s (gated-delta update, sparse read), stores its reading
//      and the rows that were already private;
//   4. copies into step s+1's rows the slots step s wrote.
// Step s+1's map entries are read before step s-1's first touches are stored
// and before step s's are known: slots written at s come from step s's
// registers and slots written at s-1 take the physical rows resolved in 1.
// Step s+1's rows are loaded before step s is computed: slots written at s
// are copied in 4, every other row was stored earlier by the same wave, in
// program order.  Row buffers alternate between even and odd steps (the loop
// is unrolled by two), so every buffer index is a compile-time constant and
// all rows stay in registers.
//
// First touches of (step t, bank b) pop free_rows[F - 1 - Q(t, b) - rank],
// where F is free_count at launch and Q the exclusive prefix of first-touch
// counts over (step, bank) pairs in step-major, bank-minor order: exactly
// the rows G single-step launches would pop.  The pair (G-1, B-1) closes the
// launch: it writes free_count and advances the scan epoch.
#pragma once

#include "common.h"
#include "lookback.h"

namespace cowsdm_impl {

constexpr int kTraceMaxWrites = 4;
constexpr int kTraceMaxReads = 16;

template <int VEC>
struct TraceMeta {
  int widx, ridx, err;
  float ww, rw;
  float gate;  // lane 0: forget log gate, lane 1: input gate, lane 2: erase gate
  float vin[VEC];
};

struct TraceClass {
  int wraw, rraw;   // physical rows of the write / read slot (-1: shared M0)
  int wfwd, rfwd;   // write lane of the previous step holding this slot, or -1
  int rsrc;         // write lane of this step holding this read slot, or -1
  int wphys;        // physical row of this write lane (first touches: after pops)
  int first;        // this write lane is a first touch
  int count, rank;  // first touches of the bank / rank of this lane among them
  int ok;           // the step runs (no error so far in this bank)
};

template <typename IDX, int VEC, bool DENSE>
__global__ __launch_bounds__(kStepThreads) void sdm_trace_kernel(StepParams P) {
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  const int bank = (blockIdx.x % P.blocks_per_layer) * kBanksPerBlock +
                   static_cast<int>(threadIdx.x) / kWave;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  if (layer_id >= P.nlayers || bank >= P.banks) return;
  const cowsdm_layer_t& L = P.layer[layer_id];

  const int N = P.slots;
  const int D = P.width;
  const int W = P.writes;
  const int R = P.reads;
  const int B = P.banks;
  const int G = P.steps;
  const int64_t C = L.capacity_rows;
  const int64_t b = bank;
  const int col = lane * VEC;
  const bool col_ok = col < D;

  // ---- launch constants of this (layer, bank)
  int base_err = 0;
  int64_t tmpl = 0;
  int64_t old_free = 0;
  uint32_t epoch = 0;
  int64_t* scan = nullptr;
  int free_top[kFreeWindow / kWave];
  if constexpr (!DENSE) {
    tmpl = L.template_indices[b];
    if (tmpl < 0 || tmpl >= P.templates) base_err |= COWSDM_ERR_TEMPLATE;
    old_free = *L.free_count;
    if (old_free < 0 || old_free > C) base_err |= COWSDM_ERR_CORRUPT;
    scan = P.scan + static_cast<int64_t>(layer_id) * P.scan_words;
    epoch = static_cast<uint32_t>(scan[COWSDM_SCRATCH_EPOCH]);
#pragma unroll
    for (int k = 0; k < kFreeWindow / kWave; ++k) {
      const int64_t pos = old_free - 1 - (k * kWave + lane);
      free_top[k] = (pos >= 0 && pos < C) ? L.free_rows[pos] : -1;
    }
  }
  int64_t* const slots = DENSE ? nullptr : scan + COWSDM_SCRATCH_SLOTS;
  const float* const m0_bank =
      DENSE ? nullptr : L.shared_initial_memory + tmpl * static_cast<int64_t>(N) * D;
  float* const table_bank = DENSE ? L.values + b * N * D : nullptr;
  int32_t* const map_bank = DENSE ? nullptr : L.logical_to_physical + b * N;

  auto step_in = [&](const void* base, int k, int s) __attribute__((always_inline)) -> const char* {
    return static_cast<const char*>(base) + (P.trace_first + s) * P.trace_stride[k];
  };

  // ---- stage helpers
  auto load_meta = [&](int s, TraceMeta<VEC>& m) __attribute__((always_inline)) {
    m.err = 0;
    m.widx = 0;
    m.ridx = 0;
    m.ww = 0.0f;
    m.rw = 0.0f;
    m.gate = 0.0f;
    const void* wi = step_in(L.write_indices, 0, s);
    const float* ww = reinterpret_cast<const float*>(step_in(L.write_weights, 1, s));
    const float* vv = reinterpret_cast<const float*>(step_in(L.step_values, 2, s));
    const void* ri = step_in(L.read_indices, 6, s);
    const float* rw = reinterpret_cast<const float*>(step_in(L.read_weights, 7, s));
    if (lane < W) {
      const int64_t x = load_index<IDX>(wi, b * W + lane);
      m.ww = ww[b * W + lane];
      if (x < 0 || x >= N) m.err |= COWSDM_ERR_WRITE_INDEX;
      else m.widx = static_cast<int>(x);
    }
    if (lane < R) {
      const int64_t x = load_index<IDX>(ri, b * R + lane);
      m.rw = rw[b * R + lane];
      if (x < 0 || x >= N) m.err |= COWSDM_ERR_READ_INDEX;
      else m.ridx = static_cast<int>(x);
    }
    // per-lane addresses keep the gates on vector loads: a scalar load here
    // would make every later scalar use wait for the newest step's gates
    if (lane < 3) {
      const int k = lane == 0 ? 5 : (lane == 1 ? 3 : 4);
      const void* base = lane == 0 ? L.forget_log_gate : (lane == 1 ? L.input_gate : L.erase_gate);
      m.gate = reinterpret_cast<const float*>(step_in(base, k, s))[b];
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) m.vin[v] = 0.0f;
    if (col_ok) load_row<VEC>(vv + b * D + col, m.vin);
  };

  auto issue_map = [&](const TraceMeta<VEC>& m, TraceClass& c) __attribute__((always_inline)) {
    c.wraw = -1;
    c.rraw = -1;
    if constexpr (!DENSE) {
      if (lane < W && !(m.err & COWSDM_ERR_WRITE_INDEX)) c.wraw = map_bank[m.widx];
      if (lane < R && !(m.err & COWSDM_ERR_READ_INDEX)) c.rraw = map_bank[m.ridx];
    }
  };

  // First touches and forwarding of step t.  p* is step t-1 (its rows in
  // registers, its first touches possibly unresolved), q* is step t-2 (its
  // physical rows resolved, its map entries possibly not yet visible in c).
  auto classify = [&](const TraceMeta<VEC>& m, TraceClass& c, const TraceMeta<VEC>& pmeta,
                      const TraceClass& pcls, const TraceMeta<VEC>& qmeta,
                      const TraceClass& qcls, bool have_p, bool have_q,
                      bool alive_in) __attribute__((always_inline)) {
    int lerr = m.err | base_err;
    if constexpr (!DENSE) {
      if (lane < W && c.wraw >= C) lerr |= COWSDM_ERR_CORRUPT;
      if (lane < R && c.rraw >= C) lerr |= COWSDM_ERR_CORRUPT;
    }
    c.rsrc = -1;
    c.wfwd = -1;
    c.rfwd = -1;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W) {
        const int other = rl(m.widx, j);
        if (lane < W && j < lane && other == m.widx) lerr |= COWSDM_ERR_DUP_WRITE;
        if (lane < R && m.ridx == other) c.rsrc = j;
      }
    }
    if (have_p) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const int prev_slot = rl(pmeta.widx, j);
          if (lane < W && m.widx == prev_slot) c.wfwd = j;
          if (lane < R && c.rsrc < 0 && m.ridx == prev_slot) c.rfwd = j;
        }
      }
    }
    if (!DENSE && have_q) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const int slot = rl(qmeta.widx, j);
          const int row = rl(qcls.wphys, j);
          if (lane < W && c.wfwd < 0 && m.widx == slot) c.wraw = row;
          if (lane < R && c.rsrc < 0 && c.rfwd < 0 && m.ridx == slot) c.rraw = row;
        }
      }
    }
    const int err = wave_or(lerr);
    c.ok = alive_in && err == 0;
    if (err && lane == 0 && !DENSE) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS], static_cast<int64_t>(err),
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    c.first = (!DENSE && c.ok && lane < W && c.wfwd < 0 && c.wraw < 0) ? 1 : 0;
    const uint64_t mask = __ballot(c.first);
    c.count = c.ok ? __popcll(mask) : 0;
    c.rank = __popcll(mask & ((1ull << lane) - 1));
    c.wphys = c.wraw;
  };

  // updated rows of the last computed step, element j * VEC + v; one vector
  // value so that the forwarding below (a wave-uniform but run-time row
  // index) stays in registers
  typedef float RowSet __attribute__((ext_vector_type(kTraceMaxWrites * VEC)));
  RowSet cur = 0.0f;
  float ncur_a[kTraceMaxWrites][VEC], ncur_b[kTraceMaxWrites][VEC];
  float rv_a[kTraceMaxReads][VEC], rv_b[kTraceMaxReads][VEC];
#pragma unroll
  for (int j = 0; j < kTraceMaxWrites; ++j) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) { ncur_a[j][v] = 0.0f; ncur_b[j][v] = 0.0f; }
  }
#pragma unroll
  for (int i = 0; i < kTraceMaxReads; ++i) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) { rv_a[i][v] = 0.0f; rv_b[i][v] = 0.0f; }
  }

  // dst = row j of cur, j wave-uniform
  auto copy_from_cur = [&](int j, float (&dst)[VEC]) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) dst[v] = cur[j * VEC + v];
  };

  // loads of the rows step m needs that the previous step did not write
  auto issue_loads = [&](const TraceMeta<VEC>& m, const TraceClass& c,
                         float (&nc)[kTraceMaxWrites][VEC],
                         float (&rv)[kTraceMaxReads][VEC]) __attribute__((always_inline)) {
    if (!c.ok) return;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W && rl(c.wfwd, j) < 0) {
        const int slot = rl(m.widx, j);
        const float* src;
        if constexpr (DENSE) {
          src = table_bank + static_cast<int64_t>(slot) * D;
        } else {
          const int p = rl(c.wraw, j);
          src = p < 0 ? m0_bank + static_cast<int64_t>(slot) * D
                      : L.values + static_cast<int64_t>(p) * D;
        }
        if (col_ok) load_row<VEC>(src + col, nc[j]);
      }
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      if (i < R && rl(c.rsrc, i) < 0 && rl(c.rfwd, i) < 0) {
        const int slot = rl(m.ridx, i);
        const float* src;
        if constexpr (DENSE) {
          src = table_bank + static_cast<int64_t>(slot) * D;
        } else {
          const int p = rl(c.rraw, i);
          src = p < 0 ? m0_bank + static_cast<int64_t>(slot) * D
                      : L.values + static_cast<int64_t>(p) * D;
        }
        if (col_ok) load_row<VEC>(src + col, rv[i]);
      }
    }
  };

  // rows of step m that the step just computed wrote, from registers
  auto copy_forwarded = [&](const TraceClass& c, float (&nc)[kTraceMaxWrites][VEC],
                            float (&rv)[kTraceMaxReads][VEC]) __attribute__((always_inline)) {
    if (!c.ok) return;
#pragma unroll
    for (int j = 0; j < kTraceMaxWrites; ++j) {
      if (j < W) {
        const int fwd = rl(c.wfwd, j);
        if (fwd >= 0) copy_from_cur(fwd, nc[j]);
      }
    }
#pragma unroll
    for (int i = 0; i < kTraceMaxReads; ++i) {
      if (i < R && rl(c.rsrc, i) < 0) {
        const int fwd = rl(c.rfwd, i);
        if (fwd >= 0) copy_from_cur(fwd, rv[i]);
      }
    }
  };

  // gated-delta update of nc into cur and the sparse read of step s
  auto compute = [&](const TraceMeta<VEC>& m, const TraceClass& c, int s,
                     float (&nc)[kTraceMaxWrites][VEC],
                     float (&rv)[kTraceMaxReads][VEC]) __attribute__((always_inline)) {
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
    if (c.ok) {
      const float forget = rlf(m.gate, 0);
      const float in_gate = rlf(m.gate, 1);
      const float er_gate = rlf(m.gate, 2);
      const float alpha = static_cast<float>(exp(static_cast<double>(forget)));
      float ret[VEC];
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const float wj = rlf(m.ww, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float d = nc[j][v] * alpha;
            cur[j * VEC + v] = d;
            const float term = wj * d;
            ret[v] = (j == 0) ? term : ret[v] + term;
          }
        }
      }
      float delta[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const float a = in_gate * m.vin[v];
        const float e = er_gate * ret[v];
        delta[v] = a - e;
      }
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W) {
          const float wj = rlf(m.ww, j);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float t = wj * delta[v];
            cur[j * VEC + v] = cur[j * VEC + v] + t;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kTraceMaxReads; ++i) {
        if (i < R) {
          const int src = rl(c.rsrc, i);
          float x[VEC];
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = rv[i][v];
          if (src >= 0) copy_from_cur(src, x);
          const float wr = rlf(m.rw, i);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float term = wr * x[v];
            acc[v] = (i == 0) ? term : acc[v] + term;
          }
        }
      }
    }
    float* out = reinterpret_cast<float*>(const_cast<char*>(step_in(L.output, 8, s)));
    if (col_ok) store_row<VEC>(out + b * D + col, acc);
    if (c.ok) {
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W && !rl(c.first, j)) {
          float* dst = DENSE ? table_bank + static_cast<int64_t>(rl(m.widx, j)) * D
                             : L.values + static_cast<int64_t>(rl(c.wphys, j)) * D;
          float row[VEC];
          copy_from_cur(j, row);
          if (col_ok) store_row<VEC>(dst + col, row);
        }
      }
    }
  };

  // pops of step s: rows, map entries; returns false when the step did not fit
  int64_t last_inclusive = 0;
  bool last_poisoned = false;
  auto resolve = [&](const TraceMeta<VEC>& m, TraceClass& c, int s) __attribute__((always_inline)) -> bool {
    bool poisoned = false;
    const int q = s * B + bank;
    const int64_t prefix = resolve_prefix(slots, q, epoch, c.count, lane, &poisoned);
    last_inclusive = prefix + c.count;
    last_poisoned = poisoned;
    bool fits = c.ok && !poisoned && (c.count == 0 || prefix + c.count <= old_free);
    const int64_t from_top = prefix + c.rank;
    const int src_lane = static_cast<int>(from_top % kWave);
    int window_row = -1;
#pragma unroll
    for (int k = 0; k < kFreeWindow / kWave; ++k) {
      const int v = __shfl(free_top[k], src_lane, kWave);
      if (from_top / kWave == k) window_row = v;
    }
    int new_row = -1;
    int bad_row = 0;
    if (fits && c.first) {
      new_row = from_top < kFreeWindow ? window_row : L.free_rows[old_free - 1 - from_top];
      if (new_row < 0 || new_row >= C) bad_row = 1;
    }
    if (__ballot(bad_row) != 0) {
      fits = false;
      if (lane == 0) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (lane == 0) {
      if (c.ok && !fits && c.count > 0 && !poisoned) *L.overflow_flag = 1;
      if (poisoned) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (fits && c.count > 0) {
      if (c.first) {
        c.wphys = new_row;
        map_bank[m.widx] = new_row;
      }
#pragma unroll
      for (int j = 0; j < kTraceMaxWrites; ++j) {
        if (j < W && rl(c.first, j)) {
          float* dst = L.values + static_cast<int64_t>(rl(c.wphys, j)) * D;
          float row[VEC];
          copy_from_cur(j, row);
          if (col_ok) store_row<VEC>(dst + col, row);
        }
      }
    }
    return fits;
  };

  // ---- prologue: step 0 classified, published, its rows in flight
  TraceMeta<VEC> cm, nm, pm;   // steps s, s+1, s-1
  TraceClass cc, nc, pc;
  bool alive = true;
  load_meta(0, cm);
  issue_map(cm, cc);
  classify(cm, cc, cm, cc, cm, cc, false, false, alive);
  if constexpr (!DENSE) publish_aggregate(slots, bank, epoch, cc.count, lane);
  issue_loads(cm, cc, ncur_a, rv_a);
  if (G > 1) load_meta(1, nm);
  pm = cm;
  pc = cc;

  auto iteration = [&](int s, float (&nc_c)[kTraceMaxWrites][VEC],
                       float (&rv_c)[kTraceMaxReads][VEC], float (&nc_n)[kTraceMaxWrites][VEC],
                       float (&rv_n)[kTraceMaxReads][VEC]) __attribute__((always_inline)) {
    const bool has_next = s + 1 < G;
    // 0. map lookups of step s+1
    if (has_next) issue_map(nm, nc);
    // 1. pops of step s-1 (its updated rows are still in cur)
    if constexpr (!DENSE) {
      if (s > 0) {
        const bool fits = resolve(pm, pc, s - 1);
        alive = alive && fits;
        if (!fits) cc.ok = 0;
        const int fwd_row = __shfl(pc.wphys, cc.wfwd < 0 ? 0 : cc.wfwd, kWave);
        if (cc.wfwd >= 0) cc.wphys = fwd_row;
      }
    }
    // 2. step s+1: classify, publish, issue its loads
    if (has_next) {
      classify(nm, nc, cm, cc, pm, pc, true, s > 0, alive && cc.ok);
      if constexpr (!DENSE) publish_aggregate(slots, (s + 1) * B + bank, epoch, nc.count, lane);
      issue_loads(nm, nc, nc_n, rv_n);
    }
    // 3. step s
    compute(cm, cc, s, nc_c, rv_c);
    // 4. rows step s wrote, into step s+1
    if (has_next) copy_forwarded(nc, nc_n, rv_n);
    // 5. rotate
    pm = cm;
    pc = cc;
    if (has_next) {
      cm = nm;
      cc = nc;
      if (s + 2 < G) load_meta(s + 2, nm);
    }
  };
  for (int s = 0; s < G; s += 2) {
    iteration(s, ncur_a, rv_a, ncur_b, rv_b);
    if (s + 1 < G) iteration(s + 1, ncur_b, rv_b, ncur_a, rv_a);
  }

  // ---- epilogue: pops of the last step; the last pair closes the launch
  if constexpr (!DENSE) {
    resolve(pm, pc, G - 1);
    if (bank == B - 1) {
      int64_t served = last_inclusive;
      if (last_poisoned || served > old_free) {
        served = fitting_prefix(slots, G * B, epoch, old_free, lane);
      }
      if (lane == 0) {
        *L.free_count = static_cast<int32_t>(old_free - served);
        atomic_store_u64(&scan[COWSDM_SCRATCH_EPOCH], static_cast<uint64_t>(epoch + 1u));
      }
    }
  }
}

// Workgroups of a persistent launch wait on one another, so every one of them
// must be resident at once.  Returns false (nothing launched) when the grid
// exceeds what the device can hold for this kernel; the caller then falls
// back to one launch per step.
template <typename IDX, bool DENSE>
bool launch_trace(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  static int resident[3] = {-1, -1, -1};
  const int which = vec == 4 ? 2 : (vec == 2 ? 1 : 0);
  const void* kernel =
      vec == 4 ? reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 4, DENSE>)
      : vec == 2 ? reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 2, DENSE>)
                 : reinterpret_cast<const void*>(&sdm_trace_kernel<IDX, 1, DENSE>);
  if (resident[which] < 0) {
    int device = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kStepThreads, 0) !=
            hipSuccess) {
      (void)hipGetLastError();
      resident[which] = 0;
    } else {
      resident[which] = cus * per_cu;
    }
  }
  if (blocks > resident[which]) return false;
  if (vec == 4) {
    hipLaunchKernelGGL((sdm_trace_kernel<IDX, 4, DENSE>), dim3(blocks), dim3(kStepThreads), 0,
                       stream, P);
  } else if (vec == 2) {
    hipLaunchKernelGGL((sdm_trace_kernel<IDX, 2, DENSE>), dim3(blocks), dim3(kStepThreads), 0,
                       stream, P);
  } else {
    hipLaunchKernelGGL((sdm_trace_kernel<IDX, 1, DENSE>), dim3(blocks), dim3(kStepThreads), 0,
                       stream, P);
  }
  return true;
}

}  // namespace cowsdm_impl
