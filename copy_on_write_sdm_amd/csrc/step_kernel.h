// The fused copy-on-write SDM step kernel (packed and dense-table forms)
// and its launchers; each step_*.hip file instantiates one index type
// and one form.
#pragma once

#include "common.h"
#include "lookback.h"

namespace cowsdm_impl {

// --------------------------------------------------------- the fused step

// One wave = one bank of one layer.  DENSE selects the dense-table control
// (allocator.py:1612-1633): rows live at values[bank, slot] and there is no
// map, free stack or scan; the row math is shared, so packed and dense
// results are bit-identical.
template <typename IDX, int MAXW, int VEC, bool DENSE>
__global__ __launch_bounds__(kStepThreads) void sdm_step_kernel(StepParams P) {
  const int layer_id = blockIdx.x / P.blocks_per_layer;
  const int bank = (blockIdx.x % P.blocks_per_layer) * kBanksPerBlock +
                   static_cast<int>(threadIdx.x) / kWave;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  if (layer_id >= P.nlayers || bank >= P.banks) return;
  const cowsdm_layer_t& L = P.layer[layer_id];
  const int64_t trace_s = P.trace_step ? P.trace_step[layer_id] : P.trace_first;
  if (P.trace_step && (trace_s < 0 || trace_s >= P.trace_len)) {
    // no recorded step left for this layer: touch no input, leave the counter
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
    return;
  }
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
  int64_t C = L.capacity_rows;
  const int64_t b = bank;
  // Planned single step of a decode trace (packed state with control
  // words): the decode loop's proof for this step, prepare_step_capacity
  // (need) (allocator.py:745-773), made identically by every wave from the
  // control words and free_count.  A growth within the slab's buffers puts
  // row ids C0 .. C0 + added - 1 on top of the found stack (grow_capacity,
  // allocator.py:691-743), so pop q from the top takes C0 + added - 1 - q
  // while q < added and the found stack's entry q - added after.
  const bool planned = !DENSE && P.control != nullptr;
  int64_t grown = 0;        // rows added on top of the found stack
  int64_t proven_after = 0;

  int lane_err = 0;

  // ---- per-bank scalars
  int64_t tmpl = 0;
  if constexpr (!DENSE) {
    tmpl = L.template_indices[b];
    if (tmpl < 0 || tmpl >= P.templates) lane_err |= COWSDM_ERR_TEMPLATE;
  }
  const float forget = forget_gate[b];
  const float in_gate = input_gate[b];
  const float er_gate = erase_gate[b];
  int64_t old_free = 0;
  uint32_t epoch = 0;
  // top kFreeWindow entries of the free stack, entry t (t-th from the top)
  // held by lane t % 64 in register t / 64: pops rarely reach deeper, so the
  // pop needs no dependent load after the bank-order scan
  int free_top[kFreeWindow / kWave];
  if constexpr (!DENSE) {
    old_free = *L.free_count;
    epoch = static_cast<uint32_t>(L.scratch[COWSDM_SCRATCH_EPOCH]);
    if (planned) {
      auto word = [&](int k) __attribute__((always_inline)) -> int64_t {
        const uint64_t v = static_cast<uint64_t>(control_word(P, layer_id, k));
        return static_cast<int64_t>(
            (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32))) << 32) |
            __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
      };
      C = word(COWSDM_CTRL_CAPACITY);
      int64_t proven = word(COWSDM_CTRL_PROVEN);
      const int64_t room = word(COWSDM_CTRL_ROOM);
      const int64_t quantum = word(COWSDM_CTRL_QUANTUM);
      const int64_t need = word(COWSDM_CTRL_NEED);
      bool refused = false;
      if (need > 0 && quantum > 0) {
        if (proven < need) {
          int64_t free_rows = old_free;
          if (free_rows < need) {
            const int64_t want = C + need - free_rows;
            const int64_t selected = (want + quantum - 1) / quantum * quantum;
            if (selected > room || selected >= (int64_t{1} << 31)) {
              refused = true;   // the host grows the slab into larger buffers
            } else {
              grown = selected - C;
              free_rows += grown;
            }
          }
          proven = free_rows;
        }
        proven_after = proven - need;
      } else {
        proven_after = proven;
      }
      if (refused) {
        // the layer takes no step: every wave of it stops here, before any
        // slot is published; the closing bank reports the refusal
        if (bank == P.banks - 1) {
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
        return;
      }
    }
    if (old_free < 0 || old_free > C) lane_err |= COWSDM_ERR_CORRUPT;
#pragma unroll
    for (int k = 0; k < kFreeWindow / kWave; ++k) {
      const int64_t pos = old_free - 1 - (k * kWave + lane);
      free_top[k] = (pos >= 0 && pos < C) ? L.free_rows[pos] : -1;
    }
  }

  // ---- write routes: lane w < W
  int widx = 0;
  float wweight = 0.0f;
  int wphys = -1;
  if (lane < W) {
    const int64_t x = load_index<IDX>(write_indices, b * W + lane);
    wweight = write_weights[b * W + lane];
    if (x < 0 || x >= N) {
      lane_err |= COWSDM_ERR_WRITE_INDEX;
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
        lane_err |= COWSDM_ERR_READ_INDEX;
      } else {
        ridx[k] = static_cast<int>(x);
      }
    }
  }

  // ---- map lookups (packed) for writes and reads
  if constexpr (!DENSE) {
    if (lane < W && !(lane_err & COWSDM_ERR_WRITE_INDEX)) {
      wphys = L.logical_to_physical[b * N + widx];
      if (wphys >= C) lane_err |= COWSDM_ERR_CORRUPT;
    }
#pragma unroll
    for (int k = 0; k < kMaxReadSlots; ++k) {
      const int r = k * kWave + lane;
      if (r < R) {
        rphys[k] = L.logical_to_physical[b * N + ridx[k]];
        if (rphys[k] >= C) lane_err |= COWSDM_ERR_CORRUPT;
      }
    }
  }

  // ---- duplicate writes and read-after-write sources
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    if (j < W) {
      const int other = rl(widx, j);
      if (lane < W && j < lane && other == widx) lane_err |= COWSDM_ERR_DUP_WRITE;
#pragma unroll
      for (int k = 0; k < kMaxReadSlots; ++k) {
        if (k * kWave + lane < R && ridx[k] == other) rsrc[k] = j;
      }
    }
  }

  const int err = wave_or(lane_err);
  const bool ok = (err == 0);
  const bool first = !DENSE && lane < W && wphys < 0;
  const uint64_t first_mask = __ballot(first);
  const int count = ok ? __popcll(first_mask) : 0;
  const int rank = __popcll(first_mask & ((1ull << lane) - 1));

  // ---- chunk 0 row loads, issued before the cross-bank wait
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
      if (j < W && ok) {
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
      if (r < R && ok && read_meta(rsrc, r) < 0) {
        const float* src = read_row_src(r);
        if (col < D) load_row<VEC>(src + col, rv[i]);
      }
    }
  };

  load_writes(0);
  load_read_batch(0, 0);

  // ---- free-stack resolution (packed): bank-major pop positions.  The row
  // math never depends on physical row ids, so the scan waits only in front
  // of the stores of first-touch rows and map entries.
  bool fits = true;
  bool poisoned = false;
  bool resolved = DENSE;
  int new_row = -1;
  int64_t prefix = 0;
  auto resolve = [&]() __attribute__((always_inline)) {
    if constexpr (!DENSE) {
      int64_t* slots = L.scratch + COWSDM_SCRATCH_SLOTS;
      prefix = bank_prefix(slots, bank, epoch, count, lane, &poisoned);
      fits = ok && !poisoned && (count == 0 || prefix + count <= old_free + grown);
      int bad_row = 0;
      const int64_t from_top = prefix + rank;  // pop position counted from the top
      const int64_t found = from_top - grown;  // ... and from the found stack's top
      const int src_lane = static_cast<int>((found < 0 ? 0 : found) % kWave);
      int window_row = -1;
#pragma unroll
      for (int k = 0; k < kFreeWindow / kWave; ++k) {
        const int v = __shfl(free_top[k], src_lane, kWave);
        if (found >= 0 && found / kWave == k) window_row = v;
      }
      if (fits && first) {
        new_row = found < 0 ? static_cast<int>(C + grown - 1 - from_top)
                : found < kFreeWindow ? window_row : L.free_rows[old_free - 1 - found];
        if (new_row < 0 || new_row >= C + grown) bad_row = 1;
      }
      if (__ballot(bad_row) != 0) {
        fits = false;
        if (lane == 0) {
          __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                                static_cast<int64_t>(COWSDM_ERR_CORRUPT),
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (lane == 0) {
        // (planned steps: the closing bank writes the flag)
        if (!planned && ok && !fits && count > 0 && !poisoned) *L.overflow_flag = 1;
        if (poisoned) {
          __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                                static_cast<int64_t>(COWSDM_ERR_LOOKBACK),
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
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

    if (ok) {
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
    if (ok) {
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
      if (ok && fits && count > 0) {
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
  const bool commit = ok && fits;

  bool closed_layer = false;
  if constexpr (!DENSE) {
    if (commit && first) L.logical_to_physical[b * N + widx] = new_row;
    if (lane == 0) {
      if (L.first_touches_out) L.first_touches_out[b] = commit ? count : 0;
      if (L.repeated_writes_out) L.repeated_writes_out[b] = ok ? W - count : W;
      if (err) {
        __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                              static_cast<int64_t>(err), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // The last bank closes the layer.  Its scan ran after every lower bank
    // had published (so all of them read free_count, the epoch and the trace
    // step already).  When it fits, every bank fit and its inclusive prefix
    // is the number of rows popped; otherwise the popped rows are the
    // largest inclusive prefix that fits, read from the other banks' slots.
    if (bank == P.banks - 1) {
      closed_layer = true;
      const int64_t top = old_free + grown;
      int64_t served = prefix + count;
      const bool short_rows = poisoned || served > top;
      if (short_rows) {
        served = fitting_prefix(L.scratch + COWSDM_SCRATCH_SLOTS, P.banks, epoch, top, lane);
      }
      const int64_t now_free = top - served;
      if (planned && now_free > old_free) {
        // the grown rows no pop took stay on the stack, above the found ones
        int32_t* const stack = const_cast<int32_t*>(L.free_rows);
        for (int64_t p = old_free + lane; p < now_free; p += kWave) {
          stack[p] = static_cast<int32_t>(C + (p - old_free));
        }
      }
      if (lane == 0) {
        *L.free_count = static_cast<int32_t>(now_free);
        if (L.allocated_rows_out) {
          *L.allocated_rows_out = static_cast<int32_t>(C + grown - now_free);
        }
        atomic_store_u64(&L.scratch[COWSDM_SCRATCH_EPOCH],
                         static_cast<uint64_t>(epoch + 1u));
        if (planned) {
          if (grown > 0) *L.overflow_flag = 0;   // grow_capacity clears it
          if (short_rows) *L.overflow_flag = 1;
          auto put = [&](int k, int64_t v) __attribute__((always_inline)) {
            atomic_store_u64(&control_word(P, layer_id, k), static_cast<uint64_t>(v));
          };
          const int64_t events = control_word(P, layer_id, COWSDM_CTRL_EVENTS);
          const int64_t added = control_word(P, layer_id, COWSDM_CTRL_ADDED);
          const int64_t copied = control_word(P, layer_id, COWSDM_CTRL_COPIED);
          put(COWSDM_CTRL_PROVEN, short_rows ? 0 : proven_after);
          put(COWSDM_CTRL_CAPACITY, C + grown);
          put(COWSDM_CTRL_EVENTS, events + (grown > 0 ? 1 : 0));
          put(COWSDM_CTRL_ADDED, added + grown);
          put(COWSDM_CTRL_COPIED, copied + (grown > 0 ? C : 0));
          put(COWSDM_CTRL_FREE, now_free);
          put(COWSDM_CTRL_STEPS, 1);
          put(COWSDM_CTRL_FIT, served);
        }
      }
    }
  } else {
    if (lane == 0 && err && L.scratch) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(err), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // device-counted trace launches: the bank that closes the layer moves the
  // layer's counter to the next step (every bank of the layer read it before:
  // packed banks before the bank-order scan, dense banks before their ticket)
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

template <typename IDX, int MAXW, int VEC, bool DENSE>
void launch_step(const StepParams& P, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((sdm_step_kernel<IDX, MAXW, VEC, DENSE>), dim3(blocks),
                     dim3(kStepThreads), 0, stream, P);
}

template <typename IDX, int MAXW, bool DENSE>
void launch_step_vec(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  if (vec == 4) launch_step<IDX, MAXW, 4, DENSE>(P, blocks, stream);
  else if (vec == 2) launch_step<IDX, MAXW, 2, DENSE>(P, blocks, stream);
  else launch_step<IDX, MAXW, 1, DENSE>(P, blocks, stream);
}

template <typename IDX, bool DENSE>
void launch_step_w(const StepParams& P, int blocks, int vec, hipStream_t stream) {
  if (P.writes <= 4) launch_step_vec<IDX, 4, DENSE>(P, blocks, vec, stream);
  else if (P.writes <= 16) launch_step_vec<IDX, 16, DENSE>(P, blocks, vec, stream);
  else launch_step_vec<IDX, 64, DENSE>(P, blocks, vec, stream);
}


}  // namespace cowsdm_impl
