// The token-serial SDM recurrence over dense route vectors: the forward
// recurrence of training and prefill (copy_on_write_sdm/sdm.py:534-607,
// _native_sdm_forward_kernel, launched at sdm.py:829-861), and the scatter
// of sparse routes into dense route vectors (sdm.py:162-172).
//
// Per batch row b and token t, over the whole [N, D] memory:
//   memory[n]  *= exp(forget_log_gate[b, t])   where write_routes[b, t, n] != 0
//   retrieved   = sum_n write_routes[b, t, n] * memory[n]
//   delta       = input_gate[b, t] * values[b, t] - erase_gate[b, t] * retrieved
//   memory[n]  += write_routes[b, t, n] * delta
//   readings[b, t] = sum_n read_routes[b, t, n] * memory[n]
//
// A wave owns 4 columns of one batch row's memory for the whole sequence,
// in registers: lane = 16 * column + row group, and row group g holds rows
// g * RPL .. g * RPL + RPL - 1 (RPL rows per lane, N <= 16 * RPL).  A
// column's 16 row groups are one DPP row of the wave, so both sums over N
// are in-register: each lane's partial sum over its rows, a DPP prefix
// within the row (lane 15 ends with the column's total) and a readlane per
// column, which gives every row of a column the same value.  The tokens of
// a sequence are serial; batch rows and column blocks are independent
// waves.  The inputs of the next tokens are in flight while a token
// computes (route vectors and values up to 8 tokens ahead, as many as 64
// registers hold; the gates of 64 tokens a lane each, a chunk ahead), and
// every load is a vector load whose value is first used tokens later.

#include "common.h"

namespace cowsdm_impl {

constexpr int kRecCols = 4;                  // columns per wave
constexpr int kRecGroups = kWave / kRecCols; // row groups per column: one DPP row
constexpr int kRecWaves = 4;                 // waves per workgroup
constexpr int kRecThreads = kRecWaves * kWave;
constexpr int kRecMaxSlots = 1024;

struct RecParams {
  int64_t batch, time;
  int slots, width, col_blocks;
  const float* m0;       // [B, N, D]
  const float* wr;       // [B, T, N]
  const float* values;   // [B, T, D]
  const float* ig;       // [B, T]
  const float* eg;       // [B, T]
  const float* flg;      // [B, T]
  const float* rr;       // [B, T, N]
  float* readings;       // [B, T, D]
  float* states;         // [B, T, N, D] or null
  float* final_memory;   // [B, N, D] or null
};

// Sum of v over the 16 lanes of each DPP row, the same value in every lane
// of the row: an inclusive DPP prefix within the row (row_shr 1, 2, 4, 8;
// lanes shifted in from outside the row add 0), lane 15 of each row read
// back, the row's value selected by the lane's column.
__device__ __forceinline__ float column_sum(float v, int col) {
  int x = __float_as_int(v);
  x = __float_as_int(__int_as_float(x) +
                     __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false)));
  x = __float_as_int(__int_as_float(x) +
                     __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false)));
  x = __float_as_int(__int_as_float(x) +
                     __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false)));
  x = __float_as_int(__int_as_float(x) +
                     __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false)));
  const float s0 = __int_as_float(__builtin_amdgcn_readlane(x, 15));
  const float s1 = __int_as_float(__builtin_amdgcn_readlane(x, 31));
  const float s2 = __int_as_float(__builtin_amdgcn_readlane(x, 47));
  const float s3 = __int_as_float(__builtin_amdgcn_readlane(x, 63));
  return col == 0 ? s0 : (col == 1 ? s1 : (col == 2 ? s2 : s3));
}

// RPL rows of one route vector (`row`, the same in every lane) from row n0
// on.  Rows at or above N are loaded from row 0 instead and must be masked
// where they are used (a select right after the load would wait for it).
// V4: N % 4 == 0, 16-byte aligned vectors and RPL % 4 == 0.
template <int RPL, bool V4>
__device__ __forceinline__ void load_rows(const float* row, int n0, int N, float (&w)[RPL]) {
  if constexpr (V4) {
#pragma unroll
    for (int j = 0; j < RPL; j += 4) {
      const uint32_t off = n0 + j < N ? static_cast<uint32_t>(n0 + j) : 0u;
      const float4 q = *reinterpret_cast<const float4*>(row + off);
      w[j] = q.x;
      w[j + 1] = q.y;
      w[j + 2] = q.z;
      w[j + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < RPL; ++j) w[j] = row[n0 + j < N ? static_cast<uint32_t>(n0 + j) : 0u];
  }
}

// The RPL rows of a lane's column to or from a [N, D] block (`base`, the
// same in every lane; lane offset n0 * D + d, row stride D): one branch when
// all of them are below N, a check per row otherwise.
template <int RPL>
__device__ __forceinline__ void store_rows(float* base, uint32_t off, uint32_t D, int n0, int N,
                                           const float (&m)[RPL]) {
  if (n0 + RPL <= N) {
#pragma unroll
    for (int i = 0; i < RPL; ++i) base[off + static_cast<uint32_t>(i) * D] = m[i];
  } else {
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      if (n0 + i < N) base[off + static_cast<uint32_t>(i) * D] = m[i];
    }
  }
}

// Tokens whose route vectors are in flight at once: as many as fit in 64
// registers (two vectors of RPL rows each), at most 8 (more spills
// registers and halves the waves a SIMD holds).
template <int RPL>
constexpr int rec_ahead() {
  return 32 / RPL < 1 ? 1 : (32 / RPL > 8 ? 8 : 32 / RPL);
}

// EXACT: N == 16 * RPL, every lane's rows are below N (no masks).
template <int RPL, bool V4, bool EXACT>
__global__ __launch_bounds__(kRecThreads) void recurrence_kernel(RecParams P) {
  constexpr int PF = rec_ahead<RPL>();
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRecWaves + wave;
  if (item >= P.batch * P.col_blocks) return;
  const int64_t b = item / P.col_blocks;
  const int cb = static_cast<int>(item - b * P.col_blocks);
  const int col = lane / kRecGroups;
  const int g = lane % kRecGroups;
  const int N = P.slots, D = P.width;
  const int64_t T = P.time;
  const int d = cb * kRecCols + col;
  const bool col_ok = d < D;
  const int n0 = g * RPL;

  // the lane's rows in a [N, D] block: offset n0 * D + d, stride D (the
  // host keeps N * D below 2^31)
  const uint32_t off = static_cast<uint32_t>(n0) * static_cast<uint32_t>(D) +
                       static_cast<uint32_t>(col_ok ? d : 0);
  float m[RPL];
  {
    const float* src = P.m0 + b * N * static_cast<int64_t>(D);
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const bool in = col_ok && n0 + i < N;
      const float v = src[in ? off + static_cast<uint32_t>(i * D) : 0u];
      m[i] = in ? v : 0.0f;
    }
  }
  const float* const wr_b = P.wr + b * T * N;
  const float* const rr_b = P.rr + b * T * N;
  // ring of PF tokens' route vectors and values: slot j holds token t0 + j
  // of the current round, and is refilled with token t + PF as soon as
  // token t is done.  Every load is a vector load, so a wait for the oldest
  // one does not wait for the newer ones.
  float w[PF][RPL], r[PF][RPL], val[PF];
  auto fetch = [&](int j, int64_t t) __attribute__((always_inline)) {
    load_rows<RPL, V4>(wr_b + t * N, n0, N, w[j]);
    load_rows<RPL, V4>(rr_b + t * N, n0, N, r[j]);
    // a lane past the width computes on column 0's values and stores nothing
    val[j] = P.values[(b * T + t) * D + (col_ok ? d : 0)];
  };
  // the gates of 64 tokens, lane k holding token 64c + k's, a chunk ahead
  float gates[2][3];
  auto fetch_gates = [&](int slot, int64_t c) __attribute__((always_inline)) {
    const int64_t t = c * kWave + lane;
    const int64_t bt = b * T + (t < T ? t : 0);
    gates[slot][0] = P.flg[bt];
    gates[slot][1] = P.ig[bt];
    gates[slot][2] = P.eg[bt];
  };
  if (T > 0) fetch_gates(0, 0);
  if (T > kWave) fetch_gates(1, 1);
  if (T > 0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) fetch(j, j < T ? j : T - 1);
  }
  for (int64_t t0 = 0; t0 < T; t0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int64_t t = t0 + j;
      if (t >= T) break;
      const int64_t bt = b * T + t;
      const int k = static_cast<int>(t % kWave);
      const int slot = static_cast<int>((t / kWave) & 1);
      float fg, in_g, er_g;
      if (slot == 0) {
        fg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[0][0]), k));
        in_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[0][1]), k));
        er_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[0][2]), k));
      } else {
        fg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[1][0]), k));
        in_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[1][1]), k));
        er_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gates[1][2]), k));
      }
      if (k == kWave - 1 && (t / kWave) + 2 < (T + kWave - 1) / kWave) {
        // chunk t / 64 is done: its slot takes the chunk after next
        if (slot == 0) fetch_gates(0, t / kWave + 2); else fetch_gates(1, t / kWave + 2);
      }
      const float alpha = expf(fg);
      float wj[RPL], rj[RPL];
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        wj[i] = EXACT || n0 + i < N ? w[j][i] : 0.0f;
        rj[i] = EXACT || n0 + i < N ? r[j][i] : 0.0f;
      }
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        m[i] = wj[i] != 0.0f ? m[i] * alpha : m[i];
        part = __builtin_fmaf(wj[i], m[i], part);
      }
      const float retrieved = column_sum(part, col);
      const float delta = in_g * val[j] - er_g * retrieved;
      float rp = 0.0f;
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        m[i] = __builtin_fmaf(wj[i], delta, m[i]);
        rp = __builtin_fmaf(rj[i], m[i], rp);
      }
      // the slot takes token t + PF (the last token again near the end, so
      // that every round loads the same registers)
      fetch(j, t + PF < T ? t + PF : T - 1);
      const float reading = column_sum(rp, col);
      if (g == 0 && col_ok) P.readings[bt * D + d] = reading;
      if (P.states && col_ok) {
        store_rows<RPL>(P.states + bt * N * static_cast<int64_t>(D), off, D, n0, N, m);
      }
    }
  }
  if (P.final_memory && col_ok) {
    store_rows<RPL>(P.final_memory + b * N * static_cast<int64_t>(D), off, D, n0, N, m);
  }
}

// Dense route vectors: out[row, n] = the weight of the last k with
// indices[row, k] == n, else 0; an index outside [0, N) sets bit 0x1 of
// *bad.  Thread = (row, n); a row's K indices are read by each of its N
// threads (from cache).
template <typename IDX>
__global__ __launch_bounds__(256) void dense_routes_kernel(const float* weights, const IDX* indices,
                                                           int64_t rows, int k, int slots,
                                                           float* out, int32_t* bad) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= rows * slots) return;
  const int64_t row = e / slots;
  const int n = static_cast<int>(e - row * slots);
  float v = 0.0f;
  bool outside = false;
  for (int j = 0; j < k; ++j) {
    const int64_t x = static_cast<int64_t>(indices[row * k + j]);
    if (x == n) v = weights[row * k + j];
    outside |= (n == 0) && (x < 0 || x >= slots);
  }
  out[e] = v;
  if (outside && bad) atomicOr(bad, 1);
}

template <int RPL>
void launch_recurrence(const RecParams& P, bool v4, unsigned grid, hipStream_t s) {
  const bool exact = P.slots == kRecGroups * RPL;
  if constexpr (RPL >= 4) {
    if (v4 && exact) {
      hipLaunchKernelGGL((recurrence_kernel<RPL, true, true>), dim3(grid), dim3(kRecThreads), 0,
                         s, P);
      return;
    }
    if (v4) {
      hipLaunchKernelGGL((recurrence_kernel<RPL, true, false>), dim3(grid), dim3(kRecThreads), 0,
                         s, P);
      return;
    }
  }
  if (exact) {
    hipLaunchKernelGGL((recurrence_kernel<RPL, false, true>), dim3(grid), dim3(kRecThreads), 0,
                       s, P);
  } else {
    hipLaunchKernelGGL((recurrence_kernel<RPL, false, false>), dim3(grid), dim3(kRecThreads), 0,
                       s, P);
  }
}

}  // namespace cowsdm_impl

using namespace cowsdm_impl;

extern "C" int32_t cowsdm_recurrence_forward(const cowsdm_recurrence_t* r, void* stream) {
  if (!r) return fail(COWSDM_EARG, "recurrence: null argument");
  if (r->batch < 0 || r->time < 0 || r->slots <= 0 || r->width <= 0) {
    return fail(COWSDM_EARG, "recurrence: invalid sizes");
  }
  if (r->slots > kRecMaxSlots) {
    return fail(COWSDM_ELIMIT, "recurrence: at most %d slots", kRecMaxSlots);
  }
  if (r->width > (int64_t{1} << 24) || r->slots * r->width >= (int64_t{1} << 31)) {
    return fail(COWSDM_ELIMIT, "recurrence: width too large");
  }
  if (r->batch == 0) return 0;
  if (!r->initial_memory || (!r->readings && r->time > 0)) {
    return fail(COWSDM_EARG, "recurrence: null pointer argument");
  }
  if (r->time > 0 && (!r->write_routes || !r->values || !r->input_gate || !r->erase_gate ||
                      !r->forget_log_gate || !r->read_routes)) {
    return fail(COWSDM_EARG, "recurrence: null pointer argument");
  }
  RecParams P{};
  P.batch = r->batch;
  P.time = r->time;
  P.slots = static_cast<int>(r->slots);
  P.width = static_cast<int>(r->width);
  P.col_blocks = static_cast<int>((r->width + kRecCols - 1) / kRecCols);
  P.m0 = r->initial_memory;
  P.wr = r->write_routes;
  P.values = r->values;
  P.ig = r->input_gate;
  P.eg = r->erase_gate;
  P.flg = r->forget_log_gate;
  P.rr = r->read_routes;
  P.readings = r->readings;
  P.states = r->states;
  P.final_memory = r->final_memory;
  const int64_t waves = P.batch * P.col_blocks;
  const int64_t grid = (waves + kRecWaves - 1) / kRecWaves;
  if (grid > (int64_t{1} << 31) - 1) return fail(COWSDM_ELIMIT, "recurrence: batch too large");
  const int groups_rows = (P.slots + kRecGroups - 1) / kRecGroups;   // rows per lane needed
  const uintptr_t align = reinterpret_cast<uintptr_t>(P.wr) | reinterpret_cast<uintptr_t>(P.rr);
  const bool v4 = P.slots % 4 == 0 && align % 16 == 0;
  const unsigned g = static_cast<unsigned>(grid);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (groups_rows <= 1) {
    launch_recurrence<1>(P, v4, g, s);
  } else if (groups_rows <= 2) {
    launch_recurrence<2>(P, v4, g, s);
  } else if (groups_rows <= 4) {
    launch_recurrence<4>(P, v4, g, s);
  } else if (groups_rows <= 8) {
    launch_recurrence<8>(P, v4, g, s);
  } else if (groups_rows <= 16) {
    launch_recurrence<16>(P, v4, g, s);
  } else if (groups_rows <= 32) {
    launch_recurrence<32>(P, v4, g, s);
  } else {
    launch_recurrence<64>(P, v4, g, s);
  }
  return launch_status("recurrence");
}

extern "C" int32_t cowsdm_dense_routes(const float* weights, const void* indices,
                                       int32_t index_dtype, int64_t rows, int64_t per_row,
                                       int64_t slots, float* dense, int32_t* bad, void* stream) {
  if (rows < 0 || per_row < 0 || slots <= 0) return fail(COWSDM_EARG, "dense routes: invalid sizes");
  if (per_row > 1024 || slots > (int64_t{1} << 30)) {
    return fail(COWSDM_ELIMIT, "dense routes: shape outside the supported range");
  }
  if (index_dtype != COWSDM_INDEX_INT32 && index_dtype != COWSDM_INDEX_INT64) {
    return fail(COWSDM_EARG, "dense routes: unknown index dtype");
  }
  if (rows == 0) return 0;
  if (!dense || (per_row > 0 && (!weights || !indices))) {
    return fail(COWSDM_EARG, "dense routes: null pointer argument");
  }
  const int64_t total = rows * slots;
  const int64_t grid = (total + 255) / 256;
  if (grid > (int64_t{1} << 31) - 1) return fail(COWSDM_ELIMIT, "dense routes: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (index_dtype == COWSDM_INDEX_INT32) {
    hipLaunchKernelGGL(dense_routes_kernel<int32_t>, dim3(static_cast<unsigned>(grid)), dim3(256),
                       0, s, weights, static_cast<const int32_t*>(indices), rows,
                       static_cast<int>(per_row), static_cast<int>(slots), dense, bad);
  } else {
    hipLaunchKernelGGL(dense_routes_kernel<int64_t>, dim3(static_cast<unsigned>(grid)), dim3(256),
                       0, s, weights, static_cast<const int64_t*>(indices), rows,
                       static_cast<int>(per_row), static_cast<int>(slots), dense, bad);
  }
  return launch_status("dense routes");
}
