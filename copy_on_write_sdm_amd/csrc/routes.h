// Product-key route selection on the device: the producer of the decode
// step's write and read routes (copy_on_write_sdm/sdm.py:96-159).  Shared by
// routes.hip (cowsdm_product_key_routes) and controller.hip (the controller's
// prepare kernel selects its tokens' routes itself).
//
// One wave per route row.  A row holds 2*root scores (root = sqrt(N)); the
// two halves are shortlisted independently to their top `sub` = min(k, root)
// entries, the sub*sub pair sums are ranked, the best min(k, sub*sub) pairs
// become slots (first * root + second), sorted by slot, and their scores go
// through a softmax.
//
// Selection ranks every candidate at once: a candidate's key is its score in
// order-preserving bits above its inverted position, so keys are unique and
// "higher key" means "selected first" (higher score, then lower position;
// torch.topk leaves the order of equal scores open, and only a tie at the
// selection boundary can change which slot is selected).  Each lane counts
// the keys of the wave, broadcast one at a time with readlane, that beat its
// own; a candidate whose rank is below the count writes itself to LDS at its
// rank.  All inputs must be finite.

#pragma once

#include <algorithm>

#include "common.h"

namespace cowsdm_impl {

constexpr int kRouteWaves = 4;                 // rows per workgroup
constexpr int kRouteMaxRoot = 1024;            // N <= 2^20
constexpr int kRouteMaxSelected = 32;          // pair-stage candidates <= 128

// -0.0 is added to +0.0 first so that equal scores get equal bits.
__device__ __forceinline__ uint64_t route_key(float v, int pos) {
  uint32_t bits = __float_as_uint(v + 0.0f);
  bits = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<uint64_t>(bits) << 32) | static_cast<uint32_t>(~pos);
}

// rank[j] = number of keys in the wave (J per lane, absent ones 0) above key[j];
// lanes from LANES on hold absent keys only (every present key is above 0),
// so only the first LANES are broadcast
template <int J, int LANES = kWave>
__device__ __forceinline__ void wave_rank(const uint64_t (&key)[J], int (&rank)[J]) {
#pragma unroll
  for (int j = 0; j < J; ++j) rank[j] = 0;
#pragma unroll
  for (int j2 = 0; j2 < J; ++j2) {
    const uint32_t lo = static_cast<uint32_t>(key[j2]);
    const uint32_t hi = static_cast<uint32_t>(key[j2] >> 32);
    auto count = [&](int u) {
      const uint64_t other =
          (static_cast<uint64_t>(static_cast<uint32_t>(rl(static_cast<int>(hi), u))) << 32) |
          static_cast<uint32_t>(rl(static_cast<int>(lo), u));
#pragma unroll
      for (int j = 0; j < J; ++j) rank[j] += other > key[j] ? 1 : 0;
    };
    if constexpr (J <= 4) {
#pragma unroll
      for (int u = 0; u < LANES; ++u) count(u);   // lane selects as immediates
    } else {
      for (int u = 0; u < LANES; ++u) count(u);
    }
  }
}

// LDS written by lanes of one wave and read by others of the same wave
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Lane t < count ends with the t-th best (value, position) of the wave's
// candidates (pos < 0: absent).  stage_val/stage_pos hold kRouteMaxSelected
// entries of this wave.
template <int J, int LANES = kWave>
__device__ __forceinline__ void wave_top(const float (&val)[J], const int (&pos)[J], int count,
                                         int lane, float* stage_val, int* stage_pos,
                                         float& top_val, int& top_pos) {
  uint64_t key[J];
  int rank[J];
#pragma unroll
  for (int j = 0; j < J; ++j) key[j] = pos[j] >= 0 ? route_key(val[j], pos[j]) : 0;
  wave_rank<J, LANES>(key, rank);
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (pos[j] >= 0 && rank[j] < count) {
      stage_val[rank[j]] = val[j];
      stage_pos[rank[j]] = pos[j];
    }
  wave_lds_sync();
  top_val = lane < count ? stage_val[lane] : -__builtin_inff();
  top_pos = lane < count ? stage_pos[lane] : 0;
  wave_lds_sync();
}

// wave_top for J > 1 (root > 64, every lane holds at least one entry).  The
// count-th largest lane maximum T bounds the selection: count lane maxima
// are >= T, so an entry below T ranks at least count and is never selected.
// The entries >= T (about count + count/4 for random scores) are compacted
// into one per lane and ranked once; if more than 64 remain (many equal
// scores), every entry is ranked.
template <int J>
__device__ __forceinline__ void wave_top_pruned(const float (&val)[J], const int (&pos)[J],
                                                int count, int lane, float* stage_val,
                                                int* stage_pos, float* pool_val, int* pool_pos,
                                                float& top_val, int& top_pos) {
  uint64_t key[J];
  uint64_t best[1] = {0};
#pragma unroll
  for (int j = 0; j < J; ++j) {
    key[j] = pos[j] >= 0 ? route_key(val[j], pos[j]) : 0;
    best[0] = key[j] > best[0] ? key[j] : best[0];
  }
  int best_rank[1];
  wave_rank<1>(best, best_rank);   // 64 unique lane maxima: ranks 0..63
  const uint64_t at = __ballot(best_rank[0] == count - 1);
  const int holder = at ? __builtin_ctzll(at) : 0;
  const uint64_t bound =
      (static_cast<uint64_t>(static_cast<uint32_t>(rl(static_cast<int>(best[0] >> 32), holder)))
       << 32) |
      static_cast<uint32_t>(rl(static_cast<int>(static_cast<uint32_t>(best[0])), holder));
  uint64_t mask[J];
  int total = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    mask[j] = __ballot(pos[j] >= 0 && key[j] >= bound);
    total += __popcll(mask[j]);
  }
  if (total > kWave) {
    wave_top<J>(val, pos, count, lane, stage_val, stage_pos, top_val, top_pos);
    return;
  }
  const uint64_t below = (uint64_t{1} << lane) - 1;
  int base = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if ((mask[j] >> lane) & 1) {
      const int slot = base + __popcll(mask[j] & below);   // < total <= 64
      pool_val[slot] = val[j];
      pool_pos[slot] = pos[j];
    }
    base += __popcll(mask[j]);
  }
  wave_lds_sync();
  float one_val[1] = {lane < total ? pool_val[lane] : -__builtin_inff()};
  int one_pos[1] = {lane < total ? pool_pos[lane] : -1};
  wave_lds_sync();
  wave_top<1>(one_val, one_pos, count, lane, stage_val, stage_pos, top_val, top_pos);
}

// Row `row` of `projected` ([rows, 2 * root]) by the calling wave: its
// final_k routes (weights and slots, sorted by slot) at row * final_k.
// stage_val/stage_pos (kRouteMaxSelected entries) and pool_val/pool_pos
// (kWave entries) are this wave's LDS.
template <int J, int M>
__device__ __forceinline__ void product_key_route_row(
    const float* __restrict__ projected, int64_t row, int root, int sub, int final_k,
    float* __restrict__ weights, int64_t* __restrict__ indices, float* stage_val,
    int* stage_pos, float* pool_val, int* pool_pos) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const float* first = projected + row * 2 * root;
  const float* second = first + root;

  // 1. shortlist each half: entry e = lane + 64 j
  float fv[J], sv[J];
  int fp[J], sp[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + kWave * j;
    const bool in = e < root;
    fv[j] = in ? first[e] : -__builtin_inff();
    sv[j] = in ? second[e] : -__builtin_inff();
    fp[j] = in ? e : -1;
    sp[j] = in ? e : -1;
  }
  float first_val, second_val;
  int first_idx, second_idx;
  if constexpr (J > 1) {
    wave_top_pruned<J>(fv, fp, sub, lane, stage_val, stage_pos, pool_val,
                       pool_pos, first_val, first_idx);
    wave_top_pruned<J>(sv, sp, sub, lane, stage_val, stage_pos, pool_val,
                       pool_pos, second_val, second_idx);
  } else if (root <= 16) {
    // root <= 64: entries only in lanes below root
    wave_top<J, 16>(fv, fp, sub, lane, stage_val, stage_pos, first_val, first_idx);
    wave_top<J, 16>(sv, sp, sub, lane, stage_val, stage_pos, second_val, second_idx);
  } else if (root <= 32) {
    wave_top<J, 32>(fv, fp, sub, lane, stage_val, stage_pos, first_val, first_idx);
    wave_top<J, 32>(sv, sp, sub, lane, stage_val, stage_pos, second_val, second_idx);
  } else {
    wave_top<J>(fv, fp, sub, lane, stage_val, stage_pos, first_val, first_idx);
    wave_top<J>(sv, sp, sub, lane, stage_val, stage_pos, second_val, second_idx);
  }

  // 2. pair c = a * sub + b scores first_val[a] + second_val[b].  Every pair
  // (a', b') <= (a, b) scores at least as high (float addition is monotone)
  // and has a lower position, so (a, b) ranks at least (a+1)(b+1) - 1 and can
  // be selected only if (a+1)(b+1) <= final_k: at most
  // sum_a min(sub, final_k / (a+1)) candidates, enumerated a-major.
  float cv[M];
  int cp[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int rest = lane + kWave * m, a = -1, b = 0;
    for (int t = 0; t < sub; ++t) {
      const int per = min(sub, final_k / (t + 1));
      if (a < 0) {
        if (rest < per) { a = t; b = rest; } else { rest -= per; }
      }
    }
    const bool in = a >= 0;
    const float va = __shfl(first_val, in ? a : 0, kWave);
    const float vb = __shfl(second_val, b, kWave);
    cv[m] = in ? va + vb : -__builtin_inff();
    cp[m] = in ? a * sub + b : -1;
  }
  float score;
  int pair;
  wave_top<M>(cv, cp, final_k, lane, stage_val, stage_pos, score, pair);

  // 3. slot of each selected pair, its rank by slot, softmax of the scores
  const bool mine = lane < final_k;
  const int a = mine ? pair / sub : 0;
  const int b = mine ? pair - a * sub : 0;
  const int fa = __shfl(first_idx, a, kWave);
  const int sb = __shfl(second_idx, b, kWave);
  const int64_t slot = static_cast<int64_t>(fa) * root + sb;
  int rank = 0;
  for (int u = 0; u < final_k; ++u) {
    const int64_t other = static_cast<int64_t>(rl(static_cast<int>(slot), u));
    rank += other < slot ? 1 : 0;
  }
  float mx = mine ? score : -__builtin_inff();
  for (int o = kWave / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  const float e = mine ? expf(score - mx) : 0.0f;
  float total = e;
  for (int o = kWave / 2; o > 0; o >>= 1) total += __shfl_xor(total, o, kWave);
  if (mine) {
    weights[row * final_k + rank] = e / total;
    indices[row * final_k + rank] = slot;
  }
}


// The selection's shape for N slots and `selected` routes a row: root =
// sqrt(N), sub = min(selected, root) entries shortlisted per half, final_k =
// min(selected, sub * sub) routes; 0, or the error of
// cowsdm_product_key_routes (recorded by fail()).
inline int32_t route_geometry(int64_t slots, int64_t selected, int& root_out, int& sub_out,
                              int& final_out) {
  int64_t root = 0;
  while ((root + 1) * (root + 1) <= slots) ++root;
  if (slots < 1 || root * root != slots)
    return fail(-1, "slot count and product-key projection do not match");
  if (selected < 1 || selected > slots)
    return fail(-1, "selected product keys must be between one and slots");
  if (root > kRouteMaxRoot)
    return fail(-2, "product_key_routes: sqrt(slots) <= %d on the HIP path (got %lld)",
                kRouteMaxRoot, static_cast<long long>(root));
  const int64_t sub = selected < root ? selected : root;
  if (sub > kRouteMaxSelected)
    return fail(-2, "product_key_routes: min(selected, sqrt(slots)) <= %d on the HIP path "
                "(got %lld)", kRouteMaxSelected, static_cast<long long>(sub));
  const int64_t final_k = selected < sub * sub ? selected : sub * sub;
  if (final_k > kRouteMaxSelected)
    return fail(-2, "product_key_routes: at most %d routes per row on the HIP path (got %lld)",
                kRouteMaxSelected, static_cast<long long>(final_k));
  root_out = static_cast<int>(root);
  sub_out = static_cast<int>(sub);
  final_out = static_cast<int>(final_k);
  return 0;
}

// Candidates of the pair stage over 64: the selection's M (1 or 2).
inline int route_pair_m(int sub, int final_k) {
  int pairs = 0;   // at most 119 for final_k <= 32
  for (int t = 0; t < sub; ++t) pairs += std::min(sub, final_k / (t + 1));
  return pairs <= kWave ? 1 : 2;
}

}  // namespace cowsdm_impl
