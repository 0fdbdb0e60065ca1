// Bank-order exclusive scan by decoupled look-back.  Each participant q
// (a bank, or a (step, bank) pair of a multi-step launch) owns one 64-bit
// slot: epoch (high 32 bits), status (2 bits), value (30 bits).  It first
// publishes its aggregate, later resolves its exclusive prefix by reading the
// slots below it, then publishes its inclusive prefix.  A participant waits
// only on lower-numbered slots; every wait is bounded, and a timed-out slot
// poisons the prefix instead of hanging.
#pragma once

#include "common.h"

namespace cowsdm_impl {

__device__ inline void publish_aggregate(int64_t* slots, int q, uint32_t epoch, int count,
                                         int lane) {
  if (lane == 0) {
    atomic_store_u64(&slots[q], slot_word(epoch, kStatusAggregate, count));
  }
}

// Exclusive prefix of slot q; publishes q's inclusive prefix.  The aggregate
// of q must have been published by publish_aggregate.
__device__ inline int64_t resolve_prefix(int64_t* slots, int q, uint32_t epoch, int count,
                                         int lane, bool* poisoned) {
  int64_t exclusive = 0;
  bool bad = false;
  int end = q;
  while (end > 0) {
    const int j = end - 1 - lane;
    uint32_t status = kStatusInclusive;
    int64_t value = 0;
    if (j >= 0) {
      uint64_t w = atomic_load_u64(&slots[j]);
      int spins = 0;
      while ((static_cast<uint32_t>(w >> 32) != epoch ||
              ((w >> 30) & 3u) == kStatusEmpty) &&
             spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
        w = atomic_load_u64(&slots[j]);
        ++spins;
      }
      if (static_cast<uint32_t>(w >> 32) != epoch ||
          ((w >> 30) & 3u) == kStatusEmpty) {
        status = kStatusPoison;
      } else {
        status = static_cast<uint32_t>((w >> 30) & 3u);
        value = static_cast<int64_t>(w & kValueMask);
      }
    }
    const uint64_t inclusive = __ballot(status == kStatusInclusive);
    const uint64_t poison = __ballot(status == kStatusPoison);
    if (inclusive != 0) {
      const int k = __ffsll(static_cast<long long>(inclusive)) - 1;
      const uint64_t upto = (k == 63) ? ~0ull : ((2ull << k) - 1);
      if (poison & upto) bad = true;
      exclusive += wave_sum64(lane <= k ? value : 0);
      break;
    }
    if (poison != 0) bad = true;
    exclusive += wave_sum64(value);
    end -= kWave;
  }
  if (lane == 0) {
    atomic_store_u64(&slots[q],
                     slot_word(epoch, bad ? kStatusPoison : kStatusInclusive,
                               static_cast<uint64_t>(exclusive + count)));
  }
  *poisoned = bad;
  return exclusive;
}

// Publish-and-resolve in one call (single-step launches).
__device__ inline int64_t bank_prefix(int64_t* slots, int q, uint32_t epoch, int count,
                                      int lane, bool* poisoned) {
  publish_aggregate(slots, q, epoch, count, lane);
  return resolve_prefix(slots, q, epoch, count, lane, poisoned);
}

// Largest inclusive prefix <= limit among slots [0, n) of this epoch: the
// rows a launch actually popped when some participant did not fit.
__device__ inline int64_t fitting_prefix(int64_t* slots, int n, uint32_t epoch, int64_t limit,
                                         int lane) {
  int64_t best = 0;
  for (int j0 = 0; j0 < n; j0 += kWave) {
    const int j = j0 + lane;
    if (j < n) {
      uint64_t w = atomic_load_u64(&slots[j]);
      int spins = 0;
      while (static_cast<uint32_t>(w >> 32) == epoch &&
             ((w >> 30) & 3u) == kStatusAggregate && spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
        w = atomic_load_u64(&slots[j]);
        ++spins;
      }
      const bool inclusive = static_cast<uint32_t>(w >> 32) == epoch &&
                             ((w >> 30) & 3u) == kStatusInclusive;
      const int64_t v = static_cast<int64_t>(w & kValueMask);
      if (inclusive && v <= limit && v > best) best = v;
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const int64_t other = __shfl_xor(best, o, kWave);
    best = other > best ? other : best;
  }
  return best;
}

}  // namespace cowsdm_impl
