// The plan of a packed decode-trace launch, made inside the persistent
// kernel (trace_kernel.h) by its control waves before any step runs.
//
// The reference's decode loop proves every step on the host before running
// it (inference.py:551-552: prepare_step_capacity(banks * W), allocator.py:
// 745-773): the proven counter drops by banks * W per step, free_count is
// read only when the counter runs short, and the slab grows by the pooled
// quantum only when free_count is below banks * W at such a read
// (grow_capacity, allocator.py:691-743: new row ids join the top of the free
// stack).  Single steps pop first-touch rows bank-major from the top of the
// stack (allocator.py:1471-1481).  Every one of those decisions depends only
// on how many first touches each (step, bank) makes, and that depends only
// on the routes and on which slots were mapped when the launch starts: slot
// x is first-touched by the first step of the launch that writes it, unless
// it was mapped already.  So the launch is settled up front, in four parts:
//
//   count (every control wave, its own bank; or the count kernel when the
//   slot map does not fit in LDS): each step's first-touch write lanes and
//   the bank's first step with an invalid route, after which the bank takes
//   no step, as count words;
//
//   prefix (every control wave, a contiguous share of the steps): for each
//   of its steps, the first touches of the lower banks at that step (a scan
//   across the banks' count words) and the step's total;
//
//   layer (the control wave of bank 0): the running totals over the steps,
//   the decode loop's proof step by step from the control words (growing
//   the capacity within the slab's buffers, or stopping the layer before a
//   growth that would not fit), free_count and the overflow flag the launch
//   leaves, and a header with the steps the layer runs, the pops that fit
//   and the capacity.  With slot maps in LDS (few first touches per launch)
//   it also lists the row every pop takes and rewrites the free stack; else
//   it publishes the launch's growth segments (the first pop, stack heights
//   and capacity of each growth) for the banks to list from;
//
//   header (every control wave): waits for the header; with slot maps in
//   global memory each control wave then lists its own bank's pops, and the
//   layer's last one to finish listing rewrites the free stack.
//
// Waves of different workgroups (on different XCDs) exchange only tagged
// words (common.h): a word is read with device-scope atomic loads until it
// carries the launch's epoch.  Every wait is bounded.  The persistent kernel
// then takes each (step, bank)'s pops at the running total of its step plus
// its prefix, so maps, slabs and free stacks equal those of the single-step
// loop bit for bit.
#pragma once

#include "common.h"

namespace cowsdm_impl {

// Loads *p (lanes with `want`) until every wanted word carries `epoch` (and,
// with `prefix`, is a prefix word); false when some never does (bounded).
__device__ __forceinline__ bool poll_tagged(const int64_t* p, bool want, uint32_t epoch,
                                            uint64_t& w, bool prefix = false) {
  const uint64_t done = prefix ? kPrefixDone : 0u;
  auto ready = [&](uint64_t x) __attribute__((always_inline)) {
    return tag_is(x, epoch) && (x & done) == done;
  };
  w = want ? atomic_load_u64(p) : tagged(epoch, static_cast<uint32_t>(done));
  for (int spins = 0; __ballot(want && !ready(w)) != 0; ++spins) {
    if (spins >= kSpinLimit) return false;
    __builtin_amdgcn_s_sleep(1);
    if (want && !ready(w)) w = atomic_load_u64(p);
  }
  return true;
}

// v, known to the compiler as the same in every lane
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// a / b for 0 <= a, 0 < b, in 32 bits when both fit
__device__ __forceinline__ int64_t plan_div(int64_t a, int64_t b) {
  if (a < (int64_t{1} << 31) && b < (int64_t{1} << 31)) {
    return static_cast<int64_t>(static_cast<uint32_t>(a) / static_cast<uint32_t>(b));
  }
  return a / b;
}

// Prefix part over steps [t_begin, t_end), each against every bank (lane =
// bank): waits for the banks' count words of the step, replaces each with
// its prefix word and publishes the step's total.  A bank's words of
// consecutive steps are contiguous, so a lane loads kBatch steps at once,
// and the batch is polled together.  False when a count never arrives.
__device__ inline bool plan_prefix(const PlanBlock& pb, int B, uint32_t epoch, int t_begin,
                                   int t_end) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  constexpr int kBatch = 8;
  for (int tb = t_begin; tb < t_end; tb += kBatch) {
    int carry[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) carry[i] = 0;
    for (int g = 0; g < B; g += kWave) {
      const int b = g + lane;
      const bool in = b < B;
      int64_t* const row = pb.word(in ? b : 0, 0);
      uint64_t w[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int t = tb + i < t_end ? tb + i : t_end - 1;
        w[i] = in ? atomic_load_u64(row + t) : tagged(epoch, 0);
      }
      // each round reloads only the words still missing, so the batch waits
      // one round trip past its last count rather than one per step
      for (int spins = 0;; ++spins) {
        bool missing = false;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) missing |= tb + i < t_end && !tag_is(w[i], epoch);
        if (__ballot(missing) == 0) break;
        if (spins >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          if (tb + i < t_end && !tag_is(w[i], epoch)) w[i] = atomic_load_u64(row + tb + i);
        }
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int t = tb + i;
        if (t >= t_end) break;
        const uint32_t v = static_cast<uint32_t>(w[i]) & (kCountStop | 15u);
        const int c = __popc(v & 15u);
        const int incl = wave_inclusive(c);
        if (in) {
          const uint32_t pre = static_cast<uint32_t>(carry[i] + incl - c);
          atomic_store_u64(row + t, tagged(epoch, v | (pre << kPrefixShift) | kPrefixDone));
        }
        carry[i] += __builtin_amdgcn_readlane(incl, kWave - 1);
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (tb + i < t_end) {
          atomic_store_u64(pb.totals + tb + i, tagged(epoch, static_cast<uint32_t>(carry[i])));
        }
      }
    }
  }
  return true;
}

// The words the layer part starts from: the control words and the free
// count the launch found.  Loaded by the layer part's wave at its start, so
// that their latency hides behind the count and prefix parts.
struct PlanControl {
  int64_t capacity, proven, room, quantum, need, events, added, copied;
  int32_t free_count;
};
__device__ __forceinline__ PlanControl plan_control(const StepParams& P, int layer) {
  PlanControl c;
  c.capacity = control_word(P, layer, COWSDM_CTRL_CAPACITY);
  c.proven = control_word(P, layer, COWSDM_CTRL_PROVEN);
  c.room = control_word(P, layer, COWSDM_CTRL_ROOM);
  c.quantum = control_word(P, layer, COWSDM_CTRL_QUANTUM);
  c.need = control_word(P, layer, COWSDM_CTRL_NEED);
  c.events = control_word(P, layer, COWSDM_CTRL_EVENTS);
  c.added = control_word(P, layer, COWSDM_CTRL_ADDED);
  c.copied = control_word(P, layer, COWSDM_CTRL_COPIED);
  c.free_count = *P.layer[layer].free_count;
  return c;
}

// ---- the local plan of a short launch
//
// A launch of at most kLocalPlanSteps steps over at most kWave banks, with
// slot maps in LDS, first tries a plan that every control wave makes by
// itself.  Each bank's count part also publishes its count words packed,
// kLocalStepsPerWord steps to a tagged word, at the end of its row of plan
// words (past the launch's steps).  Every control wave reads all banks'
// packed words (lane = bank), takes each step's first touches of the lower
// banks and its total from ballots of the banks' first-touch lanes, adds
// the totals up into running totals, and walks the decode loop's proof from
// the control words.  When the launch neither grows the slab nor overflows
// it, that is the whole plan: the bank's first touches pop the found
// stack's entries free_count - 1 - (running total + prefix + rank)
// directly, with no prefix, layer or header part and no pop list, and the
// layer's last control wave to finish writes the free count and control
// words the launch leaves.  A launch that grows, overflows, or finds a
// corrupt free count takes the central plan instead: every wave decides so
// from the same words, so all of them do.
constexpr int kLocalPlanSteps = 32;
constexpr int kLocalBits = 5;   // a count word: 4 first-touch lanes and the stop bit
constexpr int kLocalStepsPerWord = 32 / kLocalBits;
constexpr int kLocalWords = (kLocalPlanSteps + kLocalStepsPerWord - 1) / kLocalStepsPerWord;
static_assert(kLocalWords <= kPlanLocalWords, "the plan block's local rows hold every packed word");

__host__ __device__ constexpr int local_words(int steps) {
  return (steps + kLocalStepsPerWord - 1) / kLocalStepsPerWord;
}
// packed word k of a bank: row k of the plan block's local words, one word
// per bank, so that a wave reading every bank's word k (lane = bank) reads
// one contiguous row
__device__ __forceinline__ int64_t* local_word(const PlanBlock& pb, int bank, int k) {
  return pb.local + k * kWave + bank;
}

// Whether a launch of G0 steps over B banks takes the local plan first.
__device__ __forceinline__ bool local_plan_fits(int G0, int B, const PlanBlock& pb) {
  (void)pb;
  return G0 <= kLocalPlanSteps && B <= kWave;
}

struct LocalPlan {
  int fit;          // the pops the launch gives: all of its first touches
  int found;        // the stack height the launch found
  int64_t proven;   // the proof counter the launch leaves
};

// 1: planned (this bank's plan words are in plan_words[0, G0)); 0: the
// launch needs the central plan; -1: a count word never arrived (bounded).
__device__ inline int plan_local(const PlanBlock& pb, int B, int G0, uint32_t epoch, int bank,
                                 const PlanControl& pc, int* plan_words, LocalPlan& out) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const bool in = lane < B;
  const int nw = local_words(G0);
  // every bank's packed count words, lane = bank
  uint64_t w[kLocalWords];
#pragma unroll
  for (int k = 0; k < kLocalWords; ++k) {
    w[k] = k < nw && in ? atomic_load_u64(local_word(pb, lane, k)) : tagged(epoch, 0);
  }
  for (int spins = 0;; ++spins) {
    bool missing = false;
#pragma unroll
    for (int k = 0; k < kLocalWords; ++k) missing |= !tag_is(w[k], epoch);
    if (__ballot(missing) == 0) break;
    if (spins >= kSpinLimit) return -1;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < kLocalWords; ++k) {
      if (k < nw && in && !tag_is(w[k], epoch)) w[k] = atomic_load_u64(local_word(pb, lane, k));
    }
  }
  // The first touches of the lower banks at each step (pre) and the step's
  // total over all banks (tot), word by word (lane = bank): a step that no
  // bank first-touches adds nothing, so only the word's active steps are
  // summed, by ballots of their first-touch lanes when they are few, else by
  // two scans across the wave of three steps each, packed in 9-bit fields
  // (a sum over 64 banks of at most 4 each fits).  Lane t keeps the running
  // total before step t (cum_l), the lower banks' first touches at step t
  // (pre_l) and this bank's count word of step t (own_l).
  constexpr int kSumBits = 9;
  constexpr int kSumSteps = 3;
  constexpr int kBallotSteps = 3;   // active steps of a word summed by ballots
  constexpr uint32_t kField = (1u << kLocalBits) - 1;
  constexpr uint32_t kTouchFields = [] {
    uint32_t m = 0;
    for (int i = 0; i < kLocalStepsPerWord; ++i) m |= 15u << (kLocalBits * i);
    return m;
  }();
  const uint64_t lower = (uint64_t{1} << bank) - 1;   // bank < kWave
  const int lane_word = lane / kLocalStepsPerWord;
  const int lane_shift = kLocalBits * (lane % kLocalStepsPerWord);
  int cum_l = 0;
  int pre_l = 0;
  int cum_g = 0;
  uint32_t own_l = 0;
  auto add_step = [&](int t, int pre, int tot) __attribute__((always_inline)) {
    if (lane == t) pre_l = pre;
    if (lane > t) cum_l += tot;
    cum_g += tot;
  };
#pragma unroll
  for (int k = 0; k < kLocalWords; ++k) {
    if (k < nw) {
      const uint32_t lo = static_cast<uint32_t>(w[k]);
      const uint32_t own = static_cast<uint32_t>(
          __builtin_amdgcn_readlane(static_cast<int>(lo), bank));
      if (lane_word == k) own_l = (own >> lane_shift) & kField;
      const int steps_here = G0 - k * kLocalStepsPerWord;
      const uint32_t valid =
          steps_here >= kLocalStepsPerWord ? ~0u : (1u << (kLocalBits * steps_here)) - 1;
      uint32_t act = wave_or_all(lo) & kTouchFields & valid;
      // one bit per active field
      uint32_t fields = 0;
#pragma unroll
      for (int f = 0; f < kLocalStepsPerWord; ++f) {
        if ((act >> (kLocalBits * f)) & 15u) fields |= 1u << f;
      }
      if (__popc(fields) <= kBallotSteps) {
        while (fields != 0) {
          const int f = __builtin_ctz(fields);
          fields &= fields - 1;
          int pre = 0, tot = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint64_t m = __ballot((lo >> (kLocalBits * f + j)) & 1u);
            pre += __popcll(m & lower);
            tot += __popcll(m);
          }
          add_step(k * kLocalStepsPerWord + f, pre, tot);
        }
      } else {
#pragma unroll
        for (int h = 0; h < kLocalStepsPerWord / kSumSteps; ++h) {
          int packed = 0;
#pragma unroll
          for (int i = 0; i < kSumSteps; ++i) {
            const int f = h * kSumSteps + i;
            packed += __popc((lo >> (kLocalBits * f)) & 15u) << (kSumBits * i);
          }
          const int incl = wave_inclusive(packed);
          const uint32_t lw = static_cast<uint32_t>(__builtin_amdgcn_readlane(incl - packed, bank));
          const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(incl, kWave - 1));
#pragma unroll
          for (int i = 0; i < kSumSteps; ++i) {
            const int t = k * kLocalStepsPerWord + h * kSumSteps + i;
            if (t < G0) {
              add_step(t, static_cast<int>((lw >> (kSumBits * i)) & ((1u << kSumBits) - 1)),
                       static_cast<int>((total >> (kSumBits * i)) & ((1u << kSumBits) - 1)));
            }
          }
        }
      }
    }
  }
  const uint32_t word_l =
      (static_cast<uint32_t>(cum_l + pre_l) & kPlanBaseMask) | ((own_l & 15u) << kPlanMaskShift) |
      ((own_l & kCountStop) ? 1u << kPlanStopBit : 0u);
  auto cum_at = [&](int s) __attribute__((always_inline)) -> int {
    return s >= G0 ? cum_g : __builtin_amdgcn_readlane(cum_l, s);
  };

  // the decode loop's proof (plan_layer's walk, with no growth)
  const int64_t C0 = uniform64(pc.capacity);
  int64_t proven = uniform64(pc.proven);
  const int64_t quantum = uniform64(pc.quantum);
  const int64_t need = uniform64(pc.need);
  const int F0 = __builtin_amdgcn_readfirstlane(pc.free_count);
  if (F0 < 0 || F0 > C0) return 0;
  if (need > 0 && quantum > 0) {
    int s = 0;
    if (proven >= need) {
      int64_t j = plan_div(proven, need);
      if (j > G0) j = G0;
      if (cum_at(static_cast<int>(j)) > F0) return 0;   // not honest: it overflows
      proven -= j * need;
      s = static_cast<int>(j);
    }
    while (s < G0) {
      const int64_t free_rows = F0 - cum_at(s);
      if (free_rows < need) return 0;   // the slab grows at step s
      const int64_t h = plan_div(free_rows, need);
      if (s + h >= G0) {
        proven = free_rows - static_cast<int64_t>(G0 - s) * need;
        s = G0;
      } else {
        s += static_cast<int>(h);
      }
    }
  }
  // no proof (or a proof for less than the steps' first touches) and the
  // stack runs out: the central plan overflows.  Below, every pop lies in
  // the found stack: found_top - 1 - q >= 0.
  if (cum_g > F0) return 0;

  if (lane < G0) plan_words[lane] = static_cast<int>(word_l);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  out.fit = cum_g;
  out.found = F0;
  out.proven = proven;
  return 1;
}

// The stack entry at position p after growth segment k: the row the latest
// growth j <= k whose positions cover p put there, or -1 for the entry the
// launch found there.
__device__ __forceinline__ int segment_entry(const int* seg, int p, int k) {
  const int* const seg_free = seg + kPlanSegments;
  const int* const seg_old = seg + 3 * kPlanSegments;
  for (int j = k; j >= 1; --j) {
    if (p >= seg_free[j]) return seg_old[j] + (p - seg_free[j]);
  }
  return -1;
}

// The growth segment of pop q: the last one whose first pop is at or below q.
__device__ __forceinline__ int segment_of(const int* seg, int segments, int q) {
  int lo = 0, hi = segments - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (seg[mid] <= q) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Layer part, by one wave (the control wave of bank 0), from the control
// words `pc` it loaded at the launch's start.  `seg` is LDS of
// 4 * kPlanSegments ints: the launch's growth segments; `jump` LDS of
// kTraceMaxSteps ints for the proof's jump table.  Publishes the running
// totals, the pops and the header (last); false when a step total never
// arrives (the header then says the layer runs no step).
//
// Who lists the pops: with BANKS_LIST false this wave lists every pop of the
// launch and rewrites the free stack before the header (few pops: slot maps
// that fit in LDS are small, and their slots are mostly mapped after the
// first steps); with BANKS_LIST true it publishes the growth segments and
// every control wave lists its own bank's pops after the header (a large
// address space: a pop for almost every write, more than one wave lists
// while the banks step).
template <bool BANKS_LIST>
__device__ inline bool plan_layer(const StepParams& P, int layer, const PlanBlock& pb, int B,
                                  int G0, uint32_t epoch, int* seg, int* jump,
                                  const PlanControl& pc) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const cowsdm_layer_t& L = P.layer[layer];
  constexpr int K = kTraceMaxSteps / kWave;
  int* const seg_q = seg;                        // first touches before the segment
  int* const seg_free = seg + kPlanSegments;     // stack height before its growth
  int* const seg_top = seg + 2 * kPlanSegments;  // stack height after its growth
  int* const seg_old = seg + 3 * kPlanSegments;  // capacity before its growth

  // header: the steps the layer runs, the pops that fit, the capacity, and
  // when the banks list their pops the stack height the launch found and
  // its growth segments
  auto publish_head = [&](int steps, int fit, int capacity, int found = 0, int segments = 1)
      __attribute__((always_inline)) {
    if constexpr (BANKS_LIST) {
      if (lane < 5) {
        const int v = lane == 0 ? steps : lane == 1 ? fit : lane == 2 ? capacity
                    : lane == 3 ? found : segments;
        atomic_store_u64(pb.head + lane, tagged(epoch, static_cast<uint32_t>(v)));
      }
    } else if (lane < 3) {
      const int v = lane == 0 ? steps : (lane == 1 ? fit : capacity);
      atomic_store_u64(pb.head + lane, tagged(epoch, static_cast<uint32_t>(v)));
    }
  };
  auto fault = [&]() __attribute__((always_inline)) {
    if (lane == 0 && P.trace_status) {
      __hip_atomic_fetch_or(&P.trace_status[layer], int32_t{COWSDM_TRACE_FAULT},
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  const int64_t C0 = uniform64(pc.capacity);
  int64_t proven = uniform64(pc.proven);
  const int64_t room = uniform64(pc.room);
  const int64_t quantum = uniform64(pc.quantum);
  const int64_t need = uniform64(pc.need);
  const int64_t events0 = uniform64(pc.events);
  const int64_t added0 = uniform64(pc.added);
  const int64_t copied0 = uniform64(pc.copied);
  const int F0 = __builtin_amdgcn_readfirstlane(pc.free_count);

  // ---- running totals: lane l holds the first touches before steps l,
  // l + 64, ... (exclusive), cum_g all of them
  int cum[K];
  int cum_g = 0;
  bool lost = false;
  {
    // all totals loaded at once; only the ones not yet there are polled
    uint64_t w[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int t = k * kWave + lane;
      w[k] = k * kWave < G0 ? atomic_load_u64(pb.totals + (t < G0 ? t : 0)) : 0;
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int t = k * kWave + lane;
      if (k * kWave < G0 && __ballot(t < G0 && !tag_is(w[k], epoch)) != 0) {
        lost |= !poll_tagged(pb.totals + (t < G0 ? t : 0), t < G0, epoch, w[k]);
      }
      const int v = t < G0 && !lost ? static_cast<int>(static_cast<uint32_t>(w[k])) : 0;
      const int incl = wave_inclusive(v);
      cum[k] = cum_g + incl - v;
      cum_g += __builtin_amdgcn_readlane(incl, kWave - 1);
    }
  }
  if (lost) {
    if (lane == 0) {
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_LOOKBACK), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
    fault();
    publish_head(0, 0, static_cast<int>(C0));
    return false;
  }
  // lane l's value for step s = 64k + l of a per-lane array (s wave-uniform:
  // a register picked by index, then one lane read)
  auto step_value = [&](const int (&v)[K], int s) __attribute__((always_inline)) -> int {
    return G0 <= kWave ? __builtin_amdgcn_readlane(v[0], s)
                       : __builtin_amdgcn_readlane(v[s >> 6], s & (kWave - 1));
  };
  // first touches before step s (s in [0, G0]), wave-uniform
  auto cum_at = [&](int s) __attribute__((always_inline)) -> int {
    return s >= G0 ? cum_g : step_value(cum, s);
  };

  if (F0 < 0 || F0 > C0) {
    // a corrupt free count: the layer runs nothing
    if (lane == 0) {
      atomic_store_u64(&control_word(P, layer, COWSDM_CTRL_STEPS), 0);
      __hip_atomic_fetch_or(&L.scratch[COWSDM_SCRATCH_ERRORS],
                            static_cast<int64_t>(COWSDM_ERR_CORRUPT), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
    fault();
    publish_head(0, 0, static_cast<int>(C0));
    return true;
  }

  // ---- the decode loop's capacity proof, step by step (wave-uniform)
  int64_t capacity = C0;
  int64_t added = 0, events = 0, rows_added = 0, rows_copied = 0;
  int nseg = 1;
  auto put_seg = [&](int k, int q, int free_rows, int top, int old)
      __attribute__((always_inline)) {
    if (lane == 0) {
      seg_q[k] = q;
      seg_free[k] = free_rows;
      seg_top[k] = top;
      seg_old[k] = old;
    }
  };
  put_seg(0, 0, F0, F0, static_cast<int>(C0));
  int stop = G0;
  bool over = false;
  if (need > 0 && quantum > 0) {
    // hop[k] (lane l): from a step t = 64k + l whose proof re-reads
    // free_count, the steps until the next such read, given the growth so
    // far: the free rows at t over need (at most the steps left), or 0 when
    // they are short of need and the slab grows at t.  All lanes compute
    // them at once; the walk below then takes one hop per read.
    int hop[K];
    auto hops = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int t = k * kWave + lane;
        const int64_t f = F0 + added - cum[k];
        const int64_t j = t >= G0 || f < need ? 0 : plan_div(f, need);
        hop[k] = static_cast<int>(j < G0 - t ? j : G0 - t);
      }
    };
    // A long run of reads without a growth is walked through a jump table
    // (LDS): from each step, the step 2^R reads later, or the first step
    // that grows or the last read before it when one comes first (pointer
    // doubling over the hops, R rounds).
    auto build_jumps = [&](int rounds) __attribute__((always_inline)) {
      int cur[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int t = k * kWave + lane;
        cur[k] = t < G0 && hop[k] > 0 && t + hop[k] < G0 ? t + hop[k] : t;
        if (t < G0) jump[t] = cur[k];
      }
      for (int r = 0; r < rounds; ++r) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        int nxt[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int t = k * kWave + lane;
          nxt[k] = k * kWave < G0 && t < G0 ? jump[cur[k]] : t;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int t = k * kWave + lane;
          cur[k] = nxt[k];
          if (t < G0) jump[t] = cur[k];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    int s = 0;
    if (proven >= need) {
      // steps still covered by the proof the launch starts with
      int64_t j = plan_div(proven, need);
      if (j > G0) j = G0;
      if (cum_at(static_cast<int>(j)) > F0) over = true;   // the proof was not honest
      proven -= j * need;
      s = static_cast<int>(j);
    }
    if (!over && s < G0) hops();
    // from here every step whose proof runs short re-reads free_count
    bool jumps = false;   // the table matches the hops
    int walked = 0;       // reads walked one by one since the hops last changed
    while (!over && s < G0) {
      if (jumps) {
        for (int n = __builtin_amdgcn_readfirstlane(jump[s]); n != s;
             n = __builtin_amdgcn_readfirstlane(jump[s])) {
          s = n;
        }
      }
      int h = step_value(hop, s);
      if (h == 0) {
        jumps = false;
        walked = 0;
        const int64_t free_rows = F0 + added - cum_at(s);
        const int64_t want = capacity + need - free_rows;
        const int64_t selected = plan_div(want + quantum - 1, quantum) * quantum;
        if (selected > room || selected >= (int64_t{1} << 31)) {
          stop = s;   // the host grows the slab into larger buffers
          break;
        }
        const int64_t a = selected - capacity;
        put_seg(nseg, cum_at(s), static_cast<int>(free_rows),
                static_cast<int>(free_rows + a), static_cast<int>(capacity));
        ++nseg;
        ++events;
        rows_added += a;
        rows_copied += capacity;
        added += a;
        capacity = selected;
        hops();
        h = step_value(hop, s);   // >= 1 now
      }
      if (s + h >= G0) {
        // the last read of the launch: the proof left after its steps
        proven = F0 + added - cum_at(s) - static_cast<int64_t>(G0 - s) * need;
        s = G0;
      } else {
        s += h;
        if (!jumps && ++walked >= 8 && G0 - s > 16) {
          // reads keep coming without a growth: enough rounds to cross the
          // rest of the launch in a few jumps
          int rounds = 1;
          while (rounds < 9 && (1 << rounds) < G0 - s) ++rounds;
          build_jumps(rounds);
          jumps = true;
        }
      }
    }
  } else if (cum_g > F0) {
    over = true;   // no proof: the stack runs out
  }
  // LDS of one wave applies in issue order; keep the compiler from moving
  // the segment reads below above lane 0's writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // pops that can be given out: all of the planned steps', or the stack's
  const int vlen = over ? static_cast<int>(F0 + added) : cum_at(stop);
  int fit = vlen;
  if (over) {
    // the pops that fit end at a (step, bank) boundary: the last one at or
    // below the stack height, found among the banks of the step where the
    // stack runs out
    int t_out = 0;   // the last step whose running total is <= vlen
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int t = k * kWave + lane;
      const uint64_t below = __ballot(t < G0 && cum[k] <= vlen);
      if (below) t_out = k * kWave + 63 - __builtin_clzll(below);
    }
    const int base = cum_at(t_out);
    int best = base;
    for (int g = 0; g < B; g += kWave) {
      const int b = g + lane;
      uint64_t w;
      poll_tagged(pb.word(b < B ? b : 0, t_out), b < B, epoch, w, true);
      const uint32_t v = static_cast<uint32_t>(w);
      const int end = base + static_cast<int>((v & ~kPrefixDone) >> kPrefixShift) +
                      __popc(v & 15u);
      int cand = b < B && (v & kPrefixDone) && end <= vlen ? end : base;
      for (int o = kWave / 2; o > 0; o >>= 1) {
        const int y = __shfl_xor(cand, o, kWave);
        cand = y > cand ? y : cand;
      }
      best = cand > best ? cand : best;
    }
    fit = best;
  }

  // ---- running totals for the steps' waves
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int t = k * kWave + lane;
    if (t < G0) atomic_store_u64(pb.cum + t, tagged(epoch, static_cast<uint32_t>(cum[k])));
  }
  if (lane == 0) atomic_store_u64(pb.cum + G0, tagged(epoch, static_cast<uint32_t>(cum_g)));

  const int64_t height = F0 + added - fit;
  if constexpr (BANKS_LIST) {
    // ---- the growth segments, for every bank to list its own pops (when
    // the launch does not grow, a pop q is the found stack's entry
    // F0 - 1 - q); the layer's last control wave to list rewrites the stack
    if (nseg > 1) {
      for (int k = lane; k < nseg; k += kWave) {
        int64_t* const w = pb.segs + 4 * static_cast<int64_t>(k);
        atomic_store_u64(w, tagged(epoch, static_cast<uint32_t>(seg_q[k])));
        atomic_store_u64(w + 1, tagged(epoch, static_cast<uint32_t>(seg_free[k])));
        atomic_store_u64(w + 2, tagged(epoch, static_cast<uint32_t>(seg_top[k])));
        atomic_store_u64(w + 3, tagged(epoch, static_cast<uint32_t>(seg_old[k])));
      }
    }
  } else {
    // ---- the row each pop takes: segment k pops from its top down.  The
    // stack entry at position p during segment k is the row the latest
    // growth j <= k whose positions cover p put there, or the entry the
    // launch found.
    const int32_t* const found = L.free_rows;
    auto entry = [&](int p, int k) __attribute__((always_inline)) -> int {
      for (int j = k; j >= 1; --j) {
        if (p >= seg_free[j]) return seg_old[j] + (p - seg_free[j]);
      }
      return found[p];
    };
    // A pop's row is arithmetic unless it comes from the stack the launch
    // found: those are loaded kPopBatch per lane at once.
    constexpr int kPopBatch = 8;
    const int listed = vlen < cum_at(stop) ? vlen : cum_at(stop);
    for (int k = 0; k < nseg; ++k) {
      const int q0 = seg_q[k];
      const int q1 = k + 1 < nseg ? seg_q[k + 1] : listed;
      const int top = seg_top[k];
      for (int qb = q0; qb < q1; qb += kWave * kPopBatch) {
        int row[kPopBatch];
#pragma unroll
        for (int i = 0; i < kPopBatch; ++i) {
          const int q = qb + i * kWave + lane;
          const int p = top - 1 - (q - q0);
          int v = -1;   // -1: from the stack the launch found
          for (int j = k; j >= 1; --j) {
            if (p >= seg_free[j]) {
              v = seg_old[j] + (p - seg_free[j]);
              break;
            }
          }
          // the row, or -2 - p for position p of the found stack
          row[i] = q >= q1 ? 0 : (v >= 0 ? v : -2 - p);
        }
#pragma unroll
        for (int i = 0; i < kPopBatch; ++i) {
          if (row[i] <= -2) row[i] = found[-2 - row[i]];
        }
#pragma unroll
        for (int i = 0; i < kPopBatch; ++i) {
          const int q = qb + i * kWave + lane;
          if (q < q1) atomic_store_u64(pb.pops + q, tagged(epoch, static_cast<uint32_t>(row[i])));
        }
      }
    }
    // ---- the stack the launch leaves (rewritten only above the lowest
    // growth, where no pop read it: segment 0 pops read below every
    // growth's base, later segments below their own)
    if (nseg > 1) {
      // every entry the launch found was read before the stack changes
      __builtin_amdgcn_s_waitcnt(0);
      int lo = seg_free[1];
      for (int k = 2; k < nseg; ++k) lo = seg_free[k] < lo ? seg_free[k] : lo;
      // (the layer struct lists free_rows as read-only for the step
      // kernels; the plan is the one part that rewrites it)
      int32_t* const stack = const_cast<int32_t*>(L.free_rows);
      for (int64_t p = lo + lane; p < height; p += kWave) {
        stack[p] = entry(static_cast<int>(p), nseg - 1);
      }
    }
  }
  if (lane == 0) {
    *L.free_count = static_cast<int32_t>(height);
    if (over) {
      *L.overflow_flag = 1;
    } else if (nseg > 1) {
      *L.overflow_flag = 0;   // grow_capacity clears it
    }
    if (stop < G0 && P.trace_status) {
      __hip_atomic_fetch_or(&P.trace_status[layer], int32_t{COWSDM_TRACE_REFUSED},
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // the control words the launch leaves, one lane each: device-scope
  // stores, since the layer's report reads them back during the launch,
  // possibly from another XCD, whose L2 does not see this one's dirty lines
  if (lane < 8) {
    int k = COWSDM_CTRL_PROVEN;
    int64_t v = over ? 0 : proven;
    if (lane == 1) { k = COWSDM_CTRL_CAPACITY; v = capacity; }
    if (lane == 2) { k = COWSDM_CTRL_EVENTS; v = events0 + events; }
    if (lane == 3) { k = COWSDM_CTRL_ADDED; v = added0 + rows_added; }
    if (lane == 4) { k = COWSDM_CTRL_COPIED; v = copied0 + rows_copied; }
    if (lane == 5) { k = COWSDM_CTRL_FREE; v = height; }
    if (lane == 6) { k = COWSDM_CTRL_STEPS; v = stop; }
    if (lane == 7) { k = COWSDM_CTRL_FIT; v = vlen; }
    atomic_store_u64(&control_word(P, layer, k), static_cast<uint64_t>(v));
  }
  publish_head(stop, vlen, static_cast<int>(capacity), F0, nseg);
  return true;
}

// Header part: the steps the layer runs, the pops that fit, the capacity
// the launch grows to, and with BANKS_LIST the stack height it found and its
// growth segments (else left as they are).  False when the header never
// arrives.
struct PlanHeader {
  int steps, fit, capacity, found, segments;
};
template <bool BANKS_LIST>
__device__ inline bool plan_header(const PlanBlock& pb, uint32_t epoch, PlanHeader& h) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  constexpr int kWords = BANKS_LIST ? 5 : 3;
  uint64_t w;
  if (!poll_tagged(pb.head + (lane < kWords ? lane : 0), lane < kWords, epoch, w)) return false;
  const int v = static_cast<int>(static_cast<uint32_t>(w));
  h.steps = __builtin_amdgcn_readlane(v, 0);
  h.fit = __builtin_amdgcn_readlane(v, 1);
  h.capacity = __builtin_amdgcn_readlane(v, 2);
  if constexpr (BANKS_LIST) {
    h.found = __builtin_amdgcn_readlane(v, 3);
    h.segments = __builtin_amdgcn_readlane(v, 4);
  }
  return true;
}

// A launch's growth segments (plan_layer), staged into `seg` (LDS of
// 4 * kPlanSegments ints: first pops, stack heights before and after each
// growth, capacities before it) by one wave.  False when one never arrives.
__device__ inline bool plan_segments(const PlanBlock& pb, uint32_t epoch, int segments,
                                     int* seg) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  bool ok = true;
  for (int k0 = 0; k0 < segments; k0 += kWave) {
    const int k = k0 + lane;
    const bool in = k < segments;
    const int64_t* const w = pb.segs + 4 * static_cast<int64_t>(in ? k : 0);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      uint64_t x;
      ok = poll_tagged(w + f, in, epoch, x) && ok;
      if (in) seg[f * kPlanSegments + k] = static_cast<int>(static_cast<uint32_t>(x));
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return ok;
}

}  // namespace cowsdm_impl
