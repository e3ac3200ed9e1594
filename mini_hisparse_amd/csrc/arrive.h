// Split-K partials merged by the last-arriving workgroup of a launch, without
// fences: the partial words and arrival counters shared by the group attention
// (attend.hip) and the decode projections (gemm.hip).
#pragma once

#include <stdint.h>

#include <atomic>
#include <chrono>

#include <hip/hip_runtime.h>

namespace hs {

// A split-K partial value is one 64-bit word: the fp32 bits in the low half and,
// when the launch merges its own partials, a tag in the high half that names the
// launch and, for a launch replayed from a captured graph (same epoch), the replay
// (group_tag).  The workgroup that merges a group reads every partial word with
// relaxed device-scope atomic loads and takes a word only once it carries the tag:
// by coherence of each word, a read that returns the tag returns the value this
// launch's producer stored, so the merge needs no release/acquire fence (on this
// multi-XCD part those write back and invalidate the L2: ~6 us per launch,
// measured).  The producers' stores complete before their arrival is counted, so
// the first read finds the tag; a word read early is read again (at most
// kSpinReads times; stores become visible in finite time).
constexpr int kSpinReads = 1 << 22;

__device__ __forceinline__ unsigned long long partial_word(float v, uint32_t tag) {
  return (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(v);
}
__device__ __forceinline__ float partial_value(unsigned long long w) {
  return __uint_as_float(static_cast<uint32_t>(w));
}
__device__ __forceinline__ void store_partial(unsigned long long* p, float v, uint32_t tag) {
  __hip_atomic_store(p, partial_word(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static __device__ __noinline__ unsigned long long partial_reread(const unsigned long long* p, uint32_t tag) {
  unsigned long long w = 0;
  for (int i = 0; i < kSpinReads; ++i) {
    w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (static_cast<uint32_t>(w >> 32) == tag) break;
    __builtin_amdgcn_s_sleep(1);
  }
  return w;
}

// Arrival counter of a group of workgroups whose partials one of them merges (the
// splits of an attention group, or of a projection's row tile): bits 63-32 the
// identity of the launch that last used it (counter_id: the low 31 bits of its
// epoch with bit 31 set), bits 31-16 the replay round, bits 15-0 the arrivals of
// the running launch.  A counter of another launch (an earlier launch's, or memory
// never used as a counter) is round 0 with no arrival.  The merging workgroup
// leaves (id, round + 1, 0): a replay of the same launch from a captured graph then
// counts from zero again and tags its partials with the next round, so no word of
// the previous replay carries its tag.  The workspace is shared by launches of
// other shapes, so the counter of one launch may sit where another left a partial
// word: partial-word tags have bit 31 clear and counter identities have it set, so
// a partial word never reads as a counter of the running launch.
__device__ __forceinline__ uint32_t counter_id(unsigned long long epoch) {
  return static_cast<uint32_t>(epoch) | 0x80000000u;
}
__device__ __forceinline__ uint32_t counter_round(unsigned long long c, unsigned long long epoch) {
  return static_cast<uint32_t>(c >> 32) == counter_id(epoch) ? static_cast<uint32_t>(c >> 16) & 0xffffu : 0u;
}
// Partial-word tag of a group's launch in replay round `round`: odd (never 0, which
// marks a word of a launch that does not merge its own partials), bit 31 clear,
// and different for consecutive epochs and for the rounds of one epoch.
__device__ __forceinline__ uint32_t group_tag(unsigned long long epoch, uint32_t round) {
  return (2u * static_cast<uint32_t>(epoch) + 1u + 2u * 0x9e3779b9u * round) & 0x7fffffffu;
}

// Arrival of one workgroup; true for the last of `total`.  The first workgroup of a
// launch that finds another epoch installs (epoch, 0, 1) with a compare-and-swap,
// every later one adds 1 (a launch costs one swap and total - 1 additions, no retry
// loop whose length grows with the arrivals).  A failed swap means another
// workgroup changed the counter, so the loop ends after at most one installation
// and the reads that follow it.  The counter only elects the merging workgroup and
// tells it that every split has stored its partials; the partial words carry their
// own tag (partial_word).
__device__ __forceinline__ bool arrive_last(unsigned long long* counter, unsigned long long epoch, int64_t total) {
  const unsigned long long mine = static_cast<unsigned long long>(counter_id(epoch)) << 32;
  unsigned long long old = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (true) {
    if ((old >> 32) == (mine >> 32)) {
      const unsigned long long prev = atomicAdd(counter, 1ull);
      return static_cast<int64_t>((prev & 0xffffull) + 1) == total;
    }
    const unsigned long long seen = atomicCAS(counter, old, mine | 1ull);
    if (seen == old) return total == 1;
    old = seen;
  }
}

// Epoch of one launch: 48 bits, never 0, different for every launch of the process
// (a counter started from the clock, so that counters left in reused memory by
// another process are unlikely to carry it either); its low 31 bits name the
// launch in the arrival counters (counter_id) and in the partial-word tags
// (group_tag).
inline unsigned long long next_epoch() {
  static std::atomic<unsigned long long> counter{
      static_cast<unsigned long long>(std::chrono::steady_clock::now().time_since_epoch().count()) * 0x9e3779b97f4a7c15ull};
  unsigned long long e;
  do {
    e = counter.fetch_add(1, std::memory_order_relaxed) & 0xffffffffffffull;
  } while (e == 0);
  return e;
}

}  // namespace hs
