// Logical-token -> physical-row resolver for gfx950, bit-exact with
// mini_hisparse's `resolve_rows` (row_index.py:59-137).
//
// The reference sorts the selected tokens and the hot tags and uses
// searchsorted/argsort to find hits, protect them, pick least-recent victims
// and reorder the LRU.  Nothing is sorted here.  A batch of (request, layer)
// descriptors is resolved by two launches:
//
//   front   (1 WG / desc)  Everything that needs one order over the request, with
//                          the token bitmaps in LDS:
//                          - selected tokens become a bitmap over [0, length):
//                            ascending order is bit order, a duplicate input is the
//                            atomicOr that finds its bit set (the first input index
//                            of a duplicated token by atomicMin); given the union's
//                            page bitmap, the bitmap is expanded from it instead;
//                          - per page with selected tokens: resident hits are
//                            counted and host-backed non-resident tokens get a
//                            needs-hot bit;
//                          - each hot tag (host row = source[page] * P + off) finds
//                            its logical page: by subtraction when the source table
//                            is affine (host block = base + page over every
//                            host-backed page, the layout of a request's contiguous
//                            host slots; detected here), else through a hash of the
//                            needs-hot pages' host blocks.  A tag whose token needs
//                            a hot row is a hit: hit bit, the token's slot, the
//                            slot's protection bit;
//                          - miss bits = needs-hot and not hit, their per-word
//                            prefix (miss ranks in token order) and the counts;
//                          - victims = the stable partition "unprotected, then
//                            protected" of the LRU order, and the new LRU = the
//                            stable partition by category (untouched, filled, hit,
//                            hit and filled), a slot being filled iff its victim
//                            rank is below the miss count.  The filled unprotected
//                            slots are the first min(U, misses) unprotected ones and
//                            the filled protected slots the first max(0, misses - U)
//                            protected ones (U unprotected slots in all), so every
//                            new position follows from one prefix: the unprotected
//                            slots before the entry.
//   outputs (n/256 + H*W/256 WGs)  per input: its physical row (the first
//                          occurrence of a token wins), and for a miss its plan
//                          entry and the new tag of its victim slot; per head
//                          column: the row of the input it names.
//
// Preconditions, as in the reference: unique non-negative tags, an injective
// source table, and length <= n_pages * page_size (checked on the host).
#include <mutex>

#include "hs_common.h"

namespace hs {

constexpr int RT = 1024;       // threads of the front launch
constexpr int RW = 256;        // threads of the outputs launch
constexpr int NWAVES = RT / 64;
constexpr int RMAXB = 16;      // descriptors per launch (passed by value: 16 x 200 bytes)
constexpr int LRU_CHUNK = 32;  // hot_rows <= 32768 = RT * LRU_CHUNK
constexpr int TAG_BATCH = 4;   // hash probes in flight per thread
constexpr int MATCH_BATCH = 8; // tags matched per batch (needs-bit reads in flight together)
constexpr int MARK_BATCH = 8;  // pages loaded per thread before use (long tables)
constexpr int PAGE_REGS = 9;  // pages per thread loaded before the token walk (n_pages <= RT * PAGE_REGS)
constexpr int ORDER_WORDS = 8; // token-bitmap words per thread held in registers
constexpr int WALK_PRE = 5;    // page-bitmap words per thread loaded first (lengths below RT * 5 * 32)
constexpr int ST = 512;        // threads of the split front's launches
constexpr int SPLIT_MAX = 64;  // workgroups per request of the split front
constexpr int MARK_TILE = 512;                // inputs per wave and tile (8 per lane)
constexpr int MARK_TILE_PAD = MARK_TILE / 8 * 9;
constexpr uint64_t HASH_EMPTY = ~static_cast<uint64_t>(0);

// Per-thread arrays of the front launch.  Every index into them comes from fully
// unrolled loops with constant bounds, so after unrolling each one is a constant and
// the array lives in registers (a non-constant index would put it in scratch, which
// the build rejects).  Built with HS_REG_CHECK (a CPU-side check, never launched),
// every access carries a trap for an index outside [0, N); the compiler folds each
// such test away when the index is a constant inside the range, so a trap left in
// the front kernel's machine code names an index that can leave its array
// (tests/test_resolver_registers.py compiles the 16- and 32-slot fronts this way).
#ifndef HS_REG_CHECK
#define HS_REG_CHECK 0
#endif
__device__ __forceinline__ void reg_check(int i, int n) {
  if (HS_REG_CHECK && static_cast<unsigned>(i) >= static_cast<unsigned>(n)) __builtin_trap();
}
#if HS_REG_CHECK
template <typename T, int N>
struct Regs {
  T r[N];
  __device__ __forceinline__ T& operator[](int i) {
    reg_check(i, N);
    return r[i];
  }
};
#else
template <typename T, int N>
using Regs = T[N];  // the shipped build: plain arrays
#endif
struct ResolveBatch {
  hs_resolve_desc d[RMAXB];
  int count;
};
static_assert(sizeof(ResolveBatch) <= 4096, "resolver descriptors must fit the 4 KB kernel-argument block");

struct ResolveWs {
  uint32_t* hitbits;   // [wl] needs-hot tokens with a hot tag
  uint32_t* missbits;  // [wl] needs-hot tokens without one
  uint32_t* dupbits;   // [wl] tokens given more than once
  int32_t* mprefix;    // [wl] misses in the words before this one
  int32_t* first_in;   // [length] first input index of a duplicated token
  int32_t* tslot;      // [length] hot slot of a hit token
  uint64_t* hash;      // [hcap] (page << 32) | host block of needs-hot pages; all ones = empty
  int32_t* victims;    // [hot_rows] slots in victim order (ranks below the miss count written)
  int64_t* totals;     // [4] resident hits, hot hits, misses, any duplicate (2: see the split front)
  int64_t hcap;
};

// The split front's own workspace (after the regions above; a separate struct, so
// that the single-workgroup front carries none of its pointers).
struct SplitWs {
  uint32_t* prot;      // [ceil(hot_rows / 32)] protected slots
  uint16_t* lru_snap;  // [hot_rows] the LRU as read before its rewrite
  int64_t* part;       // [6 * SPLIT_MAX] per-workgroup partials
  uint32_t* needpg;    // [2 * ceil(n_pages / 64)] pages with needs-hot tokens
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); }
__host__ __device__ inline int64_t pow2_at_least(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

__host__ __device__ inline int64_t words_for(int64_t length) { return (length + 32) / 32; }

__host__ __device__ inline int64_t ws_layout(int64_t length, int64_t n_pages, int64_t hot_rows, ResolveWs* w,
                                             char* base, SplitWs* sw = nullptr) {
  const int64_t wl = words_for(length);
  const int64_t hcap = pow2_at_least(2 * (n_pages < 1 ? 1 : n_pages));
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off += align256(bytes);
    return base ? base + at : nullptr;
  };
  char* p0 = take(wl * 4);
  char* p1 = take(wl * 4);
  char* p2 = take(wl * 4);
  char* p3 = take(wl * 4);
  char* p4 = take(length * 4);
  char* p5 = take(length * 4);
  char* p6 = take(hcap * 8);
  char* p7 = take(hot_rows * 4);
  char* p8 = take(4 * 8);
  char* p9 = take((hot_rows + 31) / 32 * 4);
  char* p10 = take(hot_rows * 2);
  char* p11 = take(6 * SPLIT_MAX * 8);
  char* p12 = take((n_pages + 63) / 64 * 8);
  if (w) {
    w->hitbits = reinterpret_cast<uint32_t*>(p0);
    w->missbits = reinterpret_cast<uint32_t*>(p1);
    w->dupbits = reinterpret_cast<uint32_t*>(p2);
    w->mprefix = reinterpret_cast<int32_t*>(p3);
    w->first_in = reinterpret_cast<int32_t*>(p4);
    w->tslot = reinterpret_cast<int32_t*>(p5);
    w->hash = reinterpret_cast<uint64_t*>(p6);
    w->victims = reinterpret_cast<int32_t*>(p7);
    w->totals = reinterpret_cast<int64_t*>(p8);
    w->hcap = hcap;
  }
  if (sw) {
    sw->prot = reinterpret_cast<uint32_t*>(p9);
    sw->lru_snap = reinterpret_cast<uint16_t*>(p10);
    sw->part = reinterpret_cast<int64_t*>(p11);
    sw->needpg = reinterpret_cast<uint32_t*>(p12);
  }
  return off;
}

__device__ __forceinline__ ResolveWs ws_of(const hs_resolve_desc& d) {
  ResolveWs w;
  ws_layout(d.length, d.n_pages, d.hot_rows, &w, static_cast<char*>(d.workspace));
  return w;
}
__device__ __forceinline__ SplitWs split_ws_of(const hs_resolve_desc& d) {
  ResolveWs w;
  SplitWs sw;
  ws_layout(d.length, d.n_pages, d.hot_rows, &w, static_cast<char*>(d.workspace), &sw);
  return sw;
}

__device__ __forceinline__ uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ bool bit_of(const uint32_t* bits, int64_t t) {
  return (bits[t >> 5] >> (t & 31)) & 1u;
}

// Reads of workspace words that other threads of the same launch wrote with device
// atomics (performed in L2): device-scope loads, which bypass the CU's L1, where a
// line filled before those atomics could still hold the old value.
__device__ __forceinline__ bool bit_of_l2(const uint32_t* bits, int64_t t) {
  const uint32_t wd = __hip_atomic_load(bits + (t >> 5), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (wd >> (t & 31)) & 1u;
}
__device__ __forceinline__ uint64_t load_l2(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int64_t load_pos(const hs_resolve_desc& d, int64_t i) {
  return d.positions_i64 ? static_cast<const int64_t*>(d.positions)[i]
                         : static_cast<int64_t>(static_cast<const int32_t*>(d.positions)[i]);
}

// Bits [lo, hi) of word `word` (lo, hi absolute token indices).
__device__ __forceinline__ uint32_t range_mask(int64_t word, int64_t lo, int64_t hi) {
  const int64_t base = word << 5;
  const int64_t a = lo > base ? lo - base : 0;
  const int64_t b = hi < base + 32 ? hi - base : 32;
  if (b <= a) return 0u;
  const uint32_t upto = b >= 32 ? 0xffffffffu : ((1u << b) - 1u);
  return upto & ~((1u << a) - 1u);
}

// Division by the page size of non-negative 32-bit values (tokens, host rows, hot
// slots are all below 2^31): a shift for a power-of-two page, else a 32-bit
// division -- never the 64-bit division a plain int64_t quotient compiles to.
struct PageDiv {
  uint32_t p;
  int shift;  // -1: not a power of two
  __device__ explicit PageDiv(int64_t page_size) : p(static_cast<uint32_t>(page_size)) {
    shift = (p & (p - 1)) == 0 ? __ffs(static_cast<int>(p)) - 1 : -1;
  }
  __device__ __forceinline__ uint32_t div(uint32_t x) const { return shift >= 0 ? x >> shift : x / p; }
};

__device__ __forceinline__ int32_t wave_min_i32(int32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int32_t o = __shfl_xor(v, off, 64);
    v = o < v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int32_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int32_t lanes_below(uint64_t m) {
  return static_cast<int32_t>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// ---- front: bitmaps, hits and protection, miss ranks, victims, LRU reorder
// (row_index.py:67-113).  LDS: bits[wl] (selected tokens, then hit tokens),
// needs[wl], prot[wsw].
// POW2: page size a power of two (shifts), else 32-bit divisions.  L16: int16 LRU
// tables (two entries per 32-bit load and register), else the reference's int64.
// SR: hot slots per thread (hot_rows <= RT * SR for every descriptor): 16 or 32, so
// that the per-slot phases of smaller hot regions run no masked-off rows.
template <bool POW2, bool L16, int SR>
__global__ __launch_bounds__(RT) void resolve_front_kernel(ResolveBatch batch) {
  extern __shared__ uint32_t lds[];
  __shared__ int64_t scan64[16];
  __shared__ unsigned long long s_res;  // resident hits of the request
  __shared__ int32_t scan32[16];
  __shared__ int any_dup;
  __shared__ int32_t base_lo, base_hi;
  __shared__ int32_t mark_tile[NWAVES * MARK_TILE_PAD];
  __shared__ int32_t ucnt[SR * NWAVES];  // unprotected LRU entries per (row, wave), then their prefix
  const hs_resolve_desc& d = batch.d[blockIdx.x];
  const ResolveWs w = ws_of(d);
  const int T = threadIdx.x, lane = T & 63, wave = T >> 6;
  const int64_t n = d.n, L = d.length, P = d.page_size, NP = d.n_pages;
  const int32_t S = static_cast<int32_t>(d.hot_rows);
  const int64_t wl = words_for(L), wsw = (S + 31) / 32;
  uint32_t* bits = lds;
  uint32_t* needs = lds + wl;
  uint32_t* prot = lds + 2 * wl;
  const uint32_t pshift = static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(P)) - 1);
  auto page_of = [&](uint32_t x) -> uint32_t { return POW2 ? x >> pshift : x / static_cast<uint32_t>(P); };

  // Loads complete in issue order, so they are issued in the order of their use:
  // the page-bitmap words of the walk first, then the page tables of short histories
  // (used after the walk).
  // page-bitmap word of token words T + k * RT (one word each: a power-of-two page
  // of at most 32 tokens puts a token word's pages in one bitmap word)
  const bool pb_pre = d.page_bits && POW2 && P <= 32 && wl <= static_cast<int64_t>(RT) * WALK_PRE;
  Regs<uint32_t, WALK_PRE> pbw;
  if (pb_pre) {
#pragma unroll
    for (int k = 0; k < WALK_PRE; ++k) {
      const int64_t wd = T + static_cast<int64_t>(k) * RT;
      const bool in = wd < wl && (wd << 5) < L;  // the bitmap has ceil(pages / 32) words
      const uint32_t v = d.page_bits[in ? (wd >> pshift) : 0];
      pbw[k] = in ? v : 0u;
    }
  }
  // the page tables of short histories are loaded now and used after the token walk
  constexpr int PR = PAGE_REGS;
  const bool pages_early = NP <= static_cast<int64_t>(RT) * PR;
  Regs<int32_t, PR> src_e, res_e;  // res_e: only its sign is used
  if (pages_early) {
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int64_t p = T + static_cast<int64_t>(k) * RT;
      const int64_t pc = p < NP ? p : 0;  // unconditional loads, masked when used
      src_e[k] = d.source[pc];
      res_e[k] = d.resident[pc];
    }
  }
  // The hot tags, TR rows of RT slots per round (row k of thread T: slot k * RT + T),
  // and the LRU (slots < 32768, read before any is rewritten): row q of thread T
  // holds the entries 2 (q * RT + T) and 2 (q * RT + T) + 1 as two 16-bit halves of one
  // register (lower entry in the low half): one 32-bit load for int16 tables, the low
  // words of two entries for int64 ones.  Rows past hot_rows load entry 0 and are
  // masked where used.  (Holding every tag and every LRU entry of 32 rows in registers
  // at once made the compiler spill; a build of that form returned wrong tags in one
  // row at the 32768-slot shape, so the per-thread state is kept to 16 + 16 registers.)
  constexpr int TR = 16;
  constexpr int HALVES = 2;
  constexpr int LROWS = SR / HALVES;
  Regs<int32_t, TR> tg;
  Regs<int32_t, LROWS> slot;
  auto load_tags = [&](int r) {
#pragma unroll
    for (int kk = 0; kk < TR; ++kk) {
      const int32_t s = (r * TR + kk) * RT + T;
      const int32_t v = d.tags[s < S ? s : 0];  // unconditional load, masked afterwards
      tg[kk] = s < S ? v : -1;
    }
  };
  auto load_lru = [&]() {
    const int32_t* lru32 = static_cast<const int32_t*>(d.lru);
#pragma unroll
    for (int q = 0; q < LROWS; ++q) {
      const int32_t jp = q * RT + T;
      if constexpr (L16) {
        slot[q] = lru32[2 * jp < S ? jp : 0];  // hot_rows even for int16 (host-checked)
      } else {
        const int32_t lo = lru32[2 * (2 * jp < S ? 2 * jp : 0)];
        const int32_t hi = lru32[2 * (2 * jp + 1 < S ? 2 * jp + 1 : 0)];
        slot[q] = (lo & 0xffff) | (hi << 16);
      }
    }
  };
  for (int64_t i = T; i < 2 * wl + wsw; i += RT) lds[i] = 0u;
  if (!d.page_bits)  // a page bitmap admits no duplicate input
    for (int64_t i = T; i < wl; i += RT) w.dupbits[i] = 0u;
  if (T == 0) {
    any_dup = 0;
    s_res = 0ull;
    base_lo = INT32_MAX;
    base_hi = INT32_MIN;
  }
  __syncthreads();

  // selected tokens.  With the union's page bitmap they are the tokens below
  // length of the marked pages (no duplicates): each token word is assembled from
  // the bits of the pages it overlaps, and no input is read.  Otherwise a bit
  // already set means a duplicate input.  Each wave
  // loads 512 consecutive inputs (coalesced) into an LDS tile; lane l then
  // walks inputs 8l .. 8l+7 of the tile and gathers the bits of one bitmap
  // word in a register while consecutive tokens stay in it (selected tokens
  // mostly arrive sorted), publishing them with one atomicOr when the word
  // changes.  A token already in the register, or already in the word when
  // it is published, is a duplicate; any input order gives the same bitmap
  // and duplicate set.
  if (pb_pre) {  // the same for every thread
    const uint32_t ppw = static_cast<uint32_t>(32 / P);  // pages per token word
    const uint32_t pmask = P >= 32 ? 0xffffffffu : (1u << P) - 1u;
#pragma unroll
    for (int k = 0; k < WALK_PRE; ++k) {
      const int64_t wd = T + static_cast<int64_t>(k) * RT;
      if (wd >= wl) break;
      const uint32_t first = static_cast<uint32_t>(wd << (5 - pshift)) & 31u;  // first page bit of the word
      const uint32_t pb = (pbw[k] >> first) & (ppw >= 32 ? 0xffffffffu : (1u << ppw) - 1u);
      uint32_t m = 0u;
      for (uint32_t j = 0; j < ppw; ++j)
        if ((pb >> j) & 1u) m |= pmask << (j * static_cast<uint32_t>(P));
      bits[wd] = m & range_mask(wd, 0, L);  // each word has one writer
    }
  } else if (d.page_bits) {  // the same for every thread
    for (int64_t wd = T; wd < wl; wd += RT) {
      const int64_t t0 = wd << 5;
      const int64_t t1 = t0 + 32 < L ? t0 + 32 : L;  // tokens [t0, t1) of this word
      uint32_t m = 0u;
      if (t0 < L) {
        const uint32_t p_hi = page_of(static_cast<uint32_t>(t1 - 1));
        for (uint32_t pg = page_of(static_cast<uint32_t>(t0)); pg <= p_hi; ++pg) {
          if (!((d.page_bits[pg >> 5] >> (pg & 31)) & 1u)) continue;
          const int64_t lo = static_cast<int64_t>(pg) * P;
          m |= range_mask(wd, lo, lo + P < t1 ? lo + P : t1);
        }
      }
      bits[wd] = m;  // each word has one writer
    }
  } else {
    int32_t* tile = mark_tile + wave * MARK_TILE_PAD;
    int64_t cur = -1;
    uint32_t acc = 0u, accdup = 0u;
    auto flush = [&]() {
      if (cur < 0) return;
      const uint32_t old = atomicOr(&bits[cur], acc);
      const uint32_t dm = accdup | (old & acc);
      if (dm) {
        atomicOr(&w.dupbits[cur], dm);
        any_dup = 1;
      }
    };
    constexpr int KT = MARK_TILE / 64;
    constexpr int64_t STEP = static_cast<int64_t>(NWAVES) * MARK_TILE;
    // one loop per position type: a per-load type branch would serialise the loads
    auto walk = [&](const auto* pos) {
      Regs<int64_t, KT> nxt;  // the next tile's inputs, loaded while this one is walked
      auto load_tile = [&](int64_t base) {  // unconditional loads (clamped index), then masked
#pragma unroll
        for (int k = 0; k < KT; ++k) {
          const int64_t i = base + k * 64 + lane;
          const int64_t v = static_cast<int64_t>(pos[i < n ? i : n - 1]);
          nxt[k] = i < n ? v : -1;
        }
      };
      load_tile(static_cast<int64_t>(wave) * MARK_TILE);
      for (int64_t base = static_cast<int64_t>(wave) * MARK_TILE; base < n; base += STEP) {
#pragma unroll
        for (int k = 0; k < KT; ++k) {
          const int p = k * 64 + lane;  // tile position; stored with a stride-9 row per lane
          const int64_t t = nxt[k];
          tile[9 * (p >> 3) + (p & 7)] = (t >= 0 && t < L) ? static_cast<int32_t>(t) : -1;
        }
        load_tile(base + STEP);
        wave_lds_sync();
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int32_t t = tile[9 * lane + k];
          if (t < 0) continue;
          const int64_t word = t >> 5;
          const uint32_t bit = 1u << (t & 31);
          if (word != cur) {
            flush();
            cur = word;
            acc = accdup = 0u;
          }
          accdup |= acc & bit;
          acc |= bit;
        }
        wave_lds_sync();
      }
    };
    if (d.positions_i64) walk(static_cast<const int64_t*>(d.positions));
    else walk(static_cast<const int32_t*>(d.positions));
    flush();
  }
  __syncthreads();

  // first input index of each duplicated token (row_index.py:121-126)
  const bool dups = any_dup != 0;
  if (dups) {
    for (int64_t i = T; i < n; i += RT) {
      const int64_t t = load_pos(d, i);
      if (t >= 0 && t < L && bit_of_l2(w.dupbits, t)) w.first_in[t] = static_cast<int32_t>(n);
    }
    __syncthreads();
    for (int64_t i = T; i < n; i += RT) {
      const int64_t t = load_pos(d, i);
      if (t >= 0 && t < L && bit_of_l2(w.dupbits, t)) atomicMin(&w.first_in[t], static_cast<int32_t>(i));
    }
  }

  // per page with selected tokens: resident hits and needs-hot bits; over every
  // host-backed page of the history, the range of (host block - page)
  int64_t c_res = 0;
  int32_t my_lo = INT32_MAX, my_hi = INT32_MIN;
  // a page size dividing 32 puts every page inside one bitmap word
  const bool in_word = POW2 && P <= 32;
  const uint32_t page_bits = P >= 32 ? 0xffffffffu : (1u << (P & 31)) - 1u;
  auto page_work = [&](int64_t p, int32_t sv, int32_t rv) {
    if (sv < 0) return;  // also pages past the history
    const int32_t shift = sv - static_cast<int32_t>(p);  // both in [0, 2^31): no overflow
    my_lo = shift < my_lo ? shift : my_lo;
    my_hi = shift > my_hi ? shift : my_hi;
    if (in_word) {
      const uint32_t lo = static_cast<uint32_t>(p) << pshift;  // < length < 2^31
      const uint32_t wd = lo >> 5;
      uint32_t m = page_bits << (lo & 31);
      if (lo + static_cast<uint32_t>(P) > static_cast<uint32_t>(L))  // the history's last page, cut at the length
        m &= ((1u << (static_cast<uint32_t>(L) - lo)) - 1u) << (lo & 31);
      m &= bits[wd];
      if (!m) return;
      if (rv >= 0) c_res += __popc(m);
      else atomicOr(&needs[wd], m);
      return;
    }
    const int64_t lo = p * P;
    const int64_t hi = lo + P < L ? lo + P : L;
    for (int64_t wd = lo >> 5; wd <= (hi - 1) >> 5; ++wd) {
      const uint32_t m = bits[wd] & range_mask(wd, lo, hi);
      if (!m) continue;
      if (rv >= 0) c_res += __popc(m);
      else atomicOr(&needs[wd], m);
    }
  };
  if (pages_early) {
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int64_t p = T + static_cast<int64_t>(k) * RT;
      const bool in = p < NP && p * P < L;
      page_work(p, in ? src_e[k] : -1, res_e[k]);
    }
  } else {
    for (int64_t base = T; base < NP; base += static_cast<int64_t>(RT) * MARK_BATCH) {
      Regs<int32_t, MARK_BATCH> src, res;
#pragma unroll
      for (int k = 0; k < MARK_BATCH; ++k) {
        const int64_t p = base + static_cast<int64_t>(k) * RT;
        const bool in = p < NP && p * P < L;
        const int64_t pc = in ? p : 0;  // unconditional loads, masked afterwards
        const int32_t sv = d.source[pc], rv = d.resident[pc];
        src[k] = in ? sv : -1;
        res[k] = in ? rv : -1;
      }
#pragma unroll
      for (int k = 0; k < MARK_BATCH; ++k) page_work(base + static_cast<int64_t>(k) * RT, src[k], res[k]);
    }
  }
  my_lo = wave_min_i32(my_lo);
  my_hi = wave_max_i32(my_hi);
  if (lane == 0) {
    atomicMin(&base_lo, my_lo);
    atomicMax(&base_hi, my_hi);
  }
  // resident hits: only the request's total is needed (one LDS add per wave)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c_res += __shfl_xor(c_res, off, 64);
  if (lane == 0) atomicAdd(&s_res, static_cast<unsigned long long>(c_res));
  __syncthreads();  // the page pass and the block-range atomics are complete

  const bool affine = base_lo >= base_hi;  // one shift, or no host-backed page
  const int64_t shift = base_hi;
  for (int64_t i = T; i < wl; i += RT) bits[i] = 0u;  // from here on: hit tokens
  if (!affine) {
    // host block -> page for the pages with needs-hot tokens
    for (int64_t i = T; i < w.hcap; i += RT) w.hash[i] = HASH_EMPTY;
    __syncthreads();
    const uint32_t hmask = static_cast<uint32_t>(w.hcap - 1);
    for (int64_t p = T; p < NP; p += RT) {
      if (p * P >= L) break;
      const int64_t lo = p * P;
      const int64_t hi = lo + P < L ? lo + P : L;
      bool want = false;
      for (int64_t wd = lo >> 5; wd <= (hi - 1) >> 5; ++wd) want |= (needs[wd] & range_mask(wd, lo, hi)) != 0u;
      if (!want) continue;
      const uint32_t sv = static_cast<uint32_t>(d.source[p]);
      const uint64_t entry = (static_cast<uint64_t>(p) << 32) | sv;
      uint32_t h = hash32(sv) & hmask;
      while (true) {
        const uint64_t prev = atomicCAS(reinterpret_cast<unsigned long long*>(&w.hash[h]),
                                        static_cast<unsigned long long>(HASH_EMPTY),
                                        static_cast<unsigned long long>(entry));
        if (prev == HASH_EMPTY || static_cast<uint32_t>(prev) == sv) break;  // inserted, or first page wins
        h = (h + 1) & hmask;
      }
    }
  }
  __syncthreads();

  // hot tags -> logical pages (row_index.py:84-86).  Affine source: page = host
  // block - base.  Otherwise each tag is looked up in the hash and rewritten as
  // the host row its page would have under base 0 (page * P + offset), or -1,
  // so that one matching loop serves both.  32-bit token arithmetic: a page
  // below the history's page count times the page size stays below length +
  // page size < 2^32.
  const uint32_t Lu = static_cast<uint32_t>(L), Pu = static_cast<uint32_t>(P);
  const uint32_t hist_pages = static_cast<uint32_t>((L + P - 1) / P < NP ? (L + P - 1) / P : NP);
  const uint32_t ushift = affine ? static_cast<uint32_t>(static_cast<int32_t>(shift)) : 0u;
  // a tag whose token needs a hot row is a hit (row_index.py:84-90), TR rows per
  // round.  Batches of MATCH_BATCH tags with their needs-bit reads in flight
  // together; the slots of a wave's 64 tags form two whole protection words, which
  // lanes 2k and 2k + 1 of the wave keep (row k) and store once at the end.
  uint32_t myprot = 0u;
#pragma unroll 1
  for (int r = 0; r < SR / TR; ++r) {
    load_tags(r);
    if (!affine) {
      const uint32_t hmask = static_cast<uint32_t>(w.hcap - 1);
#pragma unroll
      for (int k0 = 0; k0 < TR; k0 += TAG_BATCH) {
        Regs<uint64_t, TAG_BATCH> e;
        Regs<uint32_t, TAG_BATCH> h, hp;
#pragma unroll
        for (int j = 0; j < TAG_BATCH; ++j) {  // first probes in flight together
          hp[j] = page_of(static_cast<uint32_t>(tg[k0 + j]));
          h[j] = hash32(hp[j]) & hmask;
          e[j] = tg[k0 + j] >= 0 ? load_l2(&w.hash[h[j]]) : HASH_EMPTY;
        }
#pragma unroll
        for (int j = 0; j < TAG_BATCH; ++j) {
          while (e[j] != HASH_EMPTY && static_cast<uint32_t>(e[j]) != hp[j]) {
            h[j] = (h[j] + 1) & hmask;
            e[j] = load_l2(&w.hash[h[j]]);
          }
          const uint32_t off = static_cast<uint32_t>(tg[k0 + j]) - hp[j] * Pu;
          tg[k0 + j] = e[j] == HASH_EMPTY || tg[k0 + j] < 0 ? -1
                                                            : static_cast<int32_t>(static_cast<uint32_t>(e[j] >> 32) * Pu + off);
        }
      }
    }

#pragma unroll
    for (int k0 = 0; k0 < TR; k0 += MATCH_BATCH) {
      Regs<uint32_t, MATCH_BATCH> t, nw;
      Regs<bool, MATCH_BATCH> ok;
#pragma unroll
      for (int j = 0; j < MATCH_BATCH; ++j) {
        const uint32_t tag = static_cast<uint32_t>(tg[k0 + j]);
        const uint32_t hp = page_of(tag);
        const uint32_t page = hp - ushift;  // a block outside the range wraps to >= 2^31
        t[j] = POW2 ? (page << pshift) | (tag & (Pu - 1u)) : page * Pu + (tag - hp * Pu);
        ok[j] = tg[k0 + j] >= 0 && page < hist_pages && t[j] < Lu;
        nw[j] = needs[ok[j] ? t[j] >> 5 : 0];
      }
#pragma unroll
      for (int j = 0; j < MATCH_BATCH; ++j) {
        const int k = r * TR + k0 + j;
        const bool hit = ok[j] && ((nw[j] >> (t[j] & 31)) & 1u);
        if (hit) {
          atomicOr(&bits[t[j] >> 5], 1u << (t[j] & 31));
          w.tslot[t[j]] = k * RT + T;
        }
        const uint64_t m = __ballot(hit);
        myprot = (lane >> 1) == k ? ((lane & 1) ? static_cast<uint32_t>(m >> 32) : static_cast<uint32_t>(m)) : myprot;
      }
    }
  }
  {
    const int32_t wi = (lane >> 1) * 32 + wave * 2 + (lane & 1);  // ((k * RT + wave * 64) >> 5) + half
    if (wi < wsw) prot[wi] = myprot;
  }

  // the LRU loads run while the miss words are counted
  load_lru();
  // slot of half h of row q, and its LRU entry index
  auto slot_at = [&](int q, int h) -> int32_t {
    return h ? static_cast<int32_t>(static_cast<uint32_t>(slot[q]) >> 16) : (slot[q] & 0xffff);
  };
  auto entry_of = [&](int q, int h) -> int32_t { return HALVES * (q * RT + T) + h; };

  __syncthreads();

  // miss bits in token order, their per-word exclusive prefix, the hit and miss counts
  const int64_t wpt = (wl + RT - 1) / RT;
  const int64_t w0 = static_cast<int64_t>(T) * wpt;
  const int64_t w1 = w0 + wpt < wl ? w0 + wpt : wl;
  int64_t c_hit = 0, c_miss = 0;
  int64_t tot_hit, tot_miss;
  // one block scan of the (hits, misses) pair packed in 64 bits (each count is below
  // 2^31, so the halves never carry into each other): the miss prefix and both totals
  auto hit_miss_scan = [&](int64_t h, int64_t m, int64_t& th, int64_t& tm_) -> int64_t {
    uint64_t tot;
    const uint64_t ex = block_exclusive_sum<uint64_t>((static_cast<uint64_t>(h) << 32) | static_cast<uint64_t>(m),
                                                      reinterpret_cast<uint64_t*>(scan64), &tot);
    th = static_cast<int64_t>(tot >> 32);
    tm_ = static_cast<int64_t>(tot & 0xffffffffull);
    return static_cast<int64_t>(ex & 0xffffffffull);
  };
  if (wpt <= ORDER_WORDS) {
    Regs<uint32_t, ORDER_WORDS> miss;
#pragma unroll
    for (int k = 0; k < ORDER_WORDS; ++k) {
      const int64_t wd = w0 + k;
      const bool in = wd < w1;
      const uint32_t hit = in ? bits[wd] : 0u;
      miss[k] = in ? needs[wd] & ~hit : 0u;
      c_hit += __popc(hit);
      c_miss += __popc(miss[k]);
      if (in) {
        w.hitbits[wd] = hit;
        w.missbits[wd] = miss[k];
      }
    }
    int64_t r = hit_miss_scan(c_hit, c_miss, tot_hit, tot_miss);
#pragma unroll
    for (int k = 0; k < ORDER_WORDS; ++k) {
      if (w0 + k < w1) w.mprefix[w0 + k] = static_cast<int32_t>(r);
      r += __popc(miss[k]);
    }
  } else {
    for (int64_t wd = w0; wd < w1; ++wd) {
      const uint32_t hit = bits[wd], miss = needs[wd] & ~hit;
      w.hitbits[wd] = hit;
      w.missbits[wd] = miss;
      c_hit += __popc(hit);
      c_miss += __popc(miss);
    }
    int64_t r = hit_miss_scan(c_hit, c_miss, tot_hit, tot_miss);
    for (int64_t wd = w0; wd < w1; ++wd) {
      w.mprefix[wd] = static_cast<int32_t>(r);
      r += __popc(needs[wd] & ~bits[wd]);
    }
  }

  // victims and the new LRU (row_index.py:94-96, 112-113).  The entries are in
  // LRU order over (row, wave, lane, half): ranks inside a wave come from ballots,
  // the counts of every (row, wave) are scanned in row-major order.
  uint32_t protmask = 0u;  // bit HALVES * q + h: that entry is protected
  static_assert(HALVES * LROWS <= 32, "one protection bit per LRU entry of the thread");
#pragma unroll
  for (int q0 = 0; q0 < LROWS; q0 += MATCH_BATCH) {
    Regs<Regs<uint32_t, HALVES>, MATCH_BATCH> pw;
#pragma unroll
    for (int j = 0; j < MATCH_BATCH; ++j) {
#pragma unroll
      for (int h = 0; h < HALVES; ++h) {
        const int32_t sl = slot_at(q0 + j, h);  // a slot outside [0, S) only with an invalid LRU
        pw[j][h] = prot[(static_cast<uint32_t>(sl) < static_cast<uint32_t>(S) ? sl : 0) >> 5];
      }
    }
#pragma unroll
    for (int j = 0; j < MATCH_BATCH; ++j) {
      const int q = q0 + j;
      int32_t cnt = 0;
#pragma unroll
      for (int h = 0; h < HALVES; ++h) {
        const bool pr = entry_of(q, h) < S && ((pw[j][h] >> (slot_at(q, h) & 31)) & 1u);
        protmask |= static_cast<uint32_t>(pr) << (HALVES * q + h);
        cnt += static_cast<int32_t>(__popcll(__ballot(entry_of(q, h) < S && !pr)));
      }
      if (lane == 0) ucnt[q * NWAVES + wave] = cnt;
    }
  }
  __syncthreads();
  int32_t U;  // unprotected slots
  {
    const int32_t v = T < LROWS * NWAVES ? ucnt[T] : 0;
    const int32_t ex = block_exclusive_sum<int32_t>(v, scan32, &U);
    if (T < LROWS * NWAVES) ucnt[T] = ex;
  }
  __syncthreads();
  const int32_t tm = tot_miss < S ? static_cast<int32_t>(tot_miss) : S;  // only rank < tm matters
  const int32_t Pn = S - U;
  const int32_t fillU = U < tm ? U : tm;
  const int32_t fillP = tm - U > 0 ? (tm - U < Pn ? tm - U : Pn) : 0;
  const int32_t start1 = U - fillU, start2 = U, start3 = S - fillP;
#pragma unroll
  for (int q = 0; q < LROWS; ++q) {
    Regs<uint64_t, HALVES> up;
    int32_t r = ucnt[q * NWAVES + wave];  // unprotected entries before the row's first of this lane
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      up[h] = __ballot(entry_of(q, h) < S && !((protmask >> (HALVES * q + h)) & 1u));
      r += lanes_below(up[h]);
    }
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      const int32_t jj = entry_of(q, h);
      const bool in = jj < S;
      const bool pr = (protmask >> (HALVES * q + h)) & 1u;
      if (in) {
        int32_t rank, at;
        if (!pr) {
          rank = r;
          at = r < fillU ? start1 + r : r - fillU;
        } else {
          const int32_t pj = jj - r;  // protected entries before jj
          rank = U + pj;
          at = pj < fillP ? start3 + pj : start2 + (pj - fillP);
        }
        const int32_t sl = slot_at(q, h);
        if (rank < tm) w.victims[rank] = sl;  // the outputs read only the ranks of misses
        if constexpr (L16) static_cast<int16_t*>(d.lru)[at] = static_cast<int16_t>(sl);
        else static_cast<int64_t*>(d.lru)[at] = sl;
      }
      r += in && !pr ? 1 : 0;  // the lower half precedes the upper one
    }
  }
  if (T == 0) {
    w.totals[0] = static_cast<int64_t>(s_res);
    w.totals[1] = tot_hit;
    w.totals[2] = tot_miss;
    w.totals[3] = dups ? 1 : 0;
  }
}

// ---- split front: the front's work spread over SW workgroups per request, in
// three launches, for the batched decode's descriptors (hs_resolve_desc.split_front):
// a union page bitmap, a power-of-two page of at most 32 tokens, and an affine source
// table whose base is source[0] (host block = source[0] + page for every host-backed
// page, the layout of a request's contiguous host slots).  The single-workgroup
// front keeps the bitmaps of a request in one CU's LDS; here every phase that needs
// the whole request waits for the launch before it instead:
//
//   match  (SW WGs / desc)  pages: resident hits, the range of (host block - page);
//                           hot slots: a slot whose tag's token needs a hot row is a
//                           hit (row_index.py:84-90): the token's slot, the slot's
//                           protection bit;
//   order  (SW WGs / desc)  token words: needs-hot bits, hits among them (a token
//                           whose slot, written by the match launch, holds its tag:
//                           slots left by earlier calls hold other tags), misses;
//                           LRU entries: protected or not, a copy of the LRU;
//   place  (SW WGs / desc)  from every workgroup's counts: the miss prefix per word,
//                           the victims and the new LRU (the same partitions as the
//                           front's, row_index.py:94-96, 112-113), the totals.
//
// Per-workgroup counts go to part[k * SPLIT_MAX + wi].  A table that is not affine
// with base source[0] (other than one with no host-backed page) is refused by the
// place launch: totals[3] = 2, and the outputs launch writes no row.
enum { PART_RES = 0, PART_LO, PART_HI, PART_HIT, PART_MISS, PART_FREE };
constexpr int SPLIT_SLOTS = 4;  // hot slots / LRU entries per thread and launch (hot_rows <= SW * ST * 4)

struct SplitGeom {
  int64_t L, P, NPh, wl;
  int32_t S;
  uint32_t pshift, base;
  __device__ explicit SplitGeom(const hs_resolve_desc& d)
      : L(d.length), P(d.page_size), NPh((d.length + d.page_size - 1) / d.page_size), wl(words_for(d.length)),
        S(static_cast<int32_t>(d.hot_rows)),
        pshift(static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(d.page_size)) - 1)),
        base(static_cast<uint32_t>(d.source[0])) {}
  // token of the host row `tag` under the affine table (-1: none of the history)
  __device__ __forceinline__ int64_t token_of(int32_t tag) const {
    if (tag < 0) return -1;
    const uint32_t page = (static_cast<uint32_t>(tag) >> pshift) - base;  // outside the range: >= 2^31
    if (page >= static_cast<uint64_t>(NPh)) return -1;
    const int64_t t = (static_cast<int64_t>(page) << pshift) | (static_cast<uint32_t>(tag) & static_cast<uint32_t>(P - 1));
    return t < L ? t : -1;
  }
};

__device__ __forceinline__ bool page_bit(const uint32_t* bits, int64_t p) { return (bits[p >> 5] >> (p & 31)) & 1u; }

// sums (and min / max) of one value per thread, published by thread 0
__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int64_t s = 0;
  for (int u = 0; u < static_cast<int>(blockDim.x >> 6); ++u) s += red[u];
  return s;
}

__global__ __launch_bounds__(ST) void resolve_split_match_kernel(ResolveBatch batch) {
  __shared__ int64_t red[ST / 64];
  __shared__ int32_t red_lo[ST / 64], red_hi[ST / 64];
  const hs_resolve_desc& d = batch.d[blockIdx.y];
  const ResolveWs w = ws_of(d);
  const SplitWs x = split_ws_of(d);
  const SplitGeom g(d);
  const int SW = gridDim.x, wi = blockIdx.x, T = threadIdx.x, lane = T & 63, wave = T >> 6;
  // the workgroup's hot slots, 64-aligned (a wave's 64 slots form two protection
  // words, which lanes 0 and 32 store); their tags load first, with the pages' tables
  const int64_t spad = (static_cast<int64_t>(g.S) + 63) / 64 * 64;
  const int64_t sp = ((g.S + SW - 1) / SW + 63) / 64 * 64;
  const int64_t s0 = wi * sp, s1 = s0 + sp < spad ? s0 + sp : spad;
  Regs<int32_t, SPLIT_SLOTS> tag;
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t s = s0 + T + static_cast<int64_t>(k) * ST;
    tag[k] = d.tags[s < g.S ? s : 0];  // unconditional load, masked below
  }
  // the workgroup's pages, 64-aligned (a wave's 64 pages form two needs-page words):
  // resident hits of the selected pages, the range of (host block - page), and the
  // pages whose selected tokens need a hot row
  const int64_t ppad = (g.NPh + 63) / 64 * 64;
  const int64_t pp = ((g.NPh + SW - 1) / SW + 63) / 64 * 64;
  const int64_t p0 = wi * pp, p1 = p0 + pp < ppad ? p0 + pp : ppad;
  int64_t c_res = 0;
  int32_t lo = INT32_MAX, hi = INT32_MIN;
  for (int64_t pb = p0; pb < p1; pb += static_cast<int64_t>(ST) * SPLIT_SLOTS) {
    Regs<int32_t, SPLIT_SLOTS> sv, rv;
    Regs<uint32_t, SPLIT_SLOTS> bw;
#pragma unroll
    for (int k = 0; k < SPLIT_SLOTS; ++k) {
      const int64_t p = pb + T + static_cast<int64_t>(k) * ST;
      const int64_t pc = p < g.NPh ? p : 0;  // unconditional loads, masked below
      sv[k] = d.source[pc];
      rv[k] = d.resident[pc];
      bw[k] = d.page_bits[pc >> 5];
    }
#pragma unroll
    for (int k = 0; k < SPLIT_SLOTS; ++k) {
      const int64_t p = pb + T + static_cast<int64_t>(k) * ST;
      if (p >= p1) break;  // the same for the whole wave (pb, p1 and ST are multiples of 64)
      const bool host = p < g.NPh && sv[k] >= 0;
      const bool sel = (bw[k] >> (p & 31)) & 1u;
      if (host) {
        const int32_t shift = sv[k] - static_cast<int32_t>(p);  // both in [0, 2^31): no overflow
        lo = shift < lo ? shift : lo;
        hi = shift > hi ? shift : hi;
        if (rv[k] >= 0 && sel) c_res += g.L - p * g.P < g.P ? g.L - p * g.P : g.P;
      }
      const uint64_t m = __ballot(host && sel && rv[k] < 0);
      if ((lane & 31) == 0) x.needpg[p >> 5] = lane ? static_cast<uint32_t>(m >> 32) : static_cast<uint32_t>(m);
    }
  }
  // hot slots: a slot whose tag's token needs a hot row is a hit
  Regs<int64_t, SPLIT_SLOTS> tok;
  Regs<bool, SPLIT_SLOTS> hit;
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t s = s0 + T + static_cast<int64_t>(k) * ST;
    tok[k] = s < s1 && s < g.S ? g.token_of(tag[k]) : -1;
  }
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t pg = tok[k] >= 0 ? tok[k] >> g.pshift : 0;
    const bool sel = page_bit(d.page_bits, pg);
    const int32_t sv = d.source[pg], rv = d.resident[pg];
    hit[k] = tok[k] >= 0 && sel && sv >= 0 && rv < 0;
  }
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t s = s0 + T + static_cast<int64_t>(k) * ST;
    if (s >= s1) break;  // the same for the whole wave (s0, s1 and ST are multiples of 64)
    if (hit[k]) w.tslot[tok[k]] = static_cast<int32_t>(s);
    const uint64_t m = __ballot(hit[k]);
    if ((lane & 31) == 0 && (s >> 5) < (g.S + 31) / 32)
      x.prot[s >> 5] = lane ? static_cast<uint32_t>(m >> 32) : static_cast<uint32_t>(m);
  }
  lo = wave_min_i32(lo);
  hi = wave_max_i32(hi);
  if (lane == 0) {
    red_lo[wave] = lo;
    red_hi[wave] = hi;
  }
  const int64_t res = block_sum64(c_res, red);  // its barriers order red_lo / red_hi too
  if (T == 0) {
    for (int u = 0; u < ST / 64; ++u) {
      lo = red_lo[u] < lo ? red_lo[u] : lo;
      hi = red_hi[u] > hi ? red_hi[u] : hi;
    }
    x.part[PART_RES * SPLIT_MAX + wi] = res;
    x.part[PART_LO * SPLIT_MAX + wi] = lo;
    x.part[PART_HI * SPLIT_MAX + wi] = hi;
  }
}

template <bool L16>
__global__ __launch_bounds__(ST) void resolve_split_order_kernel(ResolveBatch batch) {
  __shared__ int64_t red[ST / 64];
  const hs_resolve_desc& d = batch.d[blockIdx.y];
  const ResolveWs w = ws_of(d);
  const SplitWs x = split_ws_of(d);
  const SplitGeom g(d);
  const int SW = gridDim.x, wi = blockIdx.x, T = threadIdx.x;
  // LRU entries (their loads go out with the token words' first loads)
  const int64_t ep = (g.S + SW - 1) / SW, e0 = wi * ep, e1 = e0 + ep < g.S ? e0 + ep : g.S;
  Regs<uint32_t, SPLIT_SLOTS> sl;
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t j = e0 + T + static_cast<int64_t>(k) * ST;
    const int64_t jc = j < e1 ? j : 0;
    // the front's reading of an LRU entry: its low 16 bits (slots < 32768)
    sl[k] = L16 ? static_cast<uint32_t>(static_cast<uint16_t>(static_cast<const int16_t*>(d.lru)[jc]))
                : static_cast<uint32_t>(static_cast<const int64_t*>(d.lru)[jc]) & 0xffffu;
  }
  // token words: needs-hot bits from the match launch's page bitmap, hits among them
  // (a token whose slot still holds its tag), misses
  const int64_t wp = (g.wl + SW - 1) / SW, w0 = wi * wp, w1 = w0 + wp < g.wl ? w0 + wp : g.wl;
  const uint32_t ppw = 32u >> g.pshift;  // pages per token word
  const uint32_t pmask = g.P >= 32 ? 0xffffffffu : (1u << g.P) - 1u;
  int64_t c_hit = 0, c_miss = 0;
  int64_t c_free = 0;
  bool lru_done = false;
  for (int64_t wb = w0; wb < w1 || !lru_done; wb += ST) {
    const int64_t wd = wb + T;
    const int64_t t0 = wd << 5;
    const bool word = wd < w1 && t0 < g.L;
    // a multiple of ppw: the word's pages share one bitmap word
    const int64_t pf = word ? t0 >> g.pshift : 0;
    const uint32_t np = x.needpg[pf >> 5] >> (pf & 31);
    if (!lru_done) {  // the LRU's protection words, loaded beside the first needs words
#pragma unroll
      for (int k = 0; k < SPLIT_SLOTS; ++k) {
        const int64_t j = e0 + T + static_cast<int64_t>(k) * ST;
        const uint32_t pw = x.prot[(sl[k] < static_cast<uint32_t>(g.S) ? sl[k] : 0u) >> 5];
        if (j < e1) {
          x.lru_snap[j] = static_cast<uint16_t>(sl[k]);
          c_free += ((pw >> (sl[k] & 31)) & 1u) ? 0 : 1;
        }
      }
      lru_done = true;
    }
    if (wd >= w1) continue;
    uint32_t needs = 0u;
    if (word) {
      for (uint32_t j = 0; j < ppw; ++j)
        if ((np >> j) & 1u) needs |= pmask << (j * static_cast<uint32_t>(g.P));
      needs &= range_mask(wd, 0, g.L);
    }
    uint32_t hitw = 0u;
    if (needs) {
      // the word's slots (tslot has room up to the next 64 tokens), then their tags
      Regs<int32_t, 32> ts;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int4 v = *reinterpret_cast<const int4*>(w.tslot + t0 + 4 * q);
        ts[4 * q] = v.x;
        ts[4 * q + 1] = v.y;
        ts[4 * q + 2] = v.z;
        ts[4 * q + 3] = v.w;
      }
      Regs<int32_t, 32> tg;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const bool ok = ((needs >> j) & 1u) && ts[j] >= 0 && ts[j] < g.S;
        const int32_t v = d.tags[ok ? ts[j] : 0];  // unconditional load, masked afterwards
        tg[j] = ok ? v : -1;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (g.token_of(tg[j]) == t0 + j) hitw |= 1u << j;
    }
    const uint32_t missw = needs & ~hitw;
    w.hitbits[wd] = hitw;
    w.missbits[wd] = missw;
    c_hit += __popc(hitw);
    c_miss += __popc(missw);
  }
  const int64_t hits = block_sum64(c_hit, red);
  const int64_t misses = block_sum64(c_miss, red);
  const int64_t freed = block_sum64(c_free, red);
  if (T == 0) {
    x.part[PART_HIT * SPLIT_MAX + wi] = hits;
    x.part[PART_MISS * SPLIT_MAX + wi] = misses;
    x.part[PART_FREE * SPLIT_MAX + wi] = freed;
  }
}

template <bool L16>
__global__ __launch_bounds__(ST) void resolve_split_place_kernel(ResolveBatch batch) {
  __shared__ int64_t s_tot[8];  // resident, hits, misses, unprotected; miss and unprotected offsets; lo; hi
  __shared__ int32_t scan32[ST / 64];
  __shared__ int32_t wcnt[ST / 64];
  const hs_resolve_desc& d = batch.d[blockIdx.y];
  const ResolveWs w = ws_of(d);
  const SplitWs x = split_ws_of(d);
  const SplitGeom g(d);
  const int SW = gridDim.x, wi = blockIdx.x, T = threadIdx.x, lane = T & 63, wave = T >> 6;
  // one round of loads: the workgroup's miss words (contiguous runs per thread, in word
  // order; the first word of each run here), its LRU entries, every workgroup's counts
  const int64_t wp = (g.wl + SW - 1) / SW, w0 = wi * wp, w1 = w0 + wp < g.wl ? w0 + wp : g.wl;
  const int64_t run = (w1 - w0 + ST - 1) / ST;
  const int64_t a0 = w0 + T * run < w1 ? w0 + T * run : w1;
  const int64_t a1 = a0 + run < w1 ? a0 + run : w1;
  const uint32_t first_miss = w.missbits[a0 < w1 ? a0 : 0];
  const int64_t ep = (g.S + SW - 1) / SW, e0 = wi * ep, e1 = e0 + ep < g.S ? e0 + ep : g.S;
  Regs<uint32_t, SPLIT_SLOTS> sl;
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t j = e0 + T + static_cast<int64_t>(k) * ST;
    sl[k] = x.lru_snap[j < e1 ? j : 0];
  }
  if (wave == 0) {  // every workgroup's counts: totals and this workgroup's offsets
    const bool in = lane < SW;
    int64_t res = in ? x.part[PART_RES * SPLIT_MAX + lane] : 0;
    int32_t lo = in ? static_cast<int32_t>(x.part[PART_LO * SPLIT_MAX + lane]) : INT32_MAX;
    int32_t hi = in ? static_cast<int32_t>(x.part[PART_HI * SPLIT_MAX + lane]) : INT32_MIN;
    int64_t hit = in ? x.part[PART_HIT * SPLIT_MAX + lane] : 0;
    const int64_t miss = in ? x.part[PART_MISS * SPLIT_MAX + lane] : 0;
    const int64_t fr = in ? x.part[PART_FREE * SPLIT_MAX + lane] : 0;
    const int64_t miss_inc = wave_inclusive_sum(miss), free_inc = wave_inclusive_sum(fr);
    lo = wave_min_i32(lo);
    hi = wave_max_i32(hi);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      res += __shfl_xor(res, off, 64);
      hit += __shfl_xor(hit, off, 64);
    }
    if (lane == wi) {
      s_tot[4] = miss_inc - miss;
      s_tot[5] = free_inc - fr;
    }
    if (lane == 63) {
      s_tot[0] = res;
      s_tot[1] = hit;
      s_tot[2] = miss_inc;
      s_tot[3] = free_inc;
      s_tot[6] = lo;
      s_tot[7] = hi;
    }
  }
  __syncthreads();
  const int64_t tot_miss = s_tot[2];
  const int32_t lo = static_cast<int32_t>(s_tot[6]), hi = static_cast<int32_t>(s_tot[7]);
  // a table with host-backed pages must be affine with base source[0]
  const bool affine = lo > hi || (lo == hi && lo == d.source[0]);
  if (!affine) {
    if (wi == 0 && T == 0) {
      w.totals[0] = 0;
      w.totals[1] = 0;
      w.totals[2] = 0;
      w.totals[3] = 2;
    }
    return;
  }
  if (wi == 0 && T == 0) {
    w.totals[0] = s_tot[0];
    w.totals[1] = s_tot[1];
    w.totals[2] = tot_miss;
    w.totals[3] = 0;  // a page bitmap admits no duplicate input
  }
  // miss prefix of the workgroup's words
  {
    int32_t cnt = a0 < a1 ? __popc(first_miss) : 0;
    for (int64_t wd = a0 + 1; wd < a1; ++wd) cnt += __popc(w.missbits[wd]);
    int32_t all;
    int64_t r = s_tot[4] + block_exclusive_sum<int32_t>(cnt, scan32, &all);
    for (int64_t wd = a0; wd < a1; ++wd) {
      w.mprefix[wd] = static_cast<int32_t>(r);
      r += __popc(wd == a0 ? first_miss : w.missbits[wd]);
    }
  }
  // victims and the new LRU over the workgroup's LRU entries, in LRU order
  const int32_t S = g.S;
  const int32_t U = static_cast<int32_t>(s_tot[3]);
  const int32_t tm = tot_miss < S ? static_cast<int32_t>(tot_miss) : S;  // only rank < tm matters
  const int32_t Pn = S - U;
  const int32_t fillU = U < tm ? U : tm;
  const int32_t fillP = tm - U > 0 ? (tm - U < Pn ? tm - U : Pn) : 0;
  const int32_t start1 = U - fillU, start2 = U, start3 = S - fillP;
  Regs<bool, SPLIT_SLOTS> fr;
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t j = e0 + T + static_cast<int64_t>(k) * ST;
    const uint32_t pw = x.prot[(sl[k] < static_cast<uint32_t>(S) ? sl[k] : 0u) >> 5];
    fr[k] = j < e1 && !((pw >> (sl[k] & 31)) & 1u);
  }
  int32_t r = static_cast<int32_t>(s_tot[5]);  // unprotected entries before the chunk
#pragma unroll
  for (int k = 0; k < SPLIT_SLOTS; ++k) {
    const int64_t j = e0 + T + static_cast<int64_t>(k) * ST;
    const uint64_t m = __ballot(fr[k]);
    if (lane == 0) wcnt[wave] = static_cast<int32_t>(__popcll(m));
    __syncthreads();
    int32_t before = 0, chunk = 0;
    for (int u = 0; u < ST / 64; ++u) {
      const int32_t c = wcnt[u];
      before += u < wave ? c : 0;
      chunk += c;
    }
    __syncthreads();
    if (j < e1) {
      const int32_t rr = r + before + lanes_below(m);  // unprotected entries before entry j
      int32_t rank, at;
      if (fr[k]) {
        rank = rr;
        at = rr < fillU ? start1 + rr : rr - fillU;
      } else {
        const int32_t pj = static_cast<int32_t>(j) - rr;  // protected entries before entry j
        rank = U + pj;
        at = pj < fillP ? start3 + pj : start2 + (pj - fillP);
      }
      if (rank < tm) w.victims[rank] = static_cast<int32_t>(sl[k]);
      if constexpr (L16) static_cast<int16_t*>(d.lru)[at] = static_cast<int16_t>(sl[k]);
      else static_cast<int64_t*>(d.lru)[at] = static_cast<int64_t>(sl[k]);
    }
    r += chunk;
  }
}

// Physical row of input i (-1 when invalid, a later duplicate, or host-less).
// For a miss, `miss_rank` gets its rank, `slot` its victim slot and `host` its
// host row; otherwise miss_rank = -1.
__device__ __forceinline__ int64_t row_of_input(const hs_resolve_desc& d, const ResolveWs& w, bool dups,
                                                int64_t i, int64_t& miss_rank, int32_t& slot,
                                                int64_t& host) {
  miss_rank = -1;
  const int64_t t = load_pos(d, i);
  const int64_t L = d.length, P = d.page_size, S = d.hot_rows;
  if (t < 0 || t >= L) return -1;
  const PageDiv pdiv(P);
  const int64_t page = pdiv.div(static_cast<uint32_t>(t));
  const int64_t off = t - page * P;
  const int64_t word = t >> 5;
  const uint32_t bit = 1u << (t & 31);
  // everything that depends on the token alone, in one round of loads (a hit slot
  // or a first input is read whether or not it applies, and used only where it does)
  const int32_t src = d.source[page], res = d.resident[page];
  const uint32_t hw = w.hitbits[word], mw = w.missbits[word];
  const int32_t mp = w.mprefix[word], ts = w.tslot[t];
  if (dups) {
    const uint32_t dw = w.dupbits[word];
    const int32_t fi = w.first_in[t];
    if ((dw & bit) && fi != static_cast<int32_t>(i)) return -1;
  }
  if (src < 0) return -1;
  if (res >= 0) return static_cast<int64_t>(res) * P + off;
  if (hw & bit) {
    slot = ts;
  } else {
    miss_rank = mp + __popc(mw & (bit - 1u));
    slot = w.victims[miss_rank < S - 1 ? miss_rank : S - 1];
    host = static_cast<int64_t>(src) * P + off;
  }
  if (slot < 0 || slot >= S) {  // only with an LRU that is not a permutation of the slots
    host = -1;
    return -1;
  }
  const int64_t hb = pdiv.div(static_cast<uint32_t>(slot));
  return static_cast<int64_t>(d.hot[hb]) * P + (slot - hb * P);
}

// ---- outputs: rows per input and per head column, miss plan, new tags, counts
__global__ __launch_bounds__(RW) void resolve_outputs_kernel(ResolveBatch batch) {
  const hs_resolve_desc& d = batch.d[blockIdx.y];
  const ResolveWs w = ws_of(d);
  const int64_t n = d.n, S = d.hot_rows;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * RW + threadIdx.x;
  const int64_t tot_miss = w.totals[2];
  if (w.totals[3] == 2) {  // the split front refused the source table: no row, no miss, no count
    if (e < n) {
      if (d.union_physical) d.union_physical[e] = -1;
      if (!d.head_columns && d.physical != d.union_physical) d.physical[e] = -1;
      if (!d.miss_prefix_only) {
        d.miss_host_rows[e] = -1;
        d.miss_device_rows[e] = -1;
      }
      if (e == 0) d.counts[0] = d.counts[1] = d.counts[2] = 0;
    } else if (d.head_columns && e - n < d.heads * d.width) {
      d.physical[e - n] = -1;
    }
    return;
  }
  const bool dups = w.totals[3] != 0;
  if (e < n) {
    int64_t rank, host = -1;
    int32_t slot = -1;
    const int64_t r = row_of_input(d, w, dups, e, rank, slot, host);
    if (d.union_physical) d.union_physical[e] = r;
    if (!d.head_columns && d.physical != d.union_physical) d.physical[e] = r;
    if (rank >= 0) {
      d.miss_host_rows[rank] = host;
      d.miss_device_rows[rank] = r;
      if (r >= 0 && (rank < S - 1 || rank == tot_miss - 1)) d.tags[slot] = static_cast<int32_t>(host);
    }
    if (e >= tot_miss && !d.miss_prefix_only) {  // the RowPlan's -1 tail
      d.miss_host_rows[e] = -1;
      d.miss_device_rows[e] = -1;
    }
    if (e == 0) {
      const int64_t c0 = w.totals[0], c1 = w.totals[1];
      d.counts[0] = c0;
      d.counts[1] = c1;
      d.counts[2] = tot_miss;
      if (d.row_stats) {
        atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[0]), static_cast<unsigned long long>(c0));
        atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[1]), static_cast<unsigned long long>(c1));
        atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[2]), static_cast<unsigned long long>(tot_miss));
      }
    }
    return;
  }
  if (!d.head_columns) return;
  // per-head remap (row_index.py:127-131)
  const int64_t k = e - n;
  if (k >= d.heads * d.width) return;
  const int64_t h = k / d.width, jj = k - h * d.width;
  const int64_t col = d.head_columns[h * d.hc_stride_h + jj * d.hc_stride_w];
  int64_t r = -1;
  if (col >= 0 && col < n) {
    int64_t rank, host;
    int32_t slot;
    r = row_of_input(d, w, dups, col, rank, slot, host);
  }
  d.physical[k] = r;
}

static int64_t front_lds_bytes(int64_t length, int64_t hot_rows) {
  return (2 * words_for(length) + (hot_rows + 31) / 32) * 4;
}

constexpr int64_t kMaxResolverLds = 112 * 1024;  // dynamic LDS of the front launch (its tiles use ~39 KB more)

static int validate_desc(const hs_resolve_desc& d) {
  HS_CHECK_ARG(d.positions && d.n >= 1, "logical top-k must be a nonempty device integer vector");
  HS_CHECK_ARG(d.n < (static_cast<int64_t>(1) << 31), "too many positions");
  HS_CHECK_ARG(d.source && d.resident && d.hot && d.tags && d.lru, "null resolver table");
  HS_CHECK_ARG(d.physical && d.miss_host_rows && d.miss_device_rows && d.counts, "null resolver output");
  HS_CHECK_ARG(d.page_size >= 1 && d.length >= 1, "length and page size must be positive");
  HS_CHECK_ARG(d.n_pages >= 1, "source table must be nonempty");
  HS_CHECK_ARG(d.length <= d.n_pages * d.page_size, "length exceeds the page tables");
  HS_CHECK_ARG(d.hot_rows >= 1 && d.hot_rows <= RT * LRU_CHUNK, "hot_rows must be in [1, 32768]");
  HS_CHECK_ARG(d.lru_i16 == 0 || d.lru_i16 == 1, "lru_i16 must be 0 or 1");
  HS_CHECK_ARG(d.miss_prefix_only == 0 || d.miss_prefix_only == 1, "miss_prefix_only must be 0 or 1");
  HS_CHECK_ARG(d.split_front == 0 || d.split_front == 1, "split_front must be 0 or 1");
  if (d.split_front)
    HS_CHECK_ARG(d.page_bits != nullptr && d.page_size <= 32 && (d.page_size & (d.page_size - 1)) == 0,
                 "split_front needs a union page bitmap and a power-of-two page size of at most 32");
  if (d.lru_i16)  // the front launch reads an int16 LRU as 32-bit pairs
    HS_CHECK_ARG(d.hot_rows % 2 == 0 && (reinterpret_cast<uintptr_t>(d.lru) & 3) == 0,
                 "an int16 LRU needs an even hot_rows and 4-byte alignment");
  HS_CHECK_ARG(d.hot_blocks * d.page_size >= d.hot_rows, "hot block table does not cover hot_rows");
  HS_CHECK_ARG(d.length < (static_cast<int64_t>(1) << 31), "length too large");
  HS_CHECK_ARG(d.n_pages < (static_cast<int64_t>(1) << 31), "too many pages");
  HS_CHECK_ARG(front_lds_bytes(d.length, d.hot_rows) <= kMaxResolverLds,
               "length %lld too large for the LDS token bitmaps", static_cast<long long>(d.length));
  if (d.head_columns) HS_CHECK_ARG(d.heads >= 1 && d.width >= 1, "head columns must be a nonempty matrix");
  return HS_OK;
}

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace hs

using namespace hs;

extern "C" int64_t hs_resolve_workspace_bytes(int64_t n, int64_t length, int64_t n_pages,
                                              int64_t hot_rows) {
  (void)n;
  if (length < 1) length = 1;
  if (hot_rows < 1) hot_rows = 1;
  return ws_layout(length, n_pages, hot_rows, nullptr, nullptr);
}

// Validates every descriptor and returns the workspace bytes the batch needs (< 0: error).
static int64_t batch_workspace(const hs_resolve_desc* descs, int32_t count) {
  HS_CHECK_ARG(descs != nullptr && count >= 1, "resolver batch must be nonempty");
  int64_t need = 0;
  for (int32_t i = 0; i < count; ++i) {
    const int rc = validate_desc(descs[i]);
    if (rc) return rc;
    HS_CHECK_ARG(descs[i].lru_i16 == descs[0].lru_i16, "the descriptors of one batch must share lru_i16");
    HS_CHECK_ARG(descs[i].split_front == descs[0].split_front,
                 "the descriptors of one batch must share split_front");
    need += hs_resolve_workspace_bytes(descs[i].n, descs[i].length, descs[i].n_pages, descs[i].hot_rows);
  }
  return need;
}

// The two launches over validated descriptors; `workspace` holds the batch's need.
static int resolve_launch(const hs_resolve_desc* descs, int32_t count, char* workspace, hipStream_t stream);

extern "C" int hs_resolve_rows_batched(const hs_resolve_desc* descs, int32_t count, void* workspace,
                                       int64_t workspace_bytes, hipStream_t stream) {
  const int64_t need = batch_workspace(descs, count);
  if (need < 0) return static_cast<int>(need);
  HS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "resolver workspace too small: need %lld bytes", static_cast<long long>(need));
  return resolve_launch(descs, count, static_cast<char*>(workspace), stream);
}

template <int SR>
static void launch_front(bool pow2, bool l16, unsigned nb, size_t lds, hipStream_t stream, const ResolveBatch& batch) {
  if (l16) {
    if (pow2) hipLaunchKernelGGL((resolve_front_kernel<true, true, SR>), dim3(nb), dim3(RT), lds, stream, batch);
    else hipLaunchKernelGGL((resolve_front_kernel<false, true, SR>), dim3(nb), dim3(RT), lds, stream, batch);
  } else {
    if (pow2) hipLaunchKernelGGL((resolve_front_kernel<true, false, SR>), dim3(nb), dim3(RT), lds, stream, batch);
    else hipLaunchKernelGGL((resolve_front_kernel<false, false, SR>), dim3(nb), dim3(RT), lds, stream, batch);
  }
}

static int resolve_launch(const hs_resolve_desc* descs, int32_t count, char* workspace, hipStream_t stream) {
  // once per process, from whichever host thread launches first (the others wait)
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    for (const void* f : {reinterpret_cast<const void*>(resolve_front_kernel<true, false, 16>),
                          reinterpret_cast<const void*>(resolve_front_kernel<false, false, 16>),
                          reinterpret_cast<const void*>(resolve_front_kernel<true, true, 16>),
                          reinterpret_cast<const void*>(resolve_front_kernel<false, true, 16>),
                          reinterpret_cast<const void*>(resolve_front_kernel<true, false, 32>),
                          reinterpret_cast<const void*>(resolve_front_kernel<false, false, 32>),
                          reinterpret_cast<const void*>(resolve_front_kernel<true, true, 32>),
                          reinterpret_cast<const void*>(resolve_front_kernel<false, true, 32>)})
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxResolverLds));
    (void)hipGetLastError();
  });
  char* ws = workspace;
  for (int32_t start = 0; start < count; start += RMAXB) {
    ResolveBatch batch{};
    batch.count = count - start < RMAXB ? count - start : RMAXB;
    int64_t front_lds = 0, max_out = 0, max_hot = 0, max_len = 0;
    bool pow2 = true;  // every descriptor's page size a power of two
    for (int i = 0; i < batch.count; ++i) {
      hs_resolve_desc& d = batch.d[i];
      d = descs[start + i];
      d.workspace = ws;
      ws += hs_resolve_workspace_bytes(d.n, d.length, d.n_pages, d.hot_rows);
      if (front_lds_bytes(d.length, d.hot_rows) > front_lds) front_lds = front_lds_bytes(d.length, d.hot_rows);
      pow2 &= (d.page_size & (d.page_size - 1)) == 0;
      if (d.hot_rows > max_hot) max_hot = d.hot_rows;
      if (d.length > max_len) max_len = d.length;
      const int64_t outs = d.n + (d.head_columns ? d.heads * d.width : 0);
      if (outs > max_out) max_out = outs;
    }
    const unsigned nb = static_cast<unsigned>(batch.count);
    const size_t lds = static_cast<size_t>(front_lds);
    const bool l16 = batch.d[0].lru_i16 != 0;  // the same for every descriptor (validated)
    // The split front where it measured faster: hot regions above 16384 rows or histories
    // above 40000 tokens (7B layer shape, 32768 rows and 131072 tokens: 30.4 us for its three
    // launches against 37.5 us for the one-workgroup front; 32B stress shape, 2048 rows and
    // 65536 tokens: the resolve stage 4.20 -> 3.47 ms per step; 0.5B layer shape, 13504 rows
    // and 32768 tokens: 21.7 against 19.3 us, so it keeps the one-workgroup front).
    // HS_RESOLVE_SPLIT=0 / 1 forces either way for descriptors that allow it (read per call).
    const char* split_env = getenv("HS_RESOLVE_SPLIT");
    const int split_force = split_env ? atoi(split_env) : -1;
    const bool large = max_hot > 16 * RT || max_len > 40000;
    const bool split = batch.d[0].split_front && (split_force == 1 || (split_force != 0 && large));
    if (split) {
      // workgroups per request: about one round of 256 in all, and at least enough for
      // SPLIT_SLOTS hot slots per thread
      int sw = static_cast<int>(256 / nb);
      const int need = static_cast<int>(ceil_div(max_hot, static_cast<int64_t>(ST) * SPLIT_SLOTS));
      sw = sw < need ? need : sw;
      sw = sw < 1 ? 1 : (sw > SPLIT_MAX ? SPLIT_MAX : sw);
      const dim3 grid(static_cast<unsigned>(sw), nb);
      hipLaunchKernelGGL(resolve_split_match_kernel, grid, dim3(ST), 0, stream, batch);
      if (l16) {
        hipLaunchKernelGGL(resolve_split_order_kernel<true>, grid, dim3(ST), 0, stream, batch);
        hipLaunchKernelGGL(resolve_split_place_kernel<true>, grid, dim3(ST), 0, stream, batch);
      } else {
        hipLaunchKernelGGL(resolve_split_order_kernel<false>, grid, dim3(ST), 0, stream, batch);
        hipLaunchKernelGGL(resolve_split_place_kernel<false>, grid, dim3(ST), 0, stream, batch);
      }
    } else if (max_hot <= 16 * RT) {
      launch_front<16>(pow2, l16, nb, lds, stream, batch);
    } else {
      launch_front<32>(pow2, l16, nb, lds, stream, batch);
    }
    HS_CHECK_LAUNCH("resolver front");
    hipLaunchKernelGGL(resolve_outputs_kernel, dim3(static_cast<unsigned>(ceil_div(max_out, RW)), nb), dim3(RW),
                       0, stream, batch);
    HS_CHECK_LAUNCH("resolver outputs");
  }
  return HS_OK;
}

extern "C" int hs_resolve_rows(const hs_resolve_desc* desc, void* workspace, int64_t workspace_bytes,
                               hipStream_t stream) {
  return hs_resolve_rows_batched(desc, 1, workspace, workspace_bytes, stream);
}

// ---- the resolver without a caller workspace ----------------------------------
// For callers that cannot allocate (code under graph capture, serving loops,
// harnesses that forbid hipMalloc): the workspace is this file-scope device
// array, one copy per GPU, held until the process ends.  The resolver's kernels
// clear every part of the workspace they read before reading it (the front
// launch resets the duplicate bits and, when it builds one, the host-block hash;
// every other part is written before it is read), so
// nothing is left over from an earlier call; calls that overlap on one GPU
// (two streams, or two host threads) share the array and race.  The first call
// on a device looks up the array's address (and the first resolver call of the
// process sets the front kernels' LDS limit), so a caller that captures the
// call into a graph makes one uncaptured call on that device first.
namespace hs {
constexpr int64_t kNoAllocScratchBytes = static_cast<int64_t>(32) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
}  // namespace hs

extern "C" int64_t hs_resolve_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int hs_resolve_rows_noalloc(const hs_resolve_desc* descs, int32_t count, hipStream_t stream) {
  // Device address of this GPU's copy of `scratch`: in host code the array's name
  // stands for a host-side shadow, never a device address, so it is looked up once
  // per device (with that device current) and only the looked-up pointer is used.
  static void* device_scratch[kMaxDevices] = {};
  static std::mutex lock;
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess || device < 0 || device >= kMaxDevices) {
    (void)hipGetLastError();
    hs::set_error("hs_resolve_rows_noalloc: no current device (%s)", hipGetErrorString(e));
    return HS_ERUNTIME;
  }
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> guard(lock);
    ptr = device_scratch[device];
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr) {
        (void)hipGetLastError();
        hs::set_error("hs_resolve_rows_noalloc: cannot resolve the scratch array on device %d: %s", device,
                      hipGetErrorString(e));
        return HS_ERUNTIME;
      }
      device_scratch[device] = ptr;
    }
  }
  const int64_t need = batch_workspace(descs, count);
  if (need < 0) return static_cast<int>(need);
  HS_CHECK_ARG(need <= kNoAllocScratchBytes,
               "hs_resolve_rows_noalloc: the batch needs %lld bytes of scratch, above the fixed %lld; "
               "split it or call hs_resolve_rows_batched with a workspace",
               static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
  return resolve_launch(descs, count, static_cast<char*>(ptr), stream);
}
