// Logical-token -> physical-row resolver for gfx950, bit-exact with
// mini_hisparse's `resolve_rows` (row_index.py:59-137).
//
// The reference sorts the selected tokens and the hot tags and uses
// searchsorted/argsort to find hits, protect them, pick least-recent victims
// and reorder the LRU.  Here one 1024-thread workgroup resolves one
// (request, layer) without sorting anything:
//
//   * the selected tokens become a bitmap over [0, length) in LDS, so their
//     ascending order is the bit order and duplicates are found by the
//     atomicOr that sees its bit already set;
//   * hot tags are matched through a hash of the host blocks of the selected
//     non-resident pages (host row = source[page] * P + offset), so a tag maps
//     back to the logical token it caches;
//   * victims are the stable partition "unprotected then protected" of the LRU
//     order, built with one block-wide prefix sum;
//   * miss ranks are a prefix count of miss bits in token order;
//   * the new LRU is the stable partition by category (untouched, filled, hit),
//     again one block-wide prefix sum.
//
// Batched launches run one workgroup per descriptor.  Preconditions, as in the
// reference: unique non-negative tags, an injective source table, and
// length <= n_pages * page_size (checked on the host).
#include "hs_common.h"

namespace hs {

constexpr int RT = 1024;      // threads per resolver workgroup
constexpr int RMAXB = 8;      // descriptors per launch
constexpr int LRU_CHUNK = 32; // hot_rows <= 32768 = RT * LRU_CHUNK

struct ResolveBatch {
  hs_resolve_desc d[RMAXB];
  int count;
};

struct ResolveWs {
  uint32_t* dupbits;  // [wl]
  int32_t* first_in;  // [length]
  int32_t* tslot;     // [length]
  int32_t* hkeys;     // [hcap]
  int32_t* hvals;     // [hcap]
  int32_t* victims;   // [hot_rows]
  int64_t* uresult;   // [n] when the caller gives no union buffer
  int64_t hcap;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); }
__host__ __device__ inline int64_t pow2_at_least(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

__host__ __device__ inline int64_t words_for(int64_t length) { return (length + 32) / 32; }

__host__ __device__ inline int64_t ws_layout(int64_t n, int64_t length, int64_t n_pages, int64_t hot_rows, ResolveWs* w,
                         char* base) {
  const int64_t wl = words_for(length);
  const int64_t hcap = pow2_at_least(2 * (n_pages < 1 ? 1 : n_pages));
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off += align256(bytes);
    return base ? base + at : nullptr;
  };
  char* p0 = take(wl * 4);
  char* p1 = take(length * 4);
  char* p2 = take(length * 4);
  char* p3 = take(hcap * 4);
  char* p4 = take(hcap * 4);
  char* p5 = take(hot_rows * 4);
  char* p6 = take(n * 8);
  if (w) {
    w->dupbits = reinterpret_cast<uint32_t*>(p0);
    w->first_in = reinterpret_cast<int32_t*>(p1);
    w->tslot = reinterpret_cast<int32_t*>(p2);
    w->hkeys = reinterpret_cast<int32_t*>(p3);
    w->hvals = reinterpret_cast<int32_t*>(p4);
    w->victims = reinterpret_cast<int32_t*>(p5);
    w->uresult = reinterpret_cast<int64_t*>(p6);
    w->hcap = hcap;
  }
  return off;
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

__device__ __forceinline__ int64_t load_pos(const hs_resolve_desc& d, int64_t i) {
  return d.positions_i64 ? static_cast<const int64_t*>(d.positions)[i]
                         : static_cast<int64_t>(static_cast<const int32_t*>(d.positions)[i]);
}

// LDS: selbits[wl], hitbits[wl], missbits[wl], protbits[ws], insbits[ws] (u32 words)
__global__ __launch_bounds__(RT) void resolve_kernel(ResolveBatch batch) {
  extern __shared__ uint32_t lds[];
  __shared__ int64_t scan64[16];
  __shared__ int32_t scan32[16];
  __shared__ int any_dup;

  const hs_resolve_desc& d = batch.d[blockIdx.x];
  const int T = threadIdx.x;
  const int64_t n = d.n, L = d.length, P = d.page_size, NP = d.n_pages, S = d.hot_rows;
  const int64_t wl = words_for(L);
  const int64_t wsw = (S + 31) / 32;
  uint32_t* selbits = lds;
  uint32_t* hitbits = selbits + wl;
  uint32_t* missbits = hitbits + wl;
  uint32_t* protbits = missbits + wl;
  uint32_t* insbits = protbits + wsw;

  ResolveWs w;
  ws_layout(n, L, NP, S, &w, static_cast<char*>(d.workspace));
  int64_t* result = d.union_physical ? d.union_physical : (d.head_columns ? w.uresult : d.physical);

  // P0: clear bitmaps and the page hash
  for (int64_t i = T; i < 3 * wl + 2 * wsw; i += RT) lds[i] = 0u;
  for (int64_t i = T; i < wl; i += RT) w.dupbits[i] = 0u;
  for (int64_t i = T; i < w.hcap; i += RT) w.hkeys[i] = -1;
  if (T == 0) any_dup = 0;
  __syncthreads();

  // P1: mark the selected tokens; a bit already set means a duplicate input
  for (int64_t i = T; i < n; i += RT) {
    const int64_t t = load_pos(d, i);
    if (t >= 0 && t < L) {
      const uint32_t bit = 1u << (t & 31);
      const uint32_t old = atomicOr(&selbits[t >> 5], bit);
      if (old & bit) {
        atomicOr(&w.dupbits[t >> 5], bit);
        any_dup = 1;
      }
    }
  }
  __syncthreads();

  // P1b: first input index of each duplicated token (row_index.py:121-126)
  if (any_dup) {
    for (int64_t i = T; i < n; i += RT) {
      const int64_t t = load_pos(d, i);
      if (t >= 0 && t < L && bit_of(w.dupbits, t)) w.first_in[t] = static_cast<int32_t>(n);
    }
    __syncthreads();
    for (int64_t i = T; i < n; i += RT) {
      const int64_t t = load_pos(d, i);
      if (t >= 0 && t < L && bit_of(w.dupbits, t)) atomicMin(&w.first_in[t], static_cast<int32_t>(i));
    }
    __syncthreads();
  }

  // P2: hash host block -> logical page for selected, host-backed, non-resident pages
  const uint32_t hmask = static_cast<uint32_t>(w.hcap - 1);
  for (int64_t p = T; p < NP; p += RT) {
    const int64_t lo = p * P;
    if (lo >= L) continue;
    int64_t hi = lo + P;
    if (hi > L) hi = L;
    bool any = false;
    for (int64_t t = lo; t < hi && !any;) {
      const int64_t word = t >> 5;
      const int64_t wend = (word + 1) << 5;
      const int64_t stop = wend < hi ? wend : hi;
      uint32_t m = selbits[word];
      const int sh0 = static_cast<int>(t & 31);
      const int cnt = static_cast<int>(stop - t);
      m >>= sh0;
      if (cnt < 32) m &= (1u << cnt) - 1u;
      any = m != 0u;
      t = stop;
    }
    if (!any) continue;
    const int32_t src = d.source[p];
    if (src < 0 || d.resident[p] >= 0) continue;
    uint32_t h = hash32(static_cast<uint32_t>(src)) & hmask;
    while (true) {
      const int32_t prev = atomicCAS(&w.hkeys[h], -1, src);
      if (prev == -1) {
        w.hvals[h] = static_cast<int32_t>(p);
        break;
      }
      if (prev == src) break;  // non-injective source table: first page wins
      h = (h + 1) & hmask;
    }
  }
  __syncthreads();

  // P3: hot tag lookup and protection (row_index.py:84-90)
  for (int64_t s = T; s < S; s += RT) {
    const int32_t tag = d.tags[s];
    if (tag < 0) continue;
    const int32_t hp = static_cast<int32_t>(tag / P);
    const int64_t off = tag - static_cast<int64_t>(hp) * P;
    uint32_t h = hash32(static_cast<uint32_t>(hp)) & hmask;
    int32_t page = -1;
    while (true) {
      const int32_t key = w.hkeys[h];
      if (key == -1) break;
      if (key == hp) {
        page = w.hvals[h];
        break;
      }
      h = (h + 1) & hmask;
    }
    if (page < 0) continue;
    const int64_t t = static_cast<int64_t>(page) * P + off;
    if (t >= L || !bit_of(selbits, t)) continue;
    atomicOr(&hitbits[t >> 5], 1u << (t & 31));
    w.tslot[t] = static_cast<int32_t>(s);
    atomicOr(&protbits[s >> 5], 1u << (s & 31));
  }
  __syncthreads();

  // P4: victims = unprotected slots in LRU order, then protected ones (row_index.py:94-95)
  {
    const int64_t j0 = static_cast<int64_t>(T) * LRU_CHUNK;
    int32_t slot[LRU_CHUNK];
    int32_t unprot = 0;
#pragma unroll
    for (int q = 0; q < LRU_CHUNK; ++q) {
      const int64_t jj = j0 + q;
      slot[q] = jj < S ? static_cast<int32_t>(d.lru[jj]) : -1;
      if (jj < S && !bit_of(protbits, slot[q])) ++unprot;
    }
    int32_t total_unprot;
    const int32_t ubase = block_exclusive_sum<int32_t>(unprot, scan32, &total_unprot);
    int32_t u = ubase;
#pragma unroll
    for (int q = 0; q < LRU_CHUNK; ++q) {
      const int64_t jj = j0 + q;
      if (jj >= S) break;
      if (!bit_of(protbits, slot[q])) {
        w.victims[u++] = slot[q];
      } else {
        const int64_t pr = jj - (u);  // protected slots before position jj
        w.victims[total_unprot + pr] = slot[q];
      }
    }
  }
  __syncthreads();

  // P5a: classify the selected tokens in ascending order (row_index.py:72-80, 96)
  const int64_t wpt = (wl + RT - 1) / RT;
  const int64_t w0 = static_cast<int64_t>(T) * wpt;
  int64_t w1 = w0 + wpt;
  if (w1 > wl) w1 = wl;
  int64_t c_res = 0, c_hit = 0, c_miss = 0;
  for (int64_t wd = w0; wd < w1; ++wd) {
    uint32_t m = selbits[wd];
    uint32_t miss_word = 0u;
    while (m) {
      const int b = __builtin_ctz(m);
      m &= m - 1u;
      const int64_t t = (wd << 5) + b;
      const int64_t page = t / P;
      const int32_t src = d.source[page];
      if (src < 0) continue;
      if (d.resident[page] >= 0) {
        ++c_res;
      } else if ((hitbits[wd] >> b) & 1u) {
        ++c_hit;
      } else {
        ++c_miss;
        miss_word |= 1u << b;
      }
    }
    missbits[wd] = miss_word;
  }
  int64_t tot_res, tot_hit, tot_miss;
  block_exclusive_sum<int64_t>(c_res, scan64, &tot_res);
  block_exclusive_sum<int64_t>(c_hit, scan64, &tot_hit);
  const int64_t mbase = block_exclusive_sum<int64_t>(c_miss, scan64, &tot_miss);

  // P5b: assign victims to misses in token order; tags, miss plan (row_index.py:96-120)
  {
    int64_t r = mbase;
    for (int64_t wd = w0; wd < w1; ++wd) {
      uint32_t m = missbits[wd];
      while (m) {
        const int b = __builtin_ctz(m);
        m &= m - 1u;
        const int64_t t = (wd << 5) + b;
        const int64_t page = t / P;
        const int64_t off = t - page * P;
        const int64_t host = static_cast<int64_t>(d.source[page]) * P + off;
        const int64_t vi = r < S - 1 ? r : S - 1;
        const int32_t slot = w.victims[vi];
        w.tslot[t] = slot;
        const int64_t hb = slot / P;
        const int64_t hphys = static_cast<int64_t>(d.hot[hb]) * P + (slot - hb * P);
        d.miss_host_rows[r] = host;
        d.miss_device_rows[r] = hphys;
        if (r < S - 1 || r == tot_miss - 1) {
          d.tags[slot] = static_cast<int32_t>(host);
          atomicOr(&insbits[slot >> 5], 1u << (slot & 31));
        }
        ++r;
      }
    }
    for (int64_t i = tot_miss + T; i < n; i += RT) {
      d.miss_host_rows[i] = -1;
      d.miss_device_rows[i] = -1;
    }
  }
  __syncthreads();

  // P6: LRU stable reorder by category 0 untouched, 1 filled, 2 hit (3 both) (row_index.py:112-113)
  {
    const int64_t j0 = static_cast<int64_t>(T) * LRU_CHUNK;
    int32_t slot[LRU_CHUNK];
    uint64_t packed = 0;  // four 16-bit category counters
#pragma unroll
    for (int q = 0; q < LRU_CHUNK; ++q) {
      const int64_t jj = j0 + q;
      slot[q] = jj < S ? static_cast<int32_t>(d.lru[jj]) : -1;
      if (jj < S) {
        const int cat = static_cast<int>(bit_of(insbits, slot[q])) + 2 * static_cast<int>(bit_of(protbits, slot[q]));
        packed += static_cast<uint64_t>(1) << (16 * cat);
      }
    }
    uint64_t totals;
    const uint64_t before = block_exclusive_sum<uint64_t>(packed, reinterpret_cast<uint64_t*>(scan64), &totals);
    int64_t pos[4];
    int64_t catbase = 0;
#pragma unroll
    for (int cat = 0; cat < 4; ++cat) {
      pos[cat] = catbase + static_cast<int64_t>((before >> (16 * cat)) & 0xffffu);
      catbase += static_cast<int64_t>((totals >> (16 * cat)) & 0xffffu);
    }
    // every thread has read its LRU chunk (block scan above synchronises)
#pragma unroll
    for (int q = 0; q < LRU_CHUNK; ++q) {
      const int64_t jj = j0 + q;
      if (jj >= S) break;
      const int cat = static_cast<int>(bit_of(insbits, slot[q])) + 2 * static_cast<int>(bit_of(protbits, slot[q]));
      d.lru[pos[cat]++] = slot[q];
    }
  }

  // P7: physical row per input, first occurrence of each token wins (row_index.py:96-103, 121-126)
  for (int64_t i = T; i < n; i += RT) {
    const int64_t t = load_pos(d, i);
    int64_t r = -1;
    if (t >= 0 && t < L) {
      bool keep = true;
      if (any_dup && bit_of(w.dupbits, t)) keep = w.first_in[t] == static_cast<int32_t>(i);
      if (keep) {
        const int64_t page = t / P;
        const int64_t off = t - page * P;
        if (d.source[page] >= 0) {
          const int32_t res = d.resident[page];
          if (res >= 0) {
            r = static_cast<int64_t>(res) * P + off;
          } else {
            const int32_t slot = w.tslot[t];
            const int64_t hb = slot / P;
            r = static_cast<int64_t>(d.hot[hb]) * P + (slot - hb * P);
          }
        }
      }
    }
    result[i] = r;
  }
  if (d.head_columns) {
    __syncthreads();
    // P8: per-head remap (row_index.py:127-131)
    const int64_t total = d.heads * d.width;
    for (int64_t e = T; e < total; e += RT) {
      const int64_t h = e / d.width, jj = e - h * d.width;
      const int64_t col = d.head_columns[h * d.hc_stride_h + jj * d.hc_stride_w];
      d.physical[e] = (col >= 0 && col < n) ? result[col] : -1;
    }
  } else if (d.physical != result) {
    for (int64_t i = T; i < n; i += RT) d.physical[i] = result[i];
  }

  // counts (row_index.py:136), optionally accumulated into the cache's row_stats
  if (T == 0) {
    d.counts[0] = tot_res;
    d.counts[1] = tot_hit;
    d.counts[2] = tot_miss;
    if (d.row_stats) {
      atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[0]), static_cast<unsigned long long>(tot_res));
      atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[1]), static_cast<unsigned long long>(tot_hit));
      atomicAdd(reinterpret_cast<unsigned long long*>(&d.row_stats[2]), static_cast<unsigned long long>(tot_miss));
    }
  }
}

static int64_t lds_bytes_for(int64_t length, int64_t hot_rows) {
  return (3 * words_for(length) + 2 * ((hot_rows + 31) / 32)) * 4;
}

constexpr int64_t kMaxResolverLds = 150 * 1024;

static int validate_desc(const hs_resolve_desc& d) {
  HS_CHECK_ARG(d.positions && d.n >= 1, "logical top-k must be a nonempty device integer vector");
  HS_CHECK_ARG(d.n < (static_cast<int64_t>(1) << 31), "too many positions");
  HS_CHECK_ARG(d.source && d.resident && d.hot && d.tags && d.lru, "null resolver table");
  HS_CHECK_ARG(d.physical && d.miss_host_rows && d.miss_device_rows && d.counts, "null resolver output");
  HS_CHECK_ARG(d.page_size >= 1 && d.length >= 1, "length and page size must be positive");
  HS_CHECK_ARG(d.n_pages >= 1, "source table must be nonempty");
  HS_CHECK_ARG(d.length <= d.n_pages * d.page_size, "length exceeds the page tables");
  HS_CHECK_ARG(d.hot_rows >= 1 && d.hot_rows <= RT * LRU_CHUNK, "hot_rows must be in [1, 32768]");
  HS_CHECK_ARG(d.hot_blocks * d.page_size >= d.hot_rows, "hot block table does not cover hot_rows");
  HS_CHECK_ARG(d.length < (static_cast<int64_t>(1) << 31), "length too large");
  HS_CHECK_ARG(lds_bytes_for(d.length, d.hot_rows) <= kMaxResolverLds,
               "length %lld too large for the LDS token bitmaps", static_cast<long long>(d.length));
  if (d.head_columns) HS_CHECK_ARG(d.heads >= 1 && d.width >= 1, "head columns must be a nonempty matrix");
  return HS_OK;
}

}  // namespace hs

using namespace hs;

extern "C" int64_t hs_resolve_workspace_bytes(int64_t n, int64_t length, int64_t n_pages,
                                              int64_t hot_rows) {
  if (n < 1) n = 1;
  if (length < 1) length = 1;
  if (hot_rows < 1) hot_rows = 1;
  return ws_layout(n, length, n_pages, hot_rows, nullptr, nullptr);
}

extern "C" int hs_resolve_rows_batched(const hs_resolve_desc* descs, int32_t count, void* workspace,
                                       int64_t workspace_bytes, hipStream_t stream) {
  HS_CHECK_ARG(descs != nullptr && count >= 1, "resolver batch must be nonempty");
  int64_t need = 0;
  for (int32_t i = 0; i < count; ++i) {
    const int rc = validate_desc(descs[i]);
    if (rc) return rc;
    need += hs_resolve_workspace_bytes(descs[i].n, descs[i].length, descs[i].n_pages, descs[i].hot_rows);
  }
  HS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "resolver workspace too small: need %lld bytes", static_cast<long long>(need));
  char* ws = static_cast<char*>(workspace);
  for (int32_t start = 0; start < count; start += RMAXB) {
    ResolveBatch batch{};
    batch.count = count - start < RMAXB ? count - start : RMAXB;
    int64_t lds = 0;
    for (int i = 0; i < batch.count; ++i) {
      batch.d[i] = descs[start + i];
      batch.d[i].workspace = ws;
      ws += hs_resolve_workspace_bytes(batch.d[i].n, batch.d[i].length, batch.d[i].n_pages, batch.d[i].hot_rows);
      const int64_t l = lds_bytes_for(batch.d[i].length, batch.d[i].hot_rows);
      if (l > lds) lds = l;
    }
    static bool attr_set = false;
    if (!attr_set) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(resolve_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxResolverLds));
      (void)hipGetLastError();
      attr_set = true;
    }
    hipLaunchKernelGGL(resolve_kernel, dim3(batch.count), dim3(RT), static_cast<size_t>(lds), stream, batch);
    HS_CHECK_LAUNCH("resolver");
  }
  return HS_OK;
}

extern "C" int hs_resolve_rows(const hs_resolve_desc* desc, void* workspace, int64_t workspace_bytes,
                               hipStream_t stream) {
  return hs_resolve_rows_batched(desc, 1, workspace, workspace_bytes, stream);
}
