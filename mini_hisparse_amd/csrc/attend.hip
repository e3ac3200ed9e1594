// Physical-row paged GQA decode attention for gfx950.
//
// Replaces the Triton `_attend` / `attend_rows` of mini_hisparse
// (row_kernels.py:73-135) and the torch branch of `row_attention`
// (attention.py:26-35).  Per query head h with KV head h // g, the kernel
// computes softmax((K_j . q) * D^-0.5) over the rows j it selects and the
// weighted sum of V_j, accumulating in fp32; rows < 0 are masked and a head
// with no valid row returns 0.
//
// Work is organised per (request, KV head): an "entry" is one physical row
// together with the bit mask of the query heads of the group that read it.
// Each row is therefore read from HBM once per KV head however many heads
// selected it.  Entries come from one of three sources:
//   ROWS   : per-head row lists [H, W] (no cross-head deduplication),
//   SHARED : one row list read by every head of the group,
//   GROUPS : per-KV-head deduplicated union columns + head masks, with the
//            physical row of a column taken from the resolver's output.
//   WINDOW : the tokens of a window of whole pages (device slot, valid length,
//            optional per-head token mask): the page-window attention of the
//            reference's paged cache (reference/kernels.py:12-68), which returns
//            the unnormalised state (m, l, acc) per head for merging windows.
//
// bf16 / fp16 pools use MFMA (v_mfma_f32_16x16x32_{bf16,f16}): S^T = K Q^T
// with the group's query heads as the N dimension (padded to 16), then
// O^T += V^T P^T with V staged through LDS.  fp32 pools (and head dims other
// than 32, 64 and 128) use a VALU kernel with the same entry sources.  Both write
// split-K partials (m, l, acc).  The MFMA kernel combines them itself: the
// workgroup that finishes a (request, KV head, head chunk) last -- found with an
// arrival counter per group -- merges the group's partials and writes the
// output, so the launch needs no second kernel.  The VALU kernel and the
// window attention (which returns the unnormalised state) use
// `attend_merge_kernel`; both merges run the same arithmetic.
#include <float.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#include <atomic>
#include <chrono>

#include <hip/hip_ext.h>

#include "arrive.h"
#include "hs_common.h"

namespace hs {

enum { MODE_ROWS = 0, MODE_SHARED = 1, MODE_GROUPS = 2, MODE_WINDOW = 3 };

struct AttendArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* pool;
  int64_t P, Hkv, D;
  int64_t pool_rows;  // rows >= pool_rows are masked like rows < 0
  const int64_t* rows;
  int64_t r_sb, r_sh, r_sw, width;
  const int64_t* uphys;
  int64_t u_sb;
  const int32_t* ecol;
  const uint32_t* emask;
  int64_t e_sb, e_sk;
  const int32_t* ecount;
  int64_t emax;
  int mode;
  int head_chunks;
  int64_t B, Hq, g;
  int64_t splits, chunk;
  float scale;
  // split-K partials as tagged words (partial_word): [B, Hq, splits], or [slots, 16]
  // when scheduled; part_o [B, Hq, splits, D], or [slots, 16, D]
  unsigned long long* part_m;
  unsigned long long* part_l;
  unsigned long long* part_o;
  int32_t* sched; // T(0 .. B * Hkv) of the scheduled group kernel
  // in-kernel merge (fuse != 0): one arrival counter per (request, KV head, head
  // chunk), [B * Hkv * head_chunks]; `epoch` tags this launch's arrivals
  unsigned long long* arrivals;
  unsigned long long epoch;
  int fuse;
  int contiguous;     // group splits as contiguous chunks, not dealt by tile (measurement only)
  void* out;
  int64_t o_sb, o_sh;
  const int32_t* wslots;       // WINDOW: device slot of each page [wn]
  const int32_t* wlens;        // WINDOW: valid tokens of each page [wn]
  const unsigned char* wmask;  // WINDOW: [Hq, wn, P] token mask, or null (every token)
  int64_t wn;
};

// Head mask of token t of window page i for KV head k: bit hl set when query
// head k * g + hl reads it.
__device__ __forceinline__ uint32_t window_mask(const AttendArgs& a, int64_t k, int64_t i, int64_t t) {
  const uint32_t all = a.g >= 32 ? 0xffffffffu : ((1u << a.g) - 1u);
  if (!a.wmask) return all;
  uint32_t m = 0u;
  for (int64_t hl = 0; hl < a.g; ++hl)
    m |= static_cast<uint32_t>(a.wmask[((k * a.g + hl) * a.wn + i) * a.P + t] != 0) << hl;
  return m;
}

// Physical row of token t of window page i (-1 past the page's valid tokens).
__device__ __forceinline__ int64_t window_row(const AttendArgs& a, int64_t i, int64_t t) {
  const int64_t len = a.wlens[i];
  return t < len ? static_cast<int64_t>(a.wslots[i]) * a.P + t : -1;
}

__device__ __forceinline__ int64_t entry_count(const AttendArgs& a, int64_t b, int64_t k) {
  if (a.mode == MODE_ROWS) return a.g * a.width;
  if (a.mode == MODE_SHARED) return a.width;
  if (a.mode == MODE_WINDOW) return a.wn * a.P;
  int64_t e = a.ecount[b * a.Hkv + k];
  return e < 0 ? 0 : (e > a.emax ? a.emax : e);
}

__device__ __forceinline__ void entry_at(const AttendArgs& a, int64_t b, int64_t k, int64_t e,
                                         int64_t& phys, uint32_t& mask) {
  if (a.mode == MODE_ROWS) {
    const int64_t hl = e / a.width, j = e - hl * a.width;
    phys = a.rows[b * a.r_sb + (k * a.g + hl) * a.r_sh + j * a.r_sw];
    mask = 1u << hl;
  } else if (a.mode == MODE_SHARED) {
    phys = a.rows[b * a.r_sb + e * a.r_sw];
    mask = a.g >= 32 ? 0xffffffffu : ((1u << a.g) - 1u);
  } else if (a.mode == MODE_WINDOW) {
    const int64_t i = e / a.P, t = e - i * a.P;
    phys = window_row(a, i, t);
    mask = window_mask(a, k, i, t);
  } else {
    const int64_t off = b * a.e_sb + k * a.e_sk + e;
    const int32_t col = a.ecol[off];
    mask = a.emask[off];
    phys = col >= 0 ? a.uphys[b * a.u_sb + col] : -1;
  }
  if (phys < 0 || phys >= a.pool_rows) {
    phys = -1;
    mask = 0;
  }
}

// Element offset of K(row, kv) in a [blocks, 2, P, Hkv, D] pool; V is + P*Hkv*D.
__device__ __forceinline__ int64_t k_offset(int64_t row, int64_t kv, int64_t P, int64_t Hkv, int64_t D) {
  const uint32_t r = static_cast<uint32_t>(row);
  const uint32_t blk = r / static_cast<uint32_t>(P);
  const uint32_t off = r - blk * static_cast<uint32_t>(P);
  return ((static_cast<int64_t>(blk) * 2 * P + off) * Hkv + kv) * D;
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == HS_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ unsigned short to_bits(float v) {
  if constexpr (DT == HS_DTYPE_BF16) return f32_to_bf16_bits(v);
  else return f32_to_f16_bits(v);
}
template <int DT>
__device__ __forceinline__ float from_bits(unsigned short v) {
  if constexpr (DT == HS_DTYPE_BF16) return bf16_bits_to_f32(v);
  else return f16_bits_to_f32(v);
}

// Tagged read (TAGGED) of a partial word another workgroup of the running launch
// stores, possibly on another XCD; a plain read of one a finished launch stored.
template <bool TAGGED>
__device__ __forceinline__ unsigned long long partial_load(const unsigned long long* p) {
  if constexpr (TAGGED) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *p;
}
// Fold a batch of partials (m = -inf: none) into the running (M, L, O): the batch's
// maximum, the running sums rescaled to it, then the batch's terms in order.
template <int MS>
__device__ __forceinline__ void fold_partials(const float (&ms)[MS], const float (&ls)[MS], const float (&os)[MS],
                                              float& M, float& L, float& O) {
  float Mc = M;
#pragma unroll
  for (int u = 0; u < MS; ++u) Mc = fmaxf(Mc, ms[u]);
  if (Mc == -INFINITY) return;
  if (M != -INFINITY && M != Mc) {
    const float r = __expf(M - Mc);
    L *= r;
    O *= r;
  }
#pragma unroll
  for (int u = 0; u < MS; ++u) {
    if (ms[u] == -INFINITY) continue;
    const float f = __expf(ms[u] - Mc);
    L += f * ls[u];
    O += f * os[u];
  }
  M = Mc;
}

// Combine n split-K partials (m, l, acc[d]) of one head, partial u at
// base + u * stride.  Partials are read MS at a time, every load issued before
// any is used (one round of loads per MS partials); chunks after the first
// rescale the running sums, so for n <= MS the arithmetic is a plain max, then
// sums in partial order.  Returns the unnormalised (M, L, O).  TAGGED: the
// partials of the running launch, each taken once it carries `tag`.
template <bool TAGGED, int MS>
__device__ __forceinline__ void merge_partials_by(const unsigned long long* part_m, const unsigned long long* part_l,
                                                  const unsigned long long* part_o, int64_t base, int64_t stride,
                                                  int64_t n, int64_t d, int64_t D, uint32_t tag,
                                                  float& M, float& L, float& O) {
  M = -INFINITY;
  L = 0.f;
  O = 0.f;
  for (int64_t s0 = 0; s0 < n; s0 += MS) {
    float ms[MS], ls[MS], os[MS];
    unsigned long long wm[MS], wl[MS], wo[MS];
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const bool ok = s0 + u < n;
      const int64_t pi = base + (ok ? s0 + u : s0) * stride;  // s0 < n: in bounds
      wm[u] = partial_load<TAGGED>(part_m + pi);
      wl[u] = partial_load<TAGGED>(part_l + pi);
      wo[u] = partial_load<TAGGED>(part_o + pi * D + d);
    }
    if constexpr (TAGGED) {
#pragma unroll
      for (int u = 0; u < MS; ++u) {
        if (s0 + u >= n) continue;
        const int64_t pi = base + (s0 + u) * stride;
        if (static_cast<uint32_t>(wm[u] >> 32) != tag) wm[u] = partial_reread(part_m + pi, tag);
        if (static_cast<uint32_t>(wl[u] >> 32) != tag) wl[u] = partial_reread(part_l + pi, tag);
        if (static_cast<uint32_t>(wo[u] >> 32) != tag) wo[u] = partial_reread(part_o + pi * D + d, tag);
      }
    }
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const bool ok = s0 + u < n;
      ms[u] = ok ? partial_value(wm[u]) : -INFINITY;
      ls[u] = partial_value(wl[u]);
      os[u] = partial_value(wo[u]);
    }
    fold_partials<MS>(ms, ls, os, M, L, O);
  }
}

// merge_partials_by with the batch sized to n (4, 8 or 16 partials per round), so
// that the usual few splits issue no redundant loads (the merging workgroup's loads
// sit at the end of the launch, on its critical path).  The sums are the same: a
// batch covers every partial of n <= 16 in order.
template <bool TAGGED>
__device__ __forceinline__ void merge_partials(const unsigned long long* part_m, const unsigned long long* part_l,
                                               const unsigned long long* part_o, int64_t base, int64_t stride,
                                               int64_t n, int64_t d, int64_t D, uint32_t tag,
                                               float& M, float& L, float& O) {
  if (n <= 4) merge_partials_by<TAGGED, 4>(part_m, part_l, part_o, base, stride, n, d, D, tag, M, L, O);
  else if (n <= 8) merge_partials_by<TAGGED, 8>(part_m, part_l, part_o, base, stride, n, d, D, tag, M, L, O);
  else merge_partials_by<TAGGED, 16>(part_m, part_l, part_o, base, stride, n, d, D, tag, M, L, O);
}

// The merging workgroup's merge of a group of n <= NMAX partials in one round of
// loads: each thread loads one m or l word of the group (a (partial, head) pair,
// passed to every thread of that head through LDS) and the o words of its (head, d)
// pairs, PT per thread, all before the first use, then folds them exactly as
// merge_partials_by does (one batch).  `widx(head, u)` is the word index of head
// `head` of the chunk in partial u; `hc` heads are real; s_ml holds 2 * NMAX * 16
// floats.
template <int DT, int NTH, int NMAX, int PT, typename W>
__device__ __forceinline__ void merge_group_round(const AttendArgs& a, W widx, int hc, int64_t n, uint32_t tag,
                                                  float* s_ml, int64_t out_base) {
  static_assert(2 * NMAX * 16 <= NTH, "one m or l word per thread");
  const int D = static_cast<int>(a.D);
  const int which = threadIdx.x / (NMAX * 16);
  const int rem = threadIdx.x % (NMAX * 16);
  const int mu = rem / 16, mhead = rem % 16;
  const bool ml_ok = which < 2 && mu < n && mhead < hc;
  const unsigned long long* ml_part = which == 0 ? a.part_m : a.part_l;
  const int64_t ml_at = ml_ok ? widx(mhead, mu) : widx(0, 0);
  unsigned long long wml = partial_load<true>(ml_part + ml_at);
  const int pairs = hc * D;
  // only the loads of pairs and partials that exist: both conditions are the same for
  // every thread of the workgroup but the last pair round's, so the loads of a thread
  // still go out together (the merge moves splits x pairs words through one CU)
  unsigned long long wo[PT][NMAX];
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    if (p * NTH >= pairs) continue;
    const int pair = threadIdx.x + p * NTH;
    const bool ok = pair < pairs;
    const int head = ok ? pair / D : 0, d = ok ? pair % D : 0;
#pragma unroll
    for (int u = 0; u < NMAX; ++u) {
      wo[p][u] = 0;
      if (u < n) wo[p][u] = partial_load<true>(a.part_o + widx(head, u) * D + d);
    }
  }
  if (ml_ok && static_cast<uint32_t>(wml >> 32) != tag) wml = partial_reread(ml_part + ml_at, tag);
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int pair = threadIdx.x + p * NTH;
    if (pair >= pairs) continue;
    const int head = pair / D, d = pair % D;
#pragma unroll
    for (int u = 0; u < NMAX; ++u)
      if (u < n && static_cast<uint32_t>(wo[p][u] >> 32) != tag)
        wo[p][u] = partial_reread(a.part_o + widx(head, u) * D + d, tag);
  }
  if (ml_ok) s_ml[(which * NMAX + mu) * 16 + mhead] = partial_value(wml);
  __syncthreads();
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int pair = threadIdx.x + p * NTH;
    if (pair >= pairs) continue;
    const int head = pair / D, d = pair % D;
    float ms[NMAX], ls[NMAX], os[NMAX];
#pragma unroll
    for (int u = 0; u < NMAX; ++u) {
      ms[u] = u < n ? s_ml[u * 16 + head] : -INFINITY;
      ls[u] = u < n ? s_ml[(NMAX + u) * 16 + head] : 0.f;
      os[u] = partial_value(wo[p][u]);
    }
    float M = -INFINITY, L = 0.f, O = 0.f;
    fold_partials<NMAX>(ms, ls, os, M, L, O);
    store_elem<DT>(a.out, out_base + head * a.o_sh + d, L > 0.f ? O / L : 0.f);
  }
}

// The same merge for more than 16 partials (the balanced schedule's long lists): the
// (head, d) pairs one after another, merge_partials batches of 16 partials each.
template <int DT, int NTH, typename W>
__device__ __forceinline__ void merge_group_pairs(const AttendArgs& a, W widx, int hc, int64_t n, uint32_t tag,
                                                  int64_t out_base) {
  const int D = static_cast<int>(a.D);
  for (int pair = threadIdx.x; pair < hc * D; pair += NTH) {
    const int head = pair / D, d = pair % D;
    const int64_t base = widx(head, 0), stride = widx(head, 1) - base;
    float M, L, O;
    merge_partials<true>(a.part_m, a.part_l, a.part_o, base, stride, n, d, D, tag, M, L, O);
    store_elem<DT>(a.out, out_base + head * a.o_sh + d, L > 0.f ? O / L : 0.f);
  }
}


// One workgroup (8 waves) per (split, KV head x head chunk, request), or per slot
// of the balanced schedule below.  The split's entries
// (K element offset, head mask) are staged in LDS once with two batched rounds
// of loads (entry columns with the group's count and the query, then physical
// rows); each wave then walks tiles w, w+8, ... of 32 entries with two register
// buffers used in turn: the loads of tile t+8 are in flight while tile t
// computes, and no buffer is copied (a copy would make the compiler wait for
// the loads).
//
// Group entry lists (split schedule) are dealt to the splits a tile of 32 entries
// at a time: split s takes the group's tiles s, s + splits, s + 2 splits, ...  The
// splits of a group therefore differ by at most one tile whatever the group's
// entry count, with no extra round of loads: a split's entry indices do not depend
// on the count, so its entry columns load together with the count.  (Contiguous
// chunks sized for the capacity left the last split of a typical group nearly
// empty: three of four splits full at the benched shapes.)
constexpr int ATILE = 32;  // entries per tile

// Entries of split s among `splits` when a group's E entries are dealt a tile at a
// time: the splits' tiles are s, s + splits, ..., and only the group's last tile
// may be partial.
__host__ __device__ __forceinline__ int64_t dealt_count(int64_t E, int64_t s, int64_t splits) {
  const int64_t tiles = (E + ATILE - 1) / ATILE;
  if (tiles <= s) return 0;
  const int64_t mine = (tiles - s + splits - 1) / splits;
  const int64_t short_by = ((tiles - 1) % splits == s) ? tiles * ATILE - E : 0;
  return mine * ATILE - short_by;
}

// Group entry index of local entry i of split s (tile-dealt).
__host__ __device__ __forceinline__ int64_t dealt_entry(int64_t i, int64_t s, int64_t splits) {
  return ATILE * (s + splits * (i / ATILE)) + i % ATILE;
}
constexpr int ACH = 2048;        // entries per workgroup (chunk) of the MFMA kernel

// Waves per workgroup of the MFMA kernel.
__host__ __device__ constexpr int attend_waves(int DP) { return 8; }

// Physical row and head mask of entries e0 + i, i = threadIdx.x + s * NTH < cnt
// (rows outside the pool are masked); every load is issued before any use.
template <int MODE, int NTH, int SPT>
__device__ __forceinline__ void stage_entries(const AttendArgs& a, int64_t b, int64_t k, int64_t e0, int cnt,
                                              int64_t (&ph)[SPT], uint32_t (&mk)[SPT]) {
  if constexpr (MODE == MODE_GROUPS) {
    int32_t col[SPT];
    const int64_t base = b * a.e_sb + k * a.e_sk + e0;
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const int ic = i < cnt ? i : 0;
      col[s] = a.ecol[base + ic];
      mk[s] = a.emask[base + ic];
    }
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const bool ok = i < cnt && col[s] >= 0;
      const int64_t pv = a.uphys[b * a.u_sb + (ok ? col[s] : 0)];
      ph[s] = ok ? pv : -1;
    }
  } else if constexpr (MODE == MODE_ROWS) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const int64_t e = e0 + (i < cnt ? i : 0);
      const int64_t hl = e / a.width, j = e - hl * a.width;
      const int64_t pv = a.rows[b * a.r_sb + (k * a.g + hl) * a.r_sh + j * a.r_sw];
      ph[s] = i < cnt ? pv : -1;
      mk[s] = 1u << hl;
    }
  } else if constexpr (MODE == MODE_WINDOW) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const int64_t e = e0 + (i < cnt ? i : 0);
      const int64_t pi = e / a.P, t = e - pi * a.P;
      const int64_t pv = window_row(a, pi, t);
      ph[s] = i < cnt ? pv : -1;
      mk[s] = window_mask(a, k, pi, t);
    }
  } else {
    const uint32_t all = a.g >= 32 ? 0xffffffffu : ((1u << a.g) - 1u);
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const int64_t pv = a.rows[b * a.r_sb + (e0 + (i < cnt ? i : 0)) * a.r_sw];
      ph[s] = i < cnt ? pv : -1;
      mk[s] = all;
    }
  }
#pragma unroll
  for (int s = 0; s < SPT; ++s)
    if (ph[s] < 0 || ph[s] >= a.pool_rows) {
      ph[s] = -1;
      mk[s] = 0u;
    }
}

template <int MODE>
__device__ __forceinline__ int64_t entry_total(const AttendArgs& a, int64_t b, int64_t k) {
  if constexpr (MODE == MODE_ROWS) return a.g * a.width;
  else if constexpr (MODE == MODE_SHARED) return a.width;
  else if constexpr (MODE == MODE_WINDOW) return a.wn * a.P;
  else {
    const int64_t e = a.ecount[b * a.Hkv + k];
    return e < 0 ? 0 : (e > a.emax ? a.emax : e);
  }
}

// ---- balanced schedule of the group attention ----------------------------------
// The entry lists of the (request, KV head) groups differ in length and their
// lengths live on the device.  Rather than splitting every group for the
// longest possible list (which leaves the splits of short lists nearly empty
// while the others run full), every workgroup of the scheduled kernel derives
// the same schedule from the entry counts: the smallest chunk ch (a multiple of
// 32, at least ATT_MIN_CHUNK, at most ACH) for which cutting each group's head
// chunk into s_i = ceil(c_i / ch) workgroups needs at most ATT_SLOTS
// workgroups, i.e. one round on a 256-CU gfx950 (the kernel's LDS admits one
// workgroup per CU).  Group i's workgroups are T(i) + hc * s_i + j (head chunk
// hc, j < s_i), each with an even share of the group's entries rounded up to
// 32.  A group with no entries still gets one workgroup (s_i >= 1), which
// writes the empty partial its merge turns into a zero output.  The workgroup
// index is the slot of its split-K partial; T is written to the workspace for
// the merge.
constexpr int ATT_SLOTS = 256;
constexpr int ATT_MIN_CHUNK = 128;
constexpr int64_t ATT_MAX_GROUPS = 4096;

struct Assignment {
  int32_t group;  // b * Hkv + k, or -1: this workgroup has no work
  int32_t hc, e0, cnt;
  int32_t parts, part;  // workgroups of (group, hc), and this one's index among them
};

__device__ __forceinline__ int32_t wave_total(int32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// c: the groups' clamped entry counts in LDS.  Every lane of the calling wave
// takes part; `table` (or null) receives T(0..ngroups).
__device__ Assignment balanced_assignment(const int32_t* c, int32_t ngroups, int32_t hcs, int32_t w,
                                          int32_t* table) {
  const int lane = threadIdx.x & 63;
  const int32_t per = (ngroups + 63) / 64;
  const int32_t i0 = lane * per < ngroups ? lane * per : ngroups;
  const int32_t i1 = i0 + per < ngroups ? i0 + per : ngroups;
  int32_t e = 0;
  for (int32_t i = i0; i < i1; ++i) e += c[i];
  e = wave_total(e);
  auto parts_of = [](int32_t ci, int32_t ch) { return ci > 0 ? (ci + ch - 1) / ch : 1; };
  auto workgroups = [&](int32_t ch) {
    int32_t s = 0;
    for (int32_t i = i0; i < i1; ++i) s += parts_of(c[i], ch);
    return wave_total(s) * hcs;
  };
  int32_t lo = (hcs * e + ATT_SLOTS - 1) / ATT_SLOTS;
  if (lo < ATT_MIN_CHUNK) lo = ATT_MIN_CHUNK;
  int32_t mlo = (lo + 31) / 32, mhi = ACH / 32;
  if (mlo >= mhi || workgroups(ACH) > ATT_SLOTS) {
    mlo = mhi;  // one round is not possible: chunks of ACH over several rounds
  } else {
    while (mlo < mhi) {  // smallest m with workgroups(32 m) <= ATT_SLOTS (true at mhi)
      const int32_t mid = (mlo + mhi) / 2;
      if (workgroups(32 * mid) <= ATT_SLOTS) mhi = mid;
      else mlo = mid + 1;
    }
  }
  const int32_t ch = 32 * mlo;
  int32_t mine = 0;
  for (int32_t i = i0; i < i1; ++i) mine += hcs * parts_of(c[i], ch);
  const int32_t incl = wave_inclusive_sum(mine), excl = incl - mine;
  if (table) {
    int32_t t = excl;
    for (int32_t i = i0; i < i1; ++i) {
      table[i] = t;
      t += hcs * parts_of(c[i], ch);
    }
    if (lane == 63) table[ngroups] = incl;
  }
  const bool owner = excl <= w && w < incl;
  const uint64_t owners = __ballot(owner);
  Assignment r{-1, 0, 0, 0};
  if (owners == 0) return r;
  const int src = __ffsll(static_cast<unsigned long long>(owners)) - 1;
  int32_t gi = 0, gl = 0;
  if (owner) {
    int32_t t = excl;
    for (int32_t i = i0; i < i1; ++i) {
      const int32_t n = hcs * parts_of(c[i], ch);
      if (w < t + n) {
        gi = i;
        gl = w - t;
        break;
      }
      t += n;
    }
  }
  gi = __shfl(gi, src, 64);
  gl = __shfl(gl, src, 64);
  const int32_t ci = c[gi];
  const int32_t s = parts_of(ci, ch);
  const int32_t hc = gl / s, j = gl - hc * s;
  const int32_t chunk = ((ci + s - 1) / s + 31) / 32 * 32;  // <= ch, and (s - 1) * chunk < ci (ci > 0)
  r.group = gi;
  r.hc = hc;
  r.e0 = j * chunk;
  r.cnt = ci - r.e0 < chunk ? ci - r.e0 : chunk;
  r.parts = s;
  r.part = j;
  return r;
}

template <int DT, int DP, int MODE, bool SCHED>
__global__ __launch_bounds__(64 * attend_waves(DP)) void attend_mfma_kernel(AttendArgs a) {
  constexpr int AW = attend_waves(DP);
  constexpr int NTH = 64 * AW;
  constexpr int SPT = ACH / NTH;  // entries staged per thread
  constexpr int NT = DP / 16;   // PV M-tiles over d
  constexpr int KK = DP / 32;   // QK k-steps over d
  constexpr int RS = DP + 8;    // LDS row stride of the V tile (elements)
  constexpr int CPR = DP / 16 < 4 ? DP / 16 : 4;  // 16-byte V chunks per lane and row
  constexpr int LPR = DP / (8 * CPR);  // lanes per V row
  constexpr int RPI = 64 / LPR;        // V rows per pass of the wave
  constexpr int VI = 32 / RPI;         // V rows per lane and tile
  constexpr int VS_BYTES = AW * 32 * RS * 2;
  constexpr int MERGE_BYTES = AW * 16 * DP * 4;
  constexpr int SMEM = VS_BYTES > MERGE_BYTES ? VS_BYTES : MERGE_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  __shared__ int64_t s_koff[ACH];
  __shared__ uint32_t s_mask[ACH];
  __shared__ float s_m[AW][16], s_l[AW][16];
  __shared__ int s_last;

  unsigned short* vs_all = reinterpret_cast<unsigned short*>(smem);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane >> 4, c = lane & 15;
  const int64_t split = blockIdx.x;
  int64_t k, b, e0;
  int hchunk, cnt;
  int64_t parts, first_slot;  // workgroups of this (group, head chunk); the first one's index
  if constexpr (SCHED) {
    // group entry counts in the (not yet used) V-tile buffer, then the schedule
    int32_t* s_cnt = reinterpret_cast<int32_t*>(smem);
    const int32_t ng = static_cast<int32_t>(a.B * a.Hkv);
    for (int32_t i = threadIdx.x; i < ng; i += NTH) {
      const int64_t e = a.ecount[i];
      s_cnt[i] = static_cast<int32_t>(e < 0 ? 0 : (e > a.emax ? a.emax : e));
    }
    __syncthreads();
    const Assignment asg = balanced_assignment(s_cnt, ng, a.head_chunks, static_cast<int32_t>(blockIdx.x),
                                               blockIdx.x == 0 && wave == 0 ? a.sched : nullptr);
    if (asg.group < 0) return;  // the same for every wave: no barrier is left waiting
    b = asg.group / a.Hkv;
    k = asg.group - b * a.Hkv;
    hchunk = asg.hc;
    e0 = asg.e0;
    cnt = asg.cnt;
    parts = asg.parts;
    first_slot = static_cast<int64_t>(blockIdx.x) - asg.part;
  } else {
    k = blockIdx.y / a.head_chunks;
    hchunk = blockIdx.y % a.head_chunks;
    b = blockIdx.z;
    e0 = split * a.chunk;
    cnt = 0;  // set below, once the group's entry count is known
    parts = a.splits;  // the splits with entries, once the group's count is known (below)
    first_slot = 0;
  }
  // split-K partial of head `hl` of the group (16 * hchunk <= hl < 16 * hchunk + 16)
  auto partial_index = [&](int hl) -> int64_t {
    if constexpr (SCHED) return static_cast<int64_t>(blockIdx.x) * 16 + (hl - 16 * hchunk);
    else return (b * a.Hq + k * a.g + hl) * a.splits + split;
  };
  const int hh = 16 * hchunk + c;  // head index within the group owned by this lane
  const int64_t D = a.D, P = a.P, Hkv = a.Hkv;
  const unsigned short* pool = static_cast<const unsigned short*>(a.pool);
  unsigned short* vs = vs_all + wave * 32 * RS;

  // replay round of the group's arrival counter (the in-kernel merge tags its
  // partial words with it): loaded with the first loads, used after the tiles
  const unsigned long long counter0 = __hip_atomic_load(a.arrivals + (b * a.Hkv + k) * a.head_chunks + hchunk,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Q^T fragments (lane holds Q[head hh][d = 32kk + 8j .. +8]): they depend only
  // on (b, k, hchunk), so their loads go out with the first entry loads.
  u32x4 qf[KK];
  const unsigned short* qrow = static_cast<const unsigned short*>(a.q) + b * a.q_sb + k * a.g * a.q_sh;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const int d0 = 32 * kk + 8 * j;
    const bool ok = hh < a.g && d0 < D;
    const u32x4 v = load16(ok ? qrow + hh * a.q_sh + d0 : qrow);
    qf[kk] = ok ? v : u32x4{0u, 0u, 0u, 0u};
  }

  int64_t ph[SPT];
  uint32_t mk[SPT];
  if constexpr (MODE == MODE_GROUPS && !SCHED) {
    // The split's entry columns and masks are loaded together with the group's
    // entry count (one round of loads instead of two): the split's entries are
    // dealt a tile at a time, so their indices do not depend on the count; an
    // index at or past emax loads entry 0 instead (in bounds, masked below).
    int32_t col[SPT];
    const int64_t base = b * a.e_sb + k * a.e_sk;
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const int64_t e = a.contiguous ? e0 + i : dealt_entry(i, split, a.splits);
      const int64_t ic = e < a.emax ? e : 0;
      col[s] = a.ecol[base + ic];
      mk[s] = a.emask[base + ic];
    }
    const int64_t E = entry_total<MODE>(a, b, k);
    if (a.contiguous) {
      cnt = E > e0 ? static_cast<int>(E - e0 < a.chunk ? E - e0 : a.chunk) : 0;
      parts = E > 0 ? (E + a.chunk - 1) / a.chunk : 1;
    } else {
      cnt = static_cast<int>(dealt_count(E, split, a.splits));
      // splits that hold entries: the first min(splits, tiles) (one when the list is empty)
      const int64_t tiles = (E + ATILE - 1) / ATILE;
      parts = E > 0 ? (tiles < a.splits ? tiles : a.splits) : 1;
    }
    // no branch on cnt here: a conditional block would let the compiler sink the
    // column loads below the wait for the count
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = threadIdx.x + s * NTH;
      const bool ok = i < cnt && col[s] >= 0;
      const int64_t pv = a.uphys[b * a.u_sb + (ok ? col[s] : 0)];
      ph[s] = ok && pv >= 0 && pv < a.pool_rows ? pv : -1;
      if (ph[s] < 0) mk[s] = 0u;
    }
  } else if constexpr (!SCHED) {
    const int64_t E = entry_total<MODE>(a, b, k);
    cnt = E > e0 ? static_cast<int>(E - e0 < a.chunk ? E - e0 : a.chunk) : 0;
    parts = E > 0 ? (E + a.chunk - 1) / a.chunk : 1;
    stage_entries<MODE, NTH, SPT>(a, b, k, e0, cnt, ph, mk);
  } else {
    stage_entries<MODE, NTH, SPT>(a, b, k, e0, cnt, ph, mk);
  }
  // An empty split (cnt == 0, split schedule only) runs no tile and writes the
  // partial m = -inf, l = 0, o = 0 that the merge skips.  It takes the common
  // path on purpose: an early exit here would let the compiler sink every
  // other load of the prologue below the wait for the entry count.
#pragma unroll
  for (int s = 0; s < SPT; ++s) {
    const int i = threadIdx.x + s * NTH;
    s_koff[i] = ph[s] >= 0 ? k_offset(ph[s], k, P, Hkv, D) : -1;
    s_mask[i] = mk[s];
  }

  f32x4 acc[NT];
#pragma unroll
  for (int mt = 0; mt < NT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const int64_t vplane = P * Hkv * D;
  const uint32_t hbit_shift = static_cast<uint32_t>(hh);
  __syncthreads();

  const int ntiles = (cnt + 31) / 32;
  // K fragments (A operand: lane holds K[row 16rt + c][d = 32kk + 8j .. +8]) and the
  // V rows this lane stages (CPR 16-byte chunks of rows vi * RPI + lane / LPR: chunk
  // cc * LPR + lane % LPR, so that the LPR lanes of a row read 16 * LPR contiguous bytes
  // per instruction, one L1 access instead of LPR) of tile t.  Loads are unconditional and their results are used as loaded, so that
  // the loads of a tile stay in flight until the tile is processed: a masked entry
  // reads the lane's query row instead (in bounds, finite).  That data never reaches
  // the output: a masked entry's score is -inf (probability 0, so its V contributes
  // 0).  The head dim is exactly DP, so no lane reads past a row.
  // Addresses of the K rows and V rows this lane loads for tile t (a masked entry
  // reads its own query row instead), computed while earlier tiles' loads are in
  // flight, so that issuing a tile's loads needs no register the loads of the tile
  // before it may still write.
  struct TileAddr {
    const unsigned short* k[2];
    const unsigned short* v[VI];
  };
  auto tile_addr = [&](int t) {
    TileAddr ad;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int li = 32 * t + 16 * rt + c;
      const int64_t koff = s_koff[li < ACH ? li : 0];
      ad.k[rt] = li < cnt && koff >= 0 ? pool + koff + 8 * j : qrow;
    }
#pragma unroll
    for (int vi = 0; vi < VI; ++vi) {
      const int li = 32 * t + vi * RPI + lane / LPR;
      const int64_t koff = s_koff[li < ACH ? li : 0];
      ad.v[vi] = li < cnt && koff >= 0 ? pool + koff + vplane + 8 * (lane % LPR) : qrow;
    }
    return ad;
  };
  auto load_tile = [&](const TileAddr& ad, u32x4 (&kf)[2][KK], u32x4 (&vr)[VI][CPR]) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kf[rt][kk] = load16(ad.k[rt] + 32 * kk);
    }
#pragma unroll
    for (int vi = 0; vi < VI; ++vi) {
#pragma unroll
      for (int cc = 0; cc < CPR; ++cc) vr[vi][cc] = load16(ad.v[vi] + 8 * LPR * cc);
    }
  };

  auto process = [&](int t, const u32x4 (&kf)[2][KK], const u32x4 (&vr)[VI][CPR]) {
    // V rows of this tile into LDS
#pragma unroll
    for (int vi = 0; vi < VI; ++vi) {
      const int row = vi * RPI + lane / LPR;
#pragma unroll
      for (int cc = 0; cc < CPR; ++cc)
        *reinterpret_cast<u32x4*>(vs + row * RS + 8 * (lane % LPR) + 8 * LPR * cc) = vr[vi][cc];
    }

    // S^T[row][head] = K Q^T
    f32x4 st[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) sacc = mfma16x16x32<DT>(kf[rt][kk], qf[kk], sacc);
      st[rt] = sacc;
    }

    // online softmax for head hh over rows 16rt + 4j + i
    float sv[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t mkv = s_mask[32 * t + 16 * rt + 4 * j + i];
        const bool valid = (mkv >> hbit_shift) & 1u;  // hh < 32: at most two head chunks
        const float sc = valid ? st[rt][i] * a.scale : -INFINITY;
        sv[rt][i] = sc;
        tmax = fmaxf(tmax, sc);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = (m_new == -INFINITY) ? 1.f : __expf(m_run - m_new);
    unsigned short pb[8];
    float psum = 0.f;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = (sv[rt][i] == -INFINITY) ? 0.f : __expf(sv[rt][i] - m_new);
        const unsigned short bits = to_bits<DT>(pr);
        pb[4 * rt + i] = bits;
        psum += from_bits<DT>(bits);
      }
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) acc[mt] *= alpha;

    u32x4 pf;
    pf[0] = pb[0] | (static_cast<uint32_t>(pb[1]) << 16);
    pf[1] = pb[2] | (static_cast<uint32_t>(pb[3]) << 16);
    pf[2] = pb[4] | (static_cast<uint32_t>(pb[5]) << 16);
    pf[3] = pb[6] | (static_cast<uint32_t>(pb[7]) << 16);

    wave_lds_sync();  // V tile visible to every lane of the wave
    // O^T[d][head] += V^T P^T; lane holds V[row rho(j,e)][d = 16mt + c]
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) {
      unsigned short vv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int row = 16 * (e >> 2) + 4 * j + (e & 3);
        vv[e] = vs[row * RS + 16 * mt + c];
      }
      u32x4 vf;
      vf[0] = vv[0] | (static_cast<uint32_t>(vv[1]) << 16);
      vf[1] = vv[2] | (static_cast<uint32_t>(vv[3]) << 16);
      vf[2] = vv[4] | (static_cast<uint32_t>(vv[5]) << 16);
      vf[3] = vv[6] | (static_cast<uint32_t>(vv[7]) << 16);
      acc[mt] = mfma16x16x32<DT>(vf, pf, acc[mt]);
    }
    wave_lds_sync();  // all reads of this tile done before the next overwrites it
  };

  u32x4 kA[2][KK], vA[VI][CPR], kB[2][KK], vB[VI][CPR];
  int t = wave;
  if (t < ntiles) {  // uniform per wave
    TileAddr ad = tile_addr(t);
    load_tile(ad, kA, vA);
    ad = tile_addr(t + AW);
    // each half issues the next tile's loads, computes the addresses of the tile
    // after it, then processes the current tile; the scheduling barriers keep the
    // loads ahead of the wait for the current tile (the scheduler would otherwise
    // sink them below it)
    while (true) {
      load_tile(ad, kB, vB);  // past the end: every lane masked
      ad = tile_addr(t + 2 * AW);
      __builtin_amdgcn_sched_barrier(0);
      process(t, kA, vA);
      t += AW;
      if (t >= ntiles) break;
      load_tile(ad, kA, vA);
      ad = tile_addr(t + 2 * AW);
      __builtin_amdgcn_sched_barrier(0);
      process(t, kB, vB);
      t += AW;
      if (t >= ntiles) break;
    }
  }

  if constexpr (!SCHED) {
    // with the in-kernel merge, a split past the group's entries writes no partial
    // and does not arrive (the group waits for its `parts` splits with entries only);
    // the same for every wave of the workgroup, so no barrier is left waiting
    if (a.fuse && split >= parts) return;
  }

  const uint32_t round = counter_round(counter0, a.epoch);
  // per-wave totals over the four lane groups that share a head
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  __syncthreads();
  float* mo = reinterpret_cast<float*>(smem);  // [AW][16][DP]
  if (j == 0) {
    s_m[wave][c] = m_run;
    s_l[wave][c] = l_run;
  }
#pragma unroll
  for (int mt = 0; mt < NT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) mo[(wave * 16 + c) * DP + 16 * mt + 4 * j + i] = acc[mt][i];
  }
  __syncthreads();

  // merge the waves and write this split's partial for each real head
  for (int idx = threadIdx.x; idx < 16 * DP; idx += NTH) {
    const int head = idx / DP, d = idx % DP;
    const int hl = 16 * hchunk + head;
    if (hl >= a.g || d >= D) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AW; ++w) M = fmaxf(M, s_m[w][head]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < AW; ++w) {
        const float f = (s_m[w][head] == -INFINITY) ? 0.f : __expf(s_m[w][head] - M);
        L += f * s_l[w][head];
        O += f * mo[(w * 16 + head) * DP + d];
      }
    }
    const int64_t pidx = partial_index(hl);
    // device-scope stores of tagged words (partial_word): written through to where
    // every XCD's loads of the same scope see them
    const uint32_t tag = a.fuse ? group_tag(a.epoch, round) : 0u;
    if (d == 0) {
      store_partial(a.part_m + pidx, M, tag);
      store_partial(a.part_l + pidx, L, tag);
    }
    store_partial(a.part_o + pidx * D + d, O, tag);
  }
  if (!a.fuse) return;

  // The group's last workgroup merges every partial of the group and writes the
  // output.  It takes each partial word once the word carries the tag (partial_word),
  // so the arrival need not wait for this workgroup's partial stores to complete: the
  // stores and the arrival travel together (one memory round trip fewer on the
  // launch's critical path), and a word the merger reads before its store has landed
  // is read again.  The barrier orders every wave's stores before the arrival.
  __syncthreads();
  unsigned long long* counter = a.arrivals + (b * Hkv + k) * a.head_chunks + hchunk;
  if (threadIdx.x == 0) s_last = arrive_last(counter, a.epoch, parts) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  const uint32_t tag = group_tag(a.epoch, round);
  const int hc = a.g - 16 * hchunk < 16 ? static_cast<int>(a.g - 16 * hchunk) : 16;  // heads of the chunk
  const int64_t out_base = b * a.o_sb + (k * a.g + 16 * hchunk) * a.o_sh;
  auto widx = [&](int head, int64_t u) -> int64_t {  // word of head `head` of the chunk in partial u
    if constexpr (SCHED) return (first_slot + u) * 16 + head;
    else return (b * a.Hq + k * a.g + 16 * hchunk + head) * a.splits + u;
  };
  constexpr int PT = (16 * DP + NTH - 1) / NTH;  // (head, d) pairs per thread
  float* s_ml = reinterpret_cast<float*>(smem);  // free again: the partials are stored
  if (parts <= 4) {
    merge_group_round<DT, NTH, 4, PT>(a, widx, hc, parts, tag, s_ml, out_base);
  } else if (parts <= 8) {
    merge_group_round<DT, NTH, 8, PT>(a, widx, hc, parts, tag, s_ml, out_base);
  } else if (parts <= 16) {
    merge_group_round<DT, NTH, 16, PT>(a, widx, hc, parts, tag, s_ml, out_base);
  } else {
    merge_group_pairs<DT, NTH>(a, widx, hc, parts, tag, out_base);
  }
  if (threadIdx.x == 0)  // the next replay of this launch counts from zero in the next round
    __hip_atomic_store(counter,
                       (static_cast<unsigned long long>(counter_id(a.epoch)) << 32) |
                           (static_cast<unsigned long long>((round + 1) & 0xffffu) << 16),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// VALU fallback: one wave per (split, query head, request); any dtype, D <= 512.
template <int DT>
__global__ __launch_bounds__(64) void attend_valu_kernel(AttendArgs a) {
  constexpr int ND = 8;
  const int lane = threadIdx.x;
  const int64_t split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t k = h / a.g;
  const uint32_t hl = static_cast<uint32_t>(h - k * a.g);
  const int64_t D = a.D;
  float q[ND], acc[ND];
#pragma unroll
  for (int t = 0; t < ND; ++t) {
    const int64_t d = lane + 64 * t;
    q[t] = d < D ? load_elem<DT>(a.q, b * a.q_sb + h * a.q_sh + d) : 0.f;
    acc[t] = 0.f;
  }
  float m_run = -INFINITY, l_run = 0.f;
  const int64_t E = entry_count(a, b, k);
  const int64_t e0 = split * a.chunk;
  int64_t e1 = e0 + a.chunk;
  if (e1 > E) e1 = E;
  const int64_t vplane = a.P * a.Hkv * D;
  for (int64_t e = e0; e < e1; ++e) {
    int64_t ph;
    uint32_t mk;
    entry_at(a, b, k, e, ph, mk);
    if (hl >= 32 || !((mk >> hl) & 1u)) continue;
    const int64_t base = k_offset(ph, k, a.P, a.Hkv, D);
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < ND; ++t) {
      const int64_t d = lane + 64 * t;
      if (d < D) dot += q[t] * load_elem<DT>(a.pool, base + d);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
    const float s = dot * a.scale;
    const float m_new = fmaxf(m_run, s);
    const float alpha = (m_run == -INFINITY) ? 0.f : __expf(m_run - m_new);
    const float p = __expf(s - m_new);
    l_run = l_run * alpha + p;
#pragma unroll
    for (int t = 0; t < ND; ++t) {
      const int64_t d = lane + 64 * t;
      const float v = d < D ? load_elem<DT>(a.pool, base + vplane + d) : 0.f;
      acc[t] = acc[t] * alpha + p * v;
    }
    m_run = m_new;
  }
  const int64_t pidx = (b * a.Hq + h) * a.splits + split;
  if (lane == 0) {
    a.part_m[pidx] = partial_word(m_run, 0u);
    a.part_l[pidx] = partial_word(l_run, 0u);
  }
#pragma unroll
  for (int t = 0; t < ND; ++t) {
    const int64_t d = lane + 64 * t;
    if (d < D) a.part_o[pidx * D + d] = partial_word(acc[t], 0u);
  }
}

// Combine split partials: out = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s, 0 if empty.
// Split schedule: head h's partials are (b * Hq + h) * splits + s.  Scheduled
// group kernel (table != null): head hl of KV head k's group owns the slots
// T(i) + (hl / 16) * n + s, s < n = (T(i + 1) - T(i)) / head_chunks, i = b * Hkv + k,
// and its partial in slot t is t * 16 + hl % 16.
template <int DT>
__global__ __launch_bounds__(256) void attend_merge_kernel(const unsigned long long* part_m,
                                                            const unsigned long long* part_l,
                                                            const unsigned long long* part_o, int64_t splits,
                                                            const int32_t* table, int64_t Hkv, int64_t g,
                                                            int64_t head_chunks, int64_t Hq, int64_t D,
                                                            void* out, int64_t o_sb, int64_t o_sh,
                                                            float* st_m, float* st_l, float* st_o) {
  const int64_t h = blockIdx.x, b = blockIdx.y;
  int64_t base, stride, n;
  if (table) {
    const int64_t k = h / g, hl = h - k * g, i = b * Hkv + k;
    const int64_t t0 = table[i];
    n = (table[i + 1] - t0) / head_chunks;
    base = (t0 + (hl / 16) * n) * 16 + hl % 16;
    stride = 16;
  } else {
    base = (b * Hq + h) * splits;
    stride = 1;
    n = splits;
  }
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    float M, L, O;
    merge_partials<false>(part_m, part_l, part_o, base, stride, n, d, D, 0u, M, L, O);
    if (st_m) {  // the unnormalised state (m, l, acc) of the head, fp32
      if (d == 0) {
        st_m[b * Hq + h] = M;
        st_l[b * Hq + h] = L;
      }
      st_o[(b * Hq + h) * D + d] = O;
    } else {
      store_elem<DT>(out, b * o_sb + h * o_sh + d, L > 0.f ? O / L : 0.f);
    }
  }
}

// Read-only probe of a row-gather access pattern: for each of n segment pairs
// (byte offsets of a K segment; its V segment `plane_bytes` further) read every
// 16-byte unit, consecutive lanes on consecutive units, with no arithmetic
// beyond an XOR that keeps the loads alive; a fixed grid strides over the units
// with eight loads in flight per thread.  Given the K offsets of the
// attention's entries, its duration is the ceiling of the attention's memory
// traffic on the device.
constexpr int PROBE_T = 256;

constexpr int PROBE_U = 8;       // loads in flight per thread
constexpr int PROBE_BLOCKS = 2048;

__global__ __launch_bounds__(PROBE_T) void probe_row_reads_kernel(const char* base, const int64_t* offsets,
                                                                   int64_t n, int64_t seg_units,
                                                                   int64_t plane_bytes, u32x4* sink) {
  // grid-stride over the 16-byte units, PROBE_U loads issued before any is used
  const int64_t total = n * 2 * seg_units;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * PROBE_T;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t u0 = static_cast<int64_t>(blockIdx.x) * PROBE_T + threadIdx.x; u0 < total; u0 += PROBE_U * stride) {
    u32x4 v[PROBE_U];
#pragma unroll
    for (int k = 0; k < PROBE_U; ++k) {
      int64_t u = u0 + k * stride;
      if (u >= total) u = u0;  // in bounds (a repeat of this thread's first unit)
      const int64_t e = u / (2 * seg_units);
      const int64_t w = u - e * 2 * seg_units;
      const int64_t off = offsets[e] + (w >= seg_units ? plane_bytes : 0) + (w % seg_units) * 16;
      v[k] = *reinterpret_cast<const u32x4*>(base + off);
    }
#pragma unroll
    for (int k = 0; k < PROBE_U; ++k) acc ^= v[k];
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0xf39cc060u && acc[3] == 0x5ced1a2bu) sink[0] = acc;
}

// ---- host side ----------------------------------------------------------------

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Plan {
  bool mfma;
  int dp;
  int head_chunks;
  int64_t splits, chunk;
  bool sched;    // the group attention may use the balanced schedule
  int64_t grid;  // its workgroups (slots)
};

// The MFMA kernel takes 16-bit pools with a head dim of exactly 32, 64 or 128 (its
// tiles cover whole rows, with no per-lane bound); others run on the VALU kernel.
// (A head dim of 256 would need more than 256 VGPRs for the two tile buffers, the
// query fragments and the accumulators, and the build rejects kernels that spill.)
static bool mfma_shape(int dtype, int64_t D) {
  return dtype != HS_DTYPE_F32 && (D == 32 || D == 64 || D == 128);
}

static Plan plan_attend(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_entries) {
  Plan p{};
  const int64_t g = Hq / Hkv;
  p.mfma = mfma_shape(dtype, D);
  if (p.mfma) {
    p.dp = static_cast<int>(D);
    p.head_chunks = static_cast<int>(ceil_div(g, 16));
    // entries per workgroup: about one (8-wave) workgroup per CU for the
    // largest entry lists, at most ACH (the LDS entry list), at least 128
    const int64_t groups = B * Hkv * p.head_chunks;
    int64_t chunk = ceil_div(ceil_div(groups * max_entries, 256), 32) * 32;
    static const int64_t forced = [] {
      const char* env = getenv("HS_ATTEND_CHUNK");
      return env ? atoll(env) : 0;
    }();
    if (chunk < 128) chunk = 128;
    // Short lists over few groups would take more than 16 splits of 128 entries (the
    // in-kernel merge's limit; 28 at the Qwen2.5-0.5B shape): at most 12 longer
    // splits instead, merged in-kernel (0.5B end to end: 15.2 us per launch against
    // 16.6 us for 28 splits and the merge launch)
    if (ceil_div(max_entries, chunk) > 16) chunk = ceil_div(ceil_div(max_entries, 12), 32) * 32;
    if (forced > 0) chunk = ceil_div(forced, 32) * 32;
    if (chunk > ACH) chunk = ACH;
    if (chunk < 128) chunk = 128;
    p.chunk = chunk;
    p.splits = ceil_div(max_entries, p.chunk);
    if (p.splits < 1) p.splits = 1;
    // the scheduled group kernel is possible: counts held as int32, the count
    // table fits the V-tile buffer
    const int64_t ng = B * Hkv;
    p.sched = ng <= ATT_MAX_GROUPS && ng * p.head_chunks * max_entries < (int64_t{1} << 31);
    const int64_t rounds = ng * p.head_chunks * ceil_div(max_entries, ACH);
    p.grid = rounds > ATT_SLOTS ? rounds : ATT_SLOTS;
  } else {
    p.dp = 0;
    p.head_chunks = 1;
    int64_t splits = ceil_div(1024, B * Hq);
    const int64_t cap = ceil_div(max_entries, 64);
    if (splits > cap) splits = cap;
    if (splits < 1) splits = 1;
    p.chunk = ceil_div(max_entries, splits);
    if (p.chunk < 1) p.chunk = 1;
    p.splits = ceil_div(max_entries, p.chunk);
    if (p.splits < 1) p.splits = 1;
  }
  return p;
}

// Workspace of one launch: the partials [n] m, [n] l, [n, D] o, the slot table
// T(0 .. B * Hkv) when scheduled, then (8-byte aligned) the arrival counters of
// the in-kernel merge, one per (request, KV head, head chunk).
struct WsLayout {
  int64_t n, table, arrivals, bytes;
};
static WsLayout ws_layout(const Plan& p, bool sched, int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
  WsLayout w{};
  w.n = sched ? p.grid * 16 : B * Hq * p.splits;
  w.table = (2 * w.n + w.n * D) * 8;  // tagged 64-bit partial words
  const int64_t table_end = w.table + (sched ? (B * Hkv + 1) * 4 : 0);
  w.arrivals = (table_end + 7) / 8 * 8;
  w.bytes = w.arrivals + B * Hkv * p.head_chunks * 8 + 256;
  return w;
}
// Either schedule may run on a workspace sized by hs_attend_workspace_bytes.
static int64_t workspace_for(const Plan& p, int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
  const int64_t split = ws_layout(p, false, B, Hq, Hkv, D).bytes;
  const int64_t sched = p.sched ? ws_layout(p, true, B, Hq, Hkv, D).bytes : 0;
  return split > sched ? split : sched;
}


// Events of the next attention launch of this host thread (hs_attend_time_next).
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
static thread_local LaunchEvents next_events;

// Launch `kernel`, stamping `ev` from the dispatch itself when either event is set.
template <typename K, typename... Args>
static void launch_timed(K kernel, dim3 grid, dim3 block, hipStream_t s, const LaunchEvents& ev, Args... args) {
  if (ev.start || ev.stop) hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ev.start, ev.stop, 0, args...);
  else hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

template <int DT, int MODE, bool SCHED>
static void launch_mfma_mode(const Plan& p, const AttendArgs& a, hipStream_t s, const LaunchEvents& ev) {
  dim3 grid(static_cast<unsigned>(p.splits), static_cast<unsigned>(a.Hkv * p.head_chunks),
            static_cast<unsigned>(a.B));
  if (SCHED) grid = dim3(static_cast<unsigned>(p.grid));
  switch (p.dp) {
    case 32: launch_timed(attend_mfma_kernel<DT, 32, MODE, SCHED>, grid, dim3(64 * attend_waves(32)), s, ev, a); break;
    case 64: launch_timed(attend_mfma_kernel<DT, 64, MODE, SCHED>, grid, dim3(64 * attend_waves(64)), s, ev, a); break;
    default: launch_timed(attend_mfma_kernel<DT, 128, MODE, SCHED>, grid, dim3(64 * attend_waves(128)), s, ev, a); break;
  }
}

template <int DT>
static void launch_mfma(const Plan& p, const AttendArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.mode == MODE_GROUPS && a.sched) launch_mfma_mode<DT, MODE_GROUPS, true>(p, a, s, ev);
  else if (a.mode == MODE_GROUPS) launch_mfma_mode<DT, MODE_GROUPS, false>(p, a, s, ev);
  else if (a.mode == MODE_SHARED) launch_mfma_mode<DT, MODE_SHARED, false>(p, a, s, ev);
  else if (a.mode == MODE_WINDOW) launch_mfma_mode<DT, MODE_WINDOW, false>(p, a, s, ev);
  else launch_mfma_mode<DT, MODE_ROWS, false>(p, a, s, ev);
}

// out (o_sb, o_sh) receives the normalised output in the pool dtype; when st_m is
// given, st_m/st_l [B, Hq] and st_o [B, Hq, D] receive the fp32 state instead.
static int run_attend(int dtype, AttendArgs a, int64_t max_entries, void* out, int64_t o_sb,
                      int64_t o_sh, void* ws, int64_t ws_bytes, hipStream_t stream,
                      float* st_m = nullptr, float* st_l = nullptr, float* st_o = nullptr) {
  const LaunchEvents ev = next_events;  // this launch's, also when it is rejected
  next_events = LaunchEvents{};
  Plan p = plan_attend(dtype, a.B, a.Hq, a.Hkv, a.D, max_entries);
  // The split schedule is the default: its first loads (entry count, columns,
  // query) go out in one round, which the balanced schedule cannot do (it needs
  // every count first).  HS_ATTEND_SCHED=1 selects the balanced schedule, which
  // pays off when the entry lists are much shorter than max_entries.
  const char* sched_env = getenv("HS_ATTEND_SCHED");
  const bool sched = p.mfma && p.sched && a.mode == MODE_GROUPS && sched_env && atoi(sched_env) == 1;
  const WsLayout w = ws_layout(p, sched, a.B, a.Hq, a.Hkv, a.D);
  HS_CHECK_ARG(ws != nullptr && ws_bytes >= w.bytes, "attention workspace too small: need %lld bytes",
               static_cast<long long>(w.bytes));
  unsigned long long* base = static_cast<unsigned long long*>(ws);
  a.part_m = base;
  a.part_l = base + w.n;
  a.part_o = base + 2 * w.n;
  a.sched = sched ? reinterpret_cast<int32_t*>(static_cast<char*>(ws) + w.table) : nullptr;
  a.splits = p.splits;
  a.chunk = p.chunk;
  a.head_chunks = p.head_chunks;
  a.scale = 1.0f / sqrtf(static_cast<float>(a.D));
  // The MFMA kernel merges its own partials when the caller wants the normalised
  // output and a group has at most 16 splits: the last workgroup's merge replaces
  // the merge launch (measured on MI355X: 60.3 -> 58.6 us at the microbench, 68.6 ->
  // 54.1 us per launch beside the end-to-end gather), but with many short splits
  // (28 of 128 entries at the Qwen2.5-0.5B shape) the arrivals cost more than the
  // launch (15.5 -> 19.0 us).  HS_ATTEND_FUSED_MERGE=0 / 1 forces either way.
  const char* fused_env = getenv("HS_ATTEND_FUSED_MERGE");  // read per call, like HS_ATTEND_SCHED
  const int fused_merge = fused_env ? atoi(fused_env) : -1;
  const bool few_splits = sched || p.splits <= 16;
  a.fuse = p.mfma && st_m == nullptr && (fused_merge == 1 || (fused_merge != 0 && few_splits)) ? 1 : 0;
  // the arrival counter holds up to 0xffff arrivals; a group has at most
  // ceil(max_entries / 128) workgroups (chunks are at least 128 entries)
  HS_CHECK_ARG(!a.fuse || ceil_div(max_entries, 128) <= 0xffff, "too many entries per attention group");
  a.arrivals = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + w.arrivals);
  a.epoch = next_epoch();
  const char* deal_env = getenv("HS_ATTEND_DEAL");
  a.contiguous = deal_env && atoi(deal_env) == 0 ? 1 : 0;
  a.out = out;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  // the timing events of hs_attend_time_next: start on the attention kernel, stop on
  // the launch's last kernel
  const LaunchEvents first{ev.start, a.fuse ? ev.stop : nullptr};
  const LaunchEvents last{nullptr, ev.stop};
  if (p.mfma) {
    if (dtype == HS_DTYPE_BF16) launch_mfma<HS_DTYPE_BF16>(p, a, stream, first);
    else launch_mfma<HS_DTYPE_F16>(p, a, stream, first);
  } else {
    dim3 grid(static_cast<unsigned>(p.splits), static_cast<unsigned>(a.Hq), static_cast<unsigned>(a.B));
    if (dtype == HS_DTYPE_F32) launch_timed(attend_valu_kernel<HS_DTYPE_F32>, grid, dim3(64), stream, first, a);
    else if (dtype == HS_DTYPE_BF16) launch_timed(attend_valu_kernel<HS_DTYPE_BF16>, grid, dim3(64), stream, first, a);
    else launch_timed(attend_valu_kernel<HS_DTYPE_F16>, grid, dim3(64), stream, first, a);
  }
  HS_CHECK_LAUNCH("attention");
  if (a.fuse) return HS_OK;
  dim3 mgrid(static_cast<unsigned>(a.Hq), static_cast<unsigned>(a.B));
  const unsigned mthreads = a.D <= 64 ? 64 : (a.D <= 128 ? 128 : 256);
  const int64_t hcs = a.head_chunks;
  const unsigned long long* pm = a.part_m;
  const unsigned long long* pl = a.part_l;
  const unsigned long long* po = a.part_o;
  const int32_t* table = a.sched;
  const int64_t splits = p.splits, Hkv = a.Hkv, g = a.g, Hq = a.Hq, D = a.D;
  if (dtype == HS_DTYPE_F32)
    launch_timed(attend_merge_kernel<HS_DTYPE_F32>, mgrid, dim3(mthreads), stream, last, pm, pl, po, splits, table,
                 Hkv, g, hcs, Hq, D, out, o_sb, o_sh, st_m, st_l, st_o);
  else if (dtype == HS_DTYPE_BF16)
    launch_timed(attend_merge_kernel<HS_DTYPE_BF16>, mgrid, dim3(mthreads), stream, last, pm, pl, po, splits, table,
                 Hkv, g, hcs, Hq, D, out, o_sb, o_sh, st_m, st_l, st_o);
  else
    launch_timed(attend_merge_kernel<HS_DTYPE_F16>, mgrid, dim3(mthreads), stream, last, pm, pl, po, splits, table,
                 Hkv, g, hcs, Hq, D, out, o_sb, o_sh, st_m, st_l, st_o);
  HS_CHECK_LAUNCH("attention merge");
  return HS_OK;
}

static int check_common(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                        const void* q, const void* pool, const void* out) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1 && D >= 1 && P >= 1, "attention dimensions must be positive");
  HS_CHECK_ARG(Hq % Hkv == 0, "query heads must be a multiple of KV heads");
  HS_CHECK_ARG(Hq / Hkv <= 32, "at most 32 query heads per KV head are supported");
  HS_CHECK_ARG(D <= 512, "head_dim above 512 is not supported");
  HS_CHECK_ARG(q && pool && out, "null attention pointer");
  if (mfma_shape(dtype, D))
    HS_CHECK_ARG((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(pool) & 15) == 0,
                 "query and pool must be 16-byte aligned");
  return HS_OK;
}

}  // namespace hs

using namespace hs;

extern "C" int64_t hs_attend_workspace_bytes(int32_t dtype, int64_t batch, int64_t heads,
                                             int64_t kv_heads, int64_t head_dim,
                                             int64_t max_entries) {
  if (batch < 1 || heads < 1 || kv_heads < 1 || head_dim < 1 || max_entries < 1) return 256;
  Plan p = plan_attend(dtype, batch, heads, kv_heads, head_dim, max_entries);
  return workspace_for(p, batch, heads, kv_heads, head_dim);
}

extern "C" int hs_attend_rows(const void* query, int64_t q_stride_b, int64_t q_stride_h,
                              const void* pool, int32_t dtype, int64_t page_size,
                              int64_t kv_heads, int64_t head_dim, int64_t pool_rows, const int64_t* rows,
                              int64_t r_stride_b, int64_t r_stride_h, int64_t r_stride_w,
                              int64_t width, int64_t batch, int64_t heads, void* out,
                              int64_t o_stride_b, int64_t o_stride_h, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_common(dtype, batch, heads, kv_heads, head_dim, page_size, query, pool, out);
  if (rc) return rc;
  HS_CHECK_ARG(rows != nullptr && width >= 1, "attention needs a nonempty row list");
  AttendArgs a{};
  a.q = query;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.pool = pool;
  a.P = page_size;
  a.Hkv = kv_heads;
  a.D = head_dim;
  a.pool_rows = pool_rows;
  a.rows = rows;
  a.r_sb = r_stride_b;
  a.r_sh = r_stride_h;
  a.r_sw = r_stride_w;
  a.width = width;
  a.B = batch;
  a.Hq = heads;
  a.g = heads / kv_heads;
  a.mode = r_stride_h == 0 ? MODE_SHARED : MODE_ROWS;
  const int64_t max_entries = a.mode == MODE_SHARED ? width : a.g * width;
  return run_attend(dtype, a, max_entries, out, o_stride_b, o_stride_h, workspace, workspace_bytes, stream);
}

extern "C" int hs_attend_groups(const void* query, int64_t q_stride_b, int64_t q_stride_h,
                                const void* pool, int32_t dtype, int64_t page_size,
                                int64_t kv_heads, int64_t head_dim, int64_t pool_rows,
                                const int64_t* union_physical, int64_t u_stride_b,
                                const int32_t* entry_columns, const uint32_t* entry_masks,
                                int64_t e_stride_b, int64_t e_stride_k,
                                const int32_t* entry_counts, int64_t max_entries,
                                int64_t batch, int64_t heads, void* out, int64_t o_stride_b,
                                int64_t o_stride_h, void* workspace, int64_t workspace_bytes,
                                hipStream_t stream) {
  int rc = check_common(dtype, batch, heads, kv_heads, head_dim, page_size, query, pool, out);
  if (rc) return rc;
  HS_CHECK_ARG(union_physical && entry_columns && entry_masks && entry_counts && max_entries >= 1,
               "group attention needs union rows and entry lists");
  AttendArgs a{};
  a.q = query;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.pool = pool;
  a.P = page_size;
  a.Hkv = kv_heads;
  a.D = head_dim;
  a.pool_rows = pool_rows;
  a.uphys = union_physical;
  a.u_sb = u_stride_b;
  a.ecol = entry_columns;
  a.emask = entry_masks;
  a.e_sb = e_stride_b;
  a.e_sk = e_stride_k;
  a.ecount = entry_counts;
  a.emax = max_entries;
  a.B = batch;
  a.Hq = heads;
  a.g = heads / kv_heads;
  a.mode = MODE_GROUPS;
  return run_attend(dtype, a, max_entries, out, o_stride_b, o_stride_h, workspace, workspace_bytes, stream);
}

extern "C" int hs_attend_window(const void* query, int64_t q_stride_h, const void* pool, int32_t dtype,
                                int64_t page_size, int64_t kv_heads, int64_t head_dim, int64_t pool_rows,
                                const int32_t* slots, const int32_t* lengths, int64_t n_pages,
                                const uint8_t* mask, int64_t heads, float* out_m, float* out_l,
                                float* out_acc, void* workspace, int64_t workspace_bytes,
                                hipStream_t stream) {
  int rc = check_common(dtype, 1, heads, kv_heads, head_dim, page_size, query, pool, out_m);
  if (rc) return rc;
  HS_CHECK_ARG(out_l != nullptr && out_acc != nullptr, "null window attention output");
  HS_CHECK_ARG(slots && lengths && n_pages >= 1, "a window needs at least one page");
  AttendArgs a{};
  a.q = query;
  a.q_sb = 0;
  a.q_sh = q_stride_h;
  a.pool = pool;
  a.P = page_size;
  a.Hkv = kv_heads;
  a.D = head_dim;
  a.pool_rows = pool_rows;
  a.wslots = slots;
  a.wlens = lengths;
  a.wmask = mask;
  a.wn = n_pages;
  a.B = 1;
  a.Hq = heads;
  a.g = heads / kv_heads;
  a.mode = MODE_WINDOW;
  return run_attend(dtype, a, n_pages * page_size, nullptr, 0, 0, workspace, workspace_bytes, stream, out_m,
                    out_l, out_acc);
}

extern "C" int hs_attend_time_next(void* start_event, void* stop_event) {
  next_events.start = static_cast<hipEvent_t>(start_event);
  next_events.stop = static_cast<hipEvent_t>(stop_event);
  return HS_OK;
}

extern "C" int hs_probe_row_reads(const void* base, int64_t region_bytes, const int64_t* offsets, int64_t n,
                                  int64_t segment_bytes, int64_t plane_bytes, void* sink, hipStream_t stream) {
  HS_CHECK_ARG(base && offsets && sink && n >= 1, "null or empty probe");
  HS_CHECK_ARG(segment_bytes >= 16 && segment_bytes % 16 == 0 && plane_bytes % 16 == 0,
               "segments must be multiples of 16 bytes");
  HS_CHECK_ARG((reinterpret_cast<uintptr_t>(base) & 15) == 0, "region must be 16-byte aligned");
  (void)region_bytes;  // offsets are validated by the caller against region_bytes
  const int64_t seg_units = segment_bytes / 16;
  int64_t blocks = ceil_div(n * 2 * seg_units, PROBE_T * PROBE_U);
  if (blocks > PROBE_BLOCKS) blocks = PROBE_BLOCKS;
  hipLaunchKernelGGL(probe_row_reads_kernel, dim3(static_cast<unsigned>(blocks)), dim3(PROBE_T), 0, stream,
                     static_cast<const char*>(base), offsets, n, seg_units, plane_bytes, static_cast<u32x4*>(sink));
  HS_CHECK_LAUNCH("probe");
  return HS_OK;
}
