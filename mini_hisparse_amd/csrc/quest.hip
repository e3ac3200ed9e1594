// Quest page scorer, per-head top-k and the device-side union builder for gfx950.
//
// Scorer + top-k replace `quest_selection` (selection.py:80-101): for query
// head h with KV head h // g, page p scores
//     s = sum_d max(q_d * lo_d, q_d * hi_d)
// over the page's K minimum/maximum bounds; the tail page and (optionally)
// page 0 are forced; the `top` best pages per head are kept.  The sum runs over
// d in ascending order with one float32 rounding per step (for 16-bit inputs
// the product is exact, so a fused multiply-add gives the same value); ties
// go to the lower page index.  Since max(q*lo, q*hi) is q*hi for q >= 0 and
// q*lo otherwise (hi >= lo), the kernel selects the bound before multiplying.
//
// The union builder replaces the host adapter Selection -> LogicalTopK
// (row_index.py:20-31, selection.py:43-60): from the chosen pages it writes the
// ascending union of selected tokens (padded with -1), each head's union
// columns, and per KV head the deduplicated union columns its query heads read
// with a bit mask of those heads (the entry lists of the group attention).
#include <algorithm>
#include <stdlib.h>
#include <string.h>

#include "hs_common.h"

namespace hs {

constexpr int QMAXB = 16;       // requests per launch
constexpr int QHEADS = 8;       // query heads per scorer thread
constexpr int QT = 256;         // scorer / top-k threads
constexpr int UT = 1024;        // union builder threads
constexpr int64_t UMAXPAGES = 65536;

struct QuestArgs {
  const void* q;                // [B, Hq, D] in q_dtype (f32, bf16 or f16)
  int q_dtype;
  int64_t q_sb, q_sh;
  const void* kmin[QMAXB];      // per request [pages, Hkv, D]
  const void* kmax[QMAXB];
  int64_t count[QMAXB];         // ceil(length / P)
  int64_t Hq, Hkv, g, D, top;
  int keep_sink;
  float* scores;                // [B, Hq, cmax]
  int64_t cmax;
  int32_t* pages;               // [B, Hq, top]
  int64_t p_sb;
};

// Query element i widened to fp32 (exact for every query dtype).
__device__ __forceinline__ float query_value(const QuestArgs& a, int64_t i) {
  if (a.q_dtype == HS_DTYPE_BF16) return load_elem<HS_DTYPE_BF16>(a.q, i);
  if (a.q_dtype == HS_DTYPE_F16) return load_elem<HS_DTYPE_F16>(a.q, i);
  return load_elem<HS_DTYPE_F32>(a.q, i);
}

template <int DT, bool FUSED>
__global__ __launch_bounds__(QT) void quest_score_kernel(QuestArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float sq[];  // [QHEADS][D]
  const int64_t b = blockIdx.z;
  const int64_t kv = blockIdx.y / ((a.g + QHEADS - 1) / QHEADS);
  const int64_t hc = blockIdx.y % ((a.g + QHEADS - 1) / QHEADS);
  const int64_t count = a.count[b];
  if (a.top >= count) return;
  const int64_t h0 = kv * a.g + hc * QHEADS;
  int64_t nh = a.g - hc * QHEADS;
  if (nh > QHEADS) nh = QHEADS;
  const int64_t D = a.D;
  for (int64_t i = threadIdx.x; i < QHEADS * D; i += QT) {
    const int64_t hl = i / D, d = i - hl * D;
    sq[i] = hl < nh ? query_value(a, b * a.q_sb + (h0 + hl) * a.q_sh + d) : 0.f;
  }
  __syncthreads();
  const int64_t p = static_cast<int64_t>(blockIdx.x) * QT + threadIdx.x;
  if (p >= count) return;
  const int64_t row = (p * a.Hkv + kv) * D;
  const void* lo = a.kmin[b];
  const void* hi = a.kmax[b];
  float acc[QHEADS];
#pragma unroll
  for (int hl = 0; hl < QHEADS; ++hl) acc[hl] = 0.f;
  auto step = [&](int64_t d, float l, float u) {
#pragma unroll
    for (int hl = 0; hl < QHEADS; ++hl) {
      const float qv = sq[hl * D + d];
      const float bound = qv >= 0.f ? u : l;
      if constexpr (FUSED) {
        acc[hl] = __builtin_fmaf(qv, bound, acc[hl]);
      } else {
        const float prod = qv * bound;
        acc[hl] = acc[hl] + prod;
      }
    }
  };
  constexpr int EPV = DT == HS_DTYPE_F32 ? 4 : 8;  // elements per 16-byte load
  const bool vec = (D % EPV) == 0;
  if (vec) {
    for (int64_t d0 = 0; d0 < D; d0 += EPV) {
      const u32x4 L = *reinterpret_cast<const u32x4*>(static_cast<const char*>(lo) + (row + d0) * (DT == HS_DTYPE_F32 ? 4 : 2));
      const u32x4 U = *reinterpret_cast<const u32x4*>(static_cast<const char*>(hi) + (row + d0) * (DT == HS_DTYPE_F32 ? 4 : 2));
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        float l, u;
        if constexpr (DT == HS_DTYPE_F32) {
          l = __uint_as_float(L[e]);
          u = __uint_as_float(U[e]);
        } else {
          const unsigned short lb = static_cast<unsigned short>(L[e >> 1] >> (16 * (e & 1)));
          const unsigned short ub = static_cast<unsigned short>(U[e >> 1] >> (16 * (e & 1)));
          if constexpr (DT == HS_DTYPE_BF16) {
            l = bf16_bits_to_f32(lb);
            u = bf16_bits_to_f32(ub);
          } else {
            l = f16_bits_to_f32(lb);
            u = f16_bits_to_f32(ub);
          }
        }
        step(d0 + e, l, u);
      }
    }
  } else {
    for (int64_t d = 0; d < D; ++d) step(d, load_elem<DT>(lo, row + d), load_elem<DT>(hi, row + d));
  }
  for (int hl = 0; hl < nh; ++hl) a.scores[(b * a.Hq + h0 + hl) * a.cmax + p] = acc[hl];
}

// LDS-tiled scorer for the common shapes.  One workgroup scores QS_PAGES pages
// of one KV head for a chunk of up to QHEADS query heads.  The pages' lower and
// upper bound rows (D elements each, 2 KB apart in HBM for Hkv = 8, D = 128
// bf16) are staged in LDS with full-line loads (consecutive lanes read
// consecutive 16-byte units, every unit of a fetched line is used); then lane
// l of wave w scores page l for query heads 2w and 2w+1 of the chunk, reading
// its row from LDS (row stride padded by 16 bytes: conflict-free 16-byte
// reads) and the query values as wave-wide broadcasts.  The per-score
// arithmetic is that of quest_score_kernel: d ascending, one float32 rounding
// per step.
constexpr int QS_PAGES = 64;
constexpr int QS_UNITS = 8;                  // 16-byte units per thread per bound
constexpr int64_t QS_MAX_ROW_BYTES = QS_UNITS * QT * 16 / QS_PAGES;  // 512

__host__ __device__ constexpr int64_t qs_lds_bytes(int64_t row_bytes, int64_t D) {
  return 2 * QS_PAGES * (row_bytes + 16) + QHEADS * D * 4;
}

template <int DT, bool FUSED>
__global__ __launch_bounds__(QT) void quest_score_tile_kernel(QuestArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) unsigned char qs_smem[];
  constexpr int ESZ = DT == HS_DTYPE_F32 ? 4 : 2;
  constexpr int EPV = 16 / ESZ;  // elements per 16-byte unit
  const int64_t b = blockIdx.z;
  const int64_t hchunks = (a.g + QHEADS - 1) / QHEADS;
  const int64_t kv = blockIdx.y / hchunks, hc = blockIdx.y - kv * hchunks;
  const int64_t count = a.count[b];
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * QS_PAGES;
  if (a.top >= count || p0 >= count) return;
  const int64_t D = a.D, Hkv = a.Hkv;
  const int64_t rb = D * ESZ, rs = rb + 16, upr = rb / 16;
  unsigned char* tlo = qs_smem;
  unsigned char* thi = qs_smem + QS_PAGES * rs;
  float* sq = reinterpret_cast<float*>(qs_smem + 2 * QS_PAGES * rs);  // [QHEADS][D]
  int64_t nh = a.g - hc * QHEADS;
  if (nh > QHEADS) nh = QHEADS;
  const int64_t h0 = kv * a.g + hc * QHEADS;
  for (int64_t i = threadIdx.x; i < QHEADS * D; i += QT) {
    const int64_t hl = i / D, d = i - hl * D;
    sq[i] = hl < nh ? query_value(a, b * a.q_sb + (h0 + hl) * a.q_sh + d) : 0.f;
  }
  int64_t npg = count - p0;
  if (npg > QS_PAGES) npg = QS_PAGES;
  const char* lo = static_cast<const char*>(a.kmin[b]);
  const char* hi = static_cast<const char*>(a.kmax[b]);
  // 32-bit tile indexing: at most QS_PAGES * 32 units per bound
  const uint32_t units = static_cast<uint32_t>(npg * upr), upr32 = static_cast<uint32_t>(upr);
  const uint32_t rb32 = static_cast<uint32_t>(rb), rs32 = static_cast<uint32_t>(rs);
  const char* lo_t = lo + (p0 * Hkv + kv) * rb;
  const char* hi_t = hi + (p0 * Hkv + kv) * rb;
  const uint32_t gstride = static_cast<uint32_t>(Hkv) * rb32;  // bytes between consecutive pages
  // every thread issues all of its loads before the first LDS store; a unit
  // past the tile reloads unit 0 (in bounds) and is not stored
  u32x4 L[QS_UNITS], U[QS_UNITS];
#pragma unroll
  for (int k = 0; k < QS_UNITS; ++k) {
    uint32_t u = threadIdx.x + static_cast<uint32_t>(k) * QT;
    if (u >= units) u = 0;
    const uint32_t r = u / upr32, c = u - r * upr32;
    const uint64_t off = static_cast<uint64_t>(r) * gstride + c * 16u;
    L[k] = *reinterpret_cast<const u32x4*>(lo_t + off);
    U[k] = *reinterpret_cast<const u32x4*>(hi_t + off);
  }
#pragma unroll
  for (int k = 0; k < QS_UNITS; ++k) {
    const uint32_t u = threadIdx.x + static_cast<uint32_t>(k) * QT;
    const uint32_t r = u / upr32, c = u - r * upr32;
    if (u < units) {
      *reinterpret_cast<u32x4*>(tlo + r * rs32 + c * 16u) = L[k];
      *reinterpret_cast<u32x4*>(thi + r * rs32 + c * 16u) = U[k];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hA = 2 * wave, hB = 2 * wave + 1;
  if (lane >= npg || hA >= nh) return;  // no barrier follows
  const float* qa = sq + hA * D;
  const float* qb = sq + hB * D;
  const unsigned char* rlo = tlo + lane * rs;
  const unsigned char* rhi = thi + lane * rs;
  float accA = 0.f, accB = 0.f;
  auto step = [&](float qv, float l, float u, float& acc) {
    const float bound = qv >= 0.f ? u : l;
    if constexpr (FUSED) {
      acc = __builtin_fmaf(qv, bound, acc);
    } else {
      const float prod = qv * bound;
      acc = acc + prod;
    }
  };
  for (int64_t d0 = 0; d0 < D; d0 += EPV) {
    const u32x4 Lv = *reinterpret_cast<const u32x4*>(rlo + d0 * ESZ);
    const u32x4 Uv = *reinterpret_cast<const u32x4*>(rhi + d0 * ESZ);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      float l, u;
      if constexpr (DT == HS_DTYPE_F32) {
        l = __uint_as_float(Lv[e]);
        u = __uint_as_float(Uv[e]);
      } else {
        const unsigned short lb = static_cast<unsigned short>(Lv[e >> 1] >> (16 * (e & 1)));
        const unsigned short ub = static_cast<unsigned short>(Uv[e >> 1] >> (16 * (e & 1)));
        if constexpr (DT == HS_DTYPE_BF16) {
          l = bf16_bits_to_f32(lb);
          u = bf16_bits_to_f32(ub);
        } else {
          l = f16_bits_to_f32(lb);
          u = f16_bits_to_f32(ub);
        }
      }
      step(qa[d0 + e], l, u, accA);
      step(qb[d0 + e], l, u, accB);
    }
  }
  const int64_t p = p0 + lane;
  a.scores[(b * a.Hq + h0 + hA) * a.cmax + p] = accA;
  if (hB < nh) a.scores[(b * a.Hq + h0 + hB) * a.cmax + p] = accB;
}

// Scorer for bf16 bounds with the bound selection taken off the vector ALU.
// For query head h and element d, max(q*lo, q*hi) is q*hi when q >= 0 and q*lo
// otherwise, and that choice is the same for every page a wave scores: each
// wave scores one query head, reads its query words with uniform (scalar) loads
// and turns each sign into a byte selector.  One v_perm_b32 per (page, element)
// then picks the bf16 half of the chosen bound and widens it to fp32 (the bf16
// bits become the high half of the word, the low half zero), leaving one fused
// multiply-add per element for bf16 queries (their product with a bf16 bound is
// exact) and a multiply and an add for fp32 queries.  A query of -0 picks the
// lower bound here and the upper one in quest_score_kernel; both products are
// zeros, and a sum started at +0 is never -0, so adding either zero leaves it
// unchanged.  One workgroup scores QP_PAGES pages of one KV head for a chunk of
// up to QHEADS query heads (wave w: head w, lane l: pages l and l + 64), the
// bound rows staged in LDS as in quest_score_tile_kernel; two workgroups per
// CU (4 waves per SIMD).  The KV head is the fastest grid dimension, so the
// workgroups running together read whole page rows.  Measured at the microbench
// shape: 37.6 us per launch, against 30.3 us for the loads and LDS stores alone
// and 26.0 us for the arithmetic alone (LDS reads, VALU and SALU each near
// their rate: every wave reads the whole tile); tile-fastest or per-XCD grid
// orders, several tiles per workgroup with the next tile's loads in flight,
// and a persistent form with two heads per wave and 256-page tiles (2 waves
// per SIMD) were all slower.  Same arithmetic and order as quest_score_kernel.
constexpr int QP_PAGES = 128;                // pages per workgroup: two per lane
constexpr int QP_T = 64 * QHEADS;            // one wave per query head of the chunk
constexpr int QP_UNITS = 4;                  // 16-byte units per thread, bound and staging round
constexpr int64_t QP_MAX_ROW_BYTES = 256;    // D <= 128: 69.6 KB of LDS, one staging round per tile

__host__ __device__ constexpr int64_t qp_lds_bytes(int64_t row_bytes) { return 2 * QP_PAGES * (row_bytes + 16); }

template <bool QF32, int DK>
__global__ __launch_bounds__(QP_T, 4) void quest_score_perm_kernel(QuestArgs a) {  // 4 waves per SIMD: two workgroups per CU
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) unsigned char qp_smem[];
  const int64_t b = blockIdx.z;
  const int64_t hchunks = (a.g + QHEADS - 1) / QHEADS;
  const int64_t kv = blockIdx.x / hchunks, hc = blockIdx.x - kv * hchunks;
  const int64_t count = a.count[b];
  const int64_t p0 = static_cast<int64_t>(blockIdx.y) * QP_PAGES;
  if (a.top >= count || p0 >= count) return;
  const int64_t Hkv = a.Hkv;
  const uint32_t D = DK ? static_cast<uint32_t>(DK) : static_cast<uint32_t>(a.D);
  const uint32_t rb = D * 2u, rs = rb + 16u, upr = rb / 16u;
  unsigned char* tlo = qp_smem;
  unsigned char* thi = qp_smem + QP_PAGES * rs;
  int64_t npg = count - p0;
  if (npg > QP_PAGES) npg = QP_PAGES;
  const uint32_t units = static_cast<uint32_t>(npg) * upr;
  const char* lo_t = static_cast<const char*>(a.kmin[b]) + (p0 * Hkv + kv) * rb;
  const char* hi_t = static_cast<const char*>(a.kmax[b]) + (p0 * Hkv + kv) * rb;
  const uint32_t gstride = static_cast<uint32_t>(Hkv) * rb;  // bytes between consecutive pages
  {
    // one staging round (row_bytes <= 256: at most QP_UNITS * QP_T units): every
    // thread issues its loads before its LDS stores; a unit past the tile reloads
    // unit 0 (in bounds) and is not stored
    u32x4 L[QP_UNITS], U[QP_UNITS];
#pragma unroll
    for (int k = 0; k < QP_UNITS; ++k) {
      uint32_t u = threadIdx.x + static_cast<uint32_t>(k) * QP_T;
      if (u >= units) u = 0;
      const uint32_t r = u / upr, c = u - r * upr;
      const uint64_t off = static_cast<uint64_t>(r) * gstride + c * 16u;
      L[k] = *reinterpret_cast<const u32x4*>(lo_t + off);
      U[k] = *reinterpret_cast<const u32x4*>(hi_t + off);
    }
#pragma unroll
    for (int k = 0; k < QP_UNITS; ++k) {
      const uint32_t u = threadIdx.x + static_cast<uint32_t>(k) * QP_T;
      const uint32_t r = u / upr, c = u - r * upr;
      if (u < units) {
        *reinterpret_cast<u32x4*>(tlo + r * rs + c * 16u) = L[k];
        *reinterpret_cast<u32x4*>(thi + r * rs + c * 16u) = U[k];
      }
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar query loads
  int64_t nh = a.g - hc * QHEADS;
  if (nh > QHEADS) nh = QHEADS;
  if (wave >= nh) return;  // no barrier follows
  const int64_t h = kv * a.g + hc * QHEADS + wave;
  constexpr int QESZ = QF32 ? 4 : 2;
  constexpr int WPU = QF32 ? 8 : 4;  // query words per 16-byte unit of the bounds (8 elements)
  const uint32_t* qw = reinterpret_cast<const uint32_t*>(static_cast<const char*>(a.q) + (b * a.q_sb + h * a.q_sh) * QESZ);
  const unsigned char* l0 = tlo + lane * rs;
  const unsigned char* l1 = tlo + (lane + 64) * rs;
  const unsigned char* u0 = thi + lane * rs;
  const unsigned char* u1 = thi + (lane + 64) * rs;
  float acc0 = 0.f, acc1 = 0.f;  // pages l and l + 64
  // selector of bound element e (half e & 1 of word e >> 1): bytes 0-3 come from
  // the lower bound's word, 4-7 from the upper's, 0x0c is a zero byte
  auto selector = [](uint32_t qbits, int half) -> uint32_t {
    const bool neg = static_cast<int32_t>(qbits) < 0;
    return half ? (neg ? 0x03020c0cu : 0x07060c0cu) : (neg ? 0x01000c0cu : 0x05040c0cu);
  };
#pragma unroll 2
  for (uint32_t c = 0; c < upr; ++c) {
    const u32x4 L0 = *reinterpret_cast<const u32x4*>(l0 + c * 16u);
    const u32x4 L1 = *reinterpret_cast<const u32x4*>(l1 + c * 16u);
    const u32x4 U0 = *reinterpret_cast<const u32x4*>(u0 + c * 16u);
    const u32x4 U1 = *reinterpret_cast<const u32x4*>(u1 + c * 16u);
    uint32_t wq[WPU];
#pragma unroll
    for (int i = 0; i < WPU; ++i) wq[i] = qw[c * WPU + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t qbits = QF32 ? wq[e] : ((e & 1) ? (wq[e >> 1] & 0xffff0000u) : (wq[e >> 1] << 16));
      const float qf = __uint_as_float(qbits);
      const uint32_t sel = selector(qbits, e & 1);
      const float b0 = __uint_as_float(__builtin_amdgcn_perm(U0[e >> 1], L0[e >> 1], sel));
      const float b1 = __uint_as_float(__builtin_amdgcn_perm(U1[e >> 1], L1[e >> 1], sel));
      if constexpr (QF32) {
        const float p0v = qf * b0, p1v = qf * b1;
        acc0 = acc0 + p0v;
        acc1 = acc1 + p1v;
      } else {
        acc0 = __builtin_fmaf(qf, b0, acc0);
        acc1 = __builtin_fmaf(qf, b1, acc1);
      }
    }
  }
  float* out = a.scores + (b * a.Hq + h) * a.cmax + p0;
  if (lane < npg) out[lane] = acc0;
  if (lane + 64 < npg) out[lane + 64] = acc1;
}

__device__ __forceinline__ uint32_t score_key(float s) {
  if (s == 0.f) s = 0.f;  // -0 and +0 compare equal
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One workgroup per (query head, request): radix select of the top keys, ties
// to the lower page, pages written ascending.  When the page keys fit
// (`KEYS_IN_LDS`), they are computed once into LDS; the digit of each of the
// four 8-bit passes is found by wave 0 with a suffix scan over the histogram.
constexpr int64_t QTOPK_LDS_KEYS = 16384;

template <bool KEYS_IN_LDS, int TT>
__global__ __launch_bounds__(TT) void quest_topk_kernel(QuestArgs a) {
  extern __shared__ uint32_t s_keys[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_mask, s_need;
  __shared__ int64_t scan64[16];
  const int64_t h = blockIdx.x, b = blockIdx.y;
  const int64_t count = a.count[b];
  int32_t* out = a.pages + b * a.p_sb + h * a.top;
  if (a.top >= count) {
    for (int64_t j = threadIdx.x; j < count; j += TT) out[j] = static_cast<int32_t>(j);
    return;
  }
  const float* sc = a.scores + (b * a.Hq + h) * a.cmax;
  const bool sink = a.keep_sink && a.top > 1 && count > 1;
  auto key_from_scores = [&](int64_t p) -> uint32_t {
    if (p == count - 1 || (sink && p == 0)) return 0xffffffffu;
    return score_key(sc[p]);
  };
  if constexpr (KEYS_IN_LDS) {
    // TL scores per thread per round, every load issued before the first key is
    // stored (a load-then-store loop waits out one load latency per score)
    constexpr int TL = 8;
    for (int64_t p0 = threadIdx.x; p0 < count; p0 += static_cast<int64_t>(TT) * TL) {
      float v[TL];
#pragma unroll
      for (int u = 0; u < TL; ++u) {
        const int64_t p = p0 + static_cast<int64_t>(u) * TT;
        v[u] = sc[p < count ? p : p0];  // p0 < count: in bounds
      }
#pragma unroll
      for (int u = 0; u < TL; ++u) {
        const int64_t p = p0 + static_cast<int64_t>(u) * TT;
        if (p < count) s_keys[p] = (p == count - 1 || (sink && p == 0)) ? 0xffffffffu : score_key(v[u]);
      }
    }
  }
  auto key_of = [&](int64_t p) -> uint32_t {
    if constexpr (KEYS_IN_LDS) return s_keys[p];
    else return key_from_scores(p);
  };
  if (threadIdx.x == 0) {
    s_prefix = 0u;
    s_mask = 0u;
    s_need = static_cast<uint32_t>(a.top);
  }
  const int lane = threadIdx.x & 63;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += TT) hist[i] = 0u;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    for (int64_t p0 = threadIdx.x - lane; p0 < count; p0 += TT) {  // wave-uniform trip count
      const int64_t p = p0 + lane;
      const uint32_t k = p < count ? key_of(p) : 0u;
      const uint32_t digit = (k >> shift) & 255u;
      bool pending = p < count && (k & mask) == prefix;
      // Scores of one magnitude share their top digits, so most lanes of a wave
      // would add to one bin (an LDS atomic conflicting 64 ways).  Twice, the
      // lanes holding the first pending lane's digit add their count in one
      // atomic; the lanes left add their own.
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint64_t live = __ballot(pending);
        if (live == 0) break;
        const int leader = __ffsll(static_cast<unsigned long long>(live)) - 1;
        const uint32_t ld = __shfl(digit, leader, 64);
        const bool same = pending && digit == ld;
        const uint64_t group = __ballot(same);
        if (lane == leader) atomicAdd(&hist[ld], static_cast<uint32_t>(__popcll(group)));
        pending = pending && !same;
      }
      if (pending) atomicAdd(&hist[digit], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l owns digits 4l .. 4l+3; keys with a digit above d number
      // above(d) = (sum over lanes > l) + (own digits above d)
      const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2],
                     h3 = hist[4 * lane + 3];
      const uint32_t own = h0 + h1 + h2 + h3;
      uint32_t suffix = own;  // inclusive suffix sum over lanes >= l
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_down(suffix, off, 64);
        if (lane + off < 64) suffix += o;
      }
      const uint32_t need = s_need;
      uint32_t above = suffix - own;
      const uint32_t hv[4] = {h0, h1, h2, h3};
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (above < need && above + hv[i] >= need) {
          // exactly one (lane, digit) satisfies this
          s_need = need - above;
          s_prefix = prefix | (static_cast<uint32_t>(4 * lane + i) << shift);
          s_mask = mask | (255u << shift);
        }
        above += hv[i];
      }
    }
    __syncthreads();
  }
  const uint32_t kth = s_prefix, need_eq = s_need;
  // ordered compaction over contiguous page ranges
  const int64_t per = (count + TT - 1) / TT;
  const int64_t p0 = threadIdx.x * per;
  int64_t p1 = p0 + per;
  if (p1 > count) p1 = count;
  int64_t eq = 0;
  for (int64_t p = p0; p < p1; ++p) eq += key_of(p) == kth;
  int64_t tot;
  const int64_t eq_before = block_exclusive_sum<int64_t>(eq, scan64, &tot);
  int64_t sel = 0, e = eq_before;
  for (int64_t p = p0; p < p1; ++p) {
    const uint32_t k = key_of(p);
    if (k > kth) ++sel;
    else if (k == kth && e++ < static_cast<int64_t>(need_eq)) ++sel;
  }
  const int64_t sel_before = block_exclusive_sum<int64_t>(sel, scan64, &tot);
  int64_t o = sel_before;
  e = eq_before;
  for (int64_t p = p0; p < p1; ++p) {
    const uint32_t k = key_of(p);
    bool take = k > kth;
    if (!take && k == kth) take = e++ < static_cast<int64_t>(need_eq);
    if (take) out[o++] = static_cast<int32_t>(p);
  }
}

// Uniform page resampling (the miss-heavy stress workload's selector): per
// (layer, request) the tail page and top - 1 other pages drawn uniformly without
// replacement by Floyd's algorithm -- for j = n - k .. n - 1, t uniform in
// [0, j]; take t unless taken, else j -- over the count - 1 non-tail pages, with
// a counter-based generator (splitmix64 of seed, step, layer, request, j), so the
// draw depends on nothing but those.  Lane 0 draws into an LDS bitmap; the wave
// then writes the pages in ascending order (tail last) to every head's row, and
// -1 past min(top, count).  One wave per (layer, request).
struct UniformArgs {
  uint64_t seed, step;
  int64_t count[QMAXB];  // of requests b0 .. b0 + gridDim.y - 1
  int64_t b0, B, layers, top, heads;
  int32_t* out;  // [layers, B, heads, top]
};

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// Uniform in [0, bound) from a 64-bit draw: the high half of draw_hi32 * bound.
__host__ __device__ __forceinline__ uint32_t uniform_below(uint64_t draw, uint32_t bound) {
  return static_cast<uint32_t>(((draw >> 32) * static_cast<uint64_t>(bound)) >> 32);
}

constexpr int UNIFORM_MAX_PAGES = 1 << 16;

__global__ __launch_bounds__(64) void uniform_pages_kernel(UniformArgs a) {
  __shared__ uint32_t bits[UNIFORM_MAX_PAGES / 32];
  const int64_t layer = blockIdx.x, b = a.b0 + blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t count = a.count[blockIdx.y];
  const int64_t n = count - 1;  // non-tail pages
  const int64_t k = a.top - 1;  // of them drawn
  const int64_t words = (count + 31) / 32;
  for (int64_t w = lane; w < words; w += 64) bits[w] = 0u;
  __syncthreads();
  if (count <= a.top) {
    for (int64_t w = lane; w < words; w += 64) {
      const int64_t rest = count - 32 * w;
      bits[w] = rest >= 32 ? 0xffffffffu : ((1u << rest) - 1u);
    }
  } else if (lane == 0) {
    const uint64_t base = splitmix64(splitmix64(splitmix64(a.seed) ^ a.step) ^
                                     static_cast<uint64_t>(layer * a.B + b));
    for (int64_t j = n - k; j < n; ++j) {
      const uint32_t t = uniform_below(splitmix64(base ^ static_cast<uint64_t>(j)), static_cast<uint32_t>(j + 1));
      const bool taken = (bits[t >> 5] >> (t & 31)) & 1u;
      const uint32_t pick = taken ? static_cast<uint32_t>(j) : t;
      bits[pick >> 5] |= 1u << (pick & 31);
    }
    bits[n >> 5] |= 1u << (n & 31);  // the tail page
  }
  __syncthreads();
  // ascending write: lane l owns words l, l + 64, ...; a running base per round
  int32_t* row = a.out + (layer * a.B + b) * a.heads * a.top;
  int64_t written = 0;
  for (int64_t w0 = 0; w0 < words; w0 += 64) {
    const int64_t w = w0 + lane;
    uint32_t word = w < words ? bits[w] : 0u;
    const int c = __popc(word);
    int inc = c;  // inclusive prefix over the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(inc, off, 64);
      if (lane >= off) inc += o;
    }
    int64_t at = written + inc - c;
    while (word) {
      const int bit = __ffs(word) - 1;
      word &= word - 1;
      for (int64_t h = 0; h < a.heads; ++h) row[h * a.top + at] = static_cast<int32_t>(32 * w + bit);
      ++at;
    }
    written += __shfl(inc, 63, 64);
  }
  for (int64_t i = written + lane; i < a.top; i += 64)
    for (int64_t h = 0; h < a.heads; ++h) row[h * a.top + i] = -1;
}

struct UnionArgs {
  const int32_t* pages;  // [B, Hq, top], first min(top, count) ascending
  int64_t p_sb, top;
  int64_t length[QMAXB];
  int64_t P, Hq, Hkv, g;
  int32_t* positions;    // [B, cap]
  int64_t pos_cap;
  int64_t* head_columns; // [B, Hq, width]
  int64_t width;
  int32_t* union_count;  // [B]
  int32_t* ecol;         // [B, Hkv, ecap]
  uint32_t* emask;
  int64_t ecap;
  int32_t* ecount;       // [B, Hkv]
  unsigned long long* estats;  // nullable: the clamped entry counts are added here
  int32_t* status;       // nonzero on overflow
  uint32_t* page_bits;   // nullable [B, pb_stride]: the union's page bitmap
  int64_t pb_stride;
  int64_t words;         // bitmap words of the longest history
  int64_t maxcount;      // pages of the longest history
  int use_map;           // rank -> page map in LDS (maxcount <= UMAPPAGES)
};

__device__ __forceinline__ bool head_has_page(const int32_t* row, int64_t k, int32_t p) {
  int64_t lo = 0, hi = k;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (row[mid] < p) lo = mid + 1;
    else hi = mid;
  }
  return lo < k && row[lo] == p;
}

// Workgroup roles per request (blockIdx.y): blockIdx.x < Hkv builds the group
// entries of that KV head; == Hkv the union positions and size; Hkv + 1 + h
// the union columns of query head h.  Every role rebuilds the selected-page
// bitmap and its word prefix popcounts in LDS (a few hundred bits), so the
// roles run side by side.  A group entry's head mask comes from an LDS array
// indexed by the page's rank among the group's pages.
constexpr int64_t UMAXMASK = 4096;  // group pages (g * top) with an LDS mask slot
constexpr int64_t UMAPPAGES = 24576;  // longest history (pages) with an LDS rank -> page map

// Dynamic LDS: four bitmaps of `a.words` words and a rank -> page map of
// `a.maxcount` entries (longest history of the batch).  The positions and the
// entry lists are written one output element per thread through that map, so
// consecutive lanes store consecutive elements.
__global__ __launch_bounds__(UT) void build_union_kernel(UnionArgs a) {
  extern __shared__ uint32_t union_lds[];
  uint32_t* ubits = union_lds;
  uint32_t* uprefix = ubits + a.words;
  uint32_t* gbits = uprefix + a.words;
  uint32_t* gprefix = gbits + a.words;
  int32_t* rank_page = reinterpret_cast<int32_t*>(gprefix + a.words);  // [maxcount]
  __shared__ uint32_t gmask[UMAXMASK];
  __shared__ int32_t scan32[16];
  const int64_t b = blockIdx.y;
  const int64_t part = blockIdx.x;
  const int64_t L = a.length[b], P = a.P;
  const int64_t count = (L + P - 1) / P;
  const int64_t k = a.top < count ? a.top : count;
  const int64_t tail_len = L - (count - 1) * P;
  const int64_t words = (count + 31) / 32;
  const int32_t* pg = a.pages + b * a.p_sb;
  const bool group = part < a.Hkv;
  const bool masks_in_lds = a.g * k <= UMAXMASK;

  for (int64_t i = threadIdx.x; i < words; i += UT) {
    ubits[i] = 0u;
    gbits[i] = 0u;
  }
  if (group && masks_in_lds)
    for (int64_t i = threadIdx.x; i < a.g * k; i += UT) gmask[i] = 0u;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < a.Hq * k; i += UT) {
    const int64_t h = i / k, j = i - h * k;
    const int32_t p = pg[h * a.top + j];
    if (p < 0 || p >= count) continue;
    atomicOr(&ubits[p >> 5], 1u << (p & 31));
    if (group && h / a.g == part) atomicOr(&gbits[p >> 5], 1u << (p & 31));
  }
  __syncthreads();
  // word prefix popcounts (serial per thread chunk, then block scan)
  {
    const int64_t per = (words + UT - 1) / UT;
    const int64_t w0 = threadIdx.x * per;
    int64_t w1 = w0 + per;
    if (w1 > words) w1 = words;
    int32_t cu = 0, cg = 0;
    for (int64_t w = w0; w < w1; ++w) {
      cu += __popc(ubits[w]);
      cg += __popc(gbits[w]);
    }
    int32_t tu, tg;
    int32_t bu = block_exclusive_sum<int32_t>(cu, scan32, &tu);
    int32_t bg = block_exclusive_sum<int32_t>(cg, scan32, &tg);
    for (int64_t w = w0; w < w1; ++w) {
      uprefix[w] = bu;
      gprefix[w] = bg;
      bu += __popc(ubits[w]);
      bg += __popc(gbits[w]);
    }
  }
  __syncthreads();
  auto rank_of = [&](const uint32_t* bits, const uint32_t* pre, int64_t p) -> int64_t {
    const uint32_t below = (p & 31) ? (bits[p >> 5] & ((1u << (p & 31)) - 1u)) : 0u;
    return static_cast<int64_t>(pre[p >> 5]) + __popc(below);
  };

  if (part == a.Hkv) {
    const int64_t upages = rank_of(ubits, uprefix, count - 1) + 1;  // the tail page is always selected
    const int64_t n = upages * P - (P - tail_len);
    if (threadIdx.x == 0) {
      a.union_count[b] = static_cast<int32_t>(n);
      if (n > a.pos_cap) atomicOr(a.status, 1);
    }
    int32_t* pos = a.positions + b * a.pos_cap;
    const int64_t nw = n < a.pos_cap ? n : a.pos_cap;
    if (a.use_map) {
      for (int64_t p = threadIdx.x; p < count; p += UT)
        if ((ubits[p >> 5] >> (p & 31)) & 1u) rank_page[rank_of(ubits, uprefix, p)] = static_cast<int32_t>(p);
      __syncthreads();
      // position i: token i % P of the (i / P)-th union page (the tail page is the last)
      for (int64_t i = threadIdx.x; i < nw; i += UT)
        pos[i] = static_cast<int32_t>(static_cast<int64_t>(rank_page[i / P]) * P + i % P);
    } else {
      for (int64_t p = threadIdx.x; p < count; p += UT) {
        if (!((ubits[p >> 5] >> (p & 31)) & 1u)) continue;
        const int64_t base = rank_of(ubits, uprefix, p) * P;
        const int64_t plen = p == count - 1 ? tail_len : P;
        for (int64_t off = 0; off < plen; ++off)
          if (base + off < a.pos_cap) pos[base + off] = static_cast<int32_t>(p * P + off);
      }
    }
    for (int64_t i = nw + threadIdx.x; i < a.pos_cap; i += UT) pos[i] = -1;
    if (a.page_bits)
      for (int64_t w = threadIdx.x; w < words; w += UT) a.page_bits[b * a.pb_stride + w] = ubits[w];
  } else if (part > a.Hkv) {
    // union columns of head h: its j-th token (its pages ascending, tail last)
    const int64_t h = part - a.Hkv - 1;
    const int64_t W = (k - 1) * P + tail_len;
    int64_t* hc = a.head_columns + (b * a.Hq + h) * a.width;
    for (int64_t jj = threadIdx.x; jj < a.width; jj += UT) {
      int64_t col = -1;
      if (jj < W) {
        int64_t p, off;
        if (jj < (k - 1) * P) {
          p = pg[h * a.top + jj / P];
          off = jj % P;
        } else {
          p = count - 1;
          off = jj - (k - 1) * P;
        }
        col = rank_of(ubits, uprefix, p) * P + off;
      }
      hc[jj] = col;
    }
  } else {
    const int64_t kv = part;
    const int64_t gpages = rank_of(gbits, gprefix, count - 1) + 1;
    const int64_t E = gpages * P - (P - tail_len);
    if (threadIdx.x == 0) {
      a.ecount[b * a.Hkv + kv] = static_cast<int32_t>(E < a.ecap ? E : a.ecap);
      if (E > a.ecap) atomicOr(a.status, 2);
      if (a.estats) atomicAdd(a.estats, static_cast<unsigned long long>(E < a.ecap ? E : a.ecap));
    }
    if (masks_in_lds) {
      // head bits of each group page, indexed by the page's rank in the group
      for (int64_t i = threadIdx.x; i < a.g * k; i += UT) {
        const int64_t hl = i / k, j = i - hl * k;
        const int32_t p = pg[(kv * a.g + hl) * a.top + j];
        if (p < 0 || p >= count) continue;
        atomicOr(&gmask[rank_of(gbits, gprefix, p)], 1u << hl);
      }
      __syncthreads();
    }
    int32_t* ec = a.ecol + (b * a.Hkv + kv) * a.ecap;
    uint32_t* em = a.emask + (b * a.Hkv + kv) * a.ecap;
    if (masks_in_lds && a.use_map) {
      for (int64_t p = threadIdx.x; p < count; p += UT)
        if ((gbits[p >> 5] >> (p & 31)) & 1u) rank_page[rank_of(gbits, gprefix, p)] = static_cast<int32_t>(p);
      __syncthreads();
      // entry i: token i % P of the (i / P)-th group page, its union column and head mask
      const int64_t ew = E < a.ecap ? E : a.ecap;
      for (int64_t i = threadIdx.x; i < ew; i += UT) {
        const int64_t r = i / P;
        const int32_t p = rank_page[r];
        ec[i] = static_cast<int32_t>(rank_of(ubits, uprefix, p) * P + i % P);
        em[i] = gmask[r];
      }
      return;
    }
    for (int64_t p = threadIdx.x; p < count; p += UT) {
      if (!((gbits[p >> 5] >> (p & 31)) & 1u)) continue;
      const int64_t grank = rank_of(gbits, gprefix, p);
      uint32_t mask = 0u;
      if (masks_in_lds) {
        mask = gmask[grank];
      } else {
        for (int64_t hl = 0; hl < a.g; ++hl)
          if (head_has_page(pg + (kv * a.g + hl) * a.top, k, static_cast<int32_t>(p))) mask |= 1u << hl;
      }
      const int64_t gbase = grank * P;
      const int64_t ubase = rank_of(ubits, uprefix, p) * P;
      const int64_t plen = p == count - 1 ? tail_len : P;
      for (int64_t off = 0; off < plen; ++off) {
        if (gbase + off < a.ecap) {
          ec[gbase + off] = static_cast<int32_t>(ubase + off);
          em[gbase + off] = mask;
        }
      }
    }
  }
}

static int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

}  // namespace hs

using namespace hs;

extern "C" int64_t hs_quest_workspace_bytes(int64_t batch, int64_t heads, int64_t max_pages) {
  if (batch < 1 || heads < 1 || max_pages < 1) return 256;
  return ((batch * heads * max_pages * 4) + 255) & ~static_cast<int64_t>(255);
}

// At most QMAXB requests (their bounds pointers and page counts travel in the
// kernel arguments); hs_quest_topk cuts larger batches into such chunks.
static int quest_topk_chunk(const void* query, int64_t q_stride_b, int64_t q_stride_h,
                            int32_t query_dtype, const void* const* minimum,
                            const void* const* maximum, int32_t kv_dtype,
                            const int64_t* page_counts, int64_t batch, int64_t heads,
                            int64_t kv_heads, int64_t head_dim, int64_t top, int32_t keep_sink,
                            int32_t* out_pages, int64_t out_stride_b, void* workspace,
                            int64_t workspace_bytes, hipStream_t stream) {
  HS_CHECK_ARG(top >= 1 && heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0,
               "invalid page budget or GQA shape");
  HS_CHECK_ARG(batch >= 1 && batch <= QMAXB, "quest batch must be in [1, %d]", QMAXB);
  HS_CHECK_ARG(valid_dtype(kv_dtype), "invalid dtype code %d", kv_dtype);
  HS_CHECK_ARG(valid_dtype(query_dtype), "invalid query dtype code %d", query_dtype);
  HS_CHECK_ARG(head_dim >= 1 && head_dim <= 1024, "invalid head_dim");
  HS_CHECK_ARG(query && minimum && maximum && page_counts && out_pages, "null quest pointer");
  QuestArgs a{};
  a.q = query;
  a.q_dtype = query_dtype;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  int64_t cmax = 1;
  for (int64_t i = 0; i < batch; ++i) {
    HS_CHECK_ARG(page_counts[i] >= 1, "cannot select pages of an empty history");
    HS_CHECK_ARG(minimum[i] && maximum[i], "null bounds pointer");
    a.kmin[i] = minimum[i];
    a.kmax[i] = maximum[i];
    a.count[i] = page_counts[i];
    if (page_counts[i] > cmax) cmax = page_counts[i];
  }
  a.Hq = heads;
  a.Hkv = kv_heads;
  a.g = heads / kv_heads;
  a.D = head_dim;
  a.top = top;
  a.keep_sink = keep_sink;
  a.cmax = cmax;
  a.pages = out_pages;
  a.p_sb = out_stride_b;
  const int64_t need = hs_quest_workspace_bytes(batch, heads, cmax);
  HS_CHECK_ARG(workspace && workspace_bytes >= need, "quest workspace too small: need %lld bytes",
               static_cast<long long>(need));
  a.scores = static_cast<float*>(workspace);
  bool any_scored = false;
  for (int64_t i = 0; i < batch; ++i) any_scored |= top < page_counts[i];
  if (any_scored) {
    const int64_t hchunks = ceil_div(a.g, QHEADS);
    // 16-bit queries times 16-bit bounds: every product is exact in fp32, so an FMA
    // rounds like the reference's product-then-sum
    const bool fused = query_dtype != HS_DTYPE_F32 && kv_dtype != HS_DTYPE_F32;
    const int64_t epv = kv_dtype == HS_DTYPE_F32 ? 4 : 8;
    const int64_t row_bytes = head_dim * (kv_dtype == HS_DTYPE_F32 ? 4 : 2);
    bool aligned = true;
    for (int64_t i = 0; i < batch; ++i)
      aligned &= ((reinterpret_cast<uintptr_t>(minimum[i]) | reinterpret_cast<uintptr_t>(maximum[i])) & 15) == 0;
    // HS_QUEST_SCORER=tile keeps bf16 bounds on quest_score_tile_kernel (for comparisons)
    static const bool perm_off = [] {
      const char* env = getenv("HS_QUEST_SCORER");
      return env && strcmp(env, "tile") == 0;
    }();
    const bool query_words = (reinterpret_cast<uintptr_t>(query) & 3) == 0 &&
                             (query_dtype == HS_DTYPE_F32 || (q_stride_b % 2 == 0 && q_stride_h % 2 == 0));
    if (!perm_off && kv_dtype == HS_DTYPE_BF16 && (query_dtype == HS_DTYPE_BF16 || query_dtype == HS_DTYPE_F32) &&
        query_words && head_dim % 8 == 0 && aligned && row_bytes <= QP_MAX_ROW_BYTES) {
      dim3 grid(static_cast<unsigned>(kv_heads * hchunks), static_cast<unsigned>(ceil_div(cmax, QP_PAGES)),
                static_cast<unsigned>(batch));
      const size_t lds = static_cast<size_t>(qp_lds_bytes(row_bytes));
      const bool f32q = query_dtype == HS_DTYPE_F32;
      if (head_dim == 128) {
        if (f32q) hipLaunchKernelGGL((quest_score_perm_kernel<true, 128>), grid, dim3(QP_T), lds, stream, a);
        else hipLaunchKernelGGL((quest_score_perm_kernel<false, 128>), grid, dim3(QP_T), lds, stream, a);
      } else if (head_dim == 64) {
        if (f32q) hipLaunchKernelGGL((quest_score_perm_kernel<true, 64>), grid, dim3(QP_T), lds, stream, a);
        else hipLaunchKernelGGL((quest_score_perm_kernel<false, 64>), grid, dim3(QP_T), lds, stream, a);
      } else {
        if (f32q) hipLaunchKernelGGL((quest_score_perm_kernel<true, 0>), grid, dim3(QP_T), lds, stream, a);
        else hipLaunchKernelGGL((quest_score_perm_kernel<false, 0>), grid, dim3(QP_T), lds, stream, a);
      }
      HS_CHECK_LAUNCH("quest scorer");
    } else if (head_dim % epv == 0 && aligned && row_bytes <= QS_MAX_ROW_BYTES) {
      dim3 grid(static_cast<unsigned>(ceil_div(cmax, QS_PAGES)), static_cast<unsigned>(kv_heads * hchunks),
                static_cast<unsigned>(batch));
      const size_t lds = static_cast<size_t>(qs_lds_bytes(row_bytes, head_dim));
      if (kv_dtype == HS_DTYPE_BF16) {
        if (fused) hipLaunchKernelGGL((quest_score_tile_kernel<HS_DTYPE_BF16, true>), grid, dim3(QT), lds, stream, a);
        else hipLaunchKernelGGL((quest_score_tile_kernel<HS_DTYPE_BF16, false>), grid, dim3(QT), lds, stream, a);
      } else if (kv_dtype == HS_DTYPE_F16) {
        if (fused) hipLaunchKernelGGL((quest_score_tile_kernel<HS_DTYPE_F16, true>), grid, dim3(QT), lds, stream, a);
        else hipLaunchKernelGGL((quest_score_tile_kernel<HS_DTYPE_F16, false>), grid, dim3(QT), lds, stream, a);
      } else {
        hipLaunchKernelGGL((quest_score_tile_kernel<HS_DTYPE_F32, false>), grid, dim3(QT), lds, stream, a);
      }
      HS_CHECK_LAUNCH("quest scorer");
    } else {
    dim3 grid(static_cast<unsigned>(ceil_div(cmax, QT)), static_cast<unsigned>(kv_heads * hchunks),
              static_cast<unsigned>(batch));
    const size_t lds = static_cast<size_t>(QHEADS * head_dim * 4);
    if (kv_dtype == HS_DTYPE_BF16) {
      if (fused) hipLaunchKernelGGL((quest_score_kernel<HS_DTYPE_BF16, true>), grid, dim3(QT), lds, stream, a);
      else hipLaunchKernelGGL((quest_score_kernel<HS_DTYPE_BF16, false>), grid, dim3(QT), lds, stream, a);
    } else if (kv_dtype == HS_DTYPE_F16) {
      if (fused) hipLaunchKernelGGL((quest_score_kernel<HS_DTYPE_F16, true>), grid, dim3(QT), lds, stream, a);
      else hipLaunchKernelGGL((quest_score_kernel<HS_DTYPE_F16, false>), grid, dim3(QT), lds, stream, a);
    } else {
      hipLaunchKernelGGL((quest_score_kernel<HS_DTYPE_F32, false>), grid, dim3(QT), lds, stream, a);
    }
    HS_CHECK_LAUNCH("quest scorer");
    }
  }
  const dim3 tgrid(static_cast<unsigned>(heads), static_cast<unsigned>(batch));
  // 1024 threads per (request, head): measured 22 us against 28 us with 256 at the
  // microbench shape (4096 pages); HS_TOPK_THREADS=256/512 overrides
  static const int topk_threads = [] {
    const char* env = getenv("HS_TOPK_THREADS");
    const int v = env ? atoi(env) : 0;
    return v == 256 || v == 512 ? v : 1024;
  }();
  const size_t klds = cmax <= QTOPK_LDS_KEYS ? static_cast<size_t>(cmax * 4) : 0;
  if (cmax <= QTOPK_LDS_KEYS) {
    if (topk_threads == 256) hipLaunchKernelGGL((quest_topk_kernel<true, 256>), tgrid, dim3(256), klds, stream, a);
    else if (topk_threads == 512) hipLaunchKernelGGL((quest_topk_kernel<true, 512>), tgrid, dim3(512), klds, stream, a);
    else hipLaunchKernelGGL((quest_topk_kernel<true, 1024>), tgrid, dim3(1024), klds, stream, a);
  } else {
    if (topk_threads == 256) hipLaunchKernelGGL((quest_topk_kernel<false, 256>), tgrid, dim3(256), 0, stream, a);
    else if (topk_threads == 512) hipLaunchKernelGGL((quest_topk_kernel<false, 512>), tgrid, dim3(512), 0, stream, a);
    else hipLaunchKernelGGL((quest_topk_kernel<false, 1024>), tgrid, dim3(1024), 0, stream, a);
  }
  HS_CHECK_LAUNCH("quest top-k");
  return HS_OK;
}

// At most QMAXB requests (their lengths travel in the kernel arguments);
// hs_build_union cuts larger batches into such chunks.
static int build_union_chunk(const int32_t* pages, int64_t p_stride_b, int64_t top,
                             const int64_t* lengths, int64_t page_size, int64_t batch,
                             int64_t heads, int64_t kv_heads, int32_t* positions,
                             int64_t pos_capacity, int64_t* head_columns, int64_t width,
                             int32_t* union_count, int32_t* entry_columns,
                             uint32_t* entry_masks, int64_t entry_capacity,
                             int32_t* entry_counts, int32_t* status, uint32_t* page_bits,
                             int64_t pb_stride, int64_t* entry_stats, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1 && batch <= QMAXB, "union batch must be in [1, %d]", QMAXB);
  HS_CHECK_ARG(top >= 1 && page_size >= 1 && heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0,
               "invalid union shape");
  HS_CHECK_ARG(heads / kv_heads <= 32, "at most 32 query heads per KV head");
  HS_CHECK_ARG(pages && lengths && positions && head_columns && union_count && entry_columns &&
                   entry_masks && entry_counts && status,
               "null union pointer");
  HS_CHECK_ARG(pos_capacity >= 1 && entry_capacity >= 1 && width >= 1, "union capacities must be positive");
  UnionArgs a{};
  a.pages = pages;
  a.p_sb = p_stride_b;
  a.top = top;
  for (int64_t i = 0; i < batch; ++i) {
    HS_CHECK_ARG(lengths[i] >= 1, "cannot build a union over an empty history");
    HS_CHECK_ARG(ceil_div(lengths[i], page_size) <= UMAXPAGES, "too many pages for the union builder");
    const int64_t count = ceil_div(lengths[i], page_size);
    const int64_t k = top < count ? top : count;
    const int64_t W = (k - 1) * page_size + (lengths[i] - (count - 1) * page_size);
    HS_CHECK_ARG(W <= width, "head column width %lld below the selection width %lld",
                 static_cast<long long>(width), static_cast<long long>(W));
    a.length[i] = lengths[i];
  }
  a.P = page_size;
  a.Hq = heads;
  a.Hkv = kv_heads;
  a.g = heads / kv_heads;
  a.positions = positions;
  a.pos_cap = pos_capacity;
  a.page_bits = page_bits;
  a.pb_stride = pb_stride;
  a.head_columns = head_columns;
  a.width = width;
  a.union_count = union_count;
  a.ecol = entry_columns;
  a.emask = entry_masks;
  a.ecap = entry_capacity;
  a.ecount = entry_counts;
  a.estats = reinterpret_cast<unsigned long long*>(entry_stats);
  a.status = status;
  int64_t max_count = 1;
  for (int64_t i = 0; i < batch; ++i) max_count = std::max(max_count, ceil_div(lengths[i], page_size));
  a.words = (max_count + 31) / 32;
  a.maxcount = max_count;
  a.use_map = max_count <= UMAPPAGES;
  const size_t lds = static_cast<size_t>((4 * a.words + (a.use_map ? max_count : 0)) * 4);
  static bool lds_attr = false;
  if (!lds_attr) {  // up to 4 * 768 + 24576 words of dynamic LDS
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(build_union_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
    (void)hipGetLastError();
    lds_attr = true;
  }
  hipLaunchKernelGGL(build_union_kernel, dim3(static_cast<unsigned>(kv_heads + 1 + heads), static_cast<unsigned>(batch)),
                     dim3(UT), lds, stream, a);
  HS_CHECK_LAUNCH("union builder");
  return HS_OK;
}

extern "C" int hs_quest_topk(const void* query, int64_t q_stride_b, int64_t q_stride_h,
                             int32_t query_dtype, const void* const* minimum,
                             const void* const* maximum, int32_t kv_dtype,
                             const int64_t* page_counts, int64_t batch, int64_t heads,
                             int64_t kv_heads, int64_t head_dim, int64_t top, int32_t keep_sink,
                             int32_t* out_pages, int64_t out_stride_b, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1, "quest batch must be positive");
  HS_CHECK_ARG(valid_dtype(query_dtype), "invalid query dtype code %d", query_dtype);
  HS_CHECK_ARG(valid_dtype(kv_dtype), "invalid dtype code %d", kv_dtype);
  HS_CHECK_ARG(top >= 1 && heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0,
               "invalid page budget or GQA shape");
  HS_CHECK_ARG(head_dim >= 1 && head_dim <= 1024, "invalid head_dim");
  HS_CHECK_ARG(query && minimum && maximum && page_counts && out_pages, "null quest pointer");
  // every request and every chunk's workspace need are checked before the first
  // launch, so an invalid call launches nothing
  for (int64_t i = 0; i < batch; ++i) {
    HS_CHECK_ARG(page_counts[i] >= 1, "cannot select pages of an empty history");
    HS_CHECK_ARG(minimum[i] && maximum[i], "null bounds pointer");
  }
  for (int64_t s0 = 0; s0 < batch; s0 += QMAXB) {
    const int64_t n = batch - s0 < QMAXB ? batch - s0 : QMAXB;
    int64_t cmax = 1;
    for (int64_t i = s0; i < s0 + n; ++i) cmax = page_counts[i] > cmax ? page_counts[i] : cmax;
    const int64_t need = hs_quest_workspace_bytes(n, heads, cmax);
    HS_CHECK_ARG(workspace && workspace_bytes >= need, "quest workspace too small: need %lld bytes",
                 static_cast<long long>(need));
  }
  const int64_t qbytes = query_dtype == HS_DTYPE_F32 ? 4 : 2;
  // chunks run in stream order and each reuses the workspace, which holds the
  // scores of at most the whole batch
  for (int64_t s0 = 0; s0 < batch; s0 += QMAXB) {
    const int64_t n = batch - s0 < QMAXB ? batch - s0 : QMAXB;
    const int rc = quest_topk_chunk(static_cast<const char*>(query) + s0 * q_stride_b * qbytes, q_stride_b,
                                    q_stride_h, query_dtype, minimum + s0, maximum + s0, kv_dtype,
                                    page_counts + s0, n, heads, kv_heads, head_dim, top, keep_sink,
                                    out_pages + s0 * out_stride_b, out_stride_b, workspace, workspace_bytes,
                                    stream);
    if (rc != HS_OK) return rc;
  }
  return HS_OK;
}

extern "C" int hs_build_union(const int32_t* pages, int64_t p_stride_b, int64_t top,
                              const int64_t* lengths, int64_t page_size, int64_t batch,
                              int64_t heads, int64_t kv_heads, int32_t* positions,
                              int64_t pos_capacity, int64_t* head_columns, int64_t width,
                              int32_t* union_count, int32_t* entry_columns,
                              uint32_t* entry_masks, int64_t entry_capacity,
                              int32_t* entry_counts, int32_t* status, uint32_t* page_bits,
                              int64_t page_bits_stride, int64_t* entry_stats, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1, "union batch must be positive");
  HS_CHECK_ARG(top >= 1 && page_size >= 1 && lengths, "invalid union shape");
  HS_CHECK_ARG(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "invalid GQA shape");
  for (int64_t i = 0; i < batch; ++i) {  // every request, before the first launch
    HS_CHECK_ARG(lengths[i] >= 1, "cannot build a union over an empty history");
    HS_CHECK_ARG(ceil_div(lengths[i], page_size) <= UMAXPAGES, "too many pages for the union builder");
    const int64_t count = ceil_div(lengths[i], page_size);
    const int64_t k = top < count ? top : count;
    const int64_t W = (k - 1) * page_size + (lengths[i] - (count - 1) * page_size);
    HS_CHECK_ARG(W <= width, "head column width %lld below the selection width %lld",
                 static_cast<long long>(width), static_cast<long long>(W));
    HS_CHECK_ARG(!page_bits || page_bits_stride >= ceil_div(count, 32),
                 "page bitmap stride %lld below the %lld words of a history",
                 static_cast<long long>(page_bits_stride), static_cast<long long>(ceil_div(count, 32)));
  }
  for (int64_t s0 = 0; s0 < batch; s0 += QMAXB) {
    const int64_t n = batch - s0 < QMAXB ? batch - s0 : QMAXB;
    const int rc = build_union_chunk(
        pages + s0 * p_stride_b, p_stride_b, top, lengths + s0, page_size, n, heads, kv_heads,
        positions + s0 * pos_capacity, pos_capacity, head_columns + s0 * heads * width, width, union_count + s0,
        entry_columns + s0 * kv_heads * entry_capacity, entry_masks + s0 * kv_heads * entry_capacity,
        entry_capacity, entry_counts + s0 * kv_heads, status,
        page_bits ? page_bits + s0 * page_bits_stride : nullptr, page_bits_stride, entry_stats, stream);
    if (rc != HS_OK) return rc;
  }
  return HS_OK;
}

extern "C" int hs_uniform_pages(uint64_t seed, uint64_t step, const int64_t* page_counts, int64_t batch,
                                int64_t layers, int64_t top, int64_t heads, int32_t* out, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1 && layers >= 1 && layers <= 65535 && heads >= 1 && top >= 1,
               "invalid uniform pages shape");
  HS_CHECK_ARG(page_counts && out, "null uniform pages pointer");
  for (int64_t i = 0; i < batch; ++i)
    HS_CHECK_ARG(page_counts[i] >= 1 && page_counts[i] <= UNIFORM_MAX_PAGES, "page counts must be 1 to %d",
                 UNIFORM_MAX_PAGES);
  for (int64_t b0 = 0; b0 < batch; b0 += QMAXB) {  // launches of at most 16 requests, in order
    const int64_t nb = batch - b0 < QMAXB ? batch - b0 : QMAXB;
    UniformArgs a{};
    a.seed = seed;
    a.step = step;
    for (int64_t i = 0; i < nb; ++i) a.count[i] = page_counts[b0 + i];
    a.b0 = b0;
    a.B = batch;
    a.layers = layers;
    a.top = top;
    a.heads = heads;
    a.out = out;
    hipLaunchKernelGGL(uniform_pages_kernel, dim3(static_cast<unsigned>(layers), static_cast<unsigned>(nb)),
                       dim3(64), 0, stream, a);
    HS_CHECK_LAUNCH("uniform pages");
  }
  return HS_OK;
}
