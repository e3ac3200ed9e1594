// Decode projections for gfx950: y[M, N] = x[M, K] . W[N, K]^T (+ bias) with M <= 16.
//
// In a decode step every projection of the batched engine multiplies a few
// token rows by a large weight, so the weight read is the whole cost: the
// kernel is an HBM stream of W.  Tiles are v_mfma_f32_16x16x32_{bf16,f16} with
// 16 weight rows as the MFMA's M dimension and the (padded) token rows as its
// N dimension, so the MFMA's output tile is 16 weight rows x 16 tokens.
//
// A workgroup (4 waves) owns 16 or 32 weight rows and one K slice; wave w
// takes k-steps (of 32) in groups of GU consecutive steps, round-robin over
// the waves, so within a round the four waves read GU * 4 * 64 contiguous
// bytes of every row.  Per round a lane issues all of its loads (4 * GU
// weight fragments, GU token fragments) before the first MFMA.  The waves'
// partial tiles are summed in LDS.  With one K slice the workgroup adds the
// bias and writes y; with several (split-K, for tall-K shapes that would
// otherwise give too few workgroups) it writes partials and
// the last workgroup of each row tile to arrive sums them in slice order
// (deterministic), adds the bias and rounds: tagged partial words and an arrival
// counter per tile (arrive.h), so the launch needs no second kernel
// (HS_GEMM_FUSED_MERGE=0: fp32 partials summed the same way by
// gemm_finalize_kernel, a second launch).  The argmax form (the LM head of a greedy step) keeps, per
// workgroup and token, only the best rounded logit and its index as one ordered
// 64-bit key, and argmax_finalize_kernel takes the largest key per token.
#include <math.h>
#include <stdlib.h>

#include "arrive.h"
#include "hs_common.h"

namespace hs {

constexpr int GM_T = 256;  // threads per workgroup

template <int DT>
__device__ __forceinline__ f32x4 gemm_mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == HS_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
}

struct GemmArgs {
  const unsigned short* x;
  int64_t x_stride;
  const unsigned short* w;
  int64_t K, N, M;
  const unsigned short* bias;  // nullable
  void* out;
  int64_t out_stride;
  float* part;  // [splits, M, N] when splits > 1
  int64_t splits, slice_steps;
  int64_t F;  // SWIGLU: output features (N = 2 * 16 * ceil(F / 16) interleaved weight rows)
  unsigned long long* keys;  // ARGMAX: [M, gridDim.x] best key per token and workgroup
  // split-K merged in-kernel (epoch != 0): tagged partial words [splits, M, N] and one
  // arrival counter per row tile
  unsigned long long* words;
  unsigned long long* counters;
  unsigned long long epoch;
};

// Ordered key of logit v at vocabulary index n: a larger key is a larger value, or
// the same value at a smaller index, so the largest key is torch.argmax's answer
// (the first maximal index).  -0 counts as +0 (they compare equal); a NaN sits
// above every number (torch's argmax returns the first NaN).  Every key is above
// 0, the key of "no row".
__device__ __forceinline__ unsigned long long argmax_key(float v, int64_t n) {
  const uint32_t u = v == 0.f ? 0u : __float_as_uint(v);
  uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (v != v) ord = 0xffffffffu;
  return (static_cast<unsigned long long>(ord) << 32) | (0xffffffffu - static_cast<uint32_t>(n));
}

template <int DT>
__device__ __forceinline__ float gemm_round(float v) {
  if constexpr (DT == HS_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else return f16_bits_to_f32(f32_to_f16_bits(v));
}

// GM_TILES row tiles of 16 per workgroup, shared by the 4 waves, which split
// the slice's k-steps in rounds of GU.  (Measured on MI355X: splitting rows
// over the waves instead, or double-buffering the rounds in registers, is
// slower at every decode shape of the Qwen2.5 0.5B/7B/32B projections.)
// TILED: W is stored tile-major, [ceil(N/16)][K/32][16][32] (each 16-row x 32-k
// block of MFMA A fragments contiguous, rows past N zero-padded), so one wave's
// load of a block reads 1 KB of consecutive bytes instead of 16 rows x 64 bytes
// a row stride apart.
// SWIGLU (with TILED and two tiles per workgroup): the weight interleaves the
// gate and up projections tile by tile (tile 2i = gate rows 16i.., 2i+1 = up rows
// 16i..), and the workgroup writes silu(gate) * up for its 16 features with the
// arithmetic of the separate path: each projection rounded to the dtype, then
// SiLU rounded, then the product (hs_silu_mul).
// ARGMAX (one K slice): per token the workgroup's best key over its rows, each
// logit rounded to the dtype after the bias as the plain form stores it.
template <int DT, int GM_TILES, int GU, bool TILED, bool SWIGLU = false, bool ARGMAX = false>
__global__ __launch_bounds__(GM_T) void skinny_gemm_kernel(GemmArgs a) {
  constexpr int GM_ROWS = 16 * GM_TILES;  // weight rows per workgroup
  __shared__ float red[4][GM_ROWS][17];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, j = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * GM_ROWS;
  const int64_t split = blockIdx.y;
  const int64_t steps = a.K / 32;
  const int64_t s0 = split * a.slice_steps;
  int64_t s1 = s0 + a.slice_steps;
  if (s1 > steps) s1 = steps;
  // lane (c, j): weight rows n0 + 16t + c, token row c, k offset 8j within a step
  const unsigned short* wrow[GM_TILES];
#pragma unroll
  for (int t = 0; t < GM_TILES; ++t) {
    if constexpr (TILED) {
      const int64_t tiles = (a.N + 15) / 16;
      int64_t nt = n0 / 16 + t;
      if (nt >= tiles) nt = tiles - 1;  // tiles past N read the last one; their outputs are dropped
      wrow[t] = a.w + nt * steps * 512 + c * 32 + 8 * j;
    } else {
      int64_t n = n0 + 16 * t + c;
      if (n >= a.N) n = a.N - 1;  // rows past N read the last row; their outputs are dropped
      wrow[t] = a.w + n * a.K + 8 * j;
    }
  }
  const unsigned short* xrow = a.x + (c < a.M ? c : a.M - 1) * a.x_stride + 8 * j;
  // the tile's arrival counter, read with the first loads: its round tags the partials
  const unsigned long long c0 = (a.splits > 1 && a.epoch != 0)
                                    ? __hip_atomic_load(a.counters + blockIdx.x, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0ull;
  f32x4 acc[GM_TILES];
#pragma unroll
  for (int t = 0; t < GM_TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t base = s0 + static_cast<int64_t>(wave) * GU; base < s1; base += 4 * GU) {
    // every load of the round before the first MFMA; steps past the slice
    // reload its last step (in bounds) and are skipped
    u32x4 wf[GU][GM_TILES], xf[GU];
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      int64_t s = base + u;
      if (s >= s1) s = s1 - 1;
      const int64_t k = 32 * s;                   // x is row-major
      const int64_t wk = TILED ? 512 * s : k;      // a 16 x 32 block per k-step when tiled
#pragma unroll
      for (int t = 0; t < GM_TILES; ++t) wf[u][t] = *reinterpret_cast<const u32x4*>(wrow[t] + wk);
      xf[u] = *reinterpret_cast<const u32x4*>(xrow + k);
    }
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      if (base + u < s1) {  // uniform per wave
#pragma unroll
        for (int t = 0; t < GM_TILES; ++t) acc[t] = gemm_mfma<DT>(wf[u][t], xf[u], acc[t]);
      }
    }
  }
  // lane holds C[row 16t + 4j + i][token c]; the waves' partials summed in wave order
#pragma unroll
  for (int t = 0; t < GM_TILES; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][16 * t + 4 * j + i][c] = acc[t][i];
  __syncthreads();
  if constexpr (SWIGLU) {
    static_assert(TILED && GM_TILES == 2, "the fused gate/up product takes a gate tile and an up tile");
    for (int idx = threadIdx.x; idx < 16 * 16; idx += GM_T) {
      const int r = idx >> 4, m = idx & 15;
      const int64_t f = static_cast<int64_t>(blockIdx.x) * 16 + r;
      if (m >= a.M || f >= a.F) continue;
      const float g = gemm_round<DT>((red[0][r][m] + red[1][r][m] + red[2][r][m] + red[3][r][m]) + 0.f);
      const float u =
          gemm_round<DT>((red[0][16 + r][m] + red[1][16 + r][m] + red[2][16 + r][m] + red[3][16 + r][m]) + 0.f);
      const float act = gemm_round<DT>(g / (1.f + expf(-g)));
      store_elem<DT>(a.out, m * a.out_stride + f, act * u);
    }
    return;
  }
  if constexpr (ARGMAX) {
    __shared__ unsigned long long best[GM_ROWS][16];
    for (int idx = threadIdx.x; idx < GM_ROWS * 16; idx += GM_T) {
      const int r = idx >> 4, m = idx & 15;
      const int64_t n = n0 + r;
      unsigned long long key = 0;
      if (n < a.N) {
        const float b = a.bias != nullptr ? load_elem<DT>(a.bias, n) : 0.f;
        key = argmax_key(gemm_round<DT>((red[0][r][m] + red[1][r][m] + red[2][r][m] + red[3][r][m]) + b), n);
      }
      best[r][m] = key;
    }
    __syncthreads();
    if (threadIdx.x < a.M) {
      const int m = threadIdx.x;
      unsigned long long key = 0;
      for (int r = 0; r < GM_ROWS; ++r) key = best[r][m] > key ? best[r][m] : key;
      a.keys[static_cast<int64_t>(m) * gridDim.x + blockIdx.x] = key;
    }
    return;
  }
  if (a.splits > 1 && a.epoch != 0) {
    // this slice's partial words, then the arrival; the tile's last workgroup sums
    // every slice's word in slice order (reading again a word whose tag has not
    // landed yet), adds the bias, rounds, and leaves the counter to the next round
    const uint32_t round = counter_round(c0, a.epoch);
    const uint32_t tag = group_tag(a.epoch, round);
    for (int idx = threadIdx.x; idx < GM_ROWS * 16; idx += GM_T) {
      const int r = idx >> 4, m = idx & 15;
      const int64_t n = n0 + r;
      if (m >= a.M || n >= a.N) continue;
      store_partial(a.words + (split * a.M + m) * a.N + n,
                    red[0][r][m] + red[1][r][m] + red[2][r][m] + red[3][r][m], tag);
    }
    __shared__ int s_last;
    __syncthreads();
    if (threadIdx.x == 0) s_last = arrive_last(a.counters + blockIdx.x, a.epoch, a.splits) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    constexpr int MS = 8;  // slices whose words are loaded together
    const int64_t sstride = a.M * a.N;
    for (int idx = threadIdx.x; idx < GM_ROWS * 16; idx += GM_T) {
      const int r = idx >> 4, m = idx & 15;
      const int64_t n = n0 + r;
      if (m >= a.M || n >= a.N) continue;
      const unsigned long long* w0 = a.words + m * a.N + n;
      float v = 0.f;
      for (int64_t s0 = 0; s0 < a.splits; s0 += MS) {
        unsigned long long w[MS];
#pragma unroll
        for (int u = 0; u < MS; ++u) {
          const int64_t sl = s0 + u < a.splits ? s0 + u : s0;  // in bounds; not added
          w[u] = __hip_atomic_load(w0 + sl * sstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int u = 0; u < MS; ++u) {
          if (s0 + u >= a.splits) break;
          if (static_cast<uint32_t>(w[u] >> 32) != tag) w[u] = partial_reread(w0 + (s0 + u) * sstride, tag);
          v += partial_value(w[u]);
        }
      }
      const float b = a.bias != nullptr ? load_elem<DT>(a.bias, n) : 0.f;
      store_elem<DT>(a.out, m * a.out_stride + n, v + b);
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(a.counters + blockIdx.x,
                         (static_cast<unsigned long long>(counter_id(a.epoch)) << 32) |
                             (static_cast<unsigned long long>((round + 1) & 0xffffu) << 16),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  for (int idx = threadIdx.x; idx < GM_ROWS * 16; idx += GM_T) {
    const int r = idx >> 4, m = idx & 15;
    const int64_t n = n0 + r;
    if (m >= a.M || n >= a.N) continue;
    const float v = red[0][r][m] + red[1][r][m] + red[2][r][m] + red[3][r][m];
    if (a.splits > 1) {
      a.part[(split * a.M + m) * a.N + n] = v;
    } else {
      const float b = a.bias != nullptr ? load_elem<DT>(a.bias, n) : 0.f;
      store_elem<DT>(a.out, m * a.out_stride + n, v + b);
    }
  }
}

template <int DT>
__global__ __launch_bounds__(GM_T) void gemm_finalize_kernel(const float* part, int64_t splits, int64_t M, int64_t N,
                                                             const unsigned short* bias, void* out,
                                                             int64_t out_stride) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * GM_T + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;
  float v = 0.f;
  for (int64_t s = 0; s < splits; ++s) v += part[(s * M + m) * N + n];
  if (bias != nullptr) v += load_elem<DT>(bias, n);
  store_elem<DT>(out, m * out_stride + n, v);
}

// One workgroup per token: the largest of its `blocks` keys, as the vocabulary index.
__global__ __launch_bounds__(GM_T) void argmax_finalize_kernel(const unsigned long long* keys, int64_t blocks,
                                                               int64_t* tokens) {
  __shared__ unsigned long long wave_best[GM_T / 64];
  const int64_t m = blockIdx.x;
  unsigned long long key = 0;
  for (int64_t b = threadIdx.x; b < blocks; b += GM_T) {
    const unsigned long long v = keys[m * blocks + b];
    key = v > key ? v : key;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(key, off, 64);
    key = o > key ? o : key;
  }
  if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < GM_T / 64; ++w) key = wave_best[w] > key ? wave_best[w] : key;
    tokens[m] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key));
  }
}

struct GemmPlan {
  int tiles, gu;
  int64_t blocks, splits, slice_steps;
};

static int64_t gemm_ceil(int64_t a, int64_t b) { return (a + b - 1) / b; }

static int64_t env_or(const char* name, int64_t fallback) {
  const char* env = getenv(name);
  return env ? atoll(env) : fallback;
}

// 16-row workgroups up to 1024 of them, else 32-row; rounds of 8 k-steps
// (the best of 1/2/4 tiles x 2/4/8 steps measured over the Qwen2.5 decode
// shapes).  Enough K slices for about two workgroups per CU, each slice
// keeping at least two rounds per wave.  HS_GEMM_TILES / HS_GEMM_GU /
// HS_GEMM_SPLITS override the choice (read once).
static GemmPlan plan_gemm(int64_t N, int64_t K) {
  static const int64_t f_tiles = env_or("HS_GEMM_TILES", 0), f_gu = env_or("HS_GEMM_GU", 0),
                       f_splits = env_or("HS_GEMM_SPLITS", 0);
  GemmPlan p{};
  p.tiles = gemm_ceil(N, 16) <= 1024 ? 1 : 2;
  if (f_tiles == 1 || f_tiles == 2 || f_tiles == 4) p.tiles = static_cast<int>(f_tiles);
  p.gu = f_gu == 4 ? 4 : 8;
  p.blocks = gemm_ceil(N, 16 * p.tiles);
  const int64_t steps = K / 32;
  int64_t splits = gemm_ceil(512, p.blocks);
  const int64_t most = steps / (2 * 4 * p.gu);
  if (splits > most) splits = most;
  if (f_splits > 0) splits = f_splits < steps ? f_splits : steps;  // forced: at least one k-step per slice
  if (splits < 1) splits = 1;
  p.slice_steps = gemm_ceil(steps, splits);
  p.splits = gemm_ceil(steps, p.slice_steps);
  return p;
}

template <int DT, int TILES, bool TILED, bool ARGMAX>
static void launch_gemm_tiles(const GemmPlan& p, dim3 grid, const GemmArgs& a, hipStream_t s) {
  if (p.gu == 4) hipLaunchKernelGGL((skinny_gemm_kernel<DT, TILES, 4, TILED, false, ARGMAX>), grid, dim3(GM_T), 0, s, a);
  else hipLaunchKernelGGL((skinny_gemm_kernel<DT, TILES, 8, TILED, false, ARGMAX>), grid, dim3(GM_T), 0, s, a);
}

template <int DT, bool TILED, bool ARGMAX = false>
static void launch_gemm(const GemmPlan& p, dim3 grid, const GemmArgs& a, hipStream_t s) {
  if (p.tiles == 1) launch_gemm_tiles<DT, 1, TILED, ARGMAX>(p, grid, a, s);
  else if (p.tiles == 2) launch_gemm_tiles<DT, 2, TILED, ARGMAX>(p, grid, a, s);
  else launch_gemm_tiles<DT, 4, TILED, ARGMAX>(p, grid, a, s);
}

// The argmax form's plan: the plain plan's tiles and rounds, one K slice.
static GemmPlan plan_argmax(int64_t N, int64_t K) {
  GemmPlan p = plan_gemm(N, K);
  p.slice_steps = K / 32;
  p.splits = 1;
  return p;
}

}  // namespace hs

using namespace hs;

extern "C" int64_t hs_skinny_gemm_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows < 1 || n < 1 || k < 32) return 256;
  const GemmPlan p = plan_gemm(n, k);
  // tagged 64-bit partial words and a counter per row tile (the fp32 partials of the
  // two-launch form fit in the same bytes)
  return p.splits > 1 ? p.splits * rows * n * 8 + p.blocks * 8 + 256 : 256;
}

static int run_gemm(const void* x, int64_t x_stride, const void* weight, int64_t n, int64_t k, const void* bias,
                    void* out, int64_t out_stride, int64_t rows, int32_t dtype, void* workspace,
                    int64_t workspace_bytes, hipStream_t stream, bool tiled) {
  HS_CHECK_ARG(dtype == HS_DTYPE_BF16 || dtype == HS_DTYPE_F16, "the decode GEMM takes bf16 or f16");
  HS_CHECK_ARG(rows >= 1 && rows <= 16, "the decode GEMM takes 1 to 16 rows");
  HS_CHECK_ARG(n >= 1 && k >= 32 && k % 32 == 0, "K must be a positive multiple of 32");
  HS_CHECK_ARG(x_stride >= k && x_stride % 8 == 0 && out_stride >= n, "invalid row strides");
  HS_CHECK_ARG(x && weight && out, "null GEMM pointer");
  HS_CHECK_ARG((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(weight) & 15) == 0,
               "x and weight must be 16-byte aligned");
  const GemmPlan p = plan_gemm(n, k);
  HS_CHECK_ARG(p.blocks <= 0x7fffffff && p.splits <= 65535, "GEMM too large");
  GemmArgs a{};
  a.x = static_cast<const unsigned short*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const unsigned short*>(weight);
  a.K = k;
  a.N = n;
  a.M = rows;
  a.bias = static_cast<const unsigned short*>(bias);
  a.out = out;
  a.out_stride = out_stride;
  a.splits = p.splits;
  a.slice_steps = p.slice_steps;
  // the split-K partials merged in-kernel unless HS_GEMM_FUSED_MERGE=0 (read per call)
  const char* fused_env = getenv("HS_GEMM_FUSED_MERGE");
  const bool fused = !(fused_env && atoi(fused_env) == 0);
  if (p.splits > 1) {
    const int64_t need = fused ? p.splits * rows * n * 8 + p.blocks * 8 : p.splits * rows * n * 4;
    HS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 7) == 0,
                 "GEMM workspace too small or misaligned: need %lld bytes", static_cast<long long>(need));
    if (fused) {
      a.words = static_cast<unsigned long long*>(workspace);
      a.counters = a.words + p.splits * rows * n;
      a.epoch = next_epoch();
    } else {
      a.part = static_cast<float*>(workspace);
    }
  }
  const dim3 grid(static_cast<unsigned>(p.blocks), static_cast<unsigned>(p.splits));
  if (dtype == HS_DTYPE_BF16) {
    if (tiled) launch_gemm<HS_DTYPE_BF16, true>(p, grid, a, stream);
    else launch_gemm<HS_DTYPE_BF16, false>(p, grid, a, stream);
  } else {
    if (tiled) launch_gemm<HS_DTYPE_F16, true>(p, grid, a, stream);
    else launch_gemm<HS_DTYPE_F16, false>(p, grid, a, stream);
  }
  HS_CHECK_LAUNCH("skinny GEMM");
  if (p.splits > 1 && !fused) {
    const unsigned blocks = static_cast<unsigned>(gemm_ceil(rows * n, GM_T));
    if (dtype == HS_DTYPE_BF16)
      hipLaunchKernelGGL((gemm_finalize_kernel<HS_DTYPE_BF16>), dim3(blocks), dim3(GM_T), 0, stream, a.part, p.splits,
                         rows, n, a.bias, out, out_stride);
    else
      hipLaunchKernelGGL((gemm_finalize_kernel<HS_DTYPE_F16>), dim3(blocks), dim3(GM_T), 0, stream, a.part, p.splits,
                         rows, n, a.bias, out, out_stride);
    HS_CHECK_LAUNCH("skinny GEMM finalize");
  }
  return HS_OK;
}

extern "C" int hs_skinny_gemm(const void* x, int64_t x_stride, const void* weight, int64_t n, int64_t k,
                              const void* bias, void* out, int64_t out_stride, int64_t rows, int32_t dtype,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return run_gemm(x, x_stride, weight, n, k, bias, out, out_stride, rows, dtype, workspace, workspace_bytes, stream,
                  false);
}

extern "C" int hs_skinny_gemm_tiled(const void* x, int64_t x_stride, const void* weight_tiles, int64_t n, int64_t k,
                                    const void* bias, void* out, int64_t out_stride, int64_t rows, int32_t dtype,
                                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return run_gemm(x, x_stride, weight_tiles, n, k, bias, out, out_stride, rows, dtype, workspace, workspace_bytes,
                  stream, true);
}

extern "C" int hs_skinny_gemm_swiglu_tiled(const void* x, int64_t x_stride, const void* gate_up_tiles, int64_t ffn,
                                           int64_t k, void* out, int64_t out_stride, int64_t rows, int32_t dtype,
                                           hipStream_t stream) {
  HS_CHECK_ARG(dtype == HS_DTYPE_BF16 || dtype == HS_DTYPE_F16, "the decode GEMM takes bf16 or f16");
  HS_CHECK_ARG(rows >= 1 && rows <= 16, "the decode GEMM takes 1 to 16 rows");
  HS_CHECK_ARG(ffn >= 1 && k >= 32 && k % 32 == 0, "K must be a positive multiple of 32");
  HS_CHECK_ARG(x_stride >= k && x_stride % 8 == 0 && out_stride >= ffn, "invalid row strides");
  HS_CHECK_ARG(x && gate_up_tiles && out, "null GEMM pointer");
  HS_CHECK_ARG((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(gate_up_tiles) & 15) == 0,
               "x and weight must be 16-byte aligned");
  const int64_t blocks = gemm_ceil(ffn, 16);
  HS_CHECK_ARG(blocks <= 0x7fffffff, "GEMM too large");
  GemmArgs a{};
  a.x = static_cast<const unsigned short*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const unsigned short*>(gate_up_tiles);
  a.K = k;
  a.N = 2 * 16 * blocks;  // interleaved weight rows, padded
  a.M = rows;
  a.out = out;
  a.out_stride = out_stride;
  a.splits = 1;  // one K slice: the workgroup sees whole sums before the product
  a.slice_steps = k / 32;
  a.F = ffn;
  const dim3 grid(static_cast<unsigned>(blocks));
  if (dtype == HS_DTYPE_BF16)
    hipLaunchKernelGGL((skinny_gemm_kernel<HS_DTYPE_BF16, 2, 8, true, true>), grid, dim3(GM_T), 0, stream, a);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<HS_DTYPE_F16, 2, 8, true, true>), grid, dim3(GM_T), 0, stream, a);
  HS_CHECK_LAUNCH("skinny GEMM swiglu");
  return HS_OK;
}

extern "C" int64_t hs_skinny_gemm_argmax_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows < 1 || n < 1 || k < 32) return 256;
  return plan_argmax(n, k).blocks * rows * 8 + 256;
}

extern "C" int hs_skinny_gemm_argmax_tiled(const void* x, int64_t x_stride, const void* weight_tiles, int64_t n,
                                           int64_t k, const void* bias, int64_t* tokens, int64_t rows, int32_t dtype,
                                           void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  HS_CHECK_ARG(dtype == HS_DTYPE_BF16 || dtype == HS_DTYPE_F16, "the decode GEMM takes bf16 or f16");
  HS_CHECK_ARG(rows >= 1 && rows <= 16, "the decode GEMM takes 1 to 16 rows");
  HS_CHECK_ARG(n >= 1 && n <= 0x7fffffff && k >= 32 && k % 32 == 0,
               "n must be in [1, 2^31) and K a positive multiple of 32");
  HS_CHECK_ARG(x_stride >= k && x_stride % 8 == 0, "invalid row stride");
  HS_CHECK_ARG(x && weight_tiles && tokens, "null GEMM pointer");
  HS_CHECK_ARG((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(weight_tiles) & 15) == 0,
               "x and weight must be 16-byte aligned");
  const GemmPlan p = plan_argmax(n, k);
  HS_CHECK_ARG(p.blocks <= 0x7fffffff, "GEMM too large");
  const int64_t need = p.blocks * rows * 8;
  HS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 7) == 0,
               "argmax workspace too small or misaligned: need %lld bytes", static_cast<long long>(need));
  GemmArgs a{};
  a.x = static_cast<const unsigned short*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const unsigned short*>(weight_tiles);
  a.K = k;
  a.N = n;
  a.M = rows;
  a.bias = static_cast<const unsigned short*>(bias);
  a.splits = 1;
  a.slice_steps = p.slice_steps;
  a.keys = static_cast<unsigned long long*>(workspace);
  const dim3 grid(static_cast<unsigned>(p.blocks));
  if (dtype == HS_DTYPE_BF16) launch_gemm<HS_DTYPE_BF16, true, true>(p, grid, a, stream);
  else launch_gemm<HS_DTYPE_F16, true, true>(p, grid, a, stream);
  HS_CHECK_LAUNCH("skinny GEMM argmax");
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(static_cast<unsigned>(rows)), dim3(GM_T), 0, stream, a.keys,
                     p.blocks, tokens);
  HS_CHECK_LAUNCH("argmax finalize");
  return HS_OK;
}
