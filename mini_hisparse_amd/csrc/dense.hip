// Dense-layer helpers of the layer-major decode engine for gfx950.
//
// A decode step of B tokens runs, per layer, RMSNorm -> q/k/v projections ->
// rotary embedding -> sparse attention -> o_proj -> residual -> RMSNorm ->
// SiLU MLP -> residual (the reference's MiniModel.decode, model.py:183-226,
// with its Qwen2 layer math).  With B rows of a few thousand elements every
// elementwise PyTorch op is one launch of negligible work, and a layer issues
// ~30 of them.  These kernels fuse them around the projections (which stay
// PyTorch-ROCm GEMMs, with q/k/v and gate/up packed into one weight each):
//
//   add_rms_norm   x <- x + delta (in the model dtype), y = RMSNorm(x)
//   rotary_split   fused q|k|v projection output -> rotated q, rotated k, v
//   silu_mul       fused gate|up projection output -> silu(gate) * up
//
// Rounding follows the PyTorch ops they replace: the residual add rounds to
// the model dtype; RMSNorm squares and averages in fp32, rounds x * rsqrt to
// the model dtype and multiplies by the weight in that dtype; rotary rounds
// cos/sin, each product and the sum to the model dtype; SiLU rounds its fp32
// result before the product with `up`.  Only the fp32 sum order of the norm
// and the device's transcendental functions differ from PyTorch's.
#include <math.h>

#include "hs_common.h"

namespace hs {

constexpr int DN_T = 256;

// One workgroup per row.  `delta` may be null (no residual add); `x_out` may
// alias `x`.  A row of at most NR_REG * DN_T elements is held in registers: every
// load of x, delta and the weight is issued before the first is used, so the row
// costs one memory round trip (a store to x_out may alias the next load of x, so a
// loop that stores as it goes would wait out a round trip per element).  Longer
// rows go in rounds of NR_CH elements per thread, loads of a round issued together.
constexpr int NR_REG = 24;
constexpr int NR_CH = 8;

__device__ __forceinline__ float block_sum_dn(float v, float* partial) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = v;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < DN_T / 64; ++w) total += partial[w];
  return total;
}

template <int DT>
__global__ __launch_bounds__(DN_T) void add_rms_norm_kernel(const void* x, const void* delta, void* x_out, void* y,
                                                            const void* weight, int64_t width, int64_t x_stride,
                                                            int64_t y_stride, float eps) {
  __shared__ float partial[DN_T / 64];
  const int64_t row = blockIdx.x;
  const int64_t xo = row * x_stride, yo = row * y_stride;
  const bool add = delta != nullptr;
  const void* dsrc = add ? delta : x;  // always a valid row: no load sits under a branch
  if (width <= static_cast<int64_t>(NR_REG) * DN_T) {
    float v[NR_REG], dl[NR_REG], wv[NR_REG];
#pragma unroll
    for (int k = 0; k < NR_REG; ++k) {
      // unconditional loads of in-bounds elements (a load under a branch would be
      // waited for before the next), masked afterwards
      const int64_t i = threadIdx.x + static_cast<int64_t>(k) * DN_T;
      const bool in = i < width;
      const int64_t ic = in ? i : 0;
      const float xv = load_elem<DT>(x, xo + ic), wvv = load_elem<DT>(weight, ic);
      const float dv = load_elem<DT>(dsrc, xo + ic);
      v[k] = in ? xv : 0.f;
      dl[k] = in ? dv : 0.f;
      wv[k] = in ? wvv : 0.f;
    }
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < NR_REG; ++k) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(k) * DN_T;
      if (i >= width) break;
      if (add) {
        v[k] = round_to<DT>(v[k] + dl[k]);
        store_elem<DT>(x_out, xo + i, v[k]);
      }
      sq += v[k] * v[k];
    }
    const float r = rsqrtf(block_sum_dn(sq, partial) / static_cast<float>(width) + eps);
#pragma unroll
    for (int k = 0; k < NR_REG; ++k) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(k) * DN_T;
      if (i >= width) break;
      store_elem<DT>(y, yo + i, round_to<DT>(mul_rn(v[k], r)) * wv[k]);
    }
    return;
  }
  float sq = 0.f;
  for (int64_t base = threadIdx.x; base < width; base += static_cast<int64_t>(DN_T) * NR_CH) {
    float a[NR_CH], b[NR_CH];
#pragma unroll
    for (int k = 0; k < NR_CH; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * DN_T;
      const int64_t ic = i < width ? i : 0;
      const float xv = load_elem<DT>(x, xo + ic);
      const float dv = load_elem<DT>(dsrc, xo + ic);
      a[k] = i < width ? xv : 0.f;
      b[k] = i < width ? dv : 0.f;
    }
#pragma unroll
    for (int k = 0; k < NR_CH; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * DN_T;
      if (i >= width) break;
      float s = a[k];
      if (add) {
        s = round_to<DT>(s + b[k]);
        store_elem<DT>(x_out, xo + i, s);
      }
      sq += s * s;
    }
  }
  const float r = rsqrtf(block_sum_dn(sq, partial) / static_cast<float>(width) + eps);
  const void* src = add ? x_out : x;
  for (int64_t base = threadIdx.x; base < width; base += static_cast<int64_t>(DN_T) * NR_CH) {
    float a[NR_CH], b[NR_CH];
#pragma unroll
    for (int k = 0; k < NR_CH; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * DN_T;
      const int64_t ic = i < width ? i : 0;
      const float sv = load_elem<DT>(src, xo + ic), wvv = load_elem<DT>(weight, ic);
      a[k] = i < width ? sv : 0.f;
      b[k] = i < width ? wvv : 0.f;
    }
#pragma unroll
    for (int k = 0; k < NR_CH; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * DN_T;
      if (i >= width) break;
      store_elem<DT>(y, yo + i, round_to<DT>(mul_rn(a[k], r)) * b[k]);
    }
  }
}

// Grid (heads + 2 * kv_heads, rows); one thread per rotation pair (d, d + D/2).
// Heads [0, heads) are q, [heads, heads + kv_heads) k (both rotated at the
// row's position), the rest v (copied).
template <int DT>
__global__ __launch_bounds__(DN_T) void rotary_split_kernel(const void* qkv, int64_t qkv_stride, void* q, void* k,
                                                            void* v, const int64_t* positions, int64_t heads,
                                                            int64_t kv_heads, int64_t D, float theta) {
  const int64_t h = blockIdx.x, row = blockIdx.y;
  const int64_t half = D / 2;
  const int64_t src = row * qkv_stride + h * D;
  void* dst;
  int64_t doff;
  if (h < heads) {
    dst = q;
    doff = (row * heads + h) * D;
  } else if (h < heads + kv_heads) {
    dst = k;
    doff = (row * kv_heads + (h - heads)) * D;
  } else {
    dst = v;
    doff = (row * kv_heads + (h - heads - kv_heads)) * D;
  }
  if (h >= heads + kv_heads) {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) store_elem<DT>(dst, doff + d, load_elem<DT>(qkv, src + d));
    return;
  }
  const float pos = static_cast<float>(positions[row]);
  for (int64_t i = threadIdx.x; i < half; i += blockDim.x) {
    float lo, hi;
    rotary_pair<DT>(load_elem<DT>(qkv, src + i), load_elem<DT>(qkv, src + i + half), pos, i, D, theta, lo, hi);
    store_elem<DT>(dst, doff + i, lo);
    store_elem<DT>(dst, doff + i + half, hi);
  }
}

// out[row, j] = silu(gate[row, j]) * up[row, j] with gate = gate_up[row, :width],
// up = gate_up[row, width:].
template <int DT>
__global__ __launch_bounds__(DN_T) void silu_mul_kernel(const void* gate_up, int64_t gu_stride, void* out,
                                                        int64_t out_stride, int64_t width) {
  const int64_t row = blockIdx.y;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * DN_T + threadIdx.x;
  if (j >= width) return;
  const float g = load_elem<DT>(gate_up, row * gu_stride + j);
  const float u = load_elem<DT>(gate_up, row * gu_stride + width + j);
  const float act = round_to<DT>(g / (1.f + expf(-g)));
  store_elem<DT>(out, row * out_stride + j, act * u);
}

}  // namespace hs

using namespace hs;

#define HS_DENSE_DISPATCH(dtype, kernel, grid, block, stream, ...)                                              \
  do {                                                                                                          \
    if ((dtype) == HS_DTYPE_BF16) hipLaunchKernelGGL((kernel<HS_DTYPE_BF16>), grid, block, 0, stream, __VA_ARGS__); \
    else if ((dtype) == HS_DTYPE_F16) hipLaunchKernelGGL((kernel<HS_DTYPE_F16>), grid, block, 0, stream, __VA_ARGS__); \
    else hipLaunchKernelGGL((kernel<HS_DTYPE_F32>), grid, block, 0, stream, __VA_ARGS__);                     \
  } while (0)

extern "C" int hs_add_rms_norm(const void* x, const void* delta, void* x_out, void* y, const void* weight,
                               int64_t rows, int64_t width, int64_t x_stride, int64_t y_stride, float eps,
                               int32_t dtype, hipStream_t stream) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(rows >= 1 && rows <= 65535 && width >= 1, "invalid norm shape");
  HS_CHECK_ARG(x_stride >= width && y_stride >= width, "row strides below the width");
  HS_CHECK_ARG(x && y && weight && (delta == nullptr || x_out != nullptr), "null norm pointer");
  HS_DENSE_DISPATCH(dtype, add_rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(DN_T), stream, x, delta,
                    x_out, y, weight, width, x_stride, y_stride, eps);
  HS_CHECK_LAUNCH("add_rms_norm");
  return HS_OK;
}

extern "C" int hs_rotary_split(const void* qkv, int64_t qkv_stride, void* q, void* k, void* v,
                               const int64_t* positions, int64_t rows, int64_t heads, int64_t kv_heads,
                               int64_t head_dim, float theta, int32_t dtype, hipStream_t stream) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(rows >= 1 && rows <= 65535 && heads >= 1 && kv_heads >= 1 && head_dim >= 2 && head_dim % 2 == 0,
               "invalid rotary shape");
  HS_CHECK_ARG(qkv_stride >= (heads + 2 * kv_heads) * head_dim, "q|k|v row stride below its width");
  HS_CHECK_ARG(qkv && q && k && v && positions, "null rotary pointer");
  const unsigned threads = head_dim / 2 >= DN_T ? DN_T : static_cast<unsigned>(((head_dim / 2 + 63) / 64) * 64);
  HS_DENSE_DISPATCH(dtype, rotary_split_kernel, dim3(static_cast<unsigned>(heads + 2 * kv_heads), static_cast<unsigned>(rows)),
                    dim3(threads), stream, qkv, qkv_stride, q, k, v, positions, heads, kv_heads, head_dim, theta);
  HS_CHECK_LAUNCH("rotary_split");
  return HS_OK;
}

extern "C" int hs_silu_mul(const void* gate_up, int64_t gu_stride, void* out, int64_t out_stride, int64_t rows,
                           int64_t width, int32_t dtype, hipStream_t stream) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(rows >= 1 && rows <= 65535 && width >= 1, "invalid silu_mul shape");
  HS_CHECK_ARG(gu_stride >= 2 * width && out_stride >= width, "row strides below the width");
  HS_CHECK_ARG(gate_up && out, "null silu_mul pointer");
  const int64_t blocks = (width + DN_T - 1) / DN_T;
  HS_CHECK_ARG(blocks <= 0x7fffffff, "silu_mul width too large");
  HS_DENSE_DISPATCH(dtype, silu_mul_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(rows)),
                    dim3(DN_T), stream, gate_up, gu_stride, out, out_stride, width);
  HS_CHECK_LAUNCH("silu_mul");
  return HS_OK;
}
