// Shared definitions for the gfx950 kernels of the sparse decode path.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "hisparse.h"

namespace hs {

// ---- error reporting -------------------------------------------------------
void set_error(const char* fmt, ...);

#define HS_CHECK_ARG(cond, ...)                \
  do {                                         \
    if (!(cond)) {                             \
      ::hs::set_error(__VA_ARGS__);            \
      return HS_EINVAL;                        \
    }                                          \
  } while (0)

#define HS_CHECK_LAUNCH(what)                                              \
  do {                                                                     \
    hipError_t _e = hipGetLastError();                                     \
    if (_e != hipSuccess) {                                                \
      ::hs::set_error("%s launch failed: %s", what, hipGetErrorString(_e)); \
      return HS_ELAUNCH;                                                   \
    }                                                                      \
  } while (0)

// ---- element types -----------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short b) {
  return __uint_as_float(static_cast<unsigned int>(b) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(unsigned short b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}
// Round-to-nearest-even float -> bf16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float f) {
  unsigned int u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<unsigned short>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<unsigned short>(u >> 16);
}
__device__ __forceinline__ unsigned short f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  unsigned short b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Storage element -> float for the three cache dtypes.
template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
  if constexpr (DT == HS_DTYPE_F32) {
    return static_cast<const float*>(base)[i];
  } else if constexpr (DT == HS_DTYPE_BF16) {
    return bf16_bits_to_f32(static_cast<const unsigned short*>(base)[i]);
  } else {
    return f16_bits_to_f32(static_cast<const unsigned short*>(base)[i]);
  }
}
template <int DT>
__device__ __forceinline__ void store_elem(void* base, int64_t i, float v) {
  if constexpr (DT == HS_DTYPE_F32) {
    static_cast<float*>(base)[i] = v;
  } else if constexpr (DT == HS_DTYPE_BF16) {
    static_cast<unsigned short*>(base)[i] = f32_to_bf16_bits(v);
  } else {
    static_cast<unsigned short*>(base)[i] = f32_to_f16_bits(v);
  }
}

// x * y rounded to fp32, never contracted with a following conversion: the
// compiler may otherwise fold fptrunc(x * y) into one mixed-precision FMA that
// rounds the exact product to f16 once, where PyTorch's (x * y).to(float16) rounds
// to fp32 first (and it does so for some lanes of a kernel and not others).
// (The empty asm holds the product as an fp32 register value; it emits nothing.
// A contract(off) pragma does not reach that fold.)
__device__ __forceinline__ float mul_rn(float x, float y) {
  float p = x * y;
  asm("" : "+v"(p));
  return p;
}

// v rounded to the storage dtype (float32: unchanged).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == HS_DTYPE_F32) return v;
  else if constexpr (DT == HS_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else return f16_bits_to_f32(f32_to_f16_bits(v));
}

// The rotary pair (x_i, x_{i + D/2}) of a head vector at position `pos` with base
// `theta`, as the model's rotary computes it: inv_freq = theta ** (-(2i) / D) and the
// angle in fp32, cos/sin rounded to the dtype, each product rounded, then the sum
// (which the caller's store rounds).
template <int DT>
__device__ __forceinline__ void rotary_pair(float a, float b, float pos, int64_t i, int64_t D, float theta,
                                            float& lo, float& hi) {
  const float inv = powf(theta, -(static_cast<float>(2 * i) / static_cast<float>(D)));
  const float angle = pos * inv;
  const float c = round_to<DT>(cosf(angle)), s = round_to<DT>(sinf(angle));
  lo = round_to<DT>(a * c) + round_to<DT>(-b * s);
  hi = round_to<DT>(b * c) + round_to<DT>(a * s);
}

// A Quest bound element taking a new K element, as torch.minimum / torch.maximum
// compute it on this device: a NaN operand is returned (the existing bound first);
// 16-bit types return old < new ? old : new (so an equal compare -- +0 vs -0
// included -- returns the new element); float32 orders -0 below +0.  `x` is the new
// element as stored (`xbits` its 16-bit pattern).
__device__ __forceinline__ void bound16_take(unsigned short* lo, unsigned short* hi, unsigned short xbits, float x,
                                             float a, float b) {
  if (!(a != a) && (x != x || !(a < x))) *lo = xbits;
  if (!(b != b) && (x != x || !(b > x))) *hi = xbits;
}
__device__ __forceinline__ void bound32_take(float* lo, float* hi, float x) {
  const float a = *lo, b = *hi;
  const bool zero_tie = x == 0.f && a == 0.f;  // both zeros: -0 is the smaller
  if (!(a != a) && (x != x || x < a || (zero_tie && signbit(x) && !signbit(a)))) *lo = x;
  const bool zero_tie_hi = x == 0.f && b == 0.f;
  if (!(b != b) && (x != x || x > b || (zero_tie_hi && !signbit(x) && signbit(b)))) *hi = x;
}

inline int elem_bytes(int dtype) { return dtype == HS_DTYPE_F32 ? 4 : 2; }
inline bool valid_dtype(int dtype) {
  return dtype == HS_DTYPE_F32 || dtype == HS_DTYPE_F16 || dtype == HS_DTYPE_BF16;
}

// ---- wave / block primitives (wave64) -----------------------------------------
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Orders one wave's LDS writes before its later LDS reads of other lanes'
// data.  LDS executes a wave's operations in order; this waits for the wave's
// outstanding LDS operations and stops compiler reordering, without waiting
// for vector memory loads still in flight (a memory fence would).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    T o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Exclusive prefix sum over a 1-D block of up to 1024 threads.  `scratch` must
// hold 16 elements.  Returns the exclusive prefix; `total` gets the block sum.
template <typename T>
__device__ __forceinline__ T block_exclusive_sum(T v, T* scratch, T* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = (blockDim.x + 63) >> 6;
  T inc = wave_inclusive_sum(v);
  __syncthreads();
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  T base = 0, all = 0;
  for (int w = 0; w < waves; ++w) {
    T s = scratch[w];
    if (w < wave) base += s;
    all += s;
  }
  *total = all;
  __syncthreads();
  return base + inc - v;
}

}  // namespace hs
