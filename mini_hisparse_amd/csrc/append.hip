// One-token append of the decode step for gfx950: the producer of the Quest
// bounds that the page scorer reads.
//
// Replaces the single-token case of HostStore.append (storage.py:246-319) for
// a batch of (request, layer) pairs: the new K and V rows go to their pool
// row; the tail page's minimum/maximum take the element-wise min/max with the
// new K row as torch.minimum/torch.maximum compute it on this device (a NaN
// operand is returned, the existing bound first; 16-bit types otherwise return
// old < new ? old : new, so an equal compare -- +0 vs -0 included -- returns
// the new element; float32 is IEEE minimum/maximum with -0 below +0); and the
// rows are mirrored
// into the pinned host pool through its device alias (the reference queues a
// device-to-host copy on the transfer stream instead).  One workgroup per
// pair, 16-byte units.
#include "hs_common.h"

namespace hs {

constexpr int AT = 256;
constexpr int AMAXB = 32;

struct AppendArgs {
  const char* k;
  const char* v;
  int64_t kv_sb;  // bytes between requests in k and v
  char* pool;
  char* host[AMAXB];
  int64_t dev_row[AMAXB], host_row[AMAXB];
  char* kmin[AMAXB];
  char* kmax[AMAXB];
  int64_t P, row_bytes;
};

template <int DT>
__device__ __forceinline__ float from_storage(unsigned short bits) {
  if constexpr (DT == HS_DTYPE_BF16) return bf16_bits_to_f32(bits);
  else return f16_bits_to_f32(bits);
}

template <int DT>
__device__ __forceinline__ void bound_update(const unsigned short* newv, unsigned short* lo, unsigned short* hi,
                                             int n) {
  for (int e = 0; e < n; ++e)
    bound16_take(lo + e, hi + e, newv[e], from_storage<DT>(newv[e]), from_storage<DT>(lo[e]), from_storage<DT>(hi[e]));
}

template <int DT>
__global__ __launch_bounds__(AT) void append_kernel(AppendArgs a) {
  const int b = blockIdx.x;
  const int64_t units = a.row_bytes / 16;
  const uint32_t P32 = static_cast<uint32_t>(a.P);
  const int64_t dr = a.dev_row[b], hr = a.host_row[b];
  const uint32_t db = static_cast<uint32_t>(dr) / P32, dof = static_cast<uint32_t>(dr) - db * P32;
  const int64_t dk = (static_cast<int64_t>(db) * 2 * a.P + dof) * a.row_bytes;  // K row; V row + P * row_bytes
  const int64_t plane = a.P * a.row_bytes;
  int64_t hk = -1;
  if (hr >= 0) {
    const uint32_t hb = static_cast<uint32_t>(hr) / P32, hof = static_cast<uint32_t>(hr) - hb * P32;
    hk = (static_cast<int64_t>(hb) * 2 * a.P + hof) * a.row_bytes;
  }
  const char* ksrc = a.k + b * a.kv_sb;
  const char* vsrc = a.v + b * a.kv_sb;
  for (int64_t u = threadIdx.x; u < units; u += AT) {
    const u32x4 kx = *reinterpret_cast<const u32x4*>(ksrc + u * 16);
    const u32x4 vx = *reinterpret_cast<const u32x4*>(vsrc + u * 16);
    *reinterpret_cast<u32x4*>(a.pool + dk + u * 16) = kx;
    *reinterpret_cast<u32x4*>(a.pool + dk + plane + u * 16) = vx;
    if (hk >= 0) {
      *reinterpret_cast<u32x4*>(a.host[b] + hk + u * 16) = kx;
      *reinterpret_cast<u32x4*>(a.host[b] + hk + plane + u * 16) = vx;
    }
    if constexpr (DT == HS_DTYPE_F32) {
      float* lo = reinterpret_cast<float*>(a.kmin[b] + u * 16);
      float* hi = reinterpret_cast<float*>(a.kmax[b] + u * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) bound32_take(lo + e, hi + e, __uint_as_float(kx[e]));
    } else {
      unsigned short nv[8];
      __builtin_memcpy(nv, &kx, 16);
      bound_update<DT>(nv, reinterpret_cast<unsigned short*>(a.kmin[b] + u * 16),
                       reinterpret_cast<unsigned short*>(a.kmax[b] + u * 16), 8);
    }
  }
}

// The rotary + split of a q|k|v projection (rotary_split_kernel's arithmetic) fused
// with the append of the new K and V rows (append_kernel's): grid (heads + 2 kv_heads,
// rows), one thread per rotation pair.  q heads are rotated into q; k heads are rotated
// into k, the pool row and the host mirror, and fold into the tail page's bounds; v
// heads are copied to v, the pool row and the host mirror.  Every element goes out
// through the same store as the k / v buffers, so the pool, the mirror and the bounds
// hold the bits the separate launches give.
struct RotaryArgs {
  const void* qkv;
  int64_t qkv_stride;
  void* q;
  void* k;
  void* v;
  const int64_t* positions;
  int64_t heads, kv_heads, D;
  float theta;
};

template <int DT>
__device__ __forceinline__ unsigned short bits_of(float v) {
  if constexpr (DT == HS_DTYPE_BF16) return f32_to_bf16_bits(v);
  else return f32_to_f16_bits(v);
}

template <int DT>
__device__ __forceinline__ void append_elem(const AppendArgs& a, int row, int64_t pk, int64_t hk, int64_t bound,
                                            float x, bool is_k) {
  store_elem<DT>(a.pool, pk, x);
  if (hk >= 0) store_elem<DT>(a.host[row], hk, x);
  if (!is_k) return;
  if constexpr (DT == HS_DTYPE_F32) {
    bound32_take(reinterpret_cast<float*>(a.kmin[row]) + bound, reinterpret_cast<float*>(a.kmax[row]) + bound, x);
  } else {
    unsigned short* lo = reinterpret_cast<unsigned short*>(a.kmin[row]) + bound;
    unsigned short* hi = reinterpret_cast<unsigned short*>(a.kmax[row]) + bound;
    const unsigned short xb = bits_of<DT>(x);
    bound16_take(lo, hi, xb, from_storage<DT>(xb), from_storage<DT>(*lo), from_storage<DT>(*hi));
  }
}

template <int DT>
__global__ __launch_bounds__(AT) void rotary_append_kernel(RotaryArgs r, AppendArgs a) {
  const int64_t h = blockIdx.x;
  const int row = blockIdx.y;
  const int64_t D = r.D, half = D / 2, Hkv = r.kv_heads;
  const int64_t src = row * r.qkv_stride + h * D;
  const bool is_q = h < r.heads, is_k = !is_q && h < r.heads + Hkv;
  const int64_t kvh = is_q ? 0 : (is_k ? h - r.heads : h - r.heads - Hkv);
  void* dst = is_q ? r.q : (is_k ? r.k : r.v);
  const int64_t doff = is_q ? (row * r.heads + h) * D : (row * Hkv + kvh) * D;
  // the row's K (or V) segment in the pool and the host mirror ([block, 2, P, Hkv, D])
  const int64_t P = a.P, plane = P * Hkv * D, seg = kvh * D + (is_k ? 0 : plane);
  const int64_t dr = a.dev_row[row], hr = a.host_row[row];
  const int64_t pk = ((dr / P) * 2 * P + dr % P) * Hkv * D + seg;
  const int64_t hk = hr >= 0 ? ((hr / P) * 2 * P + hr % P) * Hkv * D + seg : -1;
  if (!is_q && !is_k) {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
      const float x = load_elem<DT>(r.qkv, src + d);
      store_elem<DT>(dst, doff + d, x);
      append_elem<DT>(a, row, pk + d, hk >= 0 ? hk + d : -1, 0, x, false);
    }
    return;
  }
  const float pos = static_cast<float>(r.positions[row]);
  for (int64_t i = threadIdx.x; i < half; i += blockDim.x) {
    float lo, hi;
    rotary_pair<DT>(load_elem<DT>(r.qkv, src + i), load_elem<DT>(r.qkv, src + i + half), pos, i, D, r.theta, lo, hi);
    store_elem<DT>(dst, doff + i, lo);
    store_elem<DT>(dst, doff + i + half, hi);
    if (!is_k) continue;
    append_elem<DT>(a, row, pk + i, hk >= 0 ? hk + i : -1, kvh * D + i, round_to<DT>(lo), true);
    append_elem<DT>(a, row, pk + i + half, hk >= 0 ? hk + i + half : -1, kvh * D + i + half, round_to<DT>(hi), true);
  }
}

}  // namespace hs

using namespace hs;

// At most AMAXB rows (their pointers travel in the kernel arguments);
// hs_append_rows cuts larger batches into such chunks.
static int append_chunk(const void* k, const void* v, int64_t kv_stride_b, void* pool, int64_t pool_rows,
                        int32_t dtype, int64_t page_size, int64_t kv_heads, int64_t head_dim,
                        const int64_t* device_rows, const void* const* host_alias, const int64_t* host_rows,
                        int64_t host_pool_rows, void* const* minimum, void* const* maximum, int32_t batch,
                        hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1 && batch <= AMAXB, "append batch must be in [1, %d]", AMAXB);
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(k && v && pool && device_rows && minimum && maximum, "null append pointer");
  HS_CHECK_ARG(page_size >= 1 && kv_heads >= 1 && head_dim >= 1, "invalid append shape");
  const int64_t esz = elem_bytes(dtype);
  const int64_t row_bytes = kv_heads * head_dim * esz;
  HS_CHECK_ARG(row_bytes % 16 == 0, "kv_heads * head_dim * element size must be a multiple of 16 bytes");
  uintptr_t align = reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                    reinterpret_cast<uintptr_t>(pool) | static_cast<uintptr_t>(kv_stride_b * esz);
  AppendArgs a{};
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.kv_sb = kv_stride_b * esz;
  a.pool = static_cast<char*>(pool);
  a.P = page_size;
  a.row_bytes = row_bytes;
  for (int32_t i = 0; i < batch; ++i) {
    HS_CHECK_ARG(device_rows[i] >= 0 && device_rows[i] < pool_rows, "append device row %lld outside the pool",
                 static_cast<long long>(device_rows[i]));
    HS_CHECK_ARG(!host_rows || host_rows[i] < host_pool_rows, "append host row %lld outside the host pool",
                 static_cast<long long>(host_rows[i]));
    HS_CHECK_ARG(minimum[i] && maximum[i], "null bounds pointer");
    a.dev_row[i] = device_rows[i];
    a.host_row[i] = host_rows ? host_rows[i] : -1;
    a.host[i] = host_alias ? static_cast<char*>(const_cast<void*>(host_alias[i])) : nullptr;
    HS_CHECK_ARG(a.host_row[i] < 0 || a.host[i], "a host row needs a host alias");
    a.kmin[i] = static_cast<char*>(minimum[i]);
    a.kmax[i] = static_cast<char*>(maximum[i]);
    align |= reinterpret_cast<uintptr_t>(a.kmin[i]) | reinterpret_cast<uintptr_t>(a.kmax[i]) |
             reinterpret_cast<uintptr_t>(a.host[i]);
  }
  HS_CHECK_ARG((align & 15) == 0, "append buffers must be 16-byte aligned");
  const dim3 grid(static_cast<unsigned>(batch));
  if (dtype == HS_DTYPE_BF16) hipLaunchKernelGGL(append_kernel<HS_DTYPE_BF16>, grid, dim3(AT), 0, stream, a);
  else if (dtype == HS_DTYPE_F16) hipLaunchKernelGGL(append_kernel<HS_DTYPE_F16>, grid, dim3(AT), 0, stream, a);
  else hipLaunchKernelGGL(append_kernel<HS_DTYPE_F32>, grid, dim3(AT), 0, stream, a);
  HS_CHECK_LAUNCH("append");
  return HS_OK;
}

extern "C" int hs_append_rows(const void* k, const void* v, int64_t kv_stride_b, void* pool, int64_t pool_rows,
                              int32_t dtype, int64_t page_size, int64_t kv_heads, int64_t head_dim,
                              const int64_t* device_rows, const void* const* host_alias,
                              const int64_t* host_rows, int64_t host_pool_rows, void* const* minimum,
                              void* const* maximum, int32_t batch, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1, "append batch must be positive");
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(k && v && pool && device_rows && minimum && maximum, "null append pointer");
  for (int32_t i = 0; i < batch; ++i) {  // every row, before the first launch
    HS_CHECK_ARG(device_rows[i] >= 0 && device_rows[i] < pool_rows, "append device row %lld outside the pool",
                 static_cast<long long>(device_rows[i]));
    HS_CHECK_ARG(!host_rows || host_rows[i] < host_pool_rows, "append host row %lld outside the host pool",
                 static_cast<long long>(host_rows[i]));
    HS_CHECK_ARG(minimum[i] && maximum[i], "null bounds pointer");
    HS_CHECK_ARG(!host_rows || host_rows[i] < 0 || (host_alias && host_alias[i]), "a host row needs a host alias");
  }
  const int64_t step = kv_stride_b * elem_bytes(dtype);
  for (int32_t s0 = 0; s0 < batch; s0 += AMAXB) {
    const int32_t c = batch - s0 < AMAXB ? batch - s0 : AMAXB;
    const int rc = append_chunk(static_cast<const char*>(k) + s0 * step, static_cast<const char*>(v) + s0 * step,
                                kv_stride_b, pool, pool_rows, dtype, page_size, kv_heads, head_dim, device_rows + s0,
                                host_alias ? host_alias + s0 : nullptr, host_rows ? host_rows + s0 : nullptr,
                                host_pool_rows, minimum + s0, maximum + s0, c, stream);
    if (rc != HS_OK) return rc;
  }
  return HS_OK;
}

extern "C" int hs_rotary_split_append(const void* qkv, int64_t qkv_stride, void* q, void* k, void* v,
                                      const int64_t* positions, int64_t rows, int64_t heads, int64_t kv_heads,
                                      int64_t head_dim, float theta, int32_t dtype, void* pool, int64_t pool_rows,
                                      int64_t page_size, const int64_t* device_rows, const void* const* host_alias,
                                      const int64_t* host_rows, int64_t host_pool_rows, void* const* minimum,
                                      void* const* maximum, hipStream_t stream) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(rows >= 1 && rows <= 65535 && heads >= 1 && kv_heads >= 1 && head_dim >= 2 && head_dim % 2 == 0,
               "invalid rotary shape");
  HS_CHECK_ARG(qkv_stride >= (heads + 2 * kv_heads) * head_dim, "q|k|v row stride below its width");
  HS_CHECK_ARG(qkv && q && k && v && positions && pool && device_rows && minimum && maximum,
               "null rotary/append pointer");
  HS_CHECK_ARG(page_size >= 1, "invalid append shape");
  for (int64_t i = 0; i < rows; ++i) {  // every row, before the first launch
    HS_CHECK_ARG(device_rows[i] >= 0 && device_rows[i] < pool_rows, "append device row %lld outside the pool",
                 static_cast<long long>(device_rows[i]));
    HS_CHECK_ARG(!host_rows || host_rows[i] < host_pool_rows, "append host row %lld outside the host pool",
                 static_cast<long long>(host_rows[i]));
    HS_CHECK_ARG(minimum[i] && maximum[i], "null bounds pointer");
    HS_CHECK_ARG(!host_rows || host_rows[i] < 0 || (host_alias && host_alias[i]), "a host row needs a host alias");
  }
  const int64_t esz = elem_bytes(dtype);
  const unsigned threads = head_dim / 2 >= AT ? AT : static_cast<unsigned>(((head_dim / 2 + 63) / 64) * 64);
  for (int64_t s0 = 0; s0 < rows; s0 += AMAXB) {
    const int32_t c = rows - s0 < AMAXB ? static_cast<int32_t>(rows - s0) : AMAXB;
    RotaryArgs r{};
    r.qkv = static_cast<const char*>(qkv) + s0 * qkv_stride * esz;
    r.qkv_stride = qkv_stride;
    r.q = static_cast<char*>(q) + s0 * heads * head_dim * esz;
    r.k = static_cast<char*>(k) + s0 * kv_heads * head_dim * esz;
    r.v = static_cast<char*>(v) + s0 * kv_heads * head_dim * esz;
    r.positions = positions + s0;
    r.heads = heads;
    r.kv_heads = kv_heads;
    r.D = head_dim;
    r.theta = theta;
    AppendArgs a{};
    a.pool = static_cast<char*>(pool);
    a.P = page_size;
    a.row_bytes = kv_heads * head_dim * esz;
    for (int32_t i = 0; i < c; ++i) {
      a.dev_row[i] = device_rows[s0 + i];
      a.host_row[i] = host_rows ? host_rows[s0 + i] : -1;
      a.host[i] = host_alias ? static_cast<char*>(const_cast<void*>(host_alias[s0 + i])) : nullptr;
      a.kmin[i] = static_cast<char*>(minimum[s0 + i]);
      a.kmax[i] = static_cast<char*>(maximum[s0 + i]);
    }
    const dim3 grid(static_cast<unsigned>(heads + 2 * kv_heads), static_cast<unsigned>(c));
    if (dtype == HS_DTYPE_BF16) hipLaunchKernelGGL(rotary_append_kernel<HS_DTYPE_BF16>, grid, dim3(threads), 0, stream, r, a);
    else if (dtype == HS_DTYPE_F16) hipLaunchKernelGGL(rotary_append_kernel<HS_DTYPE_F16>, grid, dim3(threads), 0, stream, r, a);
    else hipLaunchKernelGGL(rotary_append_kernel<HS_DTYPE_F32>, grid, dim3(threads), 0, stream, r, a);
    HS_CHECK_LAUNCH("rotary_split_append");
  }
  return HS_OK;
}

// ---- batched write of T tokens to one (request, layer) --------------------------
//
// Replaces the page loop of HostStore.append (storage.py:273-318) for a write
// whose page placement the caller has decided: token rows go to their page's
// device block (when the page is resident) and to its host slot (the mirror);
// each page's bounds fold its new K rows in order with the rule above; each
// page's mean-K summary is recomputed over all its valid rows (rows written
// by earlier writes are read back from the device block when resident, else
// from the host slot), summed in row order in float32 and divided.  One
// workgroup per page.

namespace hs {

constexpr int TMAXP = 64;

struct TokenAppendArgs {
  const char* k;
  const char* v;
  int64_t kv_sb;  // bytes between token rows of k and v
  char* pool;
  char* host;
  char* kmin;  // bounds of the (request, layer): [pages, Hkv, D] in the KV dtype
  char* kmax;
  float* summ;  // nullable [pages, Hkv, D] float32
  int64_t P, row_bytes, n_elem, esz;
  int64_t first_page, first_within, tokens;
  int32_t slot[TMAXP], hslot[TMAXP];
};

template <int DT>
__device__ __forceinline__ bool takes_new_min(float old, float x) {
  if (old != old) return false;
  if (x != x) return true;
  if constexpr (DT == HS_DTYPE_F32) return x < old || (x == 0.f && old == 0.f && signbit(x) && !signbit(old));
  else return !(old < x);
}
template <int DT>
__device__ __forceinline__ bool takes_new_max(float old, float x) {
  if (old != old) return false;
  if (x != x) return true;
  if constexpr (DT == HS_DTYPE_F32) return x > old || (x == 0.f && old == 0.f && !signbit(x) && signbit(old));
  else return !(old > x);
}

template <int DT, int U>
__global__ __launch_bounds__(AT) void append_tokens_kernel(TokenAppendArgs a) {
  typedef typename std::conditional<U == 16, u32x4, unsigned short>::type T;
  const int j = blockIdx.x;
  const int64_t page = a.first_page + j;
  const int64_t within = j == 0 ? a.first_within : 0;
  const int64_t t0 = j == 0 ? 0 : (a.P - a.first_within) + static_cast<int64_t>(j - 1) * a.P;
  const int64_t room = a.P - within, left = a.tokens - t0;
  const int64_t count = room < left ? room : left;
  const int64_t slot = a.slot[j], hslot = a.hslot[j];
  const int64_t plane = a.P * a.row_bytes;
  // rows: K and V of every new token, to the device block (if resident) and the host slot
  const int64_t units = a.row_bytes / U;
  for (int64_t w = threadIdx.x; w < count * units; w += AT) {
    const int64_t r = w / units, u = w - r * units;
    const T kx = *reinterpret_cast<const T*>(a.k + (t0 + r) * a.kv_sb + u * U);
    const T vx = *reinterpret_cast<const T*>(a.v + (t0 + r) * a.kv_sb + u * U);
    const int64_t in_page = (within + r) * a.row_bytes + u * U;
    if (slot >= 0) {
      char* d = a.pool + slot * 2 * plane + in_page;
      *reinterpret_cast<T*>(d) = kx;
      *reinterpret_cast<T*>(d + plane) = vx;
    }
    char* h = a.host + hslot * 2 * plane + in_page;
    *reinterpret_cast<T*>(h) = kx;
    *reinterpret_cast<T*>(h + plane) = vx;
  }
  // bounds and summary, one (kv head, channel) element per thread
  const char* old_rows = slot >= 0 ? a.pool + slot * 2 * plane : a.host + hslot * 2 * plane;
  for (int64_t e = threadIdx.x; e < a.n_elem; e += AT) {
    const int64_t at = page * a.n_elem + e;
    float lo = load_elem<DT>(a.kmin, at), hi = load_elem<DT>(a.kmax, at);
    bool lo_new = false, hi_new = false;
    float acc = 0.f;
    for (int64_t r = 0; r < within; ++r) acc += load_elem<DT>(old_rows, r * a.n_elem + e);
    for (int64_t r = 0; r < count; ++r) {
      const float x = load_elem<DT>(a.k + (t0 + r) * a.kv_sb, e);
      if (takes_new_min<DT>(lo, x)) lo = x, lo_new = true;
      if (takes_new_max<DT>(hi, x)) hi = x, hi_new = true;
      acc += x;
    }
    // a bound is rewritten only when it changed: an unchanged one keeps its exact bits
    if (lo_new) store_elem<DT>(a.kmin, at, lo);
    if (hi_new) store_elem<DT>(a.kmax, at, hi);
    if (a.summ) a.summ[at] = acc / static_cast<float>(within + count);
  }
}

}  // namespace hs

extern "C" int hs_append_tokens(const void* k, const void* v, int64_t kv_stride_t, int64_t tokens, void* pool,
                                int64_t pool_rows, const void* host_alias, int64_t host_pool_rows, int32_t dtype,
                                int64_t page_size, int64_t kv_heads, int64_t head_dim, int64_t first_page,
                                int64_t first_within, int64_t pages, const int64_t* slots,
                                const int64_t* host_slots, void* minimum, void* maximum, float* summaries,
                                int64_t bound_pages, hipStream_t stream) {
  HS_CHECK_ARG(valid_dtype(dtype), "invalid dtype code %d", dtype);
  HS_CHECK_ARG(k && v && pool && host_alias && slots && host_slots && minimum && maximum, "null append pointer");
  HS_CHECK_ARG(page_size >= 1 && kv_heads >= 1 && head_dim >= 1 && tokens >= 1, "invalid append shape");
  HS_CHECK_ARG(first_within >= 0 && first_within < page_size, "first row must lie inside its page");
  HS_CHECK_ARG(pages == (first_within + tokens + page_size - 1) / page_size,
               "%lld pages cannot hold %lld tokens from row %lld", static_cast<long long>(pages),
               static_cast<long long>(tokens), static_cast<long long>(first_within));
  HS_CHECK_ARG(first_page >= 0 && first_page + pages <= bound_pages, "pages outside the bounds tensor");
  const int64_t pool_blocks = pool_rows / page_size, host_blocks = host_pool_rows / page_size;
  for (int64_t p = 0; p < pages; ++p) {  // every page, before the first launch
    HS_CHECK_ARG(slots[p] >= -1 && slots[p] < pool_blocks, "append block %lld outside the pool",
                 static_cast<long long>(slots[p]));
    HS_CHECK_ARG(host_slots[p] >= 0 && host_slots[p] < host_blocks, "append host slot %lld outside the host pool",
                 static_cast<long long>(host_slots[p]));
  }
  const int64_t esz = elem_bytes(dtype);
  TokenAppendArgs a{};
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.kv_sb = kv_stride_t * esz;
  a.pool = static_cast<char*>(pool);
  a.host = static_cast<char*>(const_cast<void*>(host_alias));
  a.kmin = static_cast<char*>(minimum);
  a.kmax = static_cast<char*>(maximum);
  a.summ = summaries;
  a.P = page_size;
  a.n_elem = kv_heads * head_dim;
  a.esz = esz;
  a.row_bytes = a.n_elem * esz;
  const uintptr_t align = reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                          reinterpret_cast<uintptr_t>(pool) | reinterpret_cast<uintptr_t>(host_alias) |
                          static_cast<uintptr_t>(a.kv_sb) | static_cast<uintptr_t>(a.row_bytes);
  const bool wide = (align & 15) == 0;
  int64_t token = 0;
  for (int64_t p0 = 0; p0 < pages; p0 += TMAXP) {
    const int64_t n = pages - p0 < TMAXP ? pages - p0 : TMAXP;
    const int64_t within = p0 == 0 ? first_within : 0;
    a.first_page = first_page + p0;
    a.first_within = within;
    const int64_t chunk_tokens = (within + tokens - token) < n * page_size ? tokens - token : n * page_size - within;
    a.tokens = chunk_tokens;
    a.k = static_cast<const char*>(k) + token * a.kv_sb;
    a.v = static_cast<const char*>(v) + token * a.kv_sb;
    for (int64_t i = 0; i < n; ++i) {
      a.slot[i] = static_cast<int32_t>(slots[p0 + i]);
      a.hslot[i] = static_cast<int32_t>(host_slots[p0 + i]);
    }
    const dim3 grid(static_cast<unsigned>(n));
    if (dtype == HS_DTYPE_BF16) {
      if (wide) hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_BF16, 16>), grid, dim3(AT), 0, stream, a);
      else hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_BF16, 2>), grid, dim3(AT), 0, stream, a);
    } else if (dtype == HS_DTYPE_F16) {
      if (wide) hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_F16, 16>), grid, dim3(AT), 0, stream, a);
      else hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_F16, 2>), grid, dim3(AT), 0, stream, a);
    } else {
      if (wide) hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_F32, 16>), grid, dim3(AT), 0, stream, a);
      else hipLaunchKernelGGL((append_tokens_kernel<HS_DTYPE_F32, 2>), grid, dim3(AT), 0, stream, a);
    }
    HS_CHECK_LAUNCH("append tokens");
    token += chunk_tokens;
  }
  return HS_OK;
}
