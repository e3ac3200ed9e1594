// Pinned-host -> hot-row gather for gfx950.
//
// Replaces the Triton `_gather` / `gather_rows` of mini_hisparse
// (row_kernels.py:35-70) and the CPU loop of hybrid.py:466-472: for each plan
// entry i with host row h >= 0 and device row r >= 0, copy the K plane row and
// the V plane row (Hkv * D elements each) of host row h into device row r.
// Both pools are [blocks, 2, P, Hkv, D]; the kernel reads the pinned host pool
// directly through its device alias, 16 bytes per lane, many rows in flight
// per workgroup.  It is a byte copy: the dtype only sets the row size.  A plan
// entry whose host row is past the host pool or whose device row is past the
// device pool is skipped like a -1 entry, so a corrupt plan cannot read or
// write outside the two allocations.
#include <stdlib.h>

#include "hs_common.h"

namespace hs {

constexpr int GT = 256;
constexpr int GMAXB = 16;

struct GatherArgs {
  const char* host[GMAXB];
  char* pool;
  const int64_t* hrows[GMAXB];
  const int64_t* drows[GMAXB];
  const int64_t* count[GMAXB];  // nullable: number of leading valid entries
  int64_t n[GMAXB];
  int64_t host_rows[GMAXB];     // rows of each plan's host pool
  int64_t pool_rows;            // rows of the device pool
  int64_t P, row_bytes;
};

template <int U>
struct Unit;
template <> struct Unit<16> { typedef u32x4 T; };
template <> struct Unit<8> { typedef unsigned long long T; };
template <> struct Unit<4> { typedef unsigned int T; };
template <> struct Unit<2> { typedef unsigned short T; };

// Each workgroup copies GUNROLL x `per` rows per iteration, every thread
// issuing its GUNROLL loads before the first store, so that a few workgroups
// keep enough host reads in flight for the link (and leave the other CUs to
// the compute stream); a row (K plane + V plane) is 2 * row_bytes / U units.
constexpr int GUNROLL = 4;
static_assert(GUNROLL % 2 == 0 && GT % 64 == 0, "gather: whole K/V load pairs and whole waves");

template <int U, bool NT>
__device__ __forceinline__ void store_unit(char* p, typename Unit<U>::T v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<typename Unit<U>::T*>(p));
  else *reinterpret_cast<typename Unit<U>::T*>(p) = v;
}

template <int U, bool NT>
__global__ __launch_bounds__(GT) void gather_kernel(GatherArgs a) {
  typedef typename Unit<U>::T T;
  const int64_t b = blockIdx.y;
  const int64_t units_plane = a.row_bytes / U;
  const int64_t units_row = 2 * units_plane;
  int64_t per = GT / units_row;
  if (per < 1) per = 1;
  int64_t n = a.n[b];
  if (a.count[b]) {
    const int64_t c = *a.count[b];
    if (c < n) n = c;
  }
  const int64_t plane_stride = a.P * a.row_bytes;  // bytes between K and V planes
  const uint32_t P32 = static_cast<uint32_t>(a.P);
  const char* host = a.host[b];
  const int64_t* hrows = a.hrows[b];
  const int64_t* drows = a.drows[b];
  const uint64_t hlimit = static_cast<uint64_t>(a.host_rows[b]);
  const uint64_t dlimit = static_cast<uint64_t>(a.pool_rows);
  if (units_plane < 64 && 64 % units_plane == 0) {
    // Rows shorter than a wave's 64 units: a wave instruction reads one plane
    // of 64 / units_plane consecutive plan entries.  The K rows of a missed
    // page's tokens lie next to each other in the host pool (and the V rows),
    // so short rows make one contiguous run per instruction instead of a K and
    // a V piece per row (256-byte rows: 0.66 -> 0.84 of the pinned memcpy rate
    // end to end).  Rows of 64 units or more keep the per-row mapping below,
    // whose instructions are already one row plane long.  Load k of a thread
    // reads plane k % 2 of row group k / 2; a workgroup iteration covers the
    // same rows as the per-row mapping below (GUNROLL / 2 groups of GT / 64
    // waves x rw rows).
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t rw = 64 / units_plane;
    const int64_t rsub = lane / units_plane;
    const int64_t unit_off = (lane - rsub * units_plane) * U;
    const int64_t span = (GT / 64) * rw;
    const int64_t rows_iter = (GUNROLL / 2) * span;
    for (int64_t first = static_cast<int64_t>(blockIdx.x) * rows_iter; first < n;
         first += static_cast<int64_t>(gridDim.x) * rows_iter) {
      T v[GUNROLL];
      int64_t dst[GUNROLL];
#pragma unroll
      for (int g = 0; g < GUNROLL / 2; ++g) {
        const int64_t i = first + g * span + wave * rw + rsub;
        dst[2 * g] = dst[2 * g + 1] = -1;
        if (i >= n) continue;
        const int64_t h = hrows[i];
        const int64_t r = drows[i];
        if (static_cast<uint64_t>(h) >= hlimit || static_cast<uint64_t>(r) >= dlimit) continue;
        const uint32_t hb = static_cast<uint32_t>(h) / P32, ho = static_cast<uint32_t>(h) - hb * P32;
        const uint32_t rb = static_cast<uint32_t>(r) / P32, ro = static_cast<uint32_t>(r) - rb * P32;
        const int64_t src = (static_cast<int64_t>(hb) * 2 * a.P + ho) * a.row_bytes + unit_off;
        const int64_t d0 = (static_cast<int64_t>(rb) * 2 * a.P + ro) * a.row_bytes + unit_off;
        dst[2 * g] = d0;
        dst[2 * g + 1] = d0 + plane_stride;
        v[2 * g] = *reinterpret_cast<const T*>(host + src);
        v[2 * g + 1] = *reinterpret_cast<const T*>(host + src + plane_stride);
      }
#pragma unroll
      for (int k = 0; k < GUNROLL; ++k)
        if (dst[k] >= 0) store_unit<U, NT>(a.pool + dst[k], v[k]);
    }
  } else if (units_row <= GT) {
    // fixed (row slot, unit) per thread
    const int64_t slot = threadIdx.x / units_row;
    const int64_t w = threadIdx.x - slot * units_row;
    const bool active = slot < per;
    const int64_t plane = w / units_plane;
    const int64_t inrow = plane * plane_stride + (w - plane * units_plane) * U;
    for (int64_t first = static_cast<int64_t>(blockIdx.x) * per * GUNROLL; first < n;
         first += static_cast<int64_t>(gridDim.x) * per * GUNROLL) {
      T v[GUNROLL];
      int64_t dst[GUNROLL];
#pragma unroll
      for (int k = 0; k < GUNROLL; ++k) {
        const int64_t i = first + k * per + slot;
        dst[k] = -1;
        if (!active || i >= n) continue;
        const int64_t h = hrows[i];
        const int64_t r = drows[i];
        // one unsigned compare rejects both -1 and rows past the pool
        if (static_cast<uint64_t>(h) >= hlimit || static_cast<uint64_t>(r) >= dlimit) continue;
        const uint32_t hb = static_cast<uint32_t>(h) / P32, ho = static_cast<uint32_t>(h) - hb * P32;
        const uint32_t rb = static_cast<uint32_t>(r) / P32, ro = static_cast<uint32_t>(r) - rb * P32;
        const int64_t src = (static_cast<int64_t>(hb) * 2 * a.P + ho) * a.row_bytes + inrow;
        dst[k] = (static_cast<int64_t>(rb) * 2 * a.P + ro) * a.row_bytes + inrow;
        v[k] = *reinterpret_cast<const T*>(host + src);
      }
#pragma unroll
      for (int k = 0; k < GUNROLL; ++k)
        if (dst[k] >= 0) store_unit<U, NT>(a.pool + dst[k], v[k]);
    }
  } else {
    // a row wider than the workgroup: one row per iteration, strided units
    for (int64_t i = blockIdx.x; i < n; i += gridDim.x) {
      const int64_t h = hrows[i];
      const int64_t r = drows[i];
      if (static_cast<uint64_t>(h) >= hlimit || static_cast<uint64_t>(r) >= dlimit) continue;
      const uint32_t hb = static_cast<uint32_t>(h) / P32, ho = static_cast<uint32_t>(h) - hb * P32;
      const uint32_t rb = static_cast<uint32_t>(r) / P32, ro = static_cast<uint32_t>(r) - rb * P32;
      const int64_t sbase = (static_cast<int64_t>(hb) * 2 * a.P + ho) * a.row_bytes;
      const int64_t dbase = (static_cast<int64_t>(rb) * 2 * a.P + ro) * a.row_bytes;
      for (int64_t w = threadIdx.x; w < units_row; w += GT) {
        const int64_t plane = w / units_plane;
        const int64_t inrow = plane * plane_stride + (w - plane * units_plane) * U;
        store_unit<U, NT>(a.pool + dbase + inrow, *reinterpret_cast<const T*>(host + sbase + inrow));
      }
    }
  }
}

}  // namespace hs

using namespace hs;

extern "C" int hs_host_alias(const void* host_ptr, void** device_ptr) {
  HS_CHECK_ARG(host_ptr != nullptr && device_ptr != nullptr, "null host alias argument");
  void* dev = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dev, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess || dev == nullptr) {
    (void)hipGetLastError();
    hs::set_error("cannot map pinned host allocation to the device: %s", hipGetErrorString(e));
    return HS_ERUNTIME;
  }
  *device_ptr = dev;
  return HS_OK;
}

// At most GMAXB plans (their pointers travel in the kernel arguments);
// hs_gather_rows_batched cuts larger batches into such chunks.
static int gather_chunk(const void* const* host_alias, void* pool, const int64_t* const* miss_host_rows,
                        const int64_t* const* miss_device_rows, const int64_t* const* miss_counts,
                        const int64_t* n, const int64_t* host_pool_rows, int64_t pool_rows, int32_t batch,
                        int64_t page_size, int64_t row_bytes, int32_t grid_x, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1 && batch <= GMAXB, "gather batch must be in [1, %d]", GMAXB);
  HS_CHECK_ARG(pool && host_alias && miss_host_rows && miss_device_rows && n && host_pool_rows,
               "null gather pointer");
  HS_CHECK_ARG(page_size >= 1 && row_bytes >= 2 && row_bytes % 2 == 0, "invalid gather row shape");
  HS_CHECK_ARG(pool_rows >= 0 && pool_rows % page_size == 0, "device pool rows must be whole pages");
  GatherArgs a{};
  a.pool = static_cast<char*>(pool);
  a.pool_rows = pool_rows;
  a.P = page_size;
  a.row_bytes = row_bytes;
  int64_t nmax = 0;
  uintptr_t align = reinterpret_cast<uintptr_t>(pool);
  for (int32_t i = 0; i < batch; ++i) {
    HS_CHECK_ARG(host_alias[i] && miss_host_rows[i] && miss_device_rows[i], "null gather plan");
    a.host[i] = static_cast<const char*>(host_alias[i]);
    a.hrows[i] = miss_host_rows[i];
    a.drows[i] = miss_device_rows[i];
    a.count[i] = miss_counts ? miss_counts[i] : nullptr;
    a.n[i] = n[i];
    HS_CHECK_ARG(host_pool_rows[i] >= 0 && host_pool_rows[i] % page_size == 0,
                 "host pool rows must be whole pages");
    a.host_rows[i] = host_pool_rows[i];
    if (n[i] > nmax) nmax = n[i];
    align |= reinterpret_cast<uintptr_t>(host_alias[i]);
  }
  if (nmax == 0) return HS_OK;
  const int64_t per_row = 2 * row_bytes;
  int unit = 2;
  if (row_bytes % 16 == 0 && (align & 15) == 0) unit = 16;
  else if (row_bytes % 8 == 0 && (align & 7) == 0) unit = 8;
  else if (row_bytes % 4 == 0 && (align & 3) == 0) unit = 4;
  int64_t rows_per_block = (GT * unit) / per_row;
  if (rows_per_block < 1) rows_per_block = 1;
  // About 512 workgroups per launch (each thread keeps GUNROLL reads in flight):
  // enough host reads in flight for the link (~10 us per read at saturation),
  // measured at 99% of the pinned memcpy rate; more only queue behind the link.
  static const int64_t forced_gx = [] {
    const char* env = getenv("HS_GATHER_GRID");
    return env ? atoll(env) : 0;
  }();
  int64_t gx = grid_x > 0 ? grid_x : (forced_gx > 0 ? forced_gx : (512 + batch - 1) / batch);
  const int64_t useful = (nmax + rows_per_block * GUNROLL - 1) / (rows_per_block * GUNROLL);
  if (gx > useful) gx = useful;
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(batch));
  // Non-temporal stores: the gathered rows stream to HBM instead of staying as
  // dirty lines that the attention's reads right after would have to write back
  // (measured: attention 60.9 vs 65.7 us in the microbench step, gather unchanged).
  // HS_GATHER_NT=0 keeps ordinary stores.
  static const bool nt = [] {
    const char* env = getenv("HS_GATHER_NT");
    return !(env && atoi(env) == 0);
  }();
  if (nt) {
    switch (unit) {
      case 16: hipLaunchKernelGGL((gather_kernel<16, true>), grid, dim3(GT), 0, stream, a); break;
      case 8: hipLaunchKernelGGL((gather_kernel<8, true>), grid, dim3(GT), 0, stream, a); break;
      case 4: hipLaunchKernelGGL((gather_kernel<4, true>), grid, dim3(GT), 0, stream, a); break;
      default: hipLaunchKernelGGL((gather_kernel<2, true>), grid, dim3(GT), 0, stream, a); break;
    }
  } else {
    switch (unit) {
      case 16: hipLaunchKernelGGL((gather_kernel<16, false>), grid, dim3(GT), 0, stream, a); break;
      case 8: hipLaunchKernelGGL((gather_kernel<8, false>), grid, dim3(GT), 0, stream, a); break;
      case 4: hipLaunchKernelGGL((gather_kernel<4, false>), grid, dim3(GT), 0, stream, a); break;
      default: hipLaunchKernelGGL((gather_kernel<2, false>), grid, dim3(GT), 0, stream, a); break;
    }
  }
  HS_CHECK_LAUNCH("gather");
  return HS_OK;
}

extern "C" int hs_gather_rows_batched(const void* const* host_alias, void* pool,
                                      const int64_t* const* miss_host_rows,
                                      const int64_t* const* miss_device_rows,
                                      const int64_t* const* miss_counts, const int64_t* n,
                                      const int64_t* host_pool_rows, int64_t pool_rows,
                                      int32_t batch, int64_t page_size, int64_t row_bytes,
                                      int32_t grid_x, hipStream_t stream) {
  HS_CHECK_ARG(batch >= 1, "gather batch must be positive");
  HS_CHECK_ARG(host_alias && miss_host_rows && miss_device_rows && n && host_pool_rows,
               "null gather pointer");
  HS_CHECK_ARG(page_size >= 1, "invalid gather page size");
  HS_CHECK_ARG(pool_rows >= 0 && pool_rows % page_size == 0, "device pool rows must be whole pages");
  for (int32_t i = 0; i < batch; ++i) {  // every plan, before the first launch
    HS_CHECK_ARG(host_alias[i] && miss_host_rows[i] && miss_device_rows[i], "null gather plan");
    HS_CHECK_ARG(host_pool_rows[i] >= 0 && host_pool_rows[i] % page_size == 0,
                 "host pool rows must be whole pages");
  }
  for (int32_t s0 = 0; s0 < batch; s0 += GMAXB) {
    const int32_t c = batch - s0 < GMAXB ? batch - s0 : GMAXB;
    const int rc = gather_chunk(host_alias + s0, pool, miss_host_rows + s0, miss_device_rows + s0,
                                miss_counts ? miss_counts + s0 : nullptr, n + s0, host_pool_rows + s0,
                                pool_rows, c, page_size, row_bytes, grid_x, stream);
    if (rc != HS_OK) return rc;
  }
  return HS_OK;
}

extern "C" int hs_gather_rows(const void* host_alias, void* pool, const int64_t* miss_host_rows,
                              const int64_t* miss_device_rows, int64_t n, const int64_t* miss_count,
                              int64_t host_pool_rows, int64_t pool_rows, int64_t page_size,
                              int64_t row_bytes, hipStream_t stream) {
  const int64_t* counts[1] = {miss_count};
  return hs_gather_rows_batched(&host_alias, pool, &miss_host_rows, &miss_device_rows,
                                miss_count ? counts : nullptr, &n, &host_pool_rows, pool_rows, 1,
                                page_size, row_bytes, 0, stream);
}
