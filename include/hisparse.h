/*
 * hisparse.h -- C ABI of the gfx950 kernels behind mini-hisparse's per-step
 * sparse decode path (libhisparse_hip.so).
 *
 * The reference (mini-hisparse 0.2.0) has no native code and no FFI: its
 * swappable points are Python functions.  Each entry point below replaces one
 * of them; the comment names the reference function (file:line under the
 * reference checkout) whose semantics it implements.
 *
 * Conventions
 *  - All pointers are device pointers unless stated otherwise; all buffers are
 *    caller-owned; nothing is allocated persistently by the library.
 *  - Scratch memory is a caller-provided workspace sized by the matching
 *    hs_*_workspace_bytes query.
 *  - `stream` is a hipStream_t (NULL = the default stream).  Every call only
 *    enqueues work; none synchronises the host.
 *  - Return value: HS_OK (0) or a negative status; hs_last_error() gives the
 *    message of the calling thread's last failure.
 *  - Device-side invalid indices (-1, out of range) are masked, not errors,
 *    as in the reference (row_index.py:67-68, row_index.py:103).
 */
#ifndef HISPARSE_H
#define HISPARSE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; everything declared here is its
 * exported API. */
#pragma GCC visibility push(default)

#define HS_VERSION 1

#define HS_OK 0
#define HS_EINVAL (-1)
#define HS_ELAUNCH (-2)
#define HS_EWORKSPACE (-3)
#define HS_ERUNTIME (-4)

/* KV / query element types (CacheConfig.dtype, config.py:19, :27-28) */
#define HS_DTYPE_F32 0
#define HS_DTYPE_F16 1
#define HS_DTYPE_BF16 2

typedef struct ihipStream_t* hs_stream_t;

/* Message of the calling thread's last failed call ("" if none). */
const char* hs_last_error(void);

/* HS_VERSION of the loaded library. */
int hs_version(void);

/* LDS bytes available to one workgroup on `device` (diagnostic). */
int hs_device_lds_bytes(int device, int64_t* bytes);

/*
 * Exact-size pinned host allocation for a caller-owned host pool (freed with
 * hs_host_free).  No counterpart in the reference, which pins its host pool
 * with torch (storage.py:112-114); PyTorch's pinned allocator rounds every
 * request up to a power of two, which halves the usable pinned memory for
 * pools just above one.  `host_ptr` receives a host pointer.
 */
int hs_host_alloc(int64_t bytes, void** host_ptr);
int hs_host_free(void* host_ptr);

/*
 * Device alias of a pinned host allocation owned by the caller (never
 * registered or unregistered here).
 * Replaces: MappedHost (mini_hisparse/row_kernels.py:10-32), called from
 * HybridKVCache.__init__ (hybrid.py:129-132).  `host_ptr` is a host pointer.
 */
int hs_host_alias(const void* host_ptr, void** device_ptr);

/* ---------------------------------------------------------------- (1) Quest */

/* Bytes of scratch hs_quest_topk needs for `batch` requests of up to `max_pages`. */
int64_t hs_quest_workspace_bytes(int64_t batch, int64_t heads, int64_t max_pages);

/*
 * Quest page scores and per-head top-k for `batch` requests (launched in
 * chunks of at most 16, in order on `stream`).
 * Replaces: quest_selection (mini_hisparse/selection.py:80-101) up to the
 * chosen page ids (:100).
 *   query      [batch, heads, head_dim] in query_dtype (HS_DTYPE_*: the model
 *              dtype; widened to float32 exactly, as the reference's .float())
 *   minimum[b], maximum[b]  per request [pages, kv_heads, head_dim] bounds in
 *              kv_dtype (RequestPages.minimum/maximum[layer], storage.py:193-206)
 *   page_counts host array [batch]: ceil(length / page_size)
 *   out_pages  [batch, heads, top] int32: the min(top, count) chosen pages of
 *              each head, ascending; all pages when top >= count (:90-91);
 *              the tail page and, if keep_sink && top > 1 && count > 1, page 0
 *              are always chosen (:96-99).  Scores are float32 sums over the
 *              channels in ascending order; ties go to the lower page.
 * `minimum`, `maximum` and `page_counts` are host arrays of device pointers / sizes.
 */
int hs_quest_topk(const void* query, int64_t q_stride_b, int64_t q_stride_h,
                  int32_t query_dtype, const void* const* minimum, const void* const* maximum,
                  int32_t kv_dtype, const int64_t* page_counts, int64_t batch, int64_t heads,
                  int64_t kv_heads, int64_t head_dim, int64_t top, int32_t keep_sink,
                  int32_t* out_pages, int64_t out_stride_b, void* workspace,
                  int64_t workspace_bytes, hs_stream_t stream);

/*
 * Uniformly resampled page selections (BASELINE configs[4]'s miss-heavy stress
 * selector; no counterpart in the reference, whose selections come from Quest or
 * the caller): for each (layer, request), the tail page count - 1 and top - 1 other
 * pages drawn uniformly without replacement from [0, count - 1) (Floyd's
 * algorithm over a counter-based splitmix64 generator of seed, step, layer,
 * request), written ascending to every head's row of out [layers, batch, heads,
 * top] int32, then -1; a request of at most `top` pages selects all of them.  The
 * same (seed, step) always draws the same pages.  page_counts host [batch], each
 * 1 to 65536.  The rows are hs_build_union's `pages`.
 */
int hs_uniform_pages(uint64_t seed, uint64_t step, const int64_t* page_counts, int64_t batch, int64_t layers,
                     int64_t top, int64_t heads, int32_t* out, hs_stream_t stream);

/*
 * Device-side Selection -> LogicalTopK adapter for page selections.
 * Replaces: Selection.from_pages (selection.py:43-60) followed by
 * LogicalTopK.from_selection (row_index.py:20-31), without the host sync of
 * selection.py:100.
 *   pages         [batch, heads, top] from hs_quest_topk; lengths host [batch]
 *   positions     [batch, pos_capacity] int32: ascending union of the
 *                 selected tokens, then -1
 *   head_columns  [batch, heads, width] int64: union column of each head's
 *                 tokens in ascending token order, then -1
 *   union_count   [batch] int32: union size n
 *   entry_*       per (request, kv head) the deduplicated union columns read
 *                 by any query head of the group, ascending, with the bit mask
 *                 of those heads: [batch, kv_heads, entry_capacity], counts
 *                 [batch, kv_heads]
 *   status        int32 flag OR-ed with 1 (union over capacity) / 2 (entries
 *                 over capacity); the caller clears it.
 *   page_bits     nullable [batch, page_bits_stride] uint32: bit p of request b
 *                 set iff page p is in the union (page_bits_stride >= the
 *                 words of ceil(length / page_size) bits); the positions are
 *                 then exactly the tokens below length of the marked pages,
 *                 unless the union overflowed (status bit 1).  No counterpart
 *                 in the reference: it lets the resolver skip reading the
 *                 positions (hs_resolve_desc.page_bits).
 *   entry_stats   nullable int64 [1]: the (clamped) entry counts of the call are
 *                 added here on the device, so a caller can total the entries its
 *                 attention reads over many steps without a copy per call (the
 *                 attention's algorithmic bytes).  No counterpart in the reference.
 * Any batch size: launched in chunks of at most 16 requests, in order on `stream`.
 */
int hs_build_union(const int32_t* pages, int64_t p_stride_b, int64_t top, const int64_t* lengths,
                   int64_t page_size, int64_t batch, int64_t heads, int64_t kv_heads,
                   int32_t* positions, int64_t pos_capacity, int64_t* head_columns, int64_t width,
                   int32_t* union_count, int32_t* entry_columns, uint32_t* entry_masks,
                   int64_t entry_capacity, int32_t* entry_counts, int32_t* status,
                   uint32_t* page_bits, int64_t page_bits_stride, int64_t* entry_stats,
                   hs_stream_t stream);

/* ------------------------------------------------------------- (2) resolver */

/*
 * One (request, layer) resolve: the tables of LayerTables (hybrid.py:45-64)
 * and the outputs of RowPlan (row_index.py:51-56).
 */
typedef struct hs_resolve_desc {
  const void* positions;        /* [n] logical tokens, int32 or int64 */
  int64_t n;
  int32_t positions_i64;        /* 1 = int64 positions, 0 = int32 */
  int32_t lru_i16;              /* 1 = lru holds int16 slots, 0 = int64 (the reference's dtype) */
  const uint32_t* page_bits;    /* nullable: the union page bitmap of hs_build_union that produced
                                   `positions`; its valid entries are then exactly the tokens below
                                   length of the marked pages, and the resolver reads the bitmap
                                   instead of the positions to find the selected tokens */
  const int64_t* head_columns;  /* nullable [heads, width] union columns, -1 padded */
  int64_t heads, width, hc_stride_h, hc_stride_w;
  const int32_t* source;        /* [n_pages] host page of each logical page, -1 = none */
  const int32_t* resident;      /* [n_pages] device block of a resident page, -1 = none */
  int64_t n_pages;
  const int32_t* hot;           /* [hot_blocks] device block of each hot block */
  int64_t hot_blocks;
  int32_t* tags;                /* [hot_rows] in/out: host row held by each hot slot, -1 = empty */
  void* lru;                    /* [hot_rows] in/out: slots, least recent first */
  int64_t hot_rows;             /* <= 32768 (hybrid.py:34) */
  int64_t length, page_size;    /* length <= n_pages * page_size */
  int64_t* physical;            /* out [n], or [heads, width] contiguous when head_columns */
  int64_t* union_physical;      /* out, nullable: [n] physical rows in input order */
  int64_t* miss_host_rows;      /* out [n]: host rows to load, compact prefix, then -1 */
  int64_t* miss_device_rows;    /* out [n]: matching device rows */
  int64_t* counts;              /* out [3]: resident hits, hot hits, misses */
  int64_t* row_stats;           /* nullable [3]: counts are added here (hybrid.py:454) */
  void* workspace;              /* set by the library from the call's workspace */
  int32_t miss_prefix_only;     /* 1 = write the miss plan's compact prefix only (entries
                                   [0, counts[2])), not its -1 tail: for a caller whose gather
                                   stops at the miss count; 0 = the whole RowPlan */
  int32_t split_front;          /* 1 = the front's work may go over several workgroups per request
                                   (three launches instead of one; taken for hot regions above 16384
                                   rows or histories above 40000 tokens, where it measured faster;
                                   HS_RESOLVE_SPLIT=0/1 forces it off/on):
                                   needs page_bits, a power-of-two page_size <= 32 and a source table
                                   affine with base source[0] (host block = source[0] + page for every
                                   host-backed page, as a request's contiguous host slots are); a
                                   table that is not is refused on the device: no row (-1), counts 0.
                                   Every descriptor of a call shares it.  0 = one workgroup per
                                   request */
} hs_resolve_desc;

/* Scratch bytes for one descriptor (sum them for a batch). */
int64_t hs_resolve_workspace_bytes(int64_t n, int64_t length, int64_t n_pages, int64_t hot_rows);

/*
 * Resolve logical tokens to physical rows, mutating tags/lru in place.
 * Replaces: resolve_rows (mini_hisparse/row_index.py:59-137); bit-exact on
 * every output including the updated tags and LRU.  `desc` is a host pointer.
 */
int hs_resolve_rows(const hs_resolve_desc* desc, void* workspace, int64_t workspace_bytes,
                    hs_stream_t stream);

/* The same over `count` independent (request, layer) descriptors (host array). */
int hs_resolve_rows_batched(const hs_resolve_desc* descs, int32_t count, void* workspace,
                            int64_t workspace_bytes, hs_stream_t stream);

/*
 * hs_resolve_rows_batched without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The scratch
 * is a fixed device array inside the library, one per GPU, held until the
 * process ends; a batch whose hs_resolve_workspace_bytes sum exceeds
 * hs_resolve_noalloc_max_bytes() (32 MiB: 16 descriptors of the Qwen2.5-7B
 * shape at 128k tokens) is rejected with HS_EINVAL.  Nothing is allocated and
 * the outputs are those of hs_resolve_rows_batched.  Calls that overlap on one
 * GPU (other streams or threads) share the array and race: serialise them.
 * The first call on a device looks the array's address up (hipGetSymbolAddress),
 * so a caller that captures the call into a HIP graph makes one uncaptured call
 * on that device first; captured replays then run the same kernels.
 */
int64_t hs_resolve_noalloc_max_bytes(void);
int hs_resolve_rows_noalloc(const hs_resolve_desc* descs, int32_t count, hs_stream_t stream);

/* --------------------------------------------------------------- (3) gather */

/*
 * Copy the K and V planes of each planned host row into its hot device row.
 * Replaces: gather_rows (mini_hisparse/row_kernels.py:35-70) and the CPU loop
 * of HybridKVCache.resolve (hybrid.py:466-472).
 *   host_alias  device alias of the pinned host pool [host_pages, 2, P, Hkv, D]
 *   pool        device pool [gpu_pages, 2, P, Hkv, D]
 *   miss_*_rows [n] int64 plan from the resolver; entries < 0 are skipped
 *   miss_count  nullable device int64: only the first *miss_count entries are read
 *   host_pool_rows  host_pages * P; pool_rows  gpu_pages * P: an entry whose host
 *               row or device row is at or past its pool's rows is skipped like a
 *               -1 entry (the reference masks only -1, row_kernels.py:50-55)
 *   row_bytes   Hkv * D * element size
 */
int hs_gather_rows(const void* host_alias, void* pool, const int64_t* miss_host_rows,
                   const int64_t* miss_device_rows, int64_t n, const int64_t* miss_count,
                   int64_t host_pool_rows, int64_t pool_rows, int64_t page_size,
                   int64_t row_bytes, hs_stream_t stream);

/* The same for `batch` plans, one launch per chunk of at most 16; every array
 * argument is a host array of per-request values (host_pool_rows included: each
 * plan may read its own host pool); grid_x (workgroups per plan) <= 0 picks the
 * default grid. */
int hs_gather_rows_batched(const void* const* host_alias, void* pool,
                           const int64_t* const* miss_host_rows,
                           const int64_t* const* miss_device_rows,
                           const int64_t* const* miss_counts, const int64_t* n,
                           const int64_t* host_pool_rows, int64_t pool_rows, int32_t batch,
                           int64_t page_size, int64_t row_bytes, int32_t grid_x,
                           hs_stream_t stream);

/* ------------------------------------------------------- append (producer) */

/*
 * Append one token's K and V rows for each of `batch` (request, layer)
 * pairs: the decode-step producer of the Quest bounds.
 * Replaces: the single-token case of HostStore.append
 * (mini_hisparse/storage.py:246-319): the new rows go to their pool row; the
 * tail page's minimum/maximum [kv_heads, head_dim] take the element-wise
 * min/max with the new K row exactly as torch.minimum/torch.maximum compute
 * it on the device (a NaN operand is returned, the existing bound first;
 * 16-bit types: old < new ? old : new, so equal zeros give the new one;
 * float32: -0 below +0); the rows are mirrored into the pinned host pool through
 * its device alias (the reference queues a device-to-host copy).  The page
 * mean-K summary (selector "mean" only) is not produced here.
 *   k, v          [batch, kv_heads, head_dim], pool dtype, kv_stride_b elements between pairs
 *   pool          [gpu_pages, 2, P, Hkv, D]; pool_rows = gpu_pages * P
 *   device_rows   host array [batch]: pool row (block * P + offset) of the new token
 *   host_alias    host array [batch] of device aliases of pinned host pools (nullable
 *                 when host_rows is NULL); host_rows host array [batch], < 0 skips the
 *                 mirror; host_pool_rows bounds every host row
 *   minimum, maximum  host arrays [batch] of device pointers to the tail page's bounds
 * Any batch size: launched in chunks of at most 32 pairs, in order on `stream`.
 */
int hs_append_rows(const void* k, const void* v, int64_t kv_stride_b, void* pool, int64_t pool_rows,
                   int32_t dtype, int64_t page_size, int64_t kv_heads, int64_t head_dim,
                   const int64_t* device_rows, const void* const* host_alias, const int64_t* host_rows,
                   int64_t host_pool_rows, void* const* minimum, void* const* maximum, int32_t batch,
                   hs_stream_t stream);

/*
 * hs_rotary_split (below) and hs_append_rows in one launch: the decode step's
 * rotary embedding of the q|k|v projection output and the append of the rotated
 * K row and the V row of each of `rows` (request, layer) pairs to its pool row, its
 * host mirror row and its tail page's bounds.  Replaces the same reference steps as
 * the two calls it fuses (model.py:183-226's rotary; storage.py:246-319's single-token
 * append); every output holds the bits the two calls give.  Arguments: those of
 * hs_rotary_split, then those of hs_append_rows for the same rows (k and v are the
 * rotary's outputs, so no k/v source is passed).
 */
int hs_rotary_split_append(const void* qkv, int64_t qkv_stride, void* q, void* k, void* v,
                           const int64_t* positions, int64_t rows, int64_t heads, int64_t kv_heads,
                           int64_t head_dim, float theta, int32_t dtype, void* pool, int64_t pool_rows,
                           int64_t page_size, const int64_t* device_rows, const void* const* host_alias,
                           const int64_t* host_rows, int64_t host_pool_rows, void* const* minimum,
                           void* const* maximum, hs_stream_t stream);

/*
 * A write of `tokens` consecutive K/V rows to one (request, layer) whose page
 * placement the caller has decided: the page loop of HostStore.append
 * (mini_hisparse/storage.py:273-318) -- prefill or decode -- in one launch per 64
 * pages.
 *   k, v        [tokens, kv_heads, head_dim] in the pool dtype, kv_stride_t elements
 *               between token rows
 *   first_page / first_within  logical page and row of the first token; the write
 *               covers `pages` = ceil((first_within + tokens) / page_size) pages
 *   slots       host array [pages]: device block of each page, -1 = not resident
 *               (rows go to the host mirror only); host_slots host array [pages]
 *   minimum, maximum  the (request, layer)'s bounds [bound_pages, kv_heads, head_dim]
 *               in the pool dtype: each page folds its new K rows in order with the
 *               rule of hs_append_rows
 *   summaries   nullable [bound_pages, kv_heads, head_dim] float32: the mean K of all
 *               the page's valid rows (earlier rows read back from its device block,
 *               or from its host slot when not resident), summed in row order
 * Every block and host slot is checked against the pools before the first launch.
 */
int hs_append_tokens(const void* k, const void* v, int64_t kv_stride_t, int64_t tokens, void* pool,
                     int64_t pool_rows, const void* host_alias, int64_t host_pool_rows, int32_t dtype,
                     int64_t page_size, int64_t kv_heads, int64_t head_dim, int64_t first_page,
                     int64_t first_within, int64_t pages, const int64_t* slots, const int64_t* host_slots,
                     void* minimum, void* maximum, float* summaries, int64_t bound_pages,
                     hs_stream_t stream);

/* ------------------------------------------------------------ (4) attention */

/*
 * Scratch bytes of one attention call: split-K partials and, for the MFMA kernel's
 * in-kernel merge, one arrival counter per (request, KV head, head chunk).  The
 * workspace may hold anything before a call (counters carry a per-launch tag; a
 * value with another tag counts as empty) and calls that share it must run in
 * order (one stream).
 */
int64_t hs_attend_workspace_bytes(int32_t dtype, int64_t batch, int64_t heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t max_entries);

/*
 * Physical-row GQA decode attention over per-head row lists.
 * Replaces: attend_rows (mini_hisparse/row_kernels.py:73-135) and the torch
 * branch of row_attention (attention.py:26-35).
 *   query [batch, heads, head_dim] (strides in elements, head_dim contiguous)
 *   rows  [batch, heads, width] int64 physical rows, -1 masked; r_stride_h == 0
 *         means one list shared by every head (attention.py:19-21)
 *   pool_rows  blocks * page_size of the pool; rows >= pool_rows are masked
 *   out   [batch, heads, head_dim] in the pool dtype; 0 for a head with no row
 *   max_entries for the workspace query: width (shared) or width * heads / kv_heads
 */
int hs_attend_rows(const void* query, int64_t q_stride_b, int64_t q_stride_h, const void* pool,
                   int32_t dtype, int64_t page_size, int64_t kv_heads, int64_t head_dim,
                   int64_t pool_rows, const int64_t* rows, int64_t r_stride_b, int64_t r_stride_h,
                   int64_t r_stride_w, int64_t width, int64_t batch, int64_t heads, void* out,
                   int64_t o_stride_b, int64_t o_stride_h, void* workspace,
                   int64_t workspace_bytes, hs_stream_t stream);

/*
 * The same attention reading each KV head's deduplicated row set once: the
 * entry lists of hs_build_union, with physical rows taken from the
 * resolver's union_physical [batch, n].  Same result as hs_attend_rows over
 * the per-head rows physical[h, j] = union_physical[head_columns[h, j]].
 */
int hs_attend_groups(const void* query, int64_t q_stride_b, int64_t q_stride_h, const void* pool,
                     int32_t dtype, int64_t page_size, int64_t kv_heads, int64_t head_dim,
                     int64_t pool_rows, const int64_t* union_physical, int64_t u_stride_b,
                     const int32_t* entry_columns, const uint32_t* entry_masks,
                     int64_t e_stride_b, int64_t e_stride_k, const int32_t* entry_counts,
                     int64_t max_entries, int64_t batch, int64_t heads, void* out,
                     int64_t o_stride_b, int64_t o_stride_h, void* workspace,
                     int64_t workspace_bytes, hs_stream_t stream);

/*
 * Page-window attention of the paged cache: replaces the Triton
 * `_attention_window` / `triton_chunk` of the reference's optional page layout
 * (reference/kernels.py:12-97), called per window by `paged_attention`
 * (reference/attention.py:42-128).  One request; page i of the window sits in
 * device slot slots[i] of the [blocks, 2, P, Hkv, D] pool with lengths[i]
 * valid tokens; mask (null = every valid token) is a [heads, n_pages, P] byte
 * array, nonzero where the head reads the token.  Writes the unnormalised fp32
 * state per query head: out_m[h] = max score (-inf when the head reads no
 * token), out_l[h] = sum exp(s - m), out_acc[h, :] = sum exp(s - m) V, with
 * s = (K . q) * head_dim^-0.5, for the caller to merge windows.  Workspace:
 * hs_attend_workspace_bytes(dtype, 1, heads, kv_heads, head_dim, n_pages * P).
 */
int hs_attend_window(const void* query, int64_t q_stride_h, const void* pool, int32_t dtype,
                     int64_t page_size, int64_t kv_heads, int64_t head_dim, int64_t pool_rows,
                     const int32_t* slots, const int32_t* lengths, int64_t n_pages,
                     const uint8_t* mask, int64_t heads, float* out_m, float* out_l, float* out_acc,
                     void* workspace, int64_t workspace_bytes, hs_stream_t stream);

/*
 * Diagnostic (no reference counterpart): read, without computing, n segment
 * pairs of a device region -- segment i at byte offset offsets[i] (device
 * array) and its partner plane_bytes further, segment_bytes each -- with
 * consecutive lanes on consecutive 16-byte units.  Given the K offsets of the
 * attention's entries it measures the ceiling of the attention's memory
 * traffic.  The caller keeps every segment inside [base, base + region_bytes).
 * `sink` is a device buffer of at least 16 bytes (written only on an
 * impossible match).
 */
int hs_probe_row_reads(const void* base, int64_t region_bytes, const int64_t* offsets, int64_t n,
                       int64_t segment_bytes, int64_t plane_bytes, void* sink, hs_stream_t stream);

/*
 * Diagnostic (no reference counterpart): time the next attention launch of the
 * calling host thread (hs_attend_rows, hs_attend_groups or hs_attend_window)
 * with two HIP events taken from the kernel dispatches themselves
 * (hipExtLaunchKernel): `start` is stamped when the attention kernel begins and
 * `stop` when the launch's last kernel (the attention, or its merge kernel)
 * ends, so their elapsed time is the kernels' own duration, without the
 * queueing and dispatch gaps that events recorded on the stream include.  Both
 * are events created with timing enabled (hipEvent_t); either may be null.
 * The pair is used by one launch only.
 */
int hs_attend_time_next(void* start_event, void* stop_event);

/*
 * Dense-layer helpers of the batched decode engine.  They replace the
 * elementwise PyTorch ops of one decoder layer's decode step (the Qwen2 layer
 * of MiniModel.decode, model.py:183-226: RMSNorm model.py:53-57 in this build,
 * rotary, SiLU MLP) for B rows, around projections that stay PyTorch GEMMs.
 * Rounding follows those ops (each op's result rounded to `dtype`).
 *
 * hs_add_rms_norm: per row, when `delta` is non-null x_out = x + delta (x_out
 *   may alias x); then y = RMSNorm(x_out or x) * weight.  rows <= 65535.
 * hs_rotary_split: `qkv` rows hold the q|k|v projection output (heads,
 *   kv_heads, kv_heads head vectors of head_dim); writes rotated q [rows, heads,
 *   head_dim], rotated k and copied v [rows, kv_heads, head_dim] at the row's
 *   position positions[row] (device int64) with base `theta`.
 * hs_silu_mul: out[row, j] = silu(g[row, j]) * u[row, j] where a gate_up row
 *   holds g (width) then u (width).
 */
int hs_add_rms_norm(const void* x, const void* delta, void* x_out, void* y, const void* weight, int64_t rows,
                    int64_t width, int64_t x_stride, int64_t y_stride, float eps, int32_t dtype,
                    hs_stream_t stream);
int hs_rotary_split(const void* qkv, int64_t qkv_stride, void* q, void* k, void* v, const int64_t* positions,
                    int64_t rows, int64_t heads, int64_t kv_heads, int64_t head_dim, float theta, int32_t dtype,
                    hs_stream_t stream);
int hs_silu_mul(const void* gate_up, int64_t gu_stride, void* out, int64_t out_stride, int64_t rows,
                int64_t width, int32_t dtype, hs_stream_t stream);

/*
 * Decode projection of the batched engine: out[rows, n] = x[rows, k] . W[n, k]^T
 * (+ bias[n]) for 1 <= rows <= 16, bf16 or f16, fp32 accumulation; replaces
 * the PyTorch GEMMs of the decode step's projections (model.py:183-226) for
 * these skinny shapes.  k % 32 == 0, x rows 16-byte aligned (x_stride % 8 == 0),
 * W contiguous [n, k].  Tall-k shapes are split over k: the workspace
 * (hs_skinny_gemm_workspace_bytes, 8-byte aligned, any contents before a call)
 * then holds the slices' partials, which the last workgroup of each row tile sums
 * in slice order, so results are deterministic (one launch; calls sharing a
 * workspace run in order on one stream, and a call captured in a graph may be
 * replayed).
 */
int64_t hs_skinny_gemm_workspace_bytes(int64_t rows, int64_t n, int64_t k);
int hs_skinny_gemm(const void* x, int64_t x_stride, const void* weight, int64_t n, int64_t k, const void* bias,
                   void* out, int64_t out_stride, int64_t rows, int32_t dtype, void* workspace,
                   int64_t workspace_bytes, hs_stream_t stream);

/*
 * The same projection with W packed once, tile-major: weight_tiles holds
 * ceil(n/16) * (k/32) blocks of 16 rows x 32 k-values, block (t, s) =
 * W[16t .. 16t+15][32s .. 32s+31] row-major, blocks ordered by t then s, rows
 * past n zero (ceil(n/16) * 16 * k elements in all).  Each wave then reads
 * 1 KB of consecutive bytes per load instead of 16 rows a row stride apart
 * (measured 10-20% faster on the Qwen2.5 decode projections).  Same
 * arithmetic and order as hs_skinny_gemm: the outputs are bit-identical.  No
 * reference counterpart (a weight format of the batched engine).
 */
int hs_skinny_gemm_tiled(const void* x, int64_t x_stride, const void* weight_tiles, int64_t n, int64_t k,
                         const void* bias, void* out, int64_t out_stride, int64_t rows, int32_t dtype,
                         void* workspace, int64_t workspace_bytes, hs_stream_t stream);

/*
 * The MLP's gate and up projections with the SiLU gate applied on the way out:
 * out[rows, ffn] = silu(x . Wg^T) * (x . Wu^T), each projection rounded to the
 * dtype, then SiLU rounded, then the product -- the arithmetic of
 * hs_skinny_gemm_tiled on the packed gate|up weight followed by hs_silu_mul.
 * The bits are the same whenever that GEMM's plan for (rows, 2 * ffn, k) is one
 * K slice (hs_skinny_gemm_workspace_bytes at its minimum, 256) with rounds of 8
 * k-steps (HS_GEMM_GU unset); where it plans split-K the sums differ only in
 * fp32 summation order.  gate_up_tiles: 2 * ceil(ffn/16) blocks-of-tiles in
 * hs_skinny_gemm_tiled's format, the gate's tile i at position 2i and the up
 * projection's tile i at 2i + 1 (rows past ffn zero).  No workspace (one K
 * slice).  No reference counterpart (replaces two launches of the batched
 * engine's MLP, model.py:183-226).
 */
int hs_skinny_gemm_swiglu_tiled(const void* x, int64_t x_stride, const void* gate_up_tiles, int64_t ffn, int64_t k,
                                void* out, int64_t out_stride, int64_t rows, int32_t dtype, hs_stream_t stream);

/*
 * Greedy next tokens of the LM head: tokens[r] = argmax_n of the logits
 * x[r] . W[n]^T (+ bias[n]) rounded to the dtype, the first maximal index on ties
 * (-0 equal to +0; a NaN above every number), as torch.argmax over the logits of
 * hs_skinny_gemm_tiled with one K slice -- without writing the logits.  W packed as
 * for hs_skinny_gemm_tiled, n < 2^31.  Each workgroup leaves its best key per token
 * in the workspace (hs_skinny_gemm_argmax_workspace_bytes, 8-byte aligned) and a
 * second launch reduces them.  Replaces the logits GEMM and `argmax` of the
 * reference's greedy decode (engine.py:71-72, _emit: logits.argmax()).
 */
int64_t hs_skinny_gemm_argmax_workspace_bytes(int64_t rows, int64_t n, int64_t k);
int hs_skinny_gemm_argmax_tiled(const void* x, int64_t x_stride, const void* weight_tiles, int64_t n, int64_t k,
                                const void* bias, int64_t* tokens, int64_t rows, int32_t dtype, void* workspace,
                                int64_t workspace_bytes, hs_stream_t stream);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* HISPARSE_H */
