"""Row gather from pinned host memory and physical-row attention on gfx950.

Replaces mini_hisparse's ``row_kernels.py`` (Triton ``_gather``/``_attend`` and
the ctypes ``MappedHost``, row_kernels.py:10-135) with calls into
libhisparse_hip.so.  Same function names and arguments; no Triton, no CUDA
driver calls.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


class MappedHost:
    """Keep a pinned host tensor alive and expose its device alias.

    Like the reference (row_kernels.py:10-32) the allocation stays owned by
    PyTorch; the alias comes from ``hs_host_alias`` and nothing is registered
    or unregistered.
    """

    def __init__(self, tensor):
        if not tensor.is_pinned():
            raise ValueError("row gather requires pinned host backing")
        device_ptr = ctypes.c_void_p()
        status = _lib.load().hs_host_alias(tensor.data_ptr(), ctypes.byref(device_ptr))
        if status != 0:
            raise RuntimeError(
                "cannot map pinned host allocation to the device: "
                + _lib.load().hs_last_error().decode(errors="replace")
            )
        self.tensor, self.dtype, self.pointer = tensor, tensor.dtype, device_ptr.value

    def data_ptr(self):
        return self.pointer


def pinned_empty(shape, dtype):
    """A pinned host tensor of exactly ``shape`` (``hs_host_alloc``), freed when the last
    tensor viewing it is gone.  PyTorch's pinned allocator rounds a request up to a power
    of two, so a pool just above one would pin twice its size."""
    import math
    import weakref

    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    pointer = ctypes.c_void_p()
    lib = _lib.load()
    _lib.check(lib.hs_host_alloc(nbytes, ctypes.byref(pointer)), "hs_host_alloc")
    buffer = (ctypes.c_byte * nbytes).from_address(pointer.value)
    # the buffer object lives as long as any tensor storage over it
    weakref.finalize(buffer, lib.hs_host_free, pointer.value)
    return torch.frombuffer(buffer, dtype=torch.uint8).view(dtype).view(shape)


def _row_bytes(config, element_size):
    return config.kv_heads * config.head_dim * element_size


def gather_rows(host, pool, plan, config, *, miss_count=None):
    """Copy every planned host row (K and V planes) into its hot device row.

    ``host`` is a :class:`MappedHost`; ``plan`` a RowPlan (row_index.py:51-56).
    ``miss_count`` (optional device int64 scalar, e.g. ``plan.counts[2:]``)
    bounds the number of plan entries read.
    """
    if pool.device.type != "cuda":
        raise ValueError("the HIP gather needs a ROCm device pool")
    n = plan.miss_host_rows.numel()
    if n == 0:
        return
    if plan.miss_host_rows.dtype != torch.int64 or plan.miss_device_rows.dtype != torch.int64:
        raise ValueError("gather plans must be int64")
    status = _lib.load().hs_gather_rows(
        host.data_ptr(),
        pool.data_ptr(),
        plan.miss_host_rows.data_ptr(),
        plan.miss_device_rows.data_ptr(),
        n,
        _lib.ptr(miss_count),
        host.tensor.shape[0] * config.page_size,
        pool.shape[0] * config.page_size,
        config.page_size,
        _row_bytes(config, pool.element_size()),
        _lib.stream_handle(pool.device),
    )
    _lib.check(status, "hs_gather_rows")


def append_rows(k, v, pool, device_rows, minimums, maximums, config, *, host=None, host_rows=None, stream=None):
    """One token's K/V for each of B (request, layer) pairs (storage.py:246-319, one row).

    ``k``/``v`` [B, Hkv, D] in the pool dtype; ``device_rows`` / ``host_rows``
    Python ints (pool row / host row, ``-1`` skips the mirror); ``minimums`` /
    ``maximums`` the tail pages' ``[Hkv, D]`` bound tensors; ``host`` a
    :class:`MappedHost` of the pinned host pool.
    """
    batch = k.shape[0]
    if k.shape != v.shape or k.dim() != 3 or k.dtype != pool.dtype or not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("append needs contiguous [B, Hkv, D] K/V in the pool dtype")
    if not (len(device_rows) == len(minimums) == len(maximums) == batch):
        raise ValueError("one device row and one pair of bounds per appended token")
    i64, vp = ctypes.c_int64 * batch, ctypes.c_void_p * batch
    hrows = None if host_rows is None else i64(*host_rows)
    alias = None if host is None else vp(*([host.data_ptr()] * batch))
    host_pool_rows = 0 if host is None else host.tensor.shape[0] * config.page_size
    s = stream.cuda_stream if stream is not None else _lib.stream_handle(pool.device)
    status = _lib.load().hs_append_rows(
        k.data_ptr(), v.data_ptr(), k.stride(0), pool.data_ptr(), pool.shape[0] * config.page_size,
        _lib.dtype_code(pool.dtype), config.page_size, config.kv_heads, config.head_dim,
        i64(*device_rows), alias, hrows, host_pool_rows,
        vp(*[t.data_ptr() for t in minimums]), vp(*[t.data_ptr() for t in maximums]), batch, s,
    )
    _lib.check(status, "hs_append_rows")


def append_tokens(k, v, first_page, first_within, slots, host_slots, pool, host, minimum, maximum, summaries,
                  config):
    """A write of ``len(k)`` tokens to one (request, layer) with its page placement
    decided (``hs_append_tokens``; the page loop of storage.py:273-318): rows to the
    resident pages' blocks and to the host mirror, bounds and summaries of every page.

    ``slots`` / ``host_slots``: per page of the write, its device block (``-1``: not
    resident) and host slot; ``host`` a :class:`MappedHost` of the pinned host pool;
    ``minimum`` / ``maximum`` / ``summaries`` the layer's ``[pages, Hkv, D]`` tensors."""
    pages = len(slots)
    if k.shape != v.shape or k.dim() != 3 or k.dtype != pool.dtype or k.stride() != v.stride() or \
            k.stride(2) != 1 or k.stride(1) != config.head_dim:
        raise ValueError("append needs [tokens, Hkv, D] K/V rows in the pool dtype")
    i64 = ctypes.c_int64 * pages
    status = _lib.load().hs_append_tokens(
        k.data_ptr(), v.data_ptr(), k.stride(0), k.shape[0], pool.data_ptr(), pool.shape[0] * config.page_size,
        host.data_ptr(), host.tensor.shape[0] * config.page_size, _lib.dtype_code(pool.dtype), config.page_size,
        config.kv_heads, config.head_dim, first_page, first_within, pages, i64(*slots), i64(*host_slots),
        minimum.data_ptr(), maximum.data_ptr(), _lib.ptr(summaries), minimum.shape[0],
        _lib.stream_handle(pool.device),
    )
    _lib.check(status, "hs_append_tokens")


# Attention workspaces, one per (device, stream), grown on demand.  Launches on
# one stream run in order, so the calls of a stream can share its workspace.
_ATTEND_WS = {}


def _attend_workspace(dtype_code, batch, heads, kv_heads, head_dim, max_entries, device):
    size = _lib.load().hs_attend_workspace_bytes(dtype_code, batch, heads, kv_heads, head_dim, max_entries)
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _ATTEND_WS.get(key)
    if ws is None or ws.numel() < size:
        ws = torch.empty(max(size, 1 << 16), dtype=torch.uint8, device=device)
        _ATTEND_WS[key] = ws
    return ws, ws.numel()


def _check_query(query, pool, config):
    if query.device.type != "cuda" or pool.device.type != "cuda":
        raise ValueError("the HIP attention needs ROCm device tensors")
    if query.dtype != pool.dtype:
        query = query.to(pool.dtype)
    return query.contiguous()


def attend_rows(query, pool, rows, config):
    """Attention of each query head over its physical rows (row_kernels.py:116-135).

    query [Hq, D] (or [B, Hq, D]); rows [Hq, W] or [W] shared (or batched
    [B, Hq, W] / [B, W]); returns [Hq, D] (or [B, Hq, D]) in the query dtype.
    """
    batched = query.ndim == 3
    out_dtype = query.dtype
    q = _check_query(query, pool, config)
    if not batched:
        q = q[None]
        rows = rows[None]
    batch, heads, dim = q.shape
    if rows.dtype != torch.int64:
        rows = rows.to(torch.int64)
    if rows.ndim == 2:  # one row list shared by every head
        r_sb, r_sh, r_sw = rows.stride(0), 0, rows.stride(1)
        width = rows.shape[1]
        max_entries = width
    else:
        r_sb, r_sh, r_sw = rows.stride()
        width = rows.shape[2]
        if r_sh == 0:
            max_entries = width
        else:
            max_entries = width * (heads // config.kv_heads)
    out = torch.empty_like(q)
    code = _lib.dtype_code(pool.dtype)
    workspace, ws_bytes = _attend_workspace(code, batch, heads, config.kv_heads, dim, max(1, max_entries), q.device)
    status = _lib.load().hs_attend_rows(
        q.data_ptr(), q.stride(0), q.stride(1),
        pool.data_ptr(), code, config.page_size, config.kv_heads, config.head_dim,
        pool.shape[0] * config.page_size, rows.data_ptr(), r_sb, r_sh, r_sw, width, batch, heads,
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
    )
    _lib.check(status, "hs_attend_rows")
    out = out if batched else out[0]
    return out if out.dtype == out_dtype else out.to(out_dtype)


def attend_groups(query, pool, union_physical, entries, config):
    """Attention reading each KV head's deduplicated rows once (hs_attend_groups).

    ``entries`` is a GroupEntries (or a batched one with a leading batch dim)
    and ``union_physical`` the resolver's input-order physical rows.
    """
    batched = query.ndim == 3
    out_dtype = query.dtype
    q = _check_query(query, pool, config)
    cols, masks, counts = entries.columns, entries.masks, entries.counts
    up = union_physical
    if not batched:
        q, cols, masks, counts, up = q[None], cols[None], masks[None], counts[None], up[None]
    batch, heads, dim = q.shape
    out = torch.empty_like(q)
    code = _lib.dtype_code(pool.dtype)
    capacity = entries.capacity
    workspace, ws_bytes = _attend_workspace(code, batch, heads, config.kv_heads, dim, capacity, q.device)
    status = _lib.load().hs_attend_groups(
        q.data_ptr(), q.stride(0), q.stride(1),
        pool.data_ptr(), code, config.page_size, config.kv_heads, config.head_dim,
        pool.shape[0] * config.page_size, up.data_ptr(), up.stride(0),
        cols.data_ptr(), masks.data_ptr(), cols.stride(0), cols.stride(1), counts.data_ptr(), capacity,
        batch, heads, out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
    )
    _lib.check(status, "hs_attend_groups")
    out = out if batched else out[0]
    return out if out.dtype == out_dtype else out.to(out_dtype)


def attend_window(query, pool, slots, lengths, mask, config):
    """Unnormalised attention state of one window of whole pages (hs_attend_window).

    Replaces ``triton_chunk`` / ``_attention_window`` of the reference's paged
    layout (reference/kernels.py:12-97).  query [Hq, D]; slots / lengths [N]
    int32 device tensors (device slot and valid tokens of each page); mask
    [Hq, N, P] bool or None.  Returns fp32 (m [Hq], l [Hq], acc [Hq, D]).
    """
    q = _check_query(query, pool, config)
    if q.ndim != 2 or q.shape[1] != config.head_dim or q.shape[0] % config.kv_heads:
        raise ValueError("expected [query_heads, head_dim], query_heads divisible by KV heads")
    heads, dim = q.shape
    n = slots.numel()
    if n < 1 or lengths.numel() != n or slots.dtype != torch.int32 or lengths.dtype != torch.int32:
        raise ValueError("a window needs matching int32 slot and length vectors")
    if mask is not None:
        if mask.shape != (heads, n, config.page_size) or mask.dtype != torch.bool:
            raise ValueError("the window mask must be bool [query_heads, pages, page_size]")
        mask = mask.contiguous()
    m = torch.empty(heads, dtype=torch.float32, device=q.device)
    l = torch.empty_like(m)
    acc = torch.empty((heads, dim), dtype=torch.float32, device=q.device)
    code = _lib.dtype_code(pool.dtype)
    workspace, ws_bytes = _attend_workspace(code, 1, heads, config.kv_heads, dim, n * config.page_size, q.device)
    status = _lib.load().hs_attend_window(
        q.data_ptr(), q.stride(0), pool.data_ptr(), code, config.page_size, config.kv_heads, config.head_dim,
        pool.shape[0] * config.page_size, slots.contiguous().data_ptr(), lengths.contiguous().data_ptr(), n,
        None if mask is None else mask.data_ptr(), heads, m.data_ptr(), l.data_ptr(), acc.data_ptr(),
        workspace.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
    )
    _lib.check(status, "hs_attend_window")
    return m, l, acc
