"""Token selections and the Quest page selector.

``Selection`` keeps the reference's canonical host form (per-head sorted token
tuples, selection.py:11-77).  ``quest_selection`` (selection.py:80-101) runs
the gfx950 scorer + per-head top-k and returns a :class:`DeviceSelection`:
the chosen pages stay on the GPU and the union/head columns are built there
(hs_build_union), so the decode step never synchronises on the selection.
Reading ``DeviceSelection.positions`` materialises the host form (one sync),
for callers that inspect it.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import ceil

import torch

from . import _lib
from .row_index import GroupEntries, LogicalTopK


@dataclass(frozen=True)
class Selection:
    positions: tuple[tuple[int, ...], ...]  # per query head, canonical logical tokens
    length: int
    page_size: int
    source: str

    @property
    def heads(self):
        return len(self.positions)

    @classmethod
    def from_tokens(cls, rows, length, page_size, heads, source="external"):
        if length < 1 or page_size < 1 or heads < 1:
            raise ValueError("selection dimensions must be positive")
        if isinstance(rows, torch.Tensor):
            rows = rows.cpu().tolist()
        if rows and isinstance(rows[0], int):
            rows = [rows]
        if len(rows) == 1:
            rows = rows * heads
        if len(rows) != heads:
            raise ValueError("selection must be shared or have one row per query head")
        canonical = []
        for row in rows:
            if not isinstance(row, (list, tuple)):
                raise TypeError("selection rows must be integer sequences")
            for t in row:
                if not isinstance(t, int) or t < -1 or t >= length:
                    raise ValueError("token selection contains noncausal or invalid positions")
            tokens = tuple(sorted(set(row) - {-1}))
            if not tokens:
                raise ValueError("each query head must select at least one token")
            canonical.append(tokens)
        return cls(tuple(canonical), length, page_size, source)

    @classmethod
    def from_pages(cls, rows, length, page_size, heads, source="pages"):
        if isinstance(rows, torch.Tensor):
            rows = rows.cpu().tolist()
        if rows and isinstance(rows[0], int):
            rows = [rows]
        count = ceil(length / page_size)
        if any(p < 0 or p >= count for row in rows for p in row):
            raise ValueError("invalid logical page")
        expanded = [
            [t for p in row for t in range(p * page_size, min(p * page_size + page_size, length))]
            for row in rows
        ]
        return cls.from_tokens(expanded, length, page_size, heads, source)

    @property
    def pages(self):
        return sorted({t // self.page_size for row in self.positions for t in row})

    def mask(self, pages, device):
        """Bounded [heads, len(pages), page_size] token mask, never the full KV."""
        selected = [set(row) for row in self.positions]
        table = [
            [[p * self.page_size + t in row for t in range(self.page_size)] for p in pages]
            for row in selected
        ]
        mask = torch.tensor(table, dtype=torch.bool, pin_memory=torch.device(device).type == "cuda")
        return mask.to(device, non_blocking=True)


def forced_pages(count, top_pages, keep_sink=True):
    """Pages every head keeps (selection.py:96-99)."""
    required = [count - 1]
    if keep_sink and top_pages > 1 and count > 1:
        required.append(0)
    return required


def selection_width(length, page_size, top_pages):
    """Tokens per head: min(top, count) pages, the tail page partial."""
    count = ceil(length / page_size)
    k = min(top_pages, count)
    return (k - 1) * page_size + (length - (count - 1) * page_size)


def union_bound(length, page_size, top_pages, heads, keep_sink=True):
    """Upper bound on the union of ``heads`` page selections (cli.py:139-143)."""
    count = ceil(length / page_size)
    if top_pages >= count:
        return length
    forced = len(forced_pages(count, top_pages, keep_sink))
    pages = min(count, forced + (top_pages - forced) * heads)
    return min(length, pages * page_size)


class DeviceSelection:
    """Per-head Quest pages resident on the device ([heads, top] int32, ascending).

    Duck-types :class:`Selection` (``length``, ``page_size``, ``source``,
    ``heads``; ``positions``/``pages`` materialise on first access).
    """

    def __init__(self, pages, length, page_size, kv_heads, top_pages, keep_sink=True):
        self.device_pages = pages
        self.length = length
        self.page_size = page_size
        self.kv_heads = kv_heads
        self.top_pages = top_pages
        self.keep_sink = keep_sink
        self.source = "quest"
        self.heads = pages.shape[0]
        self._host = None

    def _materialize(self):
        if self._host is None:
            count = ceil(self.length / self.page_size)
            k = min(self.top_pages, count)
            rows = self.device_pages[:, :k].cpu().tolist()
            self._host = Selection.from_pages(rows, self.length, self.page_size, self.heads, "quest")
        return self._host

    @property
    def positions(self):
        return self._materialize().positions

    @property
    def pages(self):
        return self._materialize().pages

    def mask(self, pages, device):
        return self._materialize().mask(pages, device)

    def logical_topk(self, device, max_rows=None):
        """Union positions, head columns and group entries, built on the device."""
        topk = build_union(
            self.device_pages[None],
            [self.length],
            self.page_size,
            self.kv_heads,
            self.top_pages,
            keep_sink=self.keep_sink,
            max_rows=max_rows,
        )
        return topk[0]


def _quest_bounds_check(query, minimum, top_pages):
    if top_pages < 1 or query.shape[0] % minimum.shape[1]:
        raise ValueError("invalid page budget or GQA shape")


def quest_selection(query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
    """Quest-style per-head page upper bounds and top-k (selection.py:80-101).

    ``max(q_d * min(K_d), q_d * max(K_d))`` upper-bounds each page's q.K; each
    head selects independently and the cache transfers the union of pages.
    Runs on the GPU and returns a :class:`DeviceSelection`.
    """
    _quest_bounds_check(query, minimum, top_pages)
    if query.device.type != "cuda":
        raise ValueError("quest_selection needs ROCm device tensors (HIP kernels only)")
    pages = quest_topk(
        query[None], [minimum], [maximum], [length], page_size, top_pages, keep_sink
    )[0]
    return DeviceSelection(pages, length, page_size, minimum.shape[1], top_pages, keep_sink)


def quest_topk(queries, minimums, maximums, lengths, page_size, top_pages, keep_sink=True):
    """Batched scorer + top-k: queries [B, Hq, D]; per-request bounds [pages, Hkv, D].

    Returns [B, Hq, top] int32 pages, ascending per head (first min(top, count) valid).
    """
    batch, heads, dim = queries.shape
    kv_heads = minimums[0].shape[1]
    if top_pages < 1 or heads % kv_heads:
        raise ValueError("invalid page budget or GQA shape")
    device = queries.device
    # read by the kernel in the model dtype (widened exactly, like the reference's .float())
    q = queries if queries.dtype in (torch.float32, torch.bfloat16, torch.float16) else queries.float()
    if q.stride(-1) != 1:
        q = q.contiguous()
    counts = [ceil(length / page_size) for length in lengths]
    if any(c < 1 for c in counts):
        raise ValueError("cannot select pages of an empty history")
    for lo, hi, c in zip(minimums, maximums, counts):
        if lo.shape[0] < c or hi.shape != lo.shape or not (lo.is_contiguous() and hi.is_contiguous()):
            raise ValueError("Quest bounds must be contiguous [pages, kv_heads, head_dim] covering the history")
    pages = torch.empty((batch, heads, top_pages), dtype=torch.int32, device=device)
    lib = _lib.load()
    ws_bytes = lib.hs_quest_workspace_bytes(batch, heads, max(counts))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    lo_ptrs = (ctypes_void_p_array(batch))(*[t.data_ptr() for t in minimums])
    hi_ptrs = (ctypes_void_p_array(batch))(*[t.data_ptr() for t in maximums])
    count_arr = (_c_int64_array(batch))(*counts)
    status = lib.hs_quest_topk(
        q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_code(q.dtype),
        lo_ptrs, hi_ptrs, _lib.dtype_code(minimums[0].dtype), count_arr,
        batch, heads, kv_heads, dim, top_pages, int(bool(keep_sink)),
        pages.data_ptr(), pages.stride(0), workspace.data_ptr(), ws_bytes,
        _lib.stream_handle(device),
    )
    _lib.check(status, "hs_quest_topk")
    return pages


def ctypes_void_p_array(n):
    import ctypes

    return ctypes.c_void_p * n


def _c_int64_array(n):
    import ctypes

    return ctypes.c_int64 * n


def build_union(pages, lengths, page_size, kv_heads, top_pages, keep_sink=True, max_rows=None):
    """Device Selection -> LogicalTopK for a batch of page selections.

    pages [B, Hq, top] int32 (from :func:`quest_topk`); returns one
    :class:`LogicalTopK` per request, each with positions padded by -1, head
    columns and per-KV-head entry lists.  Raises the reference's
    ``max_union_rows`` error when the union exceeds ``max_rows`` (that check
    reads the union size back only when the bound alone cannot decide it).
    """
    batch, heads, top = pages.shape
    device = pages.device
    groups = heads // kv_heads
    bounds = [union_bound(l, page_size, top_pages, heads, keep_sink) for l in lengths]
    capacity = max(bounds)
    if max_rows is not None and capacity > max_rows:
        capacity = max_rows
    entry_cap = max(union_bound(l, page_size, top_pages, groups, keep_sink) for l in lengths)
    width = max(selection_width(l, page_size, top_pages) for l in lengths)
    positions = torch.empty((batch, capacity), dtype=torch.int32, device=device)
    columns = torch.empty((batch, heads, width), dtype=torch.int64, device=device)
    union_count = torch.empty(batch, dtype=torch.int32, device=device)
    ecol = torch.empty((batch, kv_heads, entry_cap), dtype=torch.int32, device=device)
    emask = torch.empty((batch, kv_heads, entry_cap), dtype=torch.int32, device=device)
    ecount = torch.empty((batch, kv_heads), dtype=torch.int32, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    length_arr = (_c_int64_array(batch))(*lengths)
    rc = _lib.load().hs_build_union(
        pages.data_ptr(), pages.stride(0), top, length_arr, page_size, batch, heads, kv_heads,
        positions.data_ptr(), capacity, columns.data_ptr(), width, union_count.data_ptr(),
        ecol.data_ptr(), emask.data_ptr(), entry_cap, ecount.data_ptr(), status.data_ptr(), None, 0, None,
        _lib.stream_handle(device),
    )
    _lib.check(rc, "hs_build_union")
    if max_rows is not None and max(bounds) > max_rows:
        if int(union_count.max().item()) > max_rows:
            raise ValueError("top-k width/union exceeds the admitted max_union_rows")
    result = []
    for b in range(batch):
        entries = GroupEntries(ecol[b], emask[b], ecount[b], entry_cap)
        result.append(LogicalTopK(positions[b], columns[b], entries, union_count[b : b + 1]))
    return result


def select_pages(cache, request_id: str, layer: int, query: torch.Tensor, top_k: int | None):
    """Page-mean selector for demonstrations (selection.py:129-155), torch ops on the
    cache device.  None selects the full causal history; sparse mode keeps the
    first and last page, then scores the rest by query-group mean . page mean K."""
    request = cache.storage.requests[request_id]
    count = ceil(request.lengths[layer] / cache.config.page_size)
    if count == 0:
        raise ValueError("cannot attend to empty KV")
    if top_k is None or top_k >= count:
        return list(range(count))
    if top_k < 1:
        raise ValueError("top_k must be positive or None")
    required = [count - 1] if top_k == 1 else [0, count - 1]
    if top_k == len(required):
        return sorted(required)
    groups = query.shape[0] // cache.config.kv_heads
    grouped = query.float().reshape(cache.config.kv_heads, groups, -1).mean(1)
    scores = torch.einsum("hd,phd->p", grouped, request.summaries[layer, :count])
    scores[required] = -torch.inf
    chosen = scores.topk(top_k - len(required)).indices.tolist()
    return sorted(required + chosen)
