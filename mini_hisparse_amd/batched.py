"""One layer of sparse decode for a batch of requests, in a fixed set of launches.

The reference decodes requests one at a time (engine.py:115-128) and, per
(request, layer), runs ~40 resolver launches, a host sync in the selector and
a host-built union (selection.py:100, row_index.py:20-31).  Here a layer of B
requests is:

    hs_quest_topk      scorer + top-k for all B x Hq heads          (compute stream)
    hs_build_union     unions, head columns, per-KV-head entry lists (compute stream)
    hs_resolve_rows    one workgroup per request, row_stats fused   (compute stream)
    hs_gather_rows     all B miss plans, host -> hot rows           (transfer stream)
    hs_attend_groups   split-K group attention + merge              (compute stream)

with the reference's event ordering (hybrid.py:443, :455-457, :473, :83-85):
the transfer stream waits for the resolve and for the previous readers of
the hot rows; attention waits for the gather.  Buffers are allocated once per
shape, so a step allocates nothing and never reads back to the host.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from math import ceil

import torch

from . import _lib
from .selection import union_bound


@dataclass
class LayerTablesView:
    """The per-(request, layer) tables the resolver reads and updates (hybrid.py:45-64)."""

    source: torch.Tensor  # [pages] int32
    resident: torch.Tensor  # [pages] int32
    hot: torch.Tensor  # [hot_blocks] int32
    tags: torch.Tensor  # [hot_rows] int32 (updated)
    lru: torch.Tensor  # [hot_rows] int64, or int16 (a quarter of the resolver's LRU bytes) (updated)


def _handle(stream, device):
    """Stream handle of ``stream``: a torch Stream, a raw handle (int), or None for the
    current stream of ``device``."""
    if stream is None:
        return _lib.stream_handle(device)
    return stream if isinstance(stream, int) else stream.cuda_stream


class BatchedSparseDecode:
    """Quest -> union -> resolve -> gather -> attention for B requests of one layer."""

    def __init__(self, config, heads, top_pages, lengths, *, keep_sink=True, device="cuda", capacity_lengths=None,
                 shared_selection=False, workspaces_from=None, head_rows=False, split_front=False):
        """``capacity_lengths`` (default ``lengths``) sizes every buffer, so that later
        ``set_lengths`` calls up to those lengths (a decode run) allocate nothing.
        ``shared_selection``: every head of a request selects the same pages
        (:meth:`select_pages`), so the union is one head's selection.
        ``workspaces_from``: a decoder of the same shape whose scorer and attention
        workspaces this one reuses (decoders whose ``select`` and ``attend`` calls run
        one after another on one stream, e.g. one decoder per layer).
        ``head_rows``: the resolver also writes each head's physical rows
        (``physical``, [B, heads, width]: row_index.py:127-131).  The group attention
        reads the union rows and the per-KV-head entry lists only, so the decode path
        leaves them out unless asked.
        ``split_front``: the tables given to :meth:`resolve` are affine with base
        ``source[0]`` (host block = source[0] + page, a request's contiguous host slots),
        so the resolver may spread its front over several workgroups per request
        (``hs_resolve_desc.split_front``; power-of-two pages of at most 32 tokens)."""
        self.split_front = split_front
        self._workspaces_from = workspaces_from
        self.head_rows = head_rows
        self.entry_stats = None  # optional int64 [1] device total of the unions' entry counts
        self.config = config
        self.heads = heads
        self.kv_heads = config.kv_heads
        self.groups = heads // config.kv_heads
        self.top = top_pages
        self.keep_sink = keep_sink
        self.shared_selection = shared_selection
        self.device = torch.device(device)
        self.batch = len(lengths)
        self._shape(list(lengths), list(capacity_lengths or lengths))

    def _shape(self, lengths, capacity_lengths):
        P, B, dev = self.config.page_size, self.batch, self.device
        caps = [max(c, l) for c, l in zip(capacity_lengths, lengths)]
        self.capacity_lengths = caps
        self.lengths = lengths
        self.counts = [ceil(l / P) for l in lengths]
        # union sizes grow with the length, and a head's width is at most top pages
        union_heads = 1 if self.shared_selection else self.heads
        group_heads = 1 if self.shared_selection else self.groups
        self.capacity = max(union_bound(l, P, self.top, union_heads, self.keep_sink) for l in caps)
        self.entry_capacity = max(union_bound(l, P, self.top, group_heads, self.keep_sink) for l in caps)
        self.width = max(min(self.top * P, l) for l in caps)
        i32, i64 = torch.int32, torch.int64
        # the selection's pages [B, heads, top]: this buffer, or a caller's expanded pages
        # (select_pages), read in place
        self.pages = self._page_buf = torch.empty((B, self.heads, self.top), dtype=i32, device=dev)
        self.positions = torch.empty((B, self.capacity), dtype=i32, device=dev)
        self.head_columns = torch.empty((B, self.heads, self.width), dtype=i64, device=dev)
        self.union_count = torch.empty(B, dtype=i32, device=dev)
        self.entry_columns = torch.empty((B, self.kv_heads, self.entry_capacity), dtype=i32, device=dev)
        self.entry_masks = torch.empty((B, self.kv_heads, self.entry_capacity), dtype=i32, device=dev)
        self.entry_counts = torch.empty((B, self.kv_heads), dtype=i32, device=dev)
        self.status = torch.zeros(1, dtype=i32, device=dev)
        # the union's page bitmap, read by the resolver instead of the positions
        self.page_bits_stride = max(ceil(ceil(l / P) / 32) for l in caps)
        self.page_bits = torch.empty((B, self.page_bits_stride), dtype=i32, device=dev)
        self.union_physical = torch.empty((B, self.capacity), dtype=i64, device=dev)
        self.physical = torch.empty((B, self.heads, self.width), dtype=i64, device=dev) if self.head_rows else None
        self.miss_host = torch.empty((B, self.capacity), dtype=i64, device=dev)
        self.miss_device = torch.empty((B, self.capacity), dtype=i64, device=dev)
        self.row_counts = torch.empty((B, 3), dtype=i64, device=dev)
        lib = _lib.load()
        self.quest_ws_bytes = lib.hs_quest_workspace_bytes(B, self.heads, max(ceil(l / P) for l in caps))
        self.resolve_ws_bytes = 0
        self.max_tables = None
        self.attend_ws_bytes = lib.hs_attend_workspace_bytes(
            _lib.HS_DTYPE_BF16, B, self.heads, self.kv_heads, self.config.head_dim, self.entry_capacity
        )
        self.attend_ws_bytes = max(
            self.attend_ws_bytes,
            lib.hs_attend_workspace_bytes(_lib.HS_DTYPE_F32, B, self.heads, self.kv_heads, self.config.head_dim, self.entry_capacity),
        )
        donor = self._workspaces_from
        if donor is not None and donor.quest_ws_bytes >= self.quest_ws_bytes and donor.attend_ws_bytes >= self.attend_ws_bytes:
            self.quest_ws, self.quest_ws_bytes = donor.quest_ws, donor.quest_ws_bytes
            self.attend_ws, self.attend_ws_bytes = donor.attend_ws, donor.attend_ws_bytes
        else:
            self.quest_ws = torch.empty(self.quest_ws_bytes, dtype=torch.uint8, device=dev)
            self.attend_ws = torch.empty(self.attend_ws_bytes, dtype=torch.uint8, device=dev)
        self._len_arr = (ctypes.c_int64 * B)(*lengths)
        self._count_arr = (ctypes.c_int64 * B)(*self.counts)
        # ctypes arguments built once per buffer set and per table / bound / host set
        # (only the lengths change between decode steps)
        self._descs = {}
        self._bounds = {}
        self._hosts = {}
        self._miss_args = (
            (ctypes.c_void_p * B)(*[self.miss_host[b].data_ptr() for b in range(B)]),
            (ctypes.c_void_p * B)(*[self.miss_device[b].data_ptr() for b in range(B)]),
            (ctypes.c_void_p * B)(*[self.row_counts[b, 2:].data_ptr() for b in range(B)]),
            (ctypes.c_int64 * B)(*([self.capacity] * B)),
        )

    def set_lengths(self, lengths):
        lengths = list(lengths)
        if lengths == self.lengths:
            return
        if any(l > c for l, c in zip(lengths, self.capacity_lengths)):
            self._shape(lengths, lengths)  # beyond the reserved sizes: new buffers
            return
        self.lengths = lengths
        self.counts = [ceil(l / self.config.page_size) for l in lengths]
        for b in range(self.batch):
            self._len_arr[b] = lengths[b]
            self._count_arr[b] = self.counts[b]

    # -- stages ------------------------------------------------------------
    def select(self, queries, minimums, maximums, stream=None):
        """Quest scorer + top-k and the device union for all B requests."""
        if self.shared_selection:
            raise RuntimeError("a shared-selection decoder takes its pages from select_pages")
        B = self.batch
        q = queries if queries.dtype in (torch.float32, torch.bfloat16, torch.float16) else queries.float()
        if q.stride(-1) != 1:  # read by the kernel in its dtype
            q = q.contiguous()
        lib = _lib.load()
        s = _handle(stream, self.device)
        key = tuple(map(id, minimums)) + tuple(map(id, maximums))
        hit = self._bounds.get(key)
        if hit is None or not all(a is b for a, b in zip(hit[0], (*minimums, *maximums))):
            hit = ((*minimums, *maximums), (ctypes.c_void_p * B)(*[t.data_ptr() for t in minimums]),
                   (ctypes.c_void_p * B)(*[t.data_ptr() for t in maximums]))
            self._bounds[key] = hit
        _, lo, hi = hit
        self.pages = self._page_buf
        _lib.check(
            lib.hs_quest_topk(
                q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_code(q.dtype),
                lo, hi, _lib.dtype_code(minimums[0].dtype), self._count_arr, B, self.heads,
                self.kv_heads, q.shape[2], self.top, int(self.keep_sink), self.pages.data_ptr(),
                self.pages.stride(0), self.quest_ws.data_ptr(), self.quest_ws_bytes, s,
            ),
            "hs_quest_topk",
        )
        self._build_union(s)

    def select_pages(self, pages, stream=None, validate=True):
        """A selection given as pages, read by every head: ``pages`` int32 on the device,
        [B, top] (copied to every head) or already [B, heads, top] with every head's row
        the same (read in place, no copy; each request's [heads, top] block contiguous);
        ascending and distinct, min(top, count) of them per request with the tail page
        last.  ``validate`` checks that on the host (a device-to-host copy); a caller that
        builds its pages that way itself may skip it."""
        expanded = pages.dim() == 3
        if pages.dtype != torch.int32 or pages.shape != ((self.batch, self.heads, self.top) if expanded
                                                           else (self.batch, self.top)):
            raise ValueError(f"pages must be int32 [{self.batch}, {self.top}] or [{self.batch}, {self.heads}, "
                             f"{self.top}]")
        if expanded and (pages.stride(2) != 1 or pages.stride(1) != self.top):
            raise ValueError("each request's [heads, top] pages must be contiguous")
        if validate:
            host = (pages[:, 0] if expanded else pages).cpu()
            for b, count in enumerate(self.counts):
                k = min(self.top, count)
                row = host[b, :k]
                if ((row < 0) | (row >= count)).any() or (row[1:] <= row[:-1]).any() or row[-1] != count - 1:
                    raise ValueError(f"request {b}: pages must be {k} ascending distinct pages below {count}, "
                                     f"the tail page {count - 1} last")
        s = _handle(stream, self.device)
        if expanded:
            self.pages = pages
        else:
            self.pages = self._page_buf
            self.pages.copy_(pages[:, None, :].expand(self.batch, self.heads, self.top))
        self._build_union(s)

    def _build_union(self, s):
        lib = _lib.load()
        _lib.check(
            lib.hs_build_union(
                self.pages.data_ptr(), self.pages.stride(0), self.top, self._len_arr,
                self.config.page_size, self.batch, self.heads, self.kv_heads, self.positions.data_ptr(),
                self.capacity, self.head_columns.data_ptr(), self.width, self.union_count.data_ptr(),
                self.entry_columns.data_ptr(), self.entry_masks.data_ptr(), self.entry_capacity,
                self.entry_counts.data_ptr(), self.status.data_ptr(), self.page_bits.data_ptr(),
                self.page_bits_stride, _lib.ptr(self.entry_stats), s,
            ),
            "hs_build_union",
        )

    def check_status(self):
        """Raise if a union of any step so far overflowed its buffers (the union builder's
        status bits: 1 = union positions, 2 = group entries; both are truncated then).
        Reads the flag back to the host."""
        bits = int(self.status.item())
        if bits:
            what = [name for bit, name in ((1, "union positions"), (2, "group entries")) if bits & bit]
            raise RuntimeError(f"union overflow ({' and '.join(what)} over capacity): the selection was truncated")

    def _resolve_descs(self, tables):
        """Resolver descriptors of one set of B tables, built once: the workspace is sized
        for the capacity lengths, and `resolve` refreshes the lengths per call."""
        key = tuple(map(id, tables))
        hit = self._descs.get(key)
        if hit is not None and all(a is b for a, b in zip(hit[0], tables)):
            return hit[1]
        B, P = self.batch, self.config.page_size
        lib = _lib.load()
        descs = (_lib.ResolveDesc * B)()
        total = 0
        for b, t in enumerate(tables):
            d = descs[b]
            d.positions = self.positions[b].data_ptr()
            d.n = self.capacity
            d.positions_i64 = 0
            d.page_bits = self.page_bits[b].data_ptr()  # the positions come from _build_union
            if self.head_rows:
                d.head_columns = self.head_columns[b].data_ptr()
                d.heads, d.width = self.heads, self.width
                d.hc_stride_h, d.hc_stride_w = self.head_columns.stride(1), 1
            d.source, d.resident = t.source.data_ptr(), t.resident.data_ptr()
            d.n_pages = t.source.numel()
            d.hot, d.hot_blocks = t.hot.data_ptr(), t.hot.numel()
            if t.lru.dtype not in (torch.int16, torch.int64):
                raise TypeError(f"lru must be int16 or int64, got {t.lru.dtype}")
            d.tags, d.lru, d.hot_rows = t.tags.data_ptr(), t.lru.data_ptr(), t.tags.numel()
            d.lru_i16 = int(t.lru.dtype == torch.int16)
            d.length, d.page_size = self.lengths[b], P
            d.union_physical = self.union_physical[b].data_ptr()
            d.physical = self.physical[b].data_ptr() if self.head_rows else d.union_physical
            d.miss_host_rows = self.miss_host[b].data_ptr()
            d.miss_device_rows = self.miss_device[b].data_ptr()
            d.miss_prefix_only = 1  # the gather stops at the miss count: no -1 tail
            d.split_front = int(self.split_front and P <= 32 and (P & (P - 1)) == 0)
            d.counts = self.row_counts[b].data_ptr()
            total += lib.hs_resolve_workspace_bytes(self.capacity, self.capacity_lengths[b], d.n_pages, d.hot_rows)
        if total > self.resolve_ws_bytes:
            self.resolve_ws = torch.empty(total, dtype=torch.uint8, device=self.device)
            self.resolve_ws_bytes = total
        self._descs[key] = (tuple(tables), descs)
        return descs

    def resolve(self, tables, row_stats=None, stream=None):
        """One resolver launch over B (request, layer) tables; counts land in row_counts."""
        if len(tables) != self.batch:
            raise ValueError(f"expected {self.batch} tables")
        descs = self._resolve_descs(tables)
        stats = _lib.ptr(row_stats)
        for b in range(self.batch):
            descs[b].length = self.lengths[b]
            descs[b].row_stats = stats
        s = _handle(stream, self.device)
        _lib.check(
            _lib.load().hs_resolve_rows_batched(descs, self.batch, self.resolve_ws.data_ptr(), self.resolve_ws_bytes, s),
            "hs_resolve_rows_batched",
        )

    def gather(self, host_alias, pool, stream, grid_x=0):
        """All B miss plans in one launch on `stream` (reads host memory directly)."""
        B, cfg = self.batch, self.config
        lib = _lib.load()
        alias = host_alias.data_ptr()
        hosts = self._hosts.get(alias)
        if hosts is None:
            host_rows = host_alias.tensor.shape[0] * cfg.page_size
            hosts = self._hosts[alias] = (
                (ctypes.c_void_p * B)(*([alias] * B)), (ctypes.c_int64 * B)(*([host_rows] * B)),
            )
        mh, md, mc, ns = self._miss_args
        row_bytes = cfg.kv_heads * cfg.head_dim * pool.element_size()
        _lib.check(
            lib.hs_gather_rows_batched(hosts[0], pool.data_ptr(), mh, md, mc, ns, hosts[1],
                                       pool.shape[0] * cfg.page_size, B, cfg.page_size, row_bytes, grid_x,
                                       _handle(stream, self.device)),
            "hs_gather_rows_batched",
        )

    def attend(self, queries, pool, out=None, stream=None):
        """Group attention over the deduplicated rows of every (request, KV head)."""
        cfg = self.config
        q = queries if queries.dtype == pool.dtype else queries.to(pool.dtype)
        q = q.contiguous()
        if out is None:
            out = torch.empty_like(q)
        lib = _lib.load()
        s = _handle(stream, self.device)
        _lib.check(
            lib.hs_attend_groups(
                q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), _lib.dtype_code(pool.dtype),
                cfg.page_size, cfg.kv_heads, cfg.head_dim, pool.shape[0] * cfg.page_size,
                self.union_physical.data_ptr(), self.union_physical.stride(0),
                self.entry_columns.data_ptr(), self.entry_masks.data_ptr(),
                self.entry_columns.stride(0), self.entry_columns.stride(1), self.entry_counts.data_ptr(),
                self.entry_capacity, self.batch, self.heads, out.data_ptr(), out.stride(0), out.stride(1),
                self.attend_ws.data_ptr(), self.attend_ws_bytes, s,
            ),
            "hs_attend_groups",
        )
        return out

    def head_physical(self):
        """[B, heads, width] physical rows of each head's columns (row_index.py:127-131):
        the union row a column names, -1 for padding.  What ``physical`` holds with
        ``head_rows``; torch ops on the device, for checks and byte counts."""
        cols = self.head_columns
        B = cols.shape[0]
        flat = cols.clamp(min=0).reshape(B, -1)
        rows = torch.gather(self.union_physical, 1, flat).view_as(cols)
        return torch.where(cols >= 0, rows, torch.full_like(rows, -1))

    def entry_offsets(self, pool):
        """Byte offsets of the K segments `attend` reads (one per valid entry; host-side
        torch ops, for the diagnostic read probe)."""
        cfg = self.config
        P, Hkv, D, esz = cfg.page_size, cfg.kv_heads, cfg.head_dim, pool.element_size()
        offsets = []
        counts = self.entry_counts.tolist()
        for b in range(self.batch):
            for k in range(Hkv):
                cols = self.entry_columns[b, k, : counts[b][k]].long()
                phys = self.union_physical[b][cols.clamp(min=0)]
                phys = phys[(cols >= 0) & (phys >= 0) & (phys < pool.shape[0] * P)]
                offsets.append((((phys // P) * 2 * P + phys % P) * Hkv + k) * D * esz)
        return torch.cat(offsets).contiguous()

    def probe_reads(self, pool, offsets, sink, stream=None):
        """Read-only pass over the K and V segments at `offsets` (diagnostic ceiling)."""
        cfg = self.config
        esz = pool.element_size()
        s = _handle(stream, self.device)
        _lib.check(
            _lib.load().hs_probe_row_reads(
                pool.data_ptr(), pool.numel() * esz, offsets.data_ptr(), offsets.numel(), cfg.head_dim * esz,
                cfg.page_size * cfg.kv_heads * cfg.head_dim * esz, sink.data_ptr(), s,
            ),
            "hs_probe_row_reads",
        )

    def step(self, queries, minimums, maximums, tables, pool, host_alias, transfer, *, row_stats=None, last_use=None):
        """The whole layer; returns (out, ready_event, done_event).

        ``last_use`` (optional event) is the previous reader of the hot rows;
        the gather waits for it, as hybrid.py:457 does.
        """
        compute = torch.cuda.current_stream(self.device)
        self.select(queries, minimums, maximums)
        self.resolve(tables, row_stats=row_stats)
        resolved = torch.cuda.Event()
        resolved.record(compute)
        transfer.wait_event(resolved)
        if last_use is not None:
            transfer.wait_event(last_use)
        self.gather(host_alias, pool, transfer)
        ready = torch.cuda.Event()
        ready.record(transfer)
        compute.wait_event(ready)
        out = self.attend(queries, pool)
        done = torch.cuda.Event()
        done.record(compute)
        return out, ready, done


class PipelinedSparseDecode:
    """The same layer for B requests as contiguous request groups, overlapped.

    Group g's gather (transfer stream) starts as soon as g is resolved, while
    the compute stream selects and resolves group g+1; group g's attention runs
    while later groups gather.  Each group is a :class:`BatchedSparseDecode`
    with its own buffers; per group the stream and event order is that of
    ``BatchedSparseDecode.step``.  ``split_front`` is passed to every group (the
    resolver's multi-workgroup front, for affine source tables).
    """

    def __init__(self, config, heads, top_pages, lengths, *, parts=2, keep_sink=True, device="cuda",
                 capacity_lengths=None, split_front=False):
        lengths = list(lengths)
        caps = list(capacity_lengths or lengths)
        parts = max(1, min(parts, len(lengths)))
        bounds = [round(i * len(lengths) / parts) for i in range(parts + 1)]
        self.slices = [slice(bounds[i], bounds[i + 1]) for i in range(parts)]
        self.parts = [
            BatchedSparseDecode(config, heads, top_pages, lengths[s], keep_sink=keep_sink, device=device,
                                capacity_lengths=caps[s], split_front=split_front)
            for s in self.slices
        ]
        self.batch = len(lengths)
        self.device = torch.device(device)

    def set_lengths(self, lengths):
        for s, part in zip(self.slices, self.parts):
            part.set_lengths(list(lengths)[s])

    def step(self, queries, minimums, maximums, tables, pool, host_alias, transfer, *, row_stats=None, out=None):
        """The whole layer for all groups; returns (out [B, Hq, D], done_event).  With
        ``transfer`` None every stage runs on the compute stream (no hand-offs, no overlap)."""
        compute = torch.cuda.current_stream(self.device)
        if out is None:
            out = torch.empty_like(queries if queries.dtype == pool.dtype else queries.to(pool.dtype))
        if transfer is None:
            for s, part in zip(self.slices, self.parts):
                part.select(queries[s], minimums[s], maximums[s])
                part.resolve(tables[s], row_stats=row_stats)
                part.gather(host_alias, pool, compute)
                part.attend(queries[s], pool, out=out[s])
        else:
            ready = []
            for s, part in zip(self.slices, self.parts):
                part.select(queries[s], minimums[s], maximums[s])
                part.resolve(tables[s], row_stats=row_stats)
                resolved = torch.cuda.Event()
                resolved.record(compute)
                transfer.wait_event(resolved)
                part.gather(host_alias, pool, transfer)
                event = torch.cuda.Event()
                event.record(transfer)
                ready.append(event)
            for s, part, event in zip(self.slices, self.parts, ready):
                compute.wait_event(event)
                part.attend(queries[s], pool, out=out[s])
        done = torch.cuda.Event()
        done.record(compute)
        return out, done
