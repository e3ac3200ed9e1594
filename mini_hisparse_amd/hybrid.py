"""Hybrid residency: resident-page block leases and per-layer token-row hot regions
on one device slab.

Policy (the reference's ``HybridKVCache``, ``mini_hisparse/hybrid.py:106-609``;
its observable decisions are kept so row statistics and counters match):

* admission reserves, per layer, the blocks of a fixed hot region
  (``ceil(hot_rows / P)``) plus the two active tail pages; resident history may
  borrow every block nobody has reserved;
* a layer *requires* its hot region when the allocatable blocks fall under the
  watermark, when its resident pages reach the window, under allocation
  pressure, or on request; it then takes the whole region at once, and its
  clean, sealed history outside the two tails becomes *reclaimable*: readable
  until another owner actually takes the block;
* an attention resolves selected tokens to physical rows on the device, loads
  the misses from pinned host memory on the transfer stream, and reads the
  rows after the load's event (:class:`RowLease`).

Structure (this module's own): the policy works on the storage's per-(request,
layer) page arrays and the allocator's block table -- candidate sets are array
masks ordered by bind stamps, not scans over page objects -- and the device
tables ``source``/``resident`` are mirrors of the host arrays, uploaded in one
copy of the changed range before the resolver reads them instead of one element
write per page event.  Kernels come from an ops backend (HIP by default).
"""

from __future__ import annotations

from collections import Counter
from contextlib import suppress
from dataclasses import dataclass, field
from math import ceil

import numpy as np
import torch

from .allocator import NO_GROUP, DeviceAllocator
from .config import CapacityError
from .row_index import LogicalTopK
from .storage import HostStore, Location, Page, PageLease

ACTIVE_TAIL_PAGES = 2  # the page being appended and the one before it stay resident


@dataclass(frozen=True)
class HotConfig:
    max_union_rows: int
    hot_rows: int | None = None
    resident_window_pages: int = 64
    transition_watermark: int | None = None

    def __post_init__(self):
        if self.max_union_rows < 1:
            raise ValueError("max_union_rows must be positive")
        if self.hot_rows is None:
            object.__setattr__(self, "hot_rows", 2 * self.max_union_rows)
        if self.hot_rows < self.max_union_rows or self.hot_rows > 32768:
            raise ValueError("hot_rows must cover max_union_rows and be <= 32768")
        if self.resident_window_pages < ACTIVE_TAIL_PAGES:
            raise ValueError("resident window must cover both active tail pages")
        if self.transition_watermark is not None and self.transition_watermark < 0:
            raise ValueError("transition watermark must be nonnegative")

    def admission_blocks(self, page_size, layers=1):
        return layers * (ceil(self.hot_rows / page_size) + ACTIVE_TAIL_PAGES)


@dataclass
class LayerTables:
    """Device tables of one (request, layer), read and updated by the resolver."""

    source: torch.Tensor  # [pages] int32 host slot of each logical page, -1
    resident: torch.Tensor  # [pages] int32 device block of a resident page, -1
    hot: torch.Tensor  # [hot_blocks] int32 device block of each hot block
    tags: torch.Tensor  # [hot_rows] int32 host row cached in each hot slot, -1
    lru: torch.Tensor  # [hot_rows] int64 hot slots, least recent first
    blocks: list[int] = field(default_factory=list)
    ready: object = None
    last_use: object = None
    busy: bool = False
    hot_required: bool = False
    trigger: str | None = None
    stale: list = field(default_factory=lambda: [0, 0])  # [lo, hi) pages whose mirrors are not uploaded

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.source, self.resident, self.hot, self.tags, self.lru))


class RowLease:
    """Resolved rows of one (request, layer), readable between ``wait`` and ``release``."""

    def __init__(self, cache, group, tables, plan, pinned):
        self.cache, self.tables, self.plan = cache, tables, plan
        self._lp, self._pinned = cache.storage.layer_pages(*group), pinned
        self.handles = cache.allocator.snapshot(np.concatenate([np.asarray(tables.blocks, np.int64),
                                                                self._lp.slot[pinned]]))
        self.released = False

    @property
    def pages(self):
        group = self.cache.allocator.group_key(self._lp.gid)
        return [Page(self._lp, (*group, int(i))) for i in self._pinned]

    def _validate(self):
        self.cache.storage.check_stream()
        if self.released:
            raise RuntimeError("row lease already released")
        self.cache.allocator.validate_snapshot(self.handles)

    def wait(self):
        self._validate()
        self.cache.storage.wait(self.cache.storage.compute, self.tables.ready)

    def release(self):
        self._validate()
        done = self.cache.storage.event(self.cache.storage.compute)
        self.tables.last_use = done
        for i in self._pinned.tolist():
            self._lp.last_use[i] = done
        self._lp.pins[self._pinned] -= 1
        self.tables.busy = False
        self.released = True

    def __enter__(self):
        self.wait()
        return self

    def __exit__(self, *_):
        self.release()


class _PendingClean:
    """Pages written since the last publication of completed host mirrors (a set of
    page keys over a per-layer flag array)."""

    def __init__(self, cache):
        self._cache = cache
        self.layers = {}  # (request, layer) -> its page arrays, for layers that may hold flags

    def add(self, key):
        lp = self._cache.storage.layer_pages(*key[:2])
        lp.unpublished[key[2]] = True
        self.layers[key[:2]] = lp

    def discard(self, key):
        if key in self._cache.storage.pages:
            self._cache.storage.layer_pages(*key[:2]).unpublished[key[2]] = False

    def __contains__(self, key):
        return key in self._cache.storage.pages and bool(self._cache.storage.layer_pages(*key[:2]).unpublished[key[2]])

    def __len__(self):
        return sum(int(np.count_nonzero(lp.unpublished)) for r in self._cache.storage.requests.values() for lp in r.pages)


class HybridKVCache:
    """One slab; resident blocks and per-layer hot regions lease from it."""

    def __init__(self, config, hot: HotConfig, ops=None):
        if ops is None:
            from .ops import default_ops

            ops = default_ops(config.device)
        self.ops = ops
        self.config = config
        self.hot_config = hot
        self.hot_blocks = ceil(hot.hot_rows / config.page_size)
        if config.host_pages * config.page_size >= 2**31:
            raise ValueError("host row tags require int32 addresses")
        self.allocator = DeviceAllocator(config)
        self.storage = HostStore(config, self.allocator, ops)
        self.pool, self.device = self.allocator.storage, self.storage.device
        self.tables: dict[tuple, LayerTables] = {}
        self.row_stats = torch.zeros(3, dtype=torch.int64, device=self.device)
        self.pending_clean = _PendingClean(self)
        self._writing = None  # (group, page index) of the page being appended
        self._dirty: set = set()  # groups whose device tables lag their page arrays

    # -- views ------------------------------------------------------------------------
    @property
    def index_bytes(self):
        return self.storage.index_bytes

    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return self.storage.owners

    def index_reservation_bytes(self, max_tokens, layers):
        per_layer = ceil(max_tokens / self.config.page_size) * 8 + self.hot_blocks * 4 + self.hot_config.hot_rows * 12
        return self.storage.index_reservation_bytes(max_tokens, layers) + layers * per_layer

    def admission_blocks(self, layers):
        return self.hot_config.admission_blocks(self.config.page_size, layers)

    @property
    def transition_watermark(self):
        configured = self.hot_config.transition_watermark
        return max(self.hot_blocks, self.budget // 10) if configured is None else configured

    def _lp(self, group):
        return self.storage.layer_pages(*group)

    def _page(self, group, index):
        return Page(self._lp(group), (*group, int(index)))

    # -- block supply -------------------------------------------------------------------
    def _readable_blocks(self):
        """Reclaimable blocks inside the budget whose page is not pinned, in queue order."""
        table = self.allocator
        queue = table.reclaim_queue(self.budget)
        if not len(queue):
            return []
        groups, index = table.owner_group[queue], table.owner_index[queue]
        pinned = np.zeros(len(queue), bool)
        for g in np.unique(groups).tolist():
            mine = groups == g
            pinned[mine] = self._lp(table.group_key(g)).pins[index[mine]] != 0
        return queue[~pinned].tolist()

    def _available_blocks(self):
        """Empty blocks (ascending) first, then readable unpinned blocks (queue order)."""
        return self.allocator.free_blocks(self.budget).tolist() + self._readable_blocks()

    def _available_count(self):
        return len(self.allocator.free_blocks(self.budget)) + len(self._readable_blocks())

    def _first_available(self):
        empty = self.allocator.free_blocks(self.budget)
        if len(empty):
            return int(empty[0])
        readable = self._readable_blocks()
        return readable[0] if readable else None

    def _take_block(self, block):
        if self.allocator.reclaim_stamp[block] >= 0:
            self.allocator.reclaim(block)
        return block

    def _on_block_reused(self, block):
        table = self.allocator
        group = table.group_key(int(table.owner_group[block]))
        index = int(table.owner_index[block])
        lp = self._lp(group)
        if lp.pins[index] or lp.committed[index] != lp.version[index]:
            raise AssertionError("a reclaimable block must hold a clean, unpinned page")
        self._detach(self._page(group, index))
        self.storage.stats["unpinned_block_reuses"] += 1

    # -- admission -------------------------------------------------------------------------
    def reserve(self, request_id, max_tokens, layers):
        self.collect()
        promised = sum(self.admission_blocks(r.layers) for r in self.storage.requests.values())
        if promised + self.admission_blocks(layers) > self.budget:
            raise CapacityError("hot-region + active-tail credits exhausted; defer admission")
        extra = self.index_reservation_bytes(max_tokens, layers) - self.storage.index_reservation_bytes(max_tokens, layers)
        self.storage.reserve(request_id, max_tokens, layers, extra_index_bytes=extra)
        pages = self.storage.requests[request_id].page_count
        for layer in range(layers):
            empty = lambda n: torch.full((n,), -1, dtype=torch.int32, device=self.device)  # noqa: E731
            self.tables[request_id, layer] = LayerTables(
                empty(pages), empty(pages), empty(self.hot_blocks), empty(self.hot_config.hot_rows),
                torch.arange(self.hot_config.hot_rows, dtype=torch.int64, device=self.device),
            )

    # -- device tables ---------------------------------------------------------------------
    def _stale(self, group, index):
        lo, hi = self.tables[group].stale
        self.tables[group].stale = [index, index + 1] if lo >= hi else [min(lo, index), max(hi, index + 1)]
        self._dirty.add(group)

    def _sync_tables(self):
        """Upload every group's changed table range: called when a public operation
        that moves pages returns, so the device tables always match the page arrays
        outside the cache's own methods."""
        for group in self._dirty:
            if group in self.tables:
                self._upload(group)
        self._dirty.clear()

    def _upload(self, group):
        """Copy the changed range of ``source``/``resident`` from the page arrays."""
        tables = self.tables[group]
        lo, hi = tables.stale
        if lo >= hi:
            return
        lp = self._lp(group)
        rows = np.stack([lp.host_slot[lo:hi], lp.slot[lo:hi]]).astype(np.int32)
        staged = torch.from_numpy(rows)
        if self.storage.cuda:
            staged = staged.pin_memory()
        tables.source[lo:hi].copy_(staged[0], non_blocking=True)
        tables.resident[lo:hi].copy_(staged[1], non_blocking=True)
        tables.stale = [0, 0]

    # -- pages -------------------------------------------------------------------------------
    def _prepare_append(self, page: Page):
        group = page.key[:2]
        self._writing = (group, page.index)
        if page.valid_tokens:
            if page.slot is None:
                raise RuntimeError("active append tail lost its resident lease")
            page.pins = page.pins + 1
            self.storage.stats["resident_hits"] += 1
            self.storage.stats["append_resident_hits"] += 1
            return PageLease(self.storage, [page])
        block = self._slot()
        self.storage.wait(self.storage.compute, self.allocator.fence[block])
        self._bind(page, block, Location.RESIDENT)  # a new page: its source and resident entries
        return None

    def _bind(self, page, block, location):
        self.storage.bind(page, block, location)
        self._stale(page.key[:2], page.index)

    def _detach(self, page):
        self.storage.detach(page)
        self._stale(page.key[:2], page.index)

    def _tail_of(self, group):
        """Index of the page the next token of ``group`` writes (the page being
        appended while a write is open)."""
        if self._writing is not None and self._writing[0] == group:
            return self._writing[1]
        return (self.storage.requests[group[0]].lengths[group[1]] - 1) // self.config.page_size

    def _history_of(self, group):
        """Page indices of one layer's sealed, unpinned resident pages at least two pages
        behind its tail, in the order their blocks were bound (the layer's page-to-block
        map holds exactly its bound page blocks, so no scan of the whole slab)."""
        lp = self._lp(group)
        idx = lp.resident()
        idx = idx[lp.sealed[idx] & (lp.pins[idx] == 0) & (idx <= self._tail_of(group) - ACTIVE_TAIL_PAGES)]
        return idx[np.argsort(self.allocator.bind_stamp[lp.slot[idx]], kind="stable")]

    def _history(self, group=None):
        """(group, index) of every sealed, unpinned resident page at least two pages
        behind its layer's tail, in the order their blocks were bound."""
        if group is not None:
            return [(group, i) for i in self._history_of(group).tolist()]
        table = self.allocator
        blocks = table.bound_pages()
        found = []
        groups = table.owner_group[blocks]
        for g in np.unique(groups).tolist():
            key = table.group_key(g)
            if key[0] not in self.storage.requests:
                continue
            lp = self._lp(key)
            mine = blocks[groups == g]
            idx = table.owner_index[mine]
            ok = lp.sealed[idx] & (lp.pins[idx] == 0) & (idx <= self._tail_of(key) - ACTIVE_TAIL_PAGES)
            found.append(np.stack([table.bind_stamp[mine[ok]], np.full(ok.sum(), g), idx[ok]], 1))
        if not found:
            return []
        rows = np.concatenate(found)
        rows = rows[np.argsort(rows[:, 0], kind="stable")]
        return [(table.group_key(int(g)), int(i)) for _, g, i in rows.tolist()]

    def _clean(self, group, index):
        lp = self._lp(group)
        return lp.committed[index] == lp.version[index]

    def _publish_clean(self):
        """Mark pages whose host mirror has completed as clean (never waits).  Only the
        layers written since their last full publication are visited."""
        layers = self.pending_clean.layers
        for group, lp in list(layers.items()):
            request = self.storage.requests.get(group[0])
            if request is None or request.pages[group[1]] is not lp:
                del layers[group]  # released: its flags went with it
                continue
            for i in np.flatnonzero(lp.unpublished).tolist():
                event = lp.host_ready[i]
                if event is None or event.query():
                    lp.committed[i] = lp.enqueued[i]
                    lp.unpublished[i] = False
                    self.storage.stats["host_mirror_completions"] += 1
            if not lp.unpublished.any():
                del layers[group]

    def _unpin_clean_pages(self, group):
        """A layer with a hot region offers its clean history as reclaimable blocks,
        nearest the tail first (the upstream release order)."""
        if not self.tables[group].blocks:
            return
        lp = self._lp(group)
        idx = np.sort(self._history_of(group))[::-1]
        blocks = lp.slot[idx]
        todo = (lp.committed[idx] == lp.version[idx]) & (self.allocator.reclaim_stamp[blocks] < 0)
        for block in blocks[todo].tolist():
            self.allocator.unpin(block, self._on_block_reused)
            self.storage.stats["clean_page_unpins"] += 1

    def _require_hot(self, group, reason):
        tables = self.tables[group]
        if not tables.hot_required:
            tables.hot_required, tables.trigger = True, reason
            self.storage.stats[f"hot_trigger_{reason}"] += 1

    # -- policy ticks ----------------------------------------------------------------------------
    def update_residency(self, request_id=None, layer=None, *, upcoming_allocation=False):
        """Publish completed mirrors and raise / serve hot-region demand, without waiting.

        A per-layer resident window stands in for vLLM's scheduler-derived in-flight
        token window; before an append allocation the projected free capacity is used,
        so demand is raised before the last free block goes."""
        self.storage.check_stream()
        self._publish_clean()
        groups = [g for g in self.tables if g[0] in self.storage.requests
                  and request_id in (None, g[0]) and layer in (None, g[1])]
        for group in groups:
            self._unpin_clean_pages(group)
        # pins and the budget hold still inside this loop, so the available count changes
        # only with the allocator's version (a bind, release or unpin)
        counted = None
        for group in groups:
            tables = self.tables[group]
            lp = self._lp(group)
            residents = len(lp.resident())
            if not residents:
                continue
            if not tables.hot_required:
                if counted is None or counted[0] != self.allocator.version:
                    counted = self.allocator.version, self._available_count()
                if counted[1] - int(upcoming_allocation) < self.transition_watermark:
                    self._require_hot(group, "watermark")
                elif residents >= self.hot_config.resident_window_pages:
                    self._require_hot(group, "window")
            if tables.hot_required and not tables.blocks and not tables.busy:
                with suppress(CapacityError):
                    self.transition_to_host(*group)
            self._unpin_clean_pages(group)
        self._sync_tables()

    def transition_to_host(self, request_id, layer):
        """Take the layer's whole hot region at once, then make its history reclaimable."""
        self.storage.check_stream()
        group = request_id, layer
        tables = self.tables[group]
        if tables.blocks:
            return
        self._require_hot(group, "explicit")
        if tables.busy:
            raise CapacityError("cannot transition an active row lease")
        self._publish_clean()
        supply = self._available_blocks()
        lp = self._lp(group)
        offered = set(supply)
        victims = [i for _, i in self._history(group) if self._clean(group, i) and int(lp.slot[i]) not in offered]
        short = max(0, self.hot_blocks - len(supply))
        if len(victims) < short:
            raise CapacityError("cannot acquire complete hot region while blocks are leased")
        for index in victims[:short]:
            block = int(lp.slot[index])
            supply.append(block)
            self.allocator.unpin(block, self._on_block_reused)
            self.storage.stats["clean_page_unpins"] += 1
        blocks = supply[: self.hot_blocks]
        for i, block in enumerate(blocks):
            self._take_block(block)
            self.storage.wait(self.storage.transfer, self.allocator.fence[block])
            self.allocator.bind(block, (request_id, layer, -i - 1))
        tables.blocks = blocks
        staged = torch.tensor(blocks, dtype=torch.int32)
        tables.hot.copy_(staged.pin_memory() if self.storage.cuda else staged, non_blocking=True)
        tables.ready = self.storage.event(self.storage.transfer)
        self.storage.stats["hot_region_allocations"] += 1
        self._unpin_clean_pages(group)
        self._sync_tables()

    def _slot(self):
        """A block for a new resident page: an allocatable one, else one freed by moving
        the layer with the most history to its hot region, else wait for a mirror."""
        while True:
            self.update_residency(upcoming_allocation=True)
            block = self._first_available()
            if block is not None:
                return self._take_block(block)
            history = self._history()
            per_group = Counter(group for group, _ in history)
            for group, count in per_group.most_common():
                if count >= self.hot_blocks + 1 and not self.tables[group].blocks:
                    self._require_hot(group, "pressure")
                    try:
                        self.transition_to_host(*group)
                    except CapacityError:
                        continue
                    block = self._first_available()
                    if block is not None:
                        return self._take_block(block)
            waiting = [(g, i) for g, i in history
                       if not self._clean(g, i) and self._lp(g).host_ready[i] is not None]
            if not waiting:
                raise CapacityError("no reclaimable resident block; tails/readers are protected")
            group, index = waiting[0]
            self._lp(group).host_ready[index].synchronize()
            self.storage.stats["pressure_mirror_waits"] += 1

    def reclaim_history(self, request_id, layer, *, evict=False):
        """Make completed history allocatable while still readable (``evict``: take it now)."""
        group = request_id, layer
        self.transition_to_host(request_id, layer)
        self._unpin_clean_pages(group)
        if evict:
            lp = self._lp(group)
            for _, index in self._history(group):
                if self.allocator.reclaim_stamp[lp.slot[index]] >= 0:
                    self._take_block(int(lp.slot[index]))
        self._sync_tables()

    def _after_write(self, page):
        self.pending_clean.add(page.key)
        self.update_residency(*page.key[:2])

    def write(self, request_id, layer, k, v):
        if self.tables[request_id, layer].busy:
            raise RuntimeError("cannot append during a row lease")
        try:
            self.storage.append(request_id, layer, k, v, self._prepare_append, self._after_write)
        finally:
            self._writing = None
            self._sync_tables()

    # -- decode ---------------------------------------------------------------------------------
    def attention(self, query, request_id, layer, selection, backend="auto"):
        from .attention import row_attention

        length = self.storage.requests[request_id].lengths[layer]
        if selection.length != length or selection.page_size != self.config.page_size:
            raise ValueError("selection has stale length or wrong page size")
        heads = getattr(selection, "heads", None)
        if heads is None:
            heads = len(selection.positions)
        if heads != query.shape[0]:
            raise ValueError("selection must have one row per query head")
        build = getattr(selection, "logical_topk", None)
        if build is not None:  # a device-resident selection builds its union on the device
            topk = build(query.device, max_rows=self.hot_config.max_union_rows)
        else:
            topk = LogicalTopK.from_selection(selection, query.device)
        return row_attention(query, self, request_id, layer, topk, backend)

    def resolve(self, request_id, layer, topk: LogicalTopK):
        storage = self.storage
        storage.check_stream()
        topk.validate(self.device, self.hot_config.max_union_rows)
        group = request_id, layer
        tables = self.tables[group]
        if tables.busy:
            raise RuntimeError("hot contents already leased by this layer")
        length = storage.requests[request_id].lengths[layer]
        if length < 1:
            raise ValueError("cannot resolve an empty history")
        lp = self._lp(group)
        pinned = lp.resident()
        lp.pins[pinned] += 1
        tables.busy = True
        try:
            self._sync_tables()
            storage.wait(storage.compute, tables.ready)
            plan = self.ops.resolve_rows(topk, tables.source, tables.resident, tables.hot, tables.tags, tables.lru,
                                         length, self.config.page_size, row_stats=self.row_stats)
            resolved = storage.event(storage.compute)
            storage.wait(storage.transfer, resolved)
            storage.wait(storage.transfer, tables.last_use)
            with storage.context(storage.transfer):
                self.ops.gather_rows(storage.host_source, self.pool, plan, self.config)
            tables.ready = storage.event(storage.transfer)
            if storage.cuda:
                for tensor in (plan.miss_host_rows, plan.miss_device_rows, plan.counts):
                    tensor.record_stream(storage.transfer)
            return RowLease(self, group, tables, plan, pinned)
        except Exception:
            lp.pins[pinned] -= 1
            tables.busy = False
            raise

    # -- release -----------------------------------------------------------------------------------
    def release_request(self, request_id, wait=True):
        storage = self.storage
        request = storage.requests[request_id]
        groups = [(g, t) for g, t in self.tables.items() if g[0] == request_id]
        if any(t.busy for _, t in groups) or any(np.any(lp.pins > 0) for lp in request.pages):
            raise RuntimeError("cannot release a request with active row leases")
        for _, tables in groups:
            storage.wait(storage.transfer, tables.ready)
            storage.wait(storage.transfer, tables.last_use)
            fence = storage.event(storage.transfer)
            for block in tables.blocks:
                self.allocator.release(block, fence)
        for key in request.keys:
            if request.pages[key[1]].slot[key[2]] >= 0:
                self._detach(storage.pages[key])
        storage.retire(request_id, keepalive=[t for _, t in groups])
        for group, _ in groups:
            del self.tables[group]
        self.collect(wait=wait)

    def collect(self, wait=False):
        self.storage.collect(wait)
        self.update_residency()

    def page_state(self, key):
        state = self.storage.page_state(key)
        page = self.storage.pages[key]
        unpinned = page.slot is not None and self.allocator.reclaim_stamp[page.slot] >= 0
        clean = page.host_committed_version == page.content_version
        if page.slot is None:
            residency = "host_only"
        elif unpinned:
            residency = "clean_unpinned"
        else:
            residency = "clean_pinned" if clean else "dirty"
        state.update(allocation_pinned=page.slot is not None and not unpinned, residency=residency)
        return state

    def set_budget(self, pages):
        if pages != self.budget:
            raise CapacityError("hybrid block budget is fixed; hot leases need readmission to resize")

    def close(self):
        self.storage.synchronize()

    def __del__(self):
        with suppress(RuntimeError, AttributeError, TypeError):
            if getattr(getattr(self, "storage", None), "cuda", False):
                self.close()

    def reset_stats(self):
        self.storage.stats.clear()
        self.row_stats.zero_()

    def snapshot(self):
        result = self.storage.snapshot()
        resident, hot, misses = self.row_stats.cpu().tolist()
        result.update(
            cache_layout="hybrid_rows",
            eviction_policy="resident-reclaim + per-layer row-LRU",
            max_union_rows=self.hot_config.max_union_rows,
            hot_rows=self.hot_config.hot_rows,
            active_tail_pages=ACTIVE_TAIL_PAGES,
            resident_window_pages=self.hot_config.resident_window_pages,
            transition_watermark=self.transition_watermark,
            empty_device_blocks=len(self.allocator.free),
            readable_unpinned_blocks=len(self.allocator.reclaimable),
            allocatable_device_blocks=self._available_count(),
            pending_clean_pages=len(self.pending_clean),
            hot_pending_groups=sum(t.hot_required and not t.blocks for t in self.tables.values()),
            hot_leased_blocks=sum(len(t.blocks) for t in self.tables.values()),
            admission_block_credits=sum(self.admission_blocks(r.layers) for r in self.storage.requests.values()),
            row_stats={
                "resident_hits": resident,
                "hot_hits": hot,
                "misses": misses,
                "h2d_bytes": misses * self.storage.page_bytes // self.config.page_size,
            },
        )
        return result

    def assert_invariants(self):
        storage, table = self.storage, self.allocator
        storage.assert_invariants()
        for name, request in storage.requests.items():
            assert request.extra_index_bytes == sum(t.nbytes for g, t in self.tables.items() if g[0] == name)
        queued = table.reclaim_queue()
        assert np.all(table.owner_group[queued] != NO_GROUP)
        for block in queued.tolist():
            group = table.group_key(int(table.owner_group[block]))
            index = int(table.owner_index[block])
            lp = self._lp(group)
            assert lp.slot[index] == block and lp.sealed[index] and self._clean(group, index)
            assert self.tables[group].blocks
            length = storage.requests[group[0]].lengths[group[1]]
            assert index <= (length - 1) // self.config.page_size - ACTIVE_TAIL_PAGES
        assert sum(self.admission_blocks(r.layers) for r in storage.requests.values()) <= self.budget
        for group, tables in self.tables.items():
            self._upload(group)
            assert len(tables.blocks) in (0, self.hot_blocks)
            lru = tables.lru.cpu().numpy()
            assert np.array_equal(np.sort(lru), np.arange(self.hot_config.hot_rows))
            tags = tables.tags.cpu().numpy()
            tags = tags[tags >= 0]
            assert len(tags) == len(np.unique(tags))
            assert tables.hot_required if tables.blocks else not len(tags)
            for i, block in enumerate(tables.blocks):
                assert table.owner_key(block) == (*group, -i - 1)
            lp = self._lp(group)
            m = lp.materialized
            source, resident = tables.source.cpu().numpy(), tables.resident.cpu().numpy()
            assert np.array_equal(source[:m], lp.host_slot[:m]) and np.all(source[m:] == -1)
            assert np.array_equal(resident[:m], lp.slot[:m]) and np.all(resident[m:] == -1)
            if np.any(lp.slot[:m] < 0):
                assert tables.blocks
