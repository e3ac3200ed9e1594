"""Hybrid residency policy: block leases on one slab, token-row hot contents.

Behaviour follows the reference ``HybridKVCache`` (hybrid.py:106-609) decision
for decision, so row statistics and residency trajectories are the same:

* admission reserves, per layer, credits for a fixed hot region
  (``ceil(hot_rows / P)`` blocks) plus two active tail pages;
* resident history may borrow every unused credit; when a layer's window,
  the free-block watermark or allocation pressure demands it, the layer
  takes its whole hot region at once and its clean, sealed history (outside
  the two tails) becomes reclaimable: still readable until a new owner
  actually takes the block;
* each attention resolves selected tokens to physical rows on the GPU, loads
  misses from pinned host memory on the transfer stream, and reads rows after
  the load's event (``RowLease``).

Differences in structure (not behaviour): kernels come from an ops backend
(HIP by default), per-layer page scans use the allocator's per-layer index,
and Quest selections may stay on the device (``DeviceSelection``).
"""

from __future__ import annotations

from collections import Counter
from contextlib import suppress
from dataclasses import dataclass, field
from math import ceil

import torch

from .allocator import DeviceAllocator
from .config import CapacityError
from .row_index import LogicalTopK
from .storage import HostStore, Location, PageLease

ACTIVE_TAIL_PAGES = 2  # the appending page and the one before it stay resident


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
    source: torch.Tensor  # [pages] int32 host slot of each logical page
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

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.source, self.resident, self.hot, self.tags, self.lru))


class RowLease:
    """Resolved rows of one (request, layer), readable between wait() and release()."""

    def __init__(self, cache, tables, plan, pages):
        self.cache, self.tables, self.plan, self.pages = cache, tables, plan, pages
        slots = cache.allocator.slots
        self.handles = [(i, slots[i].generation, slots[i].owner) for i in tables.blocks + [p.slot for p in pages]]
        self.released = False

    def _validate(self):
        self.cache.storage.check_stream()
        if self.released:
            raise RuntimeError("row lease already released")
        for handle in self.handles:
            self.cache.allocator.validate(*handle)

    def wait(self):
        self._validate()
        self.cache.storage.wait(self.cache.storage.compute, self.tables.ready)

    def release(self):
        self._validate()
        storage = self.cache.storage
        self.tables.last_use = storage.event(storage.compute)
        for page in self.pages:
            page.last_use = self.tables.last_use
            page.pins -= 1
            if not page.pins:
                storage.pinned.discard(page.key)
        self.tables.busy = False
        self.released = True

    def __enter__(self):
        self.wait()
        return self

    def __exit__(self, *_):
        self.release()


class HybridKVCache:
    """One slab; resident blocks and per-layer hot regions lease from it."""

    def __init__(self, config, hot: HotConfig, ops=None):
        if ops is None:
            from .ops import default_ops

            ops = default_ops(config.device)
        self.ops = ops
        self.hot_config = hot
        self.hot_blocks = ceil(hot.hot_rows / config.page_size)
        self.tables: dict[tuple, LayerTables] = {}
        self._writing_key = None
        self.pending_clean: set = set()
        self.config = config
        self.allocator = DeviceAllocator(config)
        self.storage = HostStore(config, self.allocator)
        self.pool, self.device = self.allocator.storage, self.storage.device
        if config.host_pages * config.page_size >= 2**31:
            raise ValueError("host row tags require int32 addresses")
        self.row_stats = torch.zeros(3, dtype=torch.int64, device=self.device)
        self._host_source = ops.host_source(self.storage.host)

    # -- views ---------------------------------------------------------------
    @property
    def index_bytes(self):
        return self.storage.index_bytes

    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return self.storage.owners

    def _owner(self, slot):
        return self.allocator.slots[slot].owner

    def index_reservation_bytes(self, max_tokens, layers):
        tables = ceil(max_tokens / self.config.page_size) * 8 + self.hot_blocks * 4 + self.hot_config.hot_rows * 12
        return self.storage.index_reservation_bytes(max_tokens, layers) + layers * tables

    def admission_blocks(self, layers):
        return self.hot_config.admission_blocks(self.config.page_size, layers)

    @property
    def transition_watermark(self):
        configured = self.hot_config.transition_watermark
        return max(self.hot_blocks, self.budget // 10) if configured is None else configured

    # -- block supply --------------------------------------------------------
    def _readable_unpinned(self):
        pages = self.storage.pages
        return [
            i for i in self.allocator.reclaimable if i < self.budget and not pages[self._owner(i)].pins
        ]

    def _available_blocks(self):
        """Empty blocks (ascending) first, then readable unpinned blocks (unpin order)."""
        empty = sorted(i for i in self.allocator.free if i < self.budget)
        return empty + self._readable_unpinned()

    def _available_count(self):
        return sum(1 for i in self.allocator.free if i < self.budget) + len(self._readable_unpinned())

    def _first_available(self):
        empty = [i for i in self.allocator.free if i < self.budget]
        if empty:
            return min(empty)
        readable = self._readable_unpinned()
        return readable[0] if readable else None

    def _take_block(self, slot):
        if slot in self.allocator.reclaimable:
            self.allocator.reclaim(slot)
        return slot

    def _on_block_reused(self, slot):
        page = self.storage.pages[self._owner(slot)]
        assert not page.pins and page.host_committed_version == page.content_version
        self._detach(page)
        self.storage.stats["unpinned_block_reuses"] += 1

    # -- admission -----------------------------------------------------------
    def reserve(self, request_id, max_tokens, layers):
        self.collect()
        promised = sum(self.admission_blocks(r.layers) for r in self.storage.requests.values())
        if promised + self.admission_blocks(layers) > self.budget:
            raise CapacityError("hot-region + active-tail credits exhausted; defer admission")
        extra = self.index_reservation_bytes(max_tokens, layers) - self.storage.index_reservation_bytes(max_tokens, layers)
        self.storage.reserve(request_id, max_tokens, layers, extra_index_bytes=extra)
        pages = self.storage.requests[request_id].page_count
        hot_rows = self.hot_config.hot_rows

        def empty(size):
            return torch.full((size,), -1, dtype=torch.int32, device=self.device)

        for layer in range(layers):
            self.tables[request_id, layer] = LayerTables(
                empty(pages),
                empty(pages),
                empty(self.hot_blocks),
                empty(hot_rows),
                torch.arange(hot_rows, device=self.device, dtype=torch.int64),
            )

    # -- append placement ----------------------------------------------------
    def _prepare_append(self, page):
        self._writing_key = page.key
        tables = self.tables[page.key[:2]]
        # table entries are set with fill kernels on the compute stream: assigning a
        # Python int to a device element is a synchronising copy on ROCm PyTorch
        tables.source[page.key[2]].fill_(page.host_slot)
        if page.valid_tokens:
            if page.slot is None:
                raise RuntimeError("active append tail lost its resident lease")
            page.pins += 1
            self.storage.pinned.add(page.key)
            self.storage.stats["resident_hits"] += 1
            self.storage.stats["append_resident_hits"] += 1
            return PageLease(self.storage, [page])
        slot = self._slot()
        self.storage.wait(self.storage.compute, self.allocator.slots[slot].fence)
        self._bind(page, slot, Location.RESIDENT)
        return None

    def _bind(self, page, slot, location):
        self.storage.bind(page, slot, location)
        self.tables[page.key[:2]].resident[page.key[2]].fill_(slot)

    def _detach(self, page):
        self.tables[page.key[:2]].resident[page.key[2]].fill_(-1)
        self.storage.detach(page)

    def _tail_of(self, group):
        if self._writing_key is not None and self._writing_key[:2] == group:
            return self._writing_key[2]
        length = self.storage.requests[group[0]].lengths[group[1]]
        return (length - 1) // self.config.page_size

    def _historical_pages(self, group=None):
        """Sealed, unleased resident pages outside the two active tails, in bind order."""
        keys = self.allocator.lru if group is None else self.allocator.group_pages(group)
        tails = {}
        candidates = []
        for key in keys:
            if key[2] < 0:  # a hot block lease, not a logical page
                continue
            page = self.storage.pages[key]
            g = key[:2]
            if g not in tails:
                tails[g] = self._tail_of(g)
            if page.sealed and not page.pins and key[2] <= tails[g] - ACTIVE_TAIL_PAGES:
                candidates.append(page)
        return candidates

    def _publish_clean(self):
        for key in list(self.pending_clean):
            page = self.storage.pages.get(key)
            if page is None:
                self.pending_clean.discard(key)
            elif page.host_ready is None or page.host_ready.query():
                page.host_committed_version = page.host_enqueued_version
                self.pending_clean.discard(key)
                self.storage.stats["host_mirror_completions"] += 1

    def _unpin_clean_pages(self, group):
        if not self.tables[group].blocks:
            return
        # tail-first, like the reference; empty blocks still take precedence
        for page in sorted(self._historical_pages(group), key=lambda p: -p.key[2]):
            if page.host_committed_version == page.content_version and page.slot not in self.allocator.reclaimable:
                self.allocator.unpin(page.slot, self._on_block_reused)
                self.storage.stats["clean_page_unpins"] += 1

    def _require_hot(self, group, reason):
        tables = self.tables[group]
        if not tables.hot_required:
            tables.hot_required, tables.trigger = True, reason
            self.storage.stats[f"hot_trigger_{reason}"] += 1

    def _groups(self, request_id, layer):
        live = self.storage.requests
        if request_id is not None and layer is not None:
            group = (request_id, layer)
            return [group] if group in self.tables and request_id in live else []
        return [
            g
            for g in self.tables
            if g[0] in live and (request_id is None or g[0] == request_id) and (layer is None or g[1] == layer)
        ]

    def update_residency(self, request_id=None, layer=None, *, upcoming_allocation=False):
        """Publish finished mirrors and raise / serve persistent hot demand; never blocks.

        A per-layer resident window stands in for a scheduler-derived window;
        before an append allocation the watermark uses projected free capacity.
        """
        self.storage.check_stream()
        self._publish_clean()
        groups = self._groups(request_id, layer)
        for group in groups:
            self._unpin_clean_pages(group)
        for group in groups:
            tables = self.tables[group]
            residents = len(self.allocator.group_pages(group))
            if not residents:
                continue
            if not tables.hot_required:
                free = self._available_count() - int(upcoming_allocation)
                if free < self.transition_watermark:
                    self._require_hot(group, "watermark")
                elif residents >= self.hot_config.resident_window_pages:
                    self._require_hot(group, "window")
            if tables.hot_required and not tables.blocks and not tables.busy:
                try:
                    self.transition_to_host(*group)
                except CapacityError:
                    pass  # retried at the next policy tick; mappings and demand are kept
            self._unpin_clean_pages(group)

    def transition_to_host(self, request_id, layer):
        """Lease the whole hot region atomically, then make history reclaimable."""
        self.storage.check_stream()
        group = request_id, layer
        tables = self.tables[group]
        if tables.blocks:
            return
        self._require_hot(group, "explicit")
        if tables.busy:
            raise CapacityError("cannot transition an active row lease")
        self._publish_clean()
        free = self._available_blocks()
        in_free = set(free)
        victims = [
            p
            for p in self._historical_pages(group)
            if p.host_committed_version == p.content_version and p.slot not in in_free
        ]
        needed = max(0, self.hot_blocks - len(free))
        if len(victims) < needed:
            raise CapacityError("cannot acquire complete hot region while blocks are leased")
        # every check precedes every mutation; fences keep copies and readers of a
        # just-detached block ordered before its reuse as a hot block
        for page in victims[:needed]:
            free.append(page.slot)
            self.allocator.unpin(page.slot, self._on_block_reused)
            self.storage.stats["clean_page_unpins"] += 1
        blocks = free[: self.hot_blocks]
        for i, block in enumerate(blocks):
            self._take_block(block)
            self.storage.wait(self.storage.transfer, self.allocator.slots[block].fence)
            self.allocator.bind(block, (request_id, layer, -i - 1))
        tables.blocks = blocks
        staged = torch.tensor(blocks, dtype=torch.int32)
        if self.storage.cuda:  # pinned staging: no host synchronisation on the decode path
            staged = staged.pin_memory()
        tables.hot.copy_(staged, non_blocking=self.storage.cuda)
        tables.ready = self.storage.event(self.storage.transfer)
        self.storage.stats["hot_region_allocations"] += 1
        self._unpin_clean_pages(group)

    def _slot(self):
        while True:
            self.update_residency(upcoming_allocation=True)
            first = self._first_available()
            if first is not None:
                return self._take_block(first)
            candidates = self._historical_pages()
            counts = Counter(p.key[:2] for p in candidates)
            for group, count in counts.most_common():
                if count >= self.hot_blocks + 1 and not self.tables[group].blocks:
                    self._require_hot(group, "pressure")
                    try:
                        self.transition_to_host(*group)
                    except CapacityError:
                        continue
                    first = self._first_available()
                    if first is not None:
                        return self._take_block(first)
            pending = [
                p for p in candidates if p.host_committed_version < p.content_version and p.host_ready is not None
            ]
            if not pending:
                raise CapacityError("no reclaimable resident block; tails/readers are protected")
            # a synchronous runner cannot suspend mid-prefill: wait for one useful
            # mirror event, never for the whole device
            pending[0].host_ready.synchronize()
            self.storage.stats["pressure_mirror_waits"] += 1

    def reclaim_history(self, request_id, layer, *, evict=False):
        """Make completed history allocatable while still readable (evict: take it now)."""
        self.transition_to_host(request_id, layer)
        self._unpin_clean_pages((request_id, layer))
        if evict:
            for page in self._historical_pages((request_id, layer)):
                if page.slot in self.allocator.reclaimable:
                    self._take_block(page.slot)

    def _after_write(self, page):
        self.pending_clean.add(page.key)
        self.update_residency(*page.key[:2])

    def write(self, request_id, layer, k, v):
        if self.tables[request_id, layer].busy:
            raise RuntimeError("cannot append during a row lease")
        try:
            self.storage.append(request_id, layer, k, v, self._prepare_append, self._after_write)
        finally:
            self._writing_key = None

    # -- decode --------------------------------------------------------------
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
        if build is not None:
            topk = build(query.device, max_rows=self.hot_config.max_union_rows)
        else:
            topk = LogicalTopK.from_selection(selection, query.device)
        return row_attention(query, self, request_id, layer, topk, backend)

    def resolve(self, request_id, layer, topk: LogicalTopK):
        storage = self.storage
        storage.check_stream()
        topk.validate(self.device, self.hot_config.max_union_rows)
        tables = self.tables[request_id, layer]
        if tables.busy:
            raise RuntimeError("hot contents already leased by this layer")
        length = storage.requests[request_id].lengths[layer]
        if length < 1:
            raise ValueError("cannot resolve an empty history")
        # pin this layer's residents: the selected rows are not read back to the host
        pages = [storage.pages[key] for key in self.allocator.group_pages((request_id, layer))]
        for page in pages:
            page.pins += 1
            storage.pinned.add(page.key)
        tables.busy = True
        try:
            storage.wait(storage.compute, tables.ready)
            plan = self.ops.resolve_rows(
                topk, tables.source, tables.resident, tables.hot, tables.tags, tables.lru,
                length, self.config.page_size, row_stats=self.row_stats,
            )
            resolved = storage.event(storage.compute)
            storage.wait(storage.transfer, resolved)
            storage.wait(storage.transfer, tables.last_use)
            # append mirrors and earlier loads already precede this on the transfer stream
            with storage.context(storage.transfer):
                self.ops.gather_rows(self._host_source, self.pool, plan, self.config)
            tables.ready = storage.event(storage.transfer)
            if storage.cuda:  # plan tensors are produced on compute, read on transfer
                plan.miss_host_rows.record_stream(storage.transfer)
                plan.miss_device_rows.record_stream(storage.transfer)
                plan.counts.record_stream(storage.transfer)
            return RowLease(self, tables, plan, pages)
        except Exception:
            for page in pages:
                page.pins -= 1
                if not page.pins:
                    storage.pinned.discard(page.key)
            tables.busy = False
            raise

    # -- release -------------------------------------------------------------
    def release_request(self, request_id, wait=True):
        storage = self.storage
        groups = [t for (name, _), t in self.tables.items() if name == request_id]
        if any(t.busy for t in groups) or any(storage.pages[key].pins for key in storage.requests[request_id].keys):
            raise RuntimeError("cannot release a request with active row leases")
        for tables in groups:
            storage.wait(storage.transfer, tables.ready)
            storage.wait(storage.transfer, tables.last_use)
            fence = storage.event(storage.transfer)
            for block in tables.blocks:
                self.allocator.release(block, fence)
        for key in storage.requests[request_id].keys:
            page = storage.pages[key]
            if page.slot is not None:
                self._detach(page)
        storage.retire(request_id, keepalive=groups)
        for key in [key for key in self.tables if key[0] == request_id]:
            del self.tables[key]
        self.collect(wait=wait)

    def collect(self, wait=False):
        self.storage.collect(wait)
        self.update_residency()

    def page_state(self, key):
        state = self.storage.page_state(key)
        page = self.storage.pages[key]
        unpinned = page.slot in self.allocator.reclaimable
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
        # the gather reads pinned memory from the GPU; drain before teardown only
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
        storage, allocator = self.storage, self.allocator
        storage.assert_invariants()
        for name, request in storage.requests.items():
            assert request.extra_index_bytes == sum(t.nbytes for g, t in self.tables.items() if g[0] == name)
        assert not (allocator.free & allocator.reclaimable.keys())
        for slot in allocator.reclaimable:
            page = storage.pages[self._owner(slot)]
            assert page.slot == slot and page.sealed
            assert page.host_committed_version == page.content_version
            assert self.tables[page.key[:2]].blocks
            length = storage.requests[page.key[0]].lengths[page.key[1]]
            assert page.key[2] <= (length - 1) // self.config.page_size - ACTIVE_TAIL_PAGES
        assert sum(self.admission_blocks(r.layers) for r in storage.requests.values()) <= self.budget
        for group, tables in self.tables.items():
            assert len(tables.blocks) in (0, self.hot_blocks)
            assert sorted(tables.lru.tolist()) == list(range(self.hot_config.hot_rows))
            tags = [tag for tag in tables.tags.tolist() if tag >= 0]
            assert len(tags) == len(set(tags))
            if not tables.blocks:
                assert not tags
            else:
                assert tables.hot_required
            for i, block in enumerate(tables.blocks):
                assert self.owners[block] == (*group, -i - 1)
            residents = tables.resident.tolist()
            for index, host in enumerate(tables.source.tolist()):
                page = storage.pages.get((*group, index))
                assert host == (-1 if page is None else page.host_slot)
                assert residents[index] == (-1 if page is None or page.slot is None else page.slot)
                if page is not None and page.slot is None:
                    assert tables.blocks
