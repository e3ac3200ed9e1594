"""Host-backed KV history: the pinned host pool, per-(request, layer) page arrays,
batched writes and event-safe retirement.

Replaces the reference's ``HostStore`` (``mini_hisparse/storage.py:101-441``)
with the same contract -- every request's full history lives in one pinned host
pool ``[host_pages, 2, P, Hkv, D]``; the device slab holds resident copies; a
write appends K/V to the tail, updates the Quest bounds (exact K extrema in the
KV dtype) and the page-mean summaries, and mirrors the new rows to host memory;
host slots of a retired request return to the free list only after its
retirement event -- organised differently:

* page state is kept per (request, layer) in :class:`LayerPages`, a set of
  arrays over that layer's logical pages (host slot, device block, valid rows,
  pins, content / mirror versions, sealed flag, events), not one object per page;
  :class:`Page` is a view onto one entry, for callers that inspect a page;
* a write first makes every placement decision page by page (the caller's
  ``prepare_page`` / ``after_write`` hooks run in page order, as the policy
  requires), then moves the data of all its pages -- pool rows, host mirror,
  bounds, summaries -- in one batched kernel launch (``ops.append_tokens``).
  The host mirror is written straight from the new K/V, so a page that the
  policy detaches again later in the same write keeps its bytes.  When the
  policy has to wait for a page of the write that is not launched yet (a
  detach, a mirror-completion wait), the pages placed so far are launched
  first (``_flush``), so every wait ends.

Storage knows no eviction policy: callers supply the placement of a new page
(``prepare_page``) and update their policy after it (``after_write``).
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Mapping
from contextlib import nullcontext
from dataclasses import dataclass, field
from enum import Enum
from math import ceil

import numpy as np
import torch

from .allocator import NO_GROUP, DeviceAllocator
from .config import CacheConfig, CapacityError
from .streams import independent_stream

PageKey = tuple[str, int, int]


class Location(str, Enum):
    HOST = "host"
    RESIDENT = "resident"
    HOT = "hot"


_LOCATIONS = (Location.HOST, Location.RESIDENT, Location.HOT)
_CODE = {loc: i for i, loc in enumerate(_LOCATIONS)}
NEVER = -1_000_000_000


class LayerPages:
    """Page state of one (request, layer) as arrays over its logical pages.

    Pages are materialized in index order (appends are sequential), so the
    materialized pages are the prefix ``[0, materialized)``.
    """

    def __init__(self, gid, pages, generation):
        self.gid = gid
        self.generation = generation
        self.materialized = 0
        self.host_slot = np.full(pages, -1, np.int64)
        self.slot = np.full(pages, -1, np.int64)
        self.location = np.zeros(pages, np.int8)
        self.valid = np.zeros(pages, np.int64)
        self.pins = np.zeros(pages, np.int64)
        self.version = np.zeros(pages, np.int64)
        self.enqueued = np.zeros(pages, np.int64)
        self.committed = np.zeros(pages, np.int64)
        self.sealed = np.zeros(pages, bool)
        self.stamp = np.zeros(pages, np.int64)  # materialization order across the store
        self.attended = np.full(pages, NEVER, np.int64)  # last attention epoch (page layout)
        self.touched = np.zeros(pages, np.int64)  # last touch of the page layout's clock
        self.unpublished = np.zeros(pages, bool)  # written since the last mirror publication
        self.ready = [None] * pages  # device contents written
        self.last_use = [None] * pages  # last reader done
        self.host_ready = [None] * pages  # host mirror written

    def resident(self):
        """Indices of the materialized pages that hold a device block."""
        return np.flatnonzero(self.slot[: self.materialized] >= 0)


class Page:
    """View of one logical page of a :class:`LayerPages` (the reference's ``Page``)."""

    __slots__ = ("_lp", "index", "key")

    def __init__(self, lp: LayerPages, key: PageKey):
        self._lp, self.index, self.key = lp, key[2], key

    def _get(self, name):
        return getattr(self._lp, name)[self.index]

    def _set(self, name, value):
        getattr(self._lp, name)[self.index] = value

    host_slot = property(lambda s: int(s._get("host_slot")))
    slot = property(lambda s: None if s._get("slot") < 0 else int(s._get("slot")))
    location = property(lambda s: _LOCATIONS[s._get("location")])
    valid_tokens = property(lambda s: int(s._get("valid")))
    sealed = property(lambda s: bool(s._get("sealed")))
    request_generation = property(lambda s: s._lp.generation)
    content_version = property(lambda s: int(s._get("version")))
    host_enqueued_version = property(lambda s: int(s._get("enqueued")))
    pins = property(lambda s: int(s._get("pins")), lambda s, v: s._set("pins", v))
    host_committed_version = property(lambda s: int(s._get("committed")), lambda s, v: s._set("committed", v))
    ready = property(lambda s: s._get("ready"), lambda s, v: s._set("ready", v))
    last_use = property(lambda s: s._get("last_use"), lambda s, v: s._set("last_use", v))
    host_ready = property(lambda s: s._get("host_ready"), lambda s, v: s._set("host_ready", v))
    last_attention_epoch = property(lambda s: int(s._get("attended")), lambda s, v: s._set("attended", v))

    def __eq__(self, other):
        return isinstance(other, Page) and other._lp is self._lp and other.index == self.index

    def __hash__(self):
        return hash((id(self._lp), self.index))

    def __repr__(self):
        return f"Page({self.key}, host_slot={self.host_slot}, slot={self.slot}, valid={self.valid_tokens})"


@dataclass
class RequestPages:
    """One admitted request: lengths, Quest bounds / summaries and its layers' pages."""

    max_tokens: int
    layers: int
    page_count: int
    lengths: list[int]
    summaries: torch.Tensor  # [layers, pages, Hkv, D] float32 page-mean K (selector "mean")
    minimum: torch.Tensor  # [layers, pages, Hkv, D] KV dtype, +inf before the first token
    maximum: torch.Tensor  # [layers, pages, Hkv, D] KV dtype, -inf before the first token
    host_credits: int
    generation: int
    pages: list[LayerPages] = field(default_factory=list)
    extra_index_bytes: int = 0
    name: str = ""
    keepalive: tuple = ()  # caller metadata retained until the retirement event

    @property
    def keys(self):
        """Materialized page keys of the request, in materialization order."""
        found = [(int(lp.stamp[i]), layer, i) for layer, lp in enumerate(self.pages) for i in range(lp.materialized)]
        return [(self.name, layer, i) for _, layer, i in sorted(found)]


class _PendingWrite:
    """Stands in for the events of pages whose data is not launched yet; asking to
    wait for it launches the pages placed so far (``HostStore._flush``)."""

    def __init__(self, store):
        self.store, self.event = store, None

    def query(self):
        return self.event is not None and self.event.query()

    def resolve(self):
        if self.event is None:
            self.store._flush()
        return self.event

    def synchronize(self):
        self.resolve().synchronize()


@dataclass
class _Write:
    """The open write of one (request, layer): pages placed, not yet launched."""

    request: RequestPages
    layer: int
    k: torch.Tensor
    v: torch.Tensor
    first_token: int  # offset into k / v of the first page not launched
    marker: _PendingWrite
    pages: list = field(default_factory=list)  # (index, within, count) in page order
    joins: list = field(default_factory=list)


class PageLease:
    """Pins protect mappings on the host; events protect bytes on the device."""

    def __init__(self, store: "HostStore", pages: list[Page]):
        self.store, self.pages, self.released = store, pages, False
        self.handles = [(p.slot, int(store.allocator.generation[p.slot]), p.key) for p in pages]

    def _validate(self):
        self.store.check_stream()
        if self.released:
            raise RuntimeError("lease already released")
        for handle in self.handles:
            self.store.allocator.validate(*handle)

    def wait(self):
        self._validate()
        for page in self.pages:
            self.store.wait(self.store.compute, page.ready)

    def release(self):
        self._validate()
        done = self.store.event(self.store.compute)
        for page in self.pages:
            page.last_use = done
            page.pins = page.pins - 1
        self.released = True

    def __enter__(self):
        self.wait()
        return self

    def __exit__(self, *_):
        self.release()


class _PageMap(Mapping):
    """``store.pages``: page key -> :class:`Page` view over every materialized page."""

    def __init__(self, store):
        self._store = store

    def _layer(self, key):
        request = self._store.requests.get(key[0])
        if request is None or not 0 <= key[1] < request.layers:
            return None
        lp = request.pages[key[1]]
        return lp if 0 <= key[2] < lp.materialized else None

    def __getitem__(self, key):
        lp = self._layer(key)
        if lp is None:
            raise KeyError(key)
        return Page(lp, key)

    def __contains__(self, key):
        return isinstance(key, tuple) and len(key) == 3 and self._layer(key) is not None

    def __iter__(self):
        for name, request in self._store.requests.items():
            for layer, lp in enumerate(request.pages):
                for i in range(lp.materialized):
                    yield (name, layer, i)

    def __len__(self):
        return sum(lp.materialized for r in self._store.requests.values() for lp in r.pages)


class HostStore:
    def __init__(self, config: CacheConfig, allocator: DeviceAllocator, ops):
        self.config, self.allocator, self.ops = config, allocator, ops
        self.pool = allocator.storage
        self.device = self.pool.device
        self.cuda = self.device.type == "cuda"
        if self.cuda and not torch.cuda.is_available():
            raise RuntimeError("no ROCm device available for a device='cuda' cache")
        shape = (config.host_pages, 2, config.page_size, config.kv_heads, config.head_dim)
        self.host = torch.empty(shape, dtype=config.dtype, pin_memory=self.cuda)
        self.host_source = ops.host_source(self.host)
        self.compute = torch.cuda.current_stream(self.device) if self.cuda else None
        self.transfer = independent_stream(self.device) if self.cuda else None
        self.requests: dict[str, RequestPages] = {}
        self.pages = _PageMap(self)
        self.free_host = list(range(config.host_pages - 1, -1, -1))  # pop() yields 0, 1, 2, ...
        self.stats: Counter = Counter()
        self.retired: list[tuple[object, RequestPages, np.ndarray]] = []
        self.request_generation = 0
        self._stamp = 0
        self._write: _Write | None = None

    # -- capacity views ----------------------------------------------------------
    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return self.allocator.owners()

    @property
    def pinned(self):
        """Keys of the pages with at least one pin."""
        return {
            (name, layer, int(i))
            for name, r in self.requests.items()
            for layer, lp in enumerate(r.pages)
            for i in np.flatnonzero(lp.pins[: lp.materialized] > 0)
        }

    def pinned_count(self):
        return sum(int(np.count_nonzero(lp.pins[: lp.materialized])) for r in self.requests.values() for lp in r.pages)

    @property
    def index_bytes(self):
        live = [*self.requests.values(), *(r for _, r, _ in self.retired)]
        tensors = sum(t.numel() * t.element_size() for r in live for t in (r.summaries, r.minimum, r.maximum))
        return tensors + sum(r.extra_index_bytes for r in live)

    def index_reservation_bytes(self, max_tokens, layers):
        pages = ceil(max_tokens / self.config.page_size)
        per_page = self.config.kv_heads * self.config.head_dim * (4 + 2 * self.pool.element_size())
        return pages * layers * per_page

    @property
    def available_host_credits(self):
        return len(self.free_host) - sum(r.host_credits for r in self.requests.values())

    @property
    def page_bytes(self):
        return self.pool[0].numel() * self.pool.element_size()

    # -- streams and events --------------------------------------------------------
    def context(self, stream):
        return torch.cuda.stream(stream) if self.cuda else nullcontext()

    def event(self, stream):
        if not self.cuda:
            return None
        event = torch.cuda.Event()
        event.record(stream)
        return event

    def wait(self, stream, event):
        if isinstance(event, _PendingWrite):
            event = event.resolve()
        if event is not None:
            stream.wait_event(event)

    def check_stream(self):
        if self.cuda and torch.cuda.current_stream(self.device) != self.compute:
            raise RuntimeError("cache operations must use the construction compute stream")

    # -- admission -------------------------------------------------------------------
    def reserve(self, request_id: str, max_tokens: int, layers: int, *, extra_index_bytes=0):
        """Reserve host backing and index bytes for the admitted lifetime."""
        self.check_stream()
        self.collect()
        if request_id in self.requests:
            raise ValueError(f"duplicate request {request_id}")
        if max_tokens < 1 or layers < 1:
            raise ValueError("max_tokens and layers must be positive")
        pages = ceil(max_tokens / self.config.page_size)
        if pages * layers > self.available_host_credits:
            raise CapacityError(f"need {pages * layers} host credits; have {self.available_host_credits}")
        if self.index_bytes + self.index_reservation_bytes(max_tokens, layers) + extra_index_bytes > \
                self.config.index_budget_bytes:
            raise CapacityError("GPU index budget exhausted; defer request admission")
        shape = (layers, pages, self.config.kv_heads, self.config.head_dim)
        summaries = torch.zeros(shape, device=self.device, dtype=torch.float32)
        # bounds are exact K extrema, exactly representable in the KV dtype
        minimum = torch.full(shape, float("inf"), device=self.device, dtype=self.config.dtype)
        maximum = torch.full(shape, float("-inf"), device=self.device, dtype=self.config.dtype)
        generation = self.request_generation
        self.request_generation += 1
        request = RequestPages(max_tokens, layers, pages, [0] * layers, summaries, minimum, maximum,
                               pages * layers, generation, extra_index_bytes=extra_index_bytes, name=request_id)
        request.pages = [LayerPages(self.allocator.group_id((request_id, l)), pages, generation) for l in range(layers)]
        self.requests[request_id] = request

    def layer_pages(self, request_id, layer) -> LayerPages:
        return self.requests[request_id].pages[layer]

    def materialize(self, request_id, layer, index) -> Page:
        request = self.requests[request_id]
        lp = request.pages[layer]
        if lp.host_slot[index] < 0:
            if request.host_credits < 1 or not self.free_host:
                raise AssertionError("host credit accounting broken")
            request.host_credits -= 1
            lp.host_slot[index] = self.free_host.pop()
            self._stamp += 1
            lp.stamp[index] = self._stamp
            lp.materialized = max(lp.materialized, index + 1)
            self.stats["materialized_pages"] += 1
        return Page(lp, (request_id, layer, index))

    # -- residency ---------------------------------------------------------------------
    def detach(self, page: Page):
        """Drop a page's device block; the block is reused only after the page's last
        readers, loads and host mirror (a fence event on the transfer stream)."""
        lp, i = page._lp, page.index
        if lp.slot[i] < 0 or lp.pins[i]:
            raise AssertionError("detach needs an unpinned resident page")
        if lp.enqueued[i] != lp.version[i]:
            raise AssertionError("detach before the page's host mirror was queued")
        for event in (lp.ready[i], lp.last_use[i], lp.host_ready[i]):
            self.wait(self.transfer, event)
        self.allocator.release(int(lp.slot[i]), self.event(self.transfer))
        lp.slot[i] = -1
        lp.location[i] = _CODE[Location.HOST]
        self.stats["evictions"] += 1

    def bind(self, page: Page, slot: int, location: Location):
        lp, i = page._lp, page.index
        lp.slot[i] = slot
        lp.location[i] = _CODE[location]
        lp.last_use[i] = None
        self.allocator.bind(slot, page.key)
        self.stats["peak_device_pages"] = max(self.stats["peak_device_pages"], self.allocator.bound)

    # -- writes ------------------------------------------------------------------------
    @torch.inference_mode()
    def append(self, request_id, layer, k, v, prepare_page, after_write=None):
        """Append projected K/V ``[tokens, Hkv, D]`` to one (request, layer).

        ``prepare_page(page)`` gives a page without rows its device block (and may
        return a read lease of an existing tail); ``after_write(page)`` updates the
        caller's policy once the page's mirror is queued.  Both run page by page, in
        order; the data of the write moves in one batched launch at the end (or
        earlier, when the policy waits for one of its pages)."""
        self.check_stream()
        request = self.requests[request_id]
        cfg = self.config
        if not 0 <= layer < request.layers:
            raise ValueError("invalid layer")
        expected = (cfg.kv_heads, cfg.head_dim)
        if k.ndim != 3 or k.shape != v.shape or tuple(k.shape[1:]) != expected:
            raise ValueError(f"expected matching [tokens, {expected[0]}, {expected[1]}] K/V")
        if k.device != self.pool.device or v.device != self.pool.device:
            raise ValueError("K/V must be on the cache device")
        if k.dtype != cfg.dtype or v.dtype != cfg.dtype:
            raise ValueError("K/V dtype must match the cache")
        start, tokens = request.lengths[layer], len(k)
        if start + tokens > request.max_tokens:
            raise CapacityError("request exceeds its reserved host capacity")
        lp = request.pages[layer]
        if np.any(lp.pins[: lp.materialized] > 0):
            raise RuntimeError("cannot append while this layer has active attention leases")
        # a pinned page holds a bound block, so fewer bound blocks than the budget
        # means fewer pinned pages too (the count is a scan over every layer)
        if self.allocator.bound >= self.budget and self.pinned_count() >= self.budget:
            raise CapacityError("no slot available for append")
        write = self._write = _Write(request, layer, k.contiguous(), v.contiguous(), 0, _PendingWrite(self))
        P = cfg.page_size
        try:
            position = start
            while position < start + tokens:
                index, within = divmod(position, P)
                count = min(P - within, start + tokens - position)
                page = self.materialize(request_id, layer, index)
                lease = prepare_page(page)
                if lease is not None:
                    lease.wait()
                # earlier readers, loads and mirrors of this page finish before it changes
                write.joins += [lp.ready[index], lp.last_use[index], lp.host_ready[index]]
                lp.valid[index] = within + count
                lp.version[index] += 1
                lp.sealed[index] = lp.valid[index] == P
                lp.location[index] = _CODE[Location.RESIDENT]
                marker = write.marker if self.cuda else None
                lp.ready[index] = lp.host_ready[index] = marker
                lp.enqueued[index] = lp.version[index]
                if not self.cuda:  # the CPU mirror is part of the (synchronous) write
                    lp.committed[index] = lp.version[index]
                write.pages.append((index, within, count))
                self.stats["d2h_bytes"] += self.page_bytes * count // P
                if lease is not None:
                    lease.release()
                if after_write is not None:
                    after_write(page)
                position += count
            request.lengths[layer] += tokens
        finally:
            self._flush()
            self._write = None

    def _flush(self):
        """Launch the data movement of the open write's placed pages: one batched
        kernel writes their rows to their current device blocks (none for a page
        detached again meanwhile) and to the host mirror, and updates their bounds
        and summaries; their events become the launch's event."""
        write = self._write
        if write is None or not write.pages:
            return
        lp = write.request.pages[write.layer]
        for event in write.joins:
            if event is not write.marker:
                self.wait(self.compute, event)
        indices = [i for i, _, _ in write.pages]
        count = sum(c for _, _, c in write.pages)
        first = write.first_token
        self.ops.append_tokens(
            write.k[first : first + count], write.v[first : first + count],
            indices[0], write.pages[0][1],
            [int(lp.slot[i]) for i in indices], [int(lp.host_slot[i]) for i in indices],
            self.pool, self.host_source, self.host,
            write.request.minimum[write.layer], write.request.maximum[write.layer],
            write.request.summaries[write.layer], self.config,
        )
        done = self.event(self.compute)
        write.marker.event = done
        for i in indices:
            if lp.ready[i] is write.marker:
                lp.ready[i] = done
            if lp.host_ready[i] is write.marker:
                lp.host_ready[i] = done
        write.first_token = first + count
        write.pages, write.joins = [], []
        write.marker = _PendingWrite(self)

    # -- retirement ------------------------------------------------------------------------
    def retire(self, request_id: str, *, keepalive=()):
        self.check_stream()
        request = self.requests[request_id]
        if any(np.any(lp.pins[: lp.materialized] > 0) for lp in request.pages):
            raise RuntimeError("cannot free a request with active leases")
        waited = set()
        for lp in request.pages:
            if np.any(lp.slot[: lp.materialized] >= 0):
                raise AssertionError("detach resident blocks before retiring host backing")
            for events in (lp.ready, lp.last_use, lp.host_ready):
                for event in events[: lp.materialized]:
                    if event is not None and id(event) not in waited:
                        waited.add(id(event))
                        self.wait(self.transfer, event)
        stamps = np.concatenate([lp.stamp[: lp.materialized] for lp in request.pages])
        slots = np.concatenate([lp.host_slot[: lp.materialized] for lp in request.pages])
        del self.requests[request_id]
        request.keepalive = tuple(keepalive)
        done = self.event(self.transfer)
        self.retired.append((done, request, slots[np.argsort(stamps, kind="stable")]))
        self.stats["retired_requests"] += 1
        return done

    def collect(self, wait=False):
        """Return host slots of retired requests whose readers have all finished.

        A normal poll never blocks; ``wait`` drains the retirement events (when idle
        or shutting down) instead of synchronising the device."""
        pending = []
        for event, request, slots in self.retired:
            if wait and event is not None:
                event.synchronize()
            if event is None or event.query():
                self.free_host.extend(slots.tolist())
                self.stats["reclaimed_requests"] += 1
            else:
                pending.append((event, request, slots))
        self.retired = pending

    # -- inspection -----------------------------------------------------------------------
    def page_state(self, key):
        page = self.pages[key]
        lp, i = page._lp, page.index
        backup_pending = lp.host_ready[i] is not None and not lp.host_ready[i].query()
        if not backup_pending:
            lp.committed[i] = lp.enqueued[i]
        loading = lp.ready[i] is not None and not lp.ready[i].query()
        return {
            "location": page.location.value,
            "loading": loading,
            "backup_pending": backup_pending,
            "content_version": page.content_version,
            "host_committed_version": page.host_committed_version,
            "sealed": page.sealed,
            "request_generation": page.request_generation,
            "slot_generation": None if page.slot is None else int(self.allocator.generation[page.slot]),
        }

    def synchronize(self):
        if self.cuda:
            self.compute.synchronize()
            self.transfer.synchronize()

    def host_kv(self, request_id: str, layer: int):
        """Blocking diagnostic read of one layer's history from the host pool."""
        self.synchronize()
        request = self.requests[request_id]
        length = request.lengths[layer]
        if not length:
            raise ValueError("layer has no KV")
        lp = request.pages[layer]
        count = ceil(length / self.config.page_size)
        rows = self.host[torch.from_numpy(lp.host_slot[:count])]  # [count, 2, P, Hkv, D]
        kv = rows.transpose(0, 1).reshape(2, count * self.config.page_size, *rows.shape[3:])[:, :length]
        return kv[0], kv[1]

    def location_counts(self):
        counts = Counter()
        for r in self.requests.values():
            for lp in r.pages:
                m = lp.materialized
                codes = lp.location[:m][lp.valid[:m] > 0]
                for code, n in zip(*np.unique(codes, return_counts=True)):
                    counts[_LOCATIONS[code].value] += int(n)
        return dict(counts)

    def snapshot(self):
        return {
            "budget_pages": self.budget,
            "allocated_device_bytes": self.pool.numel() * self.pool.element_size(),
            "allocated_host_bytes": self.host.numel() * self.host.element_size(),
            "index_bytes": self.index_bytes,
            "index_budget_bytes": self.config.index_budget_bytes,
            "host_materialized_pages": len(self.pages),
            "host_unused_credits": sum(r.host_credits for r in self.requests.values()),
            "host_available_credits": self.available_host_credits,
            "retiring_requests": len(self.retired),
            "request_device_pages": dict(self.allocator.occupancy),
            "locations": self.location_counts(),
            "stats": dict(self.stats),
        }

    def assert_invariants(self):
        table = self.allocator
        bound = np.flatnonzero(table.owner_group != NO_GROUP)
        assert not np.any(table.owner_group[self.budget :] != NO_GROUP)
        assert table.bound == len(bound)
        retired = np.concatenate([s for _, _, s in self.retired]) if self.retired else np.zeros(0, np.int64)
        live = [lp.host_slot[: lp.materialized] for r in self.requests.values() for lp in r.pages]
        live = np.concatenate(live) if live else np.zeros(0, np.int64)
        everything = np.concatenate([live, retired, np.asarray(self.free_host, np.int64)])
        assert len(everything) == self.config.host_pages
        assert len(np.unique(everything)) == self.config.host_pages
        assert self.available_host_credits >= 0
        assert self.index_bytes <= self.config.index_budget_bytes
        owned = set()
        for name, request in self.requests.items():
            assert sum(lp.materialized for lp in request.pages) + request.host_credits == request.layers * request.page_count
            for layer, lp in enumerate(request.pages):
                m = lp.materialized
                assert np.all(lp.host_slot[:m] >= 0) and np.all(lp.host_slot[m:] < 0)
                assert np.all(lp.pins[:m] >= 0) and np.all((lp.valid[:m] >= 0) & (lp.valid[:m] <= self.config.page_size))
                on_host = lp.slot[:m] < 0
                assert np.all(lp.location[:m][on_host] == _CODE[Location.HOST])
                assert np.all(lp.location[:m][~on_host] != _CODE[Location.HOST])
                assert np.all((lp.pins[:m] == 0) | ~on_host)
                assert np.all(lp.committed[:m] <= lp.enqueued[:m]) and np.all(lp.enqueued[:m] == lp.version[:m])
                for i in np.flatnonzero(~on_host).tolist():
                    block = int(lp.slot[i])
                    assert table.owner_group[block] == lp.gid and table.owner_index[block] == i
                    owned.add(block)
        for block in bound.tolist():
            if table.owner_index[block] >= 0:
                assert block in owned, f"block {block} bound to a page that does not hold it"
