"""Host-backed logical pages: append with mirrors, Quest bounds, event-safe retirement.

Same contract as the reference's ``HostStore`` (storage.py:101-441): every
request's full KV history lives in one pinned host pool ``[host_pages, 2, P,
Hkv, D]``; the device slab holds resident copies.  ``append`` writes new K/V
into the resident tail page on the compute stream, updates the page's Quest
bounds (exact K minimum / maximum in the KV dtype) and mean-K summary, and
mirrors only the new rows to host memory on the transfer stream.  Host slots
of a retired request are reused only after its retirement event completes.

Storage knows no eviction policy: callers supply the resident placement
(``prepare_page``) and update their own policy after the mirror
(``after_write``).  Pages are additionally indexed per (request, layer).
"""

from __future__ import annotations

from collections import Counter
from contextlib import nullcontext
from dataclasses import dataclass, field
from enum import Enum
from math import ceil

import torch

from .allocator import DeviceAllocator
from .config import CacheConfig, CapacityError

PageKey = tuple[str, int, int]


class Location(str, Enum):
    HOST = "host"
    RESIDENT = "resident"
    HOT = "hot"


@dataclass
class Page:
    key: PageKey
    host_slot: int
    slot: int | None = None
    location: Location = Location.HOST
    valid_tokens: int = 0
    pins: int = 0
    ready: object = None
    last_use: object = None
    host_ready: object = None
    request_generation: int = 0
    content_version: int = 0
    host_enqueued_version: int = 0
    host_committed_version: int = 0
    sealed: bool = False
    last_attention_epoch: int = -1000000000


@dataclass
class RequestPages:
    max_tokens: int
    layers: int
    page_count: int
    lengths: list[int]
    summaries: torch.Tensor  # [layers, pages, Hkv, D] float32 page-mean K (selector "mean")
    minimum: torch.Tensor  # [layers, pages, Hkv, D] KV dtype, +inf before the first token
    maximum: torch.Tensor  # [layers, pages, Hkv, D] KV dtype, -inf before the first token
    host_credits: int
    generation: int
    keys: list[PageKey] = field(default_factory=list)
    extra_index_bytes: int = 0
    keepalive: tuple = ()  # caller metadata retained until the retirement event


class PageLease:
    """Pins protect mappings on the host; events protect bytes on the device."""

    def __init__(self, store: "HostStore", pages: list[Page]):
        self.store, self.pages, self.released = store, pages, False
        self.handles = [(p.slot, store.allocator.slots[p.slot].generation, p.key) for p in pages]

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
            page.pins -= 1
            if page.pins == 0:
                self.store.pinned.discard(page.key)
        self.released = True

    def __enter__(self):
        self.wait()
        return self

    def __exit__(self, *_):
        self.release()


class HostStore:
    def __init__(self, config: CacheConfig, allocator: DeviceAllocator):
        self.config = config
        device = torch.device(config.device)
        self.cuda = device.type == "cuda"
        if self.cuda and not torch.cuda.is_available():
            raise RuntimeError("no ROCm device available for a device='cuda' cache")
        self.allocator = allocator
        self.pool = allocator.storage
        self.device = self.pool.device
        page_shape = (2, config.page_size, config.kv_heads, config.head_dim)
        self.host = torch.empty((config.host_pages, *page_shape), dtype=config.dtype, pin_memory=self.cuda)
        self.compute = torch.cuda.current_stream(self.device) if self.cuda else None
        self.transfer = torch.cuda.Stream(device=self.device) if self.cuda else None
        self.pages: dict[PageKey, Page] = {}
        self.group_pages: dict[tuple, dict[int, Page]] = {}
        self.requests: dict[str, RequestPages] = {}
        self.free_host = list(range(config.host_pages - 1, -1, -1))  # pop() yields 0, 1, 2, ...
        self.stats: Counter = Counter()
        self.pinned: set[PageKey] = set()
        self.retired: list[tuple[object, RequestPages, list[Page]]] = []
        self.request_generation = 0

    # -- capacity views ------------------------------------------------------
    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return [slot.owner for slot in self.allocator.slots]

    @property
    def index_bytes(self):
        live = list(self.requests.values()) + [r for _, r, _ in self.retired]
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

    # -- streams and events --------------------------------------------------
    def context(self, stream):
        return torch.cuda.stream(stream) if self.cuda else nullcontext()

    def event(self, stream):
        if not self.cuda:
            return None
        event = torch.cuda.Event()
        event.record(stream)
        return event

    def wait(self, stream, event):
        if event is not None:
            stream.wait_event(event)

    def check_stream(self):
        if self.cuda and torch.cuda.current_stream(self.device) != self.compute:
            raise RuntimeError("cache operations must use the construction compute stream")

    # -- admission -----------------------------------------------------------
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
        index_bytes = self.index_reservation_bytes(max_tokens, layers) + extra_index_bytes
        if self.index_bytes + index_bytes > self.config.index_budget_bytes:
            raise CapacityError("GPU index budget exhausted; defer request admission")
        shape = (layers, pages, self.config.kv_heads, self.config.head_dim)
        summaries = torch.zeros(shape, device=self.device, dtype=torch.float32)
        request = RequestPages(
            max_tokens,
            layers,
            pages,
            [0] * layers,
            summaries,
            # bounds are actual K extrema, exactly representable in the KV dtype
            torch.full(shape, torch.inf, device=self.device, dtype=self.config.dtype),
            torch.full(shape, -torch.inf, device=self.device, dtype=self.config.dtype),
            pages * layers,
            self.request_generation,
        )
        request.extra_index_bytes = extra_index_bytes
        self.request_generation += 1
        self.requests[request_id] = request

    def materialize(self, request_id, layer, index):
        key = (request_id, layer, index)
        page = self.pages.get(key)
        if page is None:
            request = self.requests[request_id]
            assert request.host_credits > 0 and self.free_host
            request.host_credits -= 1
            request.keys.append(key)
            page = Page(key, self.free_host.pop(), request_generation=request.generation)
            self.pages[key] = page
            self.group_pages.setdefault(key[:2], {})[index] = page
            self.stats["materialized_pages"] += 1
        return page

    # -- residency transitions -----------------------------------------------
    def detach(self, page: Page):
        assert page.slot is not None and page.pins == 0
        assert page.host_enqueued_version == page.content_version
        # the block is free at once, but its reuse is fenced behind every reader,
        # including a queued D2H mirror that still reads it
        for event in (page.ready, page.last_use, page.host_ready):
            self.wait(self.transfer, event)
        self.allocator.release(page.slot, self.event(self.transfer))
        page.slot, page.location = None, Location.HOST
        self.stats["evictions"] += 1

    def bind(self, page: Page, slot: int, location: Location):
        page.slot, page.location = slot, location
        page.last_use = None
        self.allocator.bind(slot, page.key)
        self.stats["peak_device_pages"] = max(self.stats["peak_device_pages"], len(self.allocator.lru))

    # -- append --------------------------------------------------------------
    @torch.inference_mode()
    def append(self, request_id, layer, k, v, prepare_page, after_write=None):
        """Append projected K/V [tokens, Hkv, D] and mirror only the new rows.

        ``prepare_page(page)`` supplies resident placement and may return a read
        lease on an existing tail; ``after_write(page)`` updates caller policy
        after the mirror is queued.  Storage never selects a victim.
        """
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
        start = request.lengths[layer]
        if start + len(k) > request.max_tokens:
            raise CapacityError("request exceeds its reserved host capacity")
        if any(key[0] == request_id and key[1] == layer for key in self.pinned):
            raise RuntimeError("cannot append while this layer has active attention leases")
        if len(self.pinned) >= self.budget:
            raise CapacityError("no slot available for append")
        done = 0
        while done < len(k):
            index, within = divmod(start + done, cfg.page_size)
            count = min(cfg.page_size - within, len(k) - done)
            page = self.materialize(request_id, layer, index)
            self._append_page(request, layer, index, page, within, k[done : done + count], v[done : done + count], prepare_page, after_write)
            done += count
        request.lengths[layer] += len(k)

    def _append_page(self, request, layer, index, page, within, k, v, prepare_page, after_write):
        cfg = self.config
        count = len(k)
        lease = prepare_page(page)
        if lease is not None:
            lease.wait()
        # join earlier readers and mirrors of this page before modifying it
        for event in (page.ready, page.last_use, page.host_ready):
            self.wait(self.compute, event)
        target = self.pool[page.slot]
        rows = slice(within, within + count)
        target[0, rows].copy_(k)
        target[1, rows].copy_(v)
        page.valid_tokens = within + count
        page.content_version += 1
        page.sealed = page.valid_tokens == cfg.page_size
        # Quest bounds (exact extrema) and the mean-K summary of the page
        request.summaries[layer, index].copy_(target[0, : page.valid_tokens].float().mean(0))
        new_keys = target[0, rows].float()
        lo, hi = request.minimum[layer, index], request.maximum[layer, index]
        lo.copy_(torch.minimum(lo, new_keys.amin(0)))
        hi.copy_(torch.maximum(hi, new_keys.amax(0)))
        page.ready = self.event(self.compute)
        page.location = Location.RESIDENT
        # mirror only the new rows to the host copy, on the transfer stream
        self.wait(self.transfer, page.ready)
        with self.context(self.transfer):
            if within == 0 and count == cfg.page_size:
                self.host[page.host_slot].copy_(target, non_blocking=self.cuda)
            else:
                for plane in (0, 1):
                    self.host[page.host_slot, plane, rows].copy_(target[plane, rows], non_blocking=self.cuda)
        page.host_ready = self.event(self.transfer)
        page.host_enqueued_version = page.content_version
        if not self.cuda:
            page.host_committed_version = page.content_version
        self.stats["d2h_bytes"] += self.page_bytes * count // cfg.page_size
        if lease is not None:
            lease.release()
        if after_write is not None:
            after_write(page)

    # -- retirement ----------------------------------------------------------
    def retire(self, request_id: str, *, keepalive=()):
        self.check_stream()
        request = self.requests[request_id]
        if any(self.pages[key].pins for key in request.keys):
            raise RuntimeError("cannot free a request with active leases")
        retired = []
        for key in request.keys:
            page = self.pages[key]
            assert page.slot is None, "detach resident blocks before retiring host backing"
            for event in (page.ready, page.last_use, page.host_ready):
                self.wait(self.transfer, event)
            retired.append(self.pages.pop(key))
            group = self.group_pages.get(key[:2])
            if group is not None:
                group.pop(key[2], None)
                if not group:
                    del self.group_pages[key[:2]]
        del self.requests[request_id]
        request.keepalive = tuple(keepalive)
        done = self.event(self.transfer)
        self.retired.append((done, request, retired))
        self.stats["retired_requests"] += 1
        return done

    def collect(self, wait=False):
        """Publish reusable host slots only after every in-flight user finished.

        A normal poll never blocks; ``wait`` drains retirement events (idle or
        shutdown) rather than synchronising the device.
        """
        pending = []
        for event, request, pages in self.retired:
            if wait and event is not None:
                event.synchronize()
            if event is None or event.query():
                self.free_host.extend(page.host_slot for page in pages)
                self.stats["reclaimed_requests"] += 1
            else:
                pending.append((event, request, pages))
        self.retired = pending

    # -- diagnostics ---------------------------------------------------------
    def page_state(self, key):
        page = self.pages[key]
        backup_pending = page.host_ready is not None and not page.host_ready.query()
        if not backup_pending:
            page.host_committed_version = page.host_enqueued_version
        loading = page.ready is not None and not page.ready.query()
        return {
            "location": page.location.value,
            "loading": loading,
            "backup_pending": backup_pending,
            "content_version": page.content_version,
            "host_committed_version": page.host_committed_version,
            "sealed": page.sealed,
            "request_generation": page.request_generation,
            "slot_generation": None if page.slot is None else self.allocator.slots[page.slot].generation,
        }

    def synchronize(self):
        if self.cuda:
            self.compute.synchronize()
            self.transfer.synchronize()

    def host_kv(self, request_id: str, layer: int):
        """Blocking diagnostic read of one layer's host history (never on the decode path)."""
        self.synchronize()
        request = self.requests[request_id]
        count = ceil(request.lengths[layer] / self.config.page_size)
        if count == 0:
            raise ValueError("layer has no KV")
        chunks = []
        for i in range(count):
            page = self.pages[(request_id, layer, i)]
            chunks.append(self.host[page.host_slot, :, : page.valid_tokens])
        kv = torch.cat(chunks, dim=1)
        return kv[0], kv[1]

    def snapshot(self):
        locations = Counter(p.location.value for p in self.pages.values() if p.valid_tokens)
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
            "locations": dict(locations),
            "stats": dict(self.stats),
        }

    def assert_invariants(self):
        owners = self.owners
        occupied = [key for key in owners if key is not None]
        assert len(occupied) == len(set(occupied))
        assert all(key is None for key in owners[self.budget :])
        retired_pages = [p for _, _, pages in self.retired for p in pages]
        assert len(self.free_host) + len(self.pages) + len(retired_pages) == self.config.host_pages
        host_slots = [p.host_slot for p in [*self.pages.values(), *retired_pages]]
        assert len(set(host_slots + self.free_host)) == self.config.host_pages
        assert self.available_host_credits >= 0
        assert self.pinned == {p.key for p in self.pages.values() if p.pins}
        assert set(self.allocator.lru) == set(occupied)
        assert self.allocator.free == {i for i, key in enumerate(owners) if key is None}
        assert +self.allocator.occupancy == Counter(key[0] for key in occupied)
        assert self.index_bytes <= self.config.index_budget_bytes
        indexed = {(g, i): p for g, pages in self.group_pages.items() for i, p in pages.items()}
        assert {(k[:2], k[2]) for k in self.pages} == set(indexed)
        for request in self.requests.values():
            assert len(request.keys) + request.host_credits == request.layers * request.page_count
        for key, page in self.pages.items():
            assert indexed[(key[:2], key[2])] is page
            assert page.pins >= 0
            assert 0 <= page.valid_tokens <= self.config.page_size
            if page.slot is None:
                assert page.location == Location.HOST
            else:
                assert owners[page.slot] == key
                assert page.location in (Location.RESIDENT, Location.HOT)
            assert page.pins == 0 or page.slot is not None
            assert page.request_generation == self.requests[key[0]].generation
            assert page.host_committed_version <= page.host_enqueued_version == page.content_version
