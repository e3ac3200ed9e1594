"""The optional page layout: whole-page leases read in bounded windows.

Same contract as the reference's comparison layout ``reference/cache.py`` and
``reference/attention.py`` (``PagedConfig``, ``PagedKVCache``,
``paged_attention``): every logical page is either resident in a device slot
or copied in whole from the pinned host pool when an attention needs it, and
an attention reads its selected pages in windows of at most ``chunk_pages``
leased pages (two windows live when ``overlap``: the next window's copies are
queued while the current one is read).  Victims come from one of three
policies (``legacy``, ``lru``, ``fair_lru``).

The window attention is the gfx950 kernel ``hs_attend_window`` (through the
cache's ops object); it returns each head's unnormalised (max, sum, weighted
V) state, and windows are merged here in fp32 exactly as the reference merges
its Triton windows.  The rest is host control logic on the shared
``HostStore`` / ``DeviceAllocator``.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import ceil

import torch

from .allocator import DeviceAllocator
from .attention import BACKENDS
from .config import CacheConfig, CapacityError
from .selection import Selection, select_pages
from .storage import HostStore, Location, Page, PageKey, PageLease

POLICIES = ("legacy", "lru", "fair_lru")


@dataclass(frozen=True)
class PagedConfig(CacheConfig):
    """CacheConfig plus the window width, overlap and eviction policy (cache.py:10-22)."""

    chunk_pages: int = 4
    overlap: bool = True
    eviction_policy: str = "fair_lru"

    def __post_init__(self):
        super().__post_init__()
        if self.chunk_pages < 1:
            raise ValueError("chunk_pages must be positive")
        if self.eviction_policy not in POLICIES:
            raise ValueError("invalid page eviction policy")


@dataclass(frozen=True)
class WindowPlan:
    """How one attention will lease its pages (cache.py:25-33)."""

    width: int
    pipelined: bool
    union_pages: int
    misses: int
    pinned_outside: int
    live_slot_limit: int
    hot_slot_target: int


class PagedKVCache:
    """Whole-page residency with window leases (cache.py:36-268)."""

    def __init__(self, config: PagedConfig, ops=None):
        if ops is None:
            from .ops import default_ops

            ops = default_ops(config.device)
        self.ops = ops
        self.config = config
        self.allocator = DeviceAllocator(config)
        self.storage = HostStore(config, self.allocator)
        self.pool, self.device = self.allocator.storage, self.storage.device
        self.lookahead: set[PageKey] = set()  # keys the running attention will still read
        self.clock = 0  # touch counter: recency order of pages
        self.attention_epoch = 0  # one per planned attention
        self.last_attention: dict[PageKey, int] = {}
        self.touched: dict[PageKey, int] = {}

    # -- views shared with the hybrid cache ----------------------------------
    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return self.storage.owners

    @property
    def index_bytes(self):
        return self.storage.index_bytes

    def index_reservation_bytes(self, max_tokens, layers):
        return self.storage.index_reservation_bytes(max_tokens, layers)

    def reserve(self, request_id, max_tokens, layers):
        self.storage.reserve(request_id, max_tokens, layers)

    def write(self, request_id, layer, k, v):
        self.storage.append(request_id, layer, k, v, self._prepare_append)

    def collect(self, wait=False):
        self.storage.collect(wait)

    def snapshot(self):
        share = max(1, self.budget // max(1, len(self.storage.requests)))
        return {**self.storage.snapshot(), "eviction_policy": self.config.eviction_policy, "fair_share_target": share}

    def assert_invariants(self):
        self.storage.assert_invariants()

    def attention(self, query, request_id, layer, selection, backend="auto"):
        return paged_attention(query, self, request_id, layer, backend=backend, selection=selection)

    @property
    def window_pages(self):
        """Window width the budget allows: two windows may coexist when overlapping."""
        windows = 2 if self.config.overlap and self.budget > 1 else 1
        return min(self.config.chunk_pages, max(1, self.budget // windows))

    # -- placement -------------------------------------------------------------
    def _prepare_append(self, page: Page):
        """A partly written tail is leased where it is (loaded if it was evicted); a
        fresh page gets a slot of its own (cache.py:67-72)."""
        if page.valid_tokens:
            return self.acquire([page.key], purpose="append")
        slot = self._slot()
        self.storage.wait(self.storage.compute, self.allocator.slots[slot].fence)
        self._bind(page, slot, Location.RESIDENT)
        return None

    def _bind(self, page: Page, slot: int, location: Location):
        self.storage.bind(page, slot, location)
        self._touch(page)

    def _touch(self, page: Page):
        self.clock += 1
        self.touched[page.key] = self.clock
        if page.slot is not None:
            self.allocator.touch(page.key)

    def release_request(self, request_id, wait=True):
        request = self.storage.requests[request_id]
        if any(self.storage.pages[key].pins for key in request.keys):
            raise RuntimeError("cannot free a request with active leases")
        for key in request.keys:
            page = self.storage.pages[key]
            if page.slot is not None:
                self.storage.detach(page)
            self.last_attention.pop(key, None)
            self.touched.pop(key, None)
        self.storage.retire(request_id)
        self.collect(wait)

    def _slot(self):
        """A slot for a new or loaded page, evicting the policy's victim (cache.py:127-153).

        Under ``fair_lru`` two kinds of page are kept when possible: tails still
        being written (append locality) and sink pages (page 0) read by an
        attention within the last two rounds over every (request, layer).
        """
        anchors = set()
        if self.config.eviction_policy == "fair_lru":
            horizon = 2 * sum(request.layers for request in self.storage.requests.values())
            for key in self.allocator.lru:
                page = self.storage.pages[key]
                recent_sink = key[2] == 0 and self.attention_epoch - self.last_attention.get(key, -(10**9)) <= horizon
                if not page.sealed or recent_sink:
                    anchors.add(key)
        slot = self._choose(anchors)
        if slot is None:
            raise CapacityError("all device slots leased; split the attention working set")
        owner = self.allocator.slots[slot].owner
        if owner is not None:
            self.storage.detach(self.storage.pages[owner])
        return slot

    def _choose(self, anchors):
        """Lowest free slot in the budget, else the policy's unpinned victim (cache.py:245-268)."""
        free = self.allocator.free & set(range(self.budget))
        if free:
            return min(free)
        pages = self.storage.pages
        candidates = [pages[key] for key in self.allocator.lru if pages[key].pins == 0]
        if not candidates:
            return None
        policy = self.config.eviction_policy
        if policy == "legacy":  # hot copies go first, then the least recently touched
            return min(candidates, key=lambda p: (p.location != Location.HOT, self.touched[p.key])).slot
        # a soft fair share: an over-share request gives up its pages first, but a
        # request may borrow the whole idle pool; leases override both
        share = max(1, self.budget // max(1, len(self.storage.requests)))

        def rank(p):
            under_share = policy == "fair_lru" and self.allocator.occupancy[p.key[0]] <= share
            return (p.key in anchors, p.key in self.lookahead, under_share, self.touched[p.key])

        return min(candidates, key=rank).slot

    # -- leases ------------------------------------------------------------------
    def acquire(self, keys: list[PageKey], purpose="attention") -> PageLease:
        """Lease pages, loading the missing ones into slots (cache.py:155-207).

        Every page is pinned before any miss is placed, so placing a miss can
        never evict a page of the same working set.
        """
        self.storage.check_stream()
        keys = list(dict.fromkeys(keys))
        if not keys:
            raise ValueError("empty working set")
        pages = [self.storage.pages[key] for key in keys]
        if any(p.valid_tokens == 0 for p in pages):
            raise ValueError("cannot read an unwritten page")
        if len(self.storage.pinned | set(keys)) > self.budget:
            raise CapacityError("working set exceeds available leases; no state changed")
        for page in pages:
            page.pins += 1
            self.storage.pinned.add(page.key)
        stats = self.storage.stats
        for page in pages:
            if purpose == "attention":
                self.last_attention[page.key] = self.attention_epoch
            if page.slot is not None:
                stats[f"{page.location.value}_hits"] += 1
                stats[f"{purpose}_{page.location.value}_hits"] += 1
            else:
                self._load(page, self._slot(), purpose)
            self._touch(page)
        return PageLease(self.storage, pages)

    def _load(self, page: Page, slot: int, purpose: str):
        """Copy a page's valid tokens from the host pool into `slot` on the transfer stream."""
        store = self.storage
        store.wait(store.transfer, self.allocator.slots[slot].fence)
        store.wait(store.transfer, page.host_ready)
        n = page.valid_tokens
        with store.context(store.transfer):
            if n == self.config.page_size:
                self.pool[slot].copy_(store.host[page.host_slot], non_blocking=store.cuda)
            else:  # each plane's prefix is contiguous; the [:, :n] view is not
                for plane in (0, 1):
                    self.pool[slot, plane, :n].copy_(store.host[page.host_slot, plane, :n], non_blocking=store.cuda)
        page.ready = store.event(store.transfer)
        self._bind(page, slot, Location.HOT)
        moved = store.page_bytes * n // self.config.page_size
        store.stats["misses"] += 1
        store.stats[f"{purpose}_misses"] += 1
        store.stats[f"{purpose}_h2d_bytes"] += moved
        store.stats["h2d_bytes"] += moved

    def plan(self, keys) -> WindowPlan:
        """Window width from the slots left by every other lease (cache.py:209-233)."""
        keys = set(keys)
        self.attention_epoch += 1
        pinned = self.storage.pinned
        outside = len(pinned - keys)
        available = self.budget - len(pinned)  # leases overlapping this selection count too
        if available < 1:
            if keys <= pinned:
                width = min(self.config.chunk_pages, len(keys))
                return WindowPlan(width, False, len(keys), 0, outside, len(keys), 0)
            raise CapacityError("no available window; all capacity leased by other consumers")
        pipelined = self.config.overlap and available > 1
        width = min(self.config.chunk_pages, max(1, available // (2 if pipelined else 1)))
        misses = sum(self.storage.pages[key].slot is None for key in keys)
        live = min(len(keys), width * (2 if pipelined else 1))
        return WindowPlan(width, pipelined, len(keys), misses, outside, live, min(misses, live))

    def set_budget(self, pages: int):
        """Limit the usable slots inside the fixed allocation (cache.py:235-243)."""
        self.storage.check_stream()
        if not 1 <= pages <= self.config.gpu_pages:
            raise ValueError("budget must be within the allocated pool")
        victims = [self.storage.pages[key] for key in self.owners[pages:] if key is not None]
        if any(p.pins for p in victims):
            raise CapacityError("cannot shrink over active leases")
        for page in victims:
            self.storage.detach(page)
        self.allocator.budget = pages


# -- attention over windows ---------------------------------------------------------
def _merge(left, right):
    """Combine two (max, sum, weighted V) states; a head may read nothing in one of
    them (attention.py:11-18)."""
    if left is None:
        return right
    m1, l1, a1 = left
    m2, l2, a2 = right
    m = torch.maximum(m1, m2)
    w1 = torch.where(torch.isfinite(m1), (m1 - m).exp(), 0.0)
    w2 = torch.where(torch.isfinite(m2), (m2 - m).exp(), 0.0)
    return m, w1 * l1 + w2 * l2, w1[:, None] * a1 + w2[:, None] * a2


def _window_state(query, cache: PagedKVCache, lease: PageLease, mask):
    pages = lease.pages
    slots = [p.slot for p in pages]
    lengths = [p.valid_tokens for p in pages]
    if cache.storage.cuda:
        slots = torch.tensor(slots, dtype=torch.int32, pin_memory=True).to(query.device, non_blocking=True)
        lengths = torch.tensor(lengths, dtype=torch.int32, pin_memory=True).to(query.device, non_blocking=True)
    else:
        slots = torch.tensor(slots, dtype=torch.int32)
        lengths = torch.tensor(lengths, dtype=torch.int32)
    return cache.ops.attend_window(query, cache.pool, slots, lengths, mask, cache.config)


@torch.inference_mode()
def paged_attention(
    query: torch.Tensor,
    cache: PagedKVCache,
    request_id: str,
    layer: int,
    pages: list[int] | None = None,
    backend: str = "auto",
    *,
    selection: Selection | None = None,
) -> torch.Tensor:
    """Attend over any number of selected pages with at most two windows live
    (attention.py:41-128).

    The next window's copies (transfer stream) may run while the current window
    is read; a lease is released only after its last kernel is queued, and its
    event keeps the slot from being overwritten before that kernel ran.
    """
    if backend not in BACKENDS:
        raise ValueError("invalid attention backend")
    cfg = cache.config
    if query.ndim != 2 or query.shape[1] != cfg.head_dim or query.shape[0] % cfg.kv_heads:
        raise ValueError("expected [query_heads, head_dim], query_heads divisible by KV heads")
    if query.device != cache.pool.device:
        raise ValueError("query must be on the cache device")
    length = cache.storage.requests[request_id].lengths[layer]
    if selection is not None:
        if (
            pages is not None
            or selection.length != length
            or selection.page_size != cfg.page_size
            or selection.heads != query.shape[0]
        ):
            raise ValueError("selection has stale length, wrong shape, or conflicts with pages")
        pages = selection.pages
    if pages is None:
        pages = select_pages(cache, request_id, layer, query, None)
    pages = list(dict.fromkeys(pages))
    count = ceil(length / cfg.page_size)
    if not pages or any(p < 0 or p >= count for p in pages):
        raise ValueError("selection must contain valid logical pages")
    keys = [(request_id, layer, p) for p in pages]
    plan = cache.plan(keys)
    previous_hint = cache.lookahead
    if cfg.eviction_policy != "legacy":
        cache.lookahead = set(keys)
    stats = cache.storage.stats
    stats["planned_union_pages"] += plan.union_pages
    stats["planned_hot_slots"] += plan.hot_slot_target
    windows = [keys[i : i + plan.width] for i in range(0, len(keys), plan.width)]
    current = future = state = None
    try:
        current = cache.acquire(windows[0])
        for i in range(len(windows)):
            if plan.pipelined and i + 1 < len(windows):
                future = cache.acquire(windows[i + 1])
                stats["prefetch_windows"] += 1
            current.wait()
            mask = selection.mask([p.key[2] for p in current.pages], query.device) if selection is not None else None
            state = _merge(state, _window_state(query, cache, current, mask))
            current.release()
            current = None
            stats["attention_windows"] += 1
            if i + 1 < len(windows):
                current = future if future is not None else cache.acquire(windows[i + 1])
                future = None
    finally:
        for lease in (current, future):
            if lease is not None and not lease.released:
                lease.release()
        cache.lookahead = previous_hint
    _, denominator, numerator = state
    return (numerator / denominator[:, None]).to(query.dtype)
