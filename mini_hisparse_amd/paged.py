"""The optional page layout: whole-page leases read in bounded windows.

Interface of the reference's comparison layout (``reference/cache.py:10-268``,
``reference/attention.py:11-128``): ``PagedConfig``, ``WindowPlan``,
``PagedKVCache`` and ``paged_attention``, with their errors and counters.  Every
logical page is either resident in a device slot or copied in whole from the
pinned host pool when a reader needs it; an attention reads its selected pages
in windows of at most ``chunk_pages`` leased pages (two windows live when
``overlap``: the next window's copies are queued while the current one is read).

Organisation (this module's own): page state lives in the storage's per-(request,
layer) arrays (touch clock, last attention epoch, pins, location); the victim is
the first block of a lexicographic sort over per-block columns
(:meth:`PagedKVCache._victim`) -- ``legacy``: loaded copies before written pages,
then least recently touched; ``lru``: pages outside the running attention's
selection first, then least recently touched; ``fair_lru``: also anchors (tails
still being written, and sink pages read within the last two rounds) last, and
pages of requests over their fair share of slots first.  The window attention is
the gfx950 kernel ``hs_attend_window`` through the ops backend; it returns each
head's unnormalised (max, sum, weighted V) state, merged across windows in fp32.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import ceil

import numpy as np
import torch

from .allocator import DeviceAllocator
from .attention import BACKENDS
from .config import CacheConfig, CapacityError
from .selection import Selection, select_pages
from .storage import _CODE, HostStore, Location, Page, PageKey, PageLease

POLICIES = ("legacy", "lru", "fair_lru")


@dataclass(frozen=True)
class PagedConfig(CacheConfig):
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
    width: int
    pipelined: bool
    union_pages: int
    misses: int
    pinned_outside: int
    live_slot_limit: int
    hot_slot_target: int


class PagedKVCache:
    def __init__(self, config: PagedConfig, ops=None):
        if ops is None:
            from .ops import default_ops

            ops = default_ops(config.device)
        self.ops = ops
        self.config = config
        self.allocator = DeviceAllocator(config)
        self.storage = HostStore(config, self.allocator, ops)
        self.pool, self.device = self.allocator.storage, self.storage.device
        self.lookahead: set[PageKey] = set()  # pages the running attention still reads
        self.clock = 0  # touch counter
        self.attention_epoch = 0  # one per planned attention

    # -- views ----------------------------------------------------------------------------
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
        return {**self.storage.snapshot(), "eviction_policy": self.config.eviction_policy,
                "fair_share_target": self._fair_share()}

    def assert_invariants(self):
        self.storage.assert_invariants()

    def attention(self, query, request_id, layer, selection, backend="auto"):
        return paged_attention(query, self, request_id, layer, backend=backend, selection=selection)

    @property
    def window_pages(self):
        """Window width the budget allows: two windows may coexist when overlapping."""
        windows = 2 if self.config.overlap and self.budget > 1 else 1
        return min(self.config.chunk_pages, max(1, self.budget // windows))

    def _fair_share(self):
        return max(1, self.budget // max(1, len(self.storage.requests)))

    # -- placement ----------------------------------------------------------------------------
    def _touch(self, page: Page):
        self.clock += 1
        page._lp.touched[page.index] = self.clock
        if page.slot is not None:
            self.allocator.touch_block(page.slot)

    def _prepare_append(self, page: Page):
        """A partly written tail is leased where it is (loaded if it was evicted); a new
        page gets a slot of its own."""
        if page.valid_tokens:
            return self.acquire([page.key], purpose="append")
        slot = self._slot()
        self.storage.wait(self.storage.compute, self.allocator.fence[slot])
        self.storage.bind(page, slot, Location.RESIDENT)
        self._touch(page)
        return None

    def _block_columns(self, blocks):
        """Per bound block: its page's (layer pages, index, request) and the columns the
        policies sort on."""
        table = self.allocator
        lps, idx, names = [], table.owner_index[blocks], []
        for g in table.owner_group[blocks].tolist():
            name, layer = table.group_key(g)
            lps.append(self.storage.requests[name].pages[layer])
            names.append(name)
        gather = lambda attr: np.array([getattr(lp, attr)[i] for lp, i in zip(lps, idx)])  # noqa: E731
        return lps, idx, names, gather

    def _victim(self):
        """The slot the next page takes: the lowest free slot in the budget, else the
        policy's first unpinned page, or None when every slot is leased."""
        table = self.allocator
        free = table.free_blocks(self.budget)
        if len(free):
            return int(free[0])
        blocks = table.bound_pages()
        if not len(blocks):
            return None
        lps, idx, names, gather = self._block_columns(blocks)
        unpinned = gather("pins") == 0
        if not unpinned.any():
            return None
        blocks, idx = blocks[unpinned], idx[unpinned]
        names = [n for n, keep in zip(names, unpinned) if keep]
        lps = [lp for lp, keep in zip(lps, unpinned) if keep]
        touched = np.array([lp.touched[i] for lp, i in zip(lps, idx)])
        policy = self.config.eviction_policy
        if policy == "legacy":  # loaded copies go first, then the least recently touched
            written = np.array([lp.location[i] != _CODE[Location.HOT] for lp, i in zip(lps, idx)])
            order = np.lexsort((touched, written))
            return int(blocks[order[0]])
        group_keys = [table.group_key(int(table.owner_group[b])) for b in blocks.tolist()]
        ahead = np.array([(*g, int(i)) in self.lookahead for g, i in zip(group_keys, idx)])
        if policy == "fair_lru":
            # anchors: tails still being written (append locality) and sink pages an
            # attention read within the last two rounds over every (request, layer)
            horizon = 2 * sum(r.layers for r in self.storage.requests.values())
            anchored = np.array([
                not lp.sealed[i] or (i == 0 and self.attention_epoch - lp.attended[i] <= horizon)
                for lp, i in zip(lps, idx)
            ])
            share = self._fair_share()
            held = table.occupancy
            within_share = np.array([held[n] <= share for n in names])
        else:
            anchored = within_share = np.zeros(len(blocks), bool)
        order = np.lexsort((touched, within_share, ahead, anchored))
        return int(blocks[order[0]])

    def _slot(self):
        slot = self._victim()
        if slot is None:
            raise CapacityError("all device slots leased; split the attention working set")
        owner = self.allocator.owner_key(slot)
        if owner is not None:
            self.storage.detach(self.storage.pages[owner])
        return slot

    def release_request(self, request_id, wait=True):
        request = self.storage.requests[request_id]
        if any(np.any(lp.pins > 0) for lp in request.pages):
            raise RuntimeError("cannot free a request with active leases")
        for key in request.keys:
            if request.pages[key[1]].slot[key[2]] >= 0:
                self.storage.detach(self.storage.pages[key])
        self.storage.retire(request_id)
        self.collect(wait)

    # -- leases -------------------------------------------------------------------------------
    def acquire(self, keys: list[PageKey], purpose="attention") -> PageLease:
        """Lease pages, loading the missing ones into slots.  Every page is pinned before
        any miss is placed, so placing a miss never evicts a page of the same set."""
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
            page.pins = page.pins + 1
        stats = self.storage.stats
        for page in pages:
            if purpose == "attention":
                page.last_attention_epoch = self.attention_epoch
            if page.slot is not None:
                where = page.location.value
                stats[f"{where}_hits"] += 1
                stats[f"{purpose}_{where}_hits"] += 1
            else:
                self._load(page, self._slot(), purpose)
            self._touch(page)
        return PageLease(self.storage, pages)

    def _load(self, page: Page, slot: int, purpose: str):
        """Copy a page's valid rows from the host pool into ``slot`` on the transfer stream."""
        store = self.storage
        store.wait(store.transfer, self.allocator.fence[slot])
        store.wait(store.transfer, page.host_ready)
        rows = page.valid_tokens
        with store.context(store.transfer):
            for plane in (0, 1):  # each plane's valid prefix is contiguous
                self.pool[slot, plane, :rows].copy_(store.host[page.host_slot, plane, :rows], non_blocking=store.cuda)
        page.ready = store.event(store.transfer)
        store.bind(page, slot, Location.HOT)
        moved = store.page_bytes * rows // self.config.page_size
        for name in ("misses", f"{purpose}_misses"):
            store.stats[name] += 1
        for name in ("h2d_bytes", f"{purpose}_h2d_bytes"):
            store.stats[name] += moved

    def plan(self, keys) -> WindowPlan:
        """Window width from the slots every other lease leaves free."""
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
        """Limit the usable slots inside the fixed allocation (no memory is freed)."""
        self.storage.check_stream()
        if not 1 <= pages <= self.config.gpu_pages:
            raise ValueError("budget must be within the allocated pool")
        victims = [self.storage.pages[key] for key in self.owners[pages:] if key is not None]
        if any(p.pins for p in victims):
            raise CapacityError("cannot shrink over active leases")
        for page in victims:
            self.storage.detach(page)
        self.allocator.budget = pages


# -- attention over windows ----------------------------------------------------------------
def merge_states(left, right):
    """Combine two per-head (max, sum, weighted V) states; a head may read nothing in
    one of them (max -inf)."""
    if left is None:
        return right
    (m1, l1, a1), (m2, l2, a2) = left, right
    m = torch.maximum(m1, m2)
    w1 = torch.where(torch.isfinite(m1), (m1 - m).exp(), 0.0)
    w2 = torch.where(torch.isfinite(m2), (m2 - m).exp(), 0.0)
    return m, w1 * l1 + w2 * l2, w1[:, None] * a1 + w2[:, None] * a2


def _window_state(query, cache: PagedKVCache, lease: PageLease, mask):
    slots = torch.tensor([p.slot for p in lease.pages], dtype=torch.int32)
    lengths = torch.tensor([p.valid_tokens for p in lease.pages], dtype=torch.int32)
    if cache.storage.cuda:
        slots = slots.pin_memory().to(query.device, non_blocking=True)
        lengths = lengths.pin_memory().to(query.device, non_blocking=True)
    return cache.ops.attend_window(query, cache.pool, slots, lengths, mask, cache.config)


@torch.inference_mode()
def paged_attention(query: torch.Tensor, cache: PagedKVCache, request_id: str, layer: int,
                    pages: list[int] | None = None, backend: str = "auto", *,
                    selection: Selection | None = None) -> torch.Tensor:
    """Attend over any number of selected pages with at most two windows live: the next
    window's copies may run while the current window is read, and a lease is released
    only after its last kernel is queued (its event keeps the slot until then)."""
    if backend not in BACKENDS:
        raise ValueError("invalid attention backend")
    cfg = cache.config
    if query.ndim != 2 or query.shape[1] != cfg.head_dim or query.shape[0] % cfg.kv_heads:
        raise ValueError("expected [query_heads, head_dim], query_heads divisible by KV heads")
    if query.device != cache.pool.device:
        raise ValueError("query must be on the cache device")
    length = cache.storage.requests[request_id].lengths[layer]
    if selection is not None:
        if pages is not None or selection.length != length or selection.page_size != cfg.page_size \
                or selection.heads != query.shape[0]:
            raise ValueError("selection has stale length, wrong shape, or conflicts with pages")
        pages = selection.pages
    if pages is None:
        pages = select_pages(cache, request_id, layer, query, None)
    pages = list(dict.fromkeys(pages))
    if not pages or min(pages) < 0 or max(pages) >= ceil(length / cfg.page_size):
        raise ValueError("selection must contain valid logical pages")
    keys = [(request_id, layer, p) for p in pages]
    plan = cache.plan(keys)
    hint = cache.lookahead
    if cfg.eviction_policy != "legacy":
        cache.lookahead = set(keys)
    stats = cache.storage.stats
    stats["planned_union_pages"] += plan.union_pages
    stats["planned_hot_slots"] += plan.hot_slot_target
    windows = [keys[i : i + plan.width] for i in range(0, len(keys), plan.width)]
    leases = {}
    state = None
    try:
        leases[0] = cache.acquire(windows[0])
        for i in range(len(windows)):
            if plan.pipelined and i + 1 < len(windows):
                leases[i + 1] = cache.acquire(windows[i + 1])
                stats["prefetch_windows"] += 1
            lease = leases.pop(i)
            lease.wait()
            mask = selection.mask([p.key[2] for p in lease.pages], query.device) if selection is not None else None
            state = merge_states(state, _window_state(query, cache, lease, mask))
            lease.release()
            stats["attention_windows"] += 1
            if i + 1 < len(windows) and i + 1 not in leases:
                leases[i + 1] = cache.acquire(windows[i + 1])
    finally:
        for lease in leases.values():
            if not lease.released:
                lease.release()
        cache.lookahead = hint
    _, denominator, numerator = state
    return (numerator / denominator[:, None]).to(query.dtype)
