"""Block placement of the hybrid residency policy, computed incrementally.

``HybridKVCache`` (hybrid.py) applies the reference's residency policy
(``mini_hisparse/hybrid.py:204-392``) to one slab of device blocks: a page gets a
block when it is first written (the lowest empty block, else the oldest readable
one of the reclaim queue); a (request, layer) requires its hot region when the
allocatable blocks fall under the watermark, when its resident pages reach the
window, or under pressure, and then takes the whole region at once and offers its
clean history outside the two active tails as reclaimable, nearest the tail first.
Its ticks visit every (request, layer) and scan the block table, which is exact
but costs O(groups + blocks) per page: at the Qwen2.5-7B shape (1.8 M pages, 224
groups, 734 k blocks) a prefill would take hours.

:class:`PlacementPlan` makes the same decisions for the same sequence of writes
in O(1) amortised per page, for writes whose host mirrors complete with the
write (the CPU semantics of the policy: every written page is clean at the next
tick) and with no row leases open (nothing is read while the plan is built).
What it exploits:

* the empty blocks are a suffix ``[next_free, blocks)`` plus the blocks released
  requests returned (a min-heap below ``next_free``) -- blocks are taken lowest
  first, like the allocator's ascending free list;
* every queued block is readable (the only pinned page is an append tail, which
  is never history);
* a page is bound once, when it is written, so a group's history in bind order
  is its pages in index order, and a group's unqueued history is the range since
  the last tick that offered it;
* a tick can change only the writing group (new history), the groups whose hot
  region is still owed, and the groups with residents and no demand yet (the
  watermark or the window may raise it); the others are skipped.

``release`` is ``HybridKVCache.release_request``: a finished request's hot blocks
and resident pages become empty blocks (queued ones leave the reclaim queue) and
its groups leave the plan.  ``tests/test_residency_plan.py`` checks every
decision, queue and counter against ``HybridKVCache`` itself on random write
sequences, with requests released and new ones admitted between them.
"""

from __future__ import annotations

import heapq
from collections import Counter, deque
from math import ceil

import numpy as np

from .config import CapacityError

ACTIVE_TAIL_PAGES = 2


class _Group:
    __slots__ = ("gid", "key", "slot", "valid", "length", "residents", "hot", "required", "trigger", "offered",
                 "released")

    def __init__(self, gid, key, pages):
        self.gid, self.key = gid, key
        self.slot = np.full(pages, -1, np.int64)  # device block of each page, -1
        self.valid = np.zeros(pages, np.int64)  # rows written to each page
        self.length = 0  # tokens of completed writes
        self.residents = 0
        self.hot: list[int] = []  # hot blocks, in region order
        self.required = False
        self.trigger = None
        self.offered = 0  # pages [0, offered) have been offered to the reclaim queue
        self.released = False


class PlacementPlan:
    """The hybrid policy's block decisions for a sequence of writes (see the module doc).

    ``blocks`` is the slab (the policy's budget), ``hot_rows`` the rows of every hot
    region, ``window`` / ``watermark`` as :class:`HotConfig` (``None``: the default
    ``max(hot blocks, blocks // 10)``).  Groups are ``(request, layer)`` keys."""

    def __init__(self, blocks, page_size, hot_rows, window=64, watermark=None):
        self.blocks, self.P = blocks, page_size
        self.hot_blocks = ceil(hot_rows / page_size)
        self.window = window
        self.watermark = max(self.hot_blocks, blocks // 10) if watermark is None else watermark
        self.next_free = 0
        self.free: list[int] = []  # empty blocks below next_free (released), a min-heap
        # reclaimable blocks in queue order as (block, ticket); an entry is live while the
        # block is queued under that ticket (a released block leaves the queue at once,
        # its entry is dropped when it reaches the head)
        self._queue: deque[tuple[int, int]] = deque()
        self.queued = np.zeros(blocks, bool)
        self.ticket = np.zeros(blocks, np.int64)
        self.n_queued = 0
        self.owner = np.full(blocks, -1, np.int64)  # group id of a page's block, -1 (free or hot)
        self.owner_page = np.zeros(blocks, np.int64)
        self.bind_order = np.zeros(blocks, np.int64)  # clock of the block's page bind
        self._clock = 0
        self.groups: list[_Group] = []
        self._by_key: dict = {}
        self.requests: dict = {}  # request -> layers
        self._open: set[int] = set()  # groups with residents and no hot demand yet
        self._owed: set[int] = set()  # groups whose hot demand is not served yet
        self._writing = None  # (group id, page) being appended
        self.stats = Counter()
        self.detached: list[tuple] = []  # (group key, page) losing their block, in order

    # -- queries -----------------------------------------------------------------
    def group(self, key) -> _Group:
        return self.groups[self._by_key[key]]

    def available(self):
        return self.blocks - self.next_free + len(self.free) + self.n_queued

    @property
    def queue(self):
        """The reclaimable blocks, in queue order."""
        return [b for b, t in self._queue if self.queued[b] and self.ticket[b] == t]

    def _queue_head(self):
        while self._queue:
            block, ticket = self._queue[0]
            if self.queued[block] and self.ticket[block] == ticket:
                return block
            self._queue.popleft()
        return None

    def _tail(self, g: _Group):
        if self._writing is not None and self._writing[0] == g.gid:
            return self._writing[1]
        return (g.length - 1) // self.P

    def _history(self, g: _Group):
        """Resident pages of ``g`` at least two behind its tail (all sealed), in bind order."""
        top = self._tail(g) - ACTIVE_TAIL_PAGES
        if top < 0:
            return np.zeros(0, np.int64)
        pages = np.arange(top + 1)
        return pages[g.slot[: top + 1] >= 0]

    # -- admission ------------------------------------------------------------------
    def admission_blocks(self, layers):
        return layers * (self.hot_blocks + ACTIVE_TAIL_PAGES)

    def reserve(self, request, max_tokens, layers):
        """``HybridKVCache.reserve``: a tick, the credit check, one group per layer."""
        self._tick(None)
        promised = sum(self.admission_blocks(n) for n in self.requests.values())
        if promised + self.admission_blocks(layers) > self.blocks:
            raise CapacityError("hot-region + active-tail credits exhausted; defer admission")
        self.requests[request] = layers
        pages = ceil(max_tokens / self.P)
        for layer in range(layers):
            gid = len(self.groups)
            self._by_key[(request, layer)] = gid
            self.groups.append(_Group(gid, (request, layer), pages))

    # -- blocks -----------------------------------------------------------------------
    def _enqueue(self, block):
        if not self.queued[block]:
            self.queued[block] = True
            self._clock += 1
            self.ticket[block] = self._clock
            self._queue.append((block, self._clock))
            self.n_queued += 1

    def _take(self, block):
        """Hand an available block to a new owner; a queued one detaches its page."""
        if self.queued[block]:
            if self._queue_head() != block:
                raise AssertionError("blocks leave the reclaim queue from its head")
            self._queue.popleft()
            self.queued[block] = False
            self.n_queued -= 1
            g = self.groups[int(self.owner[block])]
            page = int(self.owner_page[block])
            g.slot[page] = -1
            g.residents -= 1
            if g.residents == 0:
                self._open.discard(g.gid)
            self.owner[block] = -1
            self.stats["unpinned_block_reuses"] += 1
            self.stats["evictions"] += 1
            self.detached.append((g.key, page))
        elif self.free and block == self.free[0]:
            heapq.heappop(self.free)
        elif block == self.next_free and not (self.free and self.free[0] < block):
            self.next_free += 1
        else:
            raise AssertionError("empty blocks are taken lowest first")
        return block

    def _first_available(self):
        if self.free:
            return self.free[0]  # below next_free
        if self.next_free < self.blocks:
            return self.next_free
        return self._queue_head()

    # -- policy --------------------------------------------------------------------------
    def _offer(self, g: _Group):
        """``_unpin_clean_pages``: with a hot region, history not yet queued joins the
        reclaim queue nearest the tail first."""
        if not g.hot:
            return
        top = self._tail(g) - ACTIVE_TAIL_PAGES
        if top < g.offered:
            return
        for page in range(top, g.offered - 1, -1):
            block = g.slot[page]
            if block >= 0 and not self.queued[block]:
                self._enqueue(int(block))
                self.stats["clean_page_unpins"] += 1
        g.offered = top + 1

    def _require(self, g: _Group, reason):
        if not g.required:
            g.required, g.trigger = True, reason
            self.stats[f"hot_trigger_{reason}"] += 1
            self._open.discard(g.gid)
            if not g.hot:
                self._owed.add(g.gid)

    def transition(self, g: _Group):
        """``transition_to_host``: the whole hot region at once, from the empty blocks,
        then the queue, then the group's own unqueued history (bind order)."""
        if g.hot:
            return
        self._require(g, "explicit")
        supply = self.available()
        short = max(0, self.hot_blocks - supply)
        if short:
            victims = [int(g.slot[p]) for p in self._history(g) if not self.queued[g.slot[p]]]
            if len(victims) < short:
                raise CapacityError("cannot acquire complete hot region while blocks are leased")
            for block in victims[:short]:
                self._enqueue(block)
                self.stats["clean_page_unpins"] += 1
        region = []
        for _ in range(self.hot_blocks):
            block = self._take(self._first_available())
            self._clock += 1
            region.append(block)
        g.hot = region
        self._owed.discard(g.gid)
        self.stats["hot_region_allocations"] += 1
        self._offer(g)

    def _visit(self, g: _Group, upcoming):
        """One group's part of a tick (``update_residency``'s second loop)."""
        if not g.residents:
            return
        if not g.required:
            if self.available() - int(upcoming) < self.watermark:
                self._require(g, "watermark")
            elif g.residents >= self.window:
                self._require(g, "window")
        if g.required and not g.hot:
            try:
                self.transition(g)
            except CapacityError:
                pass  # demand and residents stay; the next tick retries
        self._offer(g)

    def _tick(self, only: _Group | None, upcoming=False):
        """``update_residency``: over every group, or one.  Groups a tick cannot change
        (no residents, or served demand and no new history) are skipped."""
        if only is not None:
            self._offer(only)
            self._visit(only, upcoming)
            return
        writing = None if self._writing is None else self.groups[self._writing[0]]
        if writing is not None:
            self._offer(writing)
        # the groups a visit can change: demand owed, residents without demand (the
        # watermark or the window may raise it), and the writer (new history)
        visit = set(self._owed) | set(self._open)
        if writing is not None:
            visit.add(writing.gid)
        for gid in sorted(visit):
            self._visit(self.groups[gid], upcoming)

    def _slot(self):
        """``_slot``: a block for a new page."""
        self._tick(None, upcoming=True)
        block = self._first_available()
        if block is not None:
            return self._take(block)
        history = []
        for g in self.groups:
            for page in self._history(g):
                history.append((int(self.bind_order[g.slot[page]]), g.gid))
        history.sort()
        counts = Counter(gid for _, gid in history)
        for gid, count in counts.most_common():
            g = self.groups[gid]
            if count >= self.hot_blocks + 1 and not g.hot:
                self._require(g, "pressure")
                try:
                    self.transition(g)
                except CapacityError:
                    continue
                block = self._first_available()
                if block is not None:
                    return self._take(block)
        raise CapacityError("no reclaimable resident block; tails/readers are protected")

    # -- writes ----------------------------------------------------------------------------
    def write(self, key, tokens):
        """Place the pages of a write of ``tokens`` rows to group ``key`` (page by page,
        with the policy's ticks); returns the (page, block) pairs of the pages it opened."""
        g = self.group(key)
        opened = []
        position, end = g.length, g.length + tokens
        if end > len(g.slot) * self.P:
            raise CapacityError("request exceeds its reserved host capacity")
        try:
            while position < end:
                page, within = divmod(position, self.P)
                count = min(self.P - within, end - position)
                self._writing = (g.gid, page)
                if g.valid[page]:
                    if g.slot[page] < 0:
                        raise RuntimeError("active append tail lost its resident lease")
                    self.stats["resident_hits"] += 1
                    self.stats["append_resident_hits"] += 1
                else:
                    block = self._slot()
                    self._clock += 1
                    g.slot[page] = block
                    self.owner[block], self.owner_page[block] = g.gid, page
                    self.bind_order[block] = self._clock
                    g.residents += 1
                    if not g.required:
                        self._open.add(g.gid)
                    opened.append((page, block))
                g.valid[page] = within + count
                self._tick(g)  # after_write
                position += count
            g.length = end
        finally:
            self._writing = None
        return opened

    def append_within(self, keys):
        """One row for each group of ``keys`` into its tail page, when that equals
        ``write(key, 1)`` for each without placing anything: every tail page already
        has rows and every group's hot region is served, so each write's tick offers no
        new history and raises no demand.  Returns False (and changes nothing) when a
        group does not qualify."""
        groups = [self.group(key) for key in keys]
        for g in groups:
            if not g.hot or g.gid in self._owed or g.length % self.P == 0:
                return False
        for g in groups:
            g.valid[g.length // self.P] += 1
            g.length += 1
        self.stats["resident_hits"] += len(groups)
        self.stats["append_resident_hits"] += len(groups)
        return True

    # -- release ------------------------------------------------------------------------
    def release(self, request):
        """``HybridKVCache.release_request`` and its collect: every hot block and resident
        page of the request's groups becomes an empty block (a queued one leaves the
        reclaim queue), the groups leave the plan, then a tick over every group.
        Returns the groups' keys."""
        layers = self.requests.pop(request)
        groups = [self.groups[self._by_key.pop((request, layer))] for layer in range(layers)]
        for g in groups:
            for block in g.hot:
                heapq.heappush(self.free, int(block))
            g.hot = []
        for g in groups:
            for page in np.flatnonzero(g.slot >= 0).tolist():
                block = int(g.slot[page])
                if self.queued[block]:
                    self.queued[block] = False
                    self.n_queued -= 1
                self.owner[block] = -1
                heapq.heappush(self.free, block)
                g.slot[page] = -1
                self.stats["evictions"] += 1
            g.residents = 0
            g.released = True
            self._open.discard(g.gid)
            self._owed.discard(g.gid)
        self.detached = [(key, page) for key, page in self.detached if key[0] != request]
        self.stats["retired_requests"] += 1
        self._tick(None)
        return [g.key for g in groups]

    def resident_pages(self, key):
        """(pages, blocks) of the group's resident pages."""
        g = self.group(key)
        pages = np.flatnonzero(g.slot >= 0)
        return pages, g.slot[pages]
