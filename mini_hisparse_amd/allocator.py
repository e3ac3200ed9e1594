"""Device block table: the one slab that holds every resident page and hot block.

Replaces ``DeviceAllocator`` of the reference (``mini_hisparse/allocator.py:16-66``)
with the same lease semantics, kept as flat per-block arrays instead of one
object per block and ordered dictionaries of owner keys:

* a block is *free*, *bound* to an owner, or bound and *reclaimable* (still
  readable by its owner until a new owner actually takes it; taking it runs the
  owner's ``on_reuse`` callback first);
* every bind increments the block's generation, so a ``(block, generation,
  owner)`` handle taken before a re-bind is detected as stale (ABA);
* the orders the cache policies need are carried by stamps drawn from one
  counter: ``bind_stamp`` (set at bind, renewed by ``touch``) orders bound blocks
  least recently bound/touched first, ``reclaim_stamp`` orders the reclaimable
  queue by the time each block joined it.

Owners are ``(request, layer, index)`` keys; ``index < 0`` names hot block
``-index - 1`` of that layer's hot region.  Internally an owner is a (group,
index) pair of integers with a group number per (request, layer).

Read-only views (``slots``, ``free``, ``reclaimable``, ``lru``, ``occupancy``)
present the table in the reference's shapes for callers and tests that inspect
it; the policies use the array queries (``free_blocks``, ``reclaim_queue``,
``bound_pages``).
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass

import numpy as np
import torch

NO_GROUP = -1


@dataclass(frozen=True)
class SlotView:
    """One block as the reference's ``DeviceSlot`` shows it (owner, generation, fence)."""

    owner: tuple | None
    generation: int
    fence: object


class _Slots:
    def __init__(self, table):
        self._t = table

    def __len__(self):
        return self._t.blocks

    def __getitem__(self, block):
        t = self._t
        return SlotView(t.owner_key(block), int(t.generation[block]), t.fence[block])

    def __iter__(self):
        return (self[i] for i in range(len(self)))


class _ReclaimQueue:
    """Reclaimable blocks in queue order (mapping block -> on_reuse callback)."""

    def __init__(self, table):
        self._t = table

    def __contains__(self, block):
        return isinstance(block, (int, np.integer)) and 0 <= block < self._t.blocks and \
            self._t.reclaim_stamp[block] >= 0

    def __iter__(self):
        return iter(self._t.reclaim_queue().tolist())

    def __len__(self):
        return int(np.count_nonzero(self._t.reclaim_stamp >= 0))

    def __getitem__(self, block):
        return self._t.on_reuse[block]

    def keys(self):
        return set(self._t.reclaim_queue().tolist())


class DeviceAllocator:
    def __init__(self, config):
        n = config.gpu_pages
        self.storage = torch.empty(
            (n, 2, config.page_size, config.kv_heads, config.head_dim), device=config.device, dtype=config.dtype
        )
        self.blocks = n
        self.budget = n
        self.owner_group = np.full(n, NO_GROUP, np.int64)
        self.owner_index = np.zeros(n, np.int64)
        self.generation = np.zeros(n, np.int64)
        self.bind_stamp = np.full(n, -1, np.int64)
        self.reclaim_stamp = np.full(n, -1, np.int64)
        self.fence = [None] * n
        self.on_reuse = [None] * n
        self._clock = 0
        # bumped by every bind, release and unpin: a count of free or reclaimable blocks
        # taken at one version holds until the version changes
        self.version = 0
        self.bound = 0  # blocks bound to a group
        # (request, layer) <-> group number
        self._group_of: dict[tuple, int] = {}
        self._group_key: list[tuple] = []

    # -- groups ----------------------------------------------------------------
    def group_id(self, group) -> int:
        gid = self._group_of.get(group)
        if gid is None:
            gid = self._group_of[group] = len(self._group_key)
            self._group_key.append(group)
        return gid

    def group_key(self, gid):
        return self._group_key[gid]

    def owner_key(self, block):
        gid = int(self.owner_group[block])
        if gid == NO_GROUP:
            return None
        return (*self._group_key[gid], int(self.owner_index[block]))

    def _stamp(self):
        self._clock += 1
        return self._clock

    # -- leases ------------------------------------------------------------------
    def bind(self, block, key):
        if self.owner_group[block] != NO_GROUP or block >= self.budget:
            raise AssertionError(f"block {block} is not free within the budget")
        self.version += 1
        self.bound += 1
        self.owner_group[block] = self.group_id(key[:2])
        self.owner_index[block] = key[2]
        self.generation[block] += 1
        self.bind_stamp[block] = self._stamp()

    def release(self, block, fence):
        if self.owner_group[block] == NO_GROUP:
            raise AssertionError(f"block {block} is not bound")
        self.version += 1
        self.bound -= 1
        self.owner_group[block] = NO_GROUP
        self.bind_stamp[block] = -1
        self.reclaim_stamp[block] = -1
        self.on_reuse[block] = None
        self.fence[block] = fence

    def touch_block(self, block):
        self.bind_stamp[block] = self._stamp()

    def unpin(self, block, on_reuse):
        """Queue a bound block as reclaimable (idempotent: keeps its first place)."""
        if self.owner_group[block] == NO_GROUP:
            raise AssertionError(f"block {block} is not bound")
        if self.reclaim_stamp[block] < 0:
            self.version += 1
            self.reclaim_stamp[block] = self._stamp()
            self.on_reuse[block] = on_reuse

    def reclaim(self, block):
        """Hand a reclaimable block back as free: its owner's callback detaches it."""
        self.on_reuse[block](block)
        if self.owner_group[block] != NO_GROUP or self.reclaim_stamp[block] >= 0:
            raise AssertionError("on_reuse callback must release the block")

    def validate(self, block, generation, owner):
        if self.owner_key(block) != owner or self.generation[block] != generation:
            raise RuntimeError("stale device-slot generation (ABA)")

    def snapshot(self, blocks):
        """(blocks, generations, owner groups, owner indices) of ``blocks`` now: the
        handles of a lease over many blocks, checked at once by ``validate_snapshot``."""
        blocks = np.asarray(blocks, np.int64)
        return blocks, self.generation[blocks].copy(), self.owner_group[blocks].copy(), self.owner_index[blocks].copy()

    def validate_snapshot(self, snapshot):
        """``validate`` of every block of a snapshot: same owner (or still free) and
        same generation."""
        blocks, generation, group, index = snapshot
        same = (self.owner_group[blocks] == group) & ((group == NO_GROUP) | (self.owner_index[blocks] == index))
        if not np.all(same & (self.generation[blocks] == generation)):
            raise RuntimeError("stale device-slot generation (ABA)")

    # -- queries for the policies -----------------------------------------------
    def is_free(self, block):
        return self.owner_group[block] == NO_GROUP

    def free_blocks(self, limit=None):
        """Free blocks below ``limit`` (default: the budget), ascending."""
        limit = self.budget if limit is None else limit
        return np.flatnonzero(self.owner_group[:limit] == NO_GROUP)

    def reclaim_queue(self, limit=None):
        """Reclaimable blocks below ``limit`` (default: all), in queue order."""
        stamps = self.reclaim_stamp if limit is None else self.reclaim_stamp[:limit]
        queued = np.flatnonzero(stamps >= 0)
        return queued[np.argsort(stamps[queued], kind="stable")]

    def bound_pages(self, gid=None):
        """Blocks bound to logical pages (hot blocks excluded), least recently
        bound/touched first; restricted to one group when ``gid`` is given."""
        mask = (self.owner_group != NO_GROUP) & (self.owner_index >= 0)
        if gid is not None:
            mask &= self.owner_group == gid
        blocks = np.flatnonzero(mask)
        return blocks[np.argsort(self.bind_stamp[blocks], kind="stable")]

    def owned_count(self, request_id):
        gids = [g for g, key in enumerate(self._group_key) if key[0] == request_id]
        return int(np.count_nonzero(np.isin(self.owner_group, gids))) if gids else 0

    # -- views in the reference's shapes -------------------------------------------
    @property
    def slots(self):
        return _Slots(self)

    @property
    def free(self):
        return set(np.flatnonzero(self.owner_group == NO_GROUP).tolist())

    @property
    def reclaimable(self):
        return _ReclaimQueue(self)

    @property
    def lru(self):
        """Owner keys of every bound block, least recently bound/touched first."""
        bound = np.flatnonzero(self.owner_group != NO_GROUP)
        order = bound[np.argsort(self.bind_stamp[bound], kind="stable")]
        return [self.owner_key(b) for b in order.tolist()]

    @property
    def occupancy(self):
        return Counter(self._group_key[g][0] for g in self.owner_group[self.owner_group != NO_GROUP].tolist())

    def owners(self):
        return [self.owner_key(b) for b in range(self.blocks)]
