"""The device block slab and its leases (same semantics as allocator.py:9-66 of the
reference).

One tensor ``storage`` of ``[gpu_pages, 2, P, Hkv, D]`` holds every resident
page and every hot block.  A block is either free (empty), bound to an owner
key, or bound but *reclaimable* (its bytes still readable until it is taken).
Each bind bumps the block's generation, so a stale (slot, generation, owner)
handle is detected (ABA).

Beyond the reference, bound page keys are also indexed per (request, layer)
in bind order, so per-layer scans do not walk every block of the device.
"""

from __future__ import annotations

from collections import Counter, OrderedDict
from dataclasses import dataclass

import torch


@dataclass
class DeviceSlot:
    owner: tuple | None = None
    generation: int = 0
    fence: object = None


class DeviceAllocator:
    def __init__(self, config):
        self.storage = torch.empty(
            (config.gpu_pages, 2, config.page_size, config.kv_heads, config.head_dim),
            device=config.device,
            dtype=config.dtype,
        )
        self.slots = [DeviceSlot() for _ in range(config.gpu_pages)]
        self.free = set(range(config.gpu_pages))
        # slot -> callback run when a readable-but-unpinned block is actually taken
        self.reclaimable: OrderedDict[int, object] = OrderedDict()
        # owner key -> slot, in bind order
        self.lru: OrderedDict[tuple, int] = OrderedDict()
        # (request, layer) -> OrderedDict(page key -> slot) for logical pages only
        self.by_group: dict[tuple, OrderedDict] = {}
        self.occupancy: Counter = Counter()
        self.budget = config.gpu_pages

    def touch(self, key):
        self.lru.move_to_end(key)

    def bind(self, slot, key):
        assert slot in self.free and slot < self.budget
        self.free.discard(slot)
        frame = self.slots[slot]
        frame.generation += 1
        frame.owner = key
        self.lru[key] = slot
        if key[2] >= 0:
            self.by_group.setdefault(key[:2], OrderedDict())[key] = slot
        self.occupancy[key[0]] += 1

    def release(self, slot, fence):
        frame = self.slots[slot]
        key = frame.owner
        assert key is not None
        self.reclaimable.pop(slot, None)
        del self.lru[key]
        if key[2] >= 0:
            group = self.by_group[key[:2]]
            del group[key]
            if not group:
                del self.by_group[key[:2]]
        self.occupancy[key[0]] -= 1
        frame.owner, frame.fence = None, fence
        self.free.add(slot)

    def unpin(self, slot, on_reuse):
        assert self.slots[slot].owner is not None and slot not in self.free
        self.reclaimable.setdefault(slot, on_reuse)

    def reclaim(self, slot):
        """Run the owner's callback only when the block is actually taken."""
        self.reclaimable[slot](slot)
        assert slot in self.free and slot not in self.reclaimable

    def group_pages(self, group):
        """Bound logical page keys of one (request, layer), in bind order."""
        return self.by_group.get(group, {})

    def validate(self, slot, generation, owner):
        frame = self.slots[slot]
        if frame.owner != owner or frame.generation != generation:
            raise RuntimeError("stale device-slot generation (ABA)")
