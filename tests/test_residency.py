"""Residency policy of the hybrid cache: readable-but-reclaimable history, completion
publication of host mirrors, and the three triggers of a hot region (window,
watermark, pressure).  The scenarios and their known answers are those of the
reference's residency tests (mini-hisparse tests/test_residency.py); the mirror
completion doubles stand in for device events on the CPU."""

import pytest
import torch

from mini_hisparse_amd.config import CapacityError
from mini_hisparse_amd.hybrid import ACTIVE_TAIL_PAGES
from mini_hisparse_amd.row_index import LogicalTopK
from tests.cache_harness import Harness
from tests.conftest import gpu_available


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    if request.param.startswith("cuda") and not gpu_available():
        pytest.skip("no ROCm GPU")
    torch.set_num_threads(1)
    return request.param


def cache_of(device, pages=7, watermark=0, window=64, seed=0):
    """One KV head of 8 dims, pages of 4 tokens, a hot region of one block (4 rows)."""
    return Harness.hybrid(device, gpu_pages=pages, host_pages=128, window=window, watermark=watermark, seed=seed)


def positions(device, values):
    return LogicalTopK(torch.tensor(values, dtype=torch.int32, device=device))


class FakeCompletion:
    """A host-mirror event under the test's control."""

    def __init__(self, on_wait=None):
        self.done, self.waits, self.on_wait = False, 0, on_wait

    def query(self):
        return self.done

    def synchronize(self):
        if self.on_wait is not None:
            self.on_wait()
        self.done = True
        self.waits += 1


def test_reclaimable_history_hits_until_its_block_is_taken(device):
    h = cache_of(device)
    for name in "ab":
        h.cache.reserve(name, 64, 1)
    h.write("a", 12)
    h.cache.storage.synchronize()
    page = h.page("a", 0)
    slot, host, generation = page.slot, page.host_slot, h.cache.allocator.slots[page.slot].generation
    h.cache.reclaim_history("a", 0)
    assert h.cache.page_state(page.key)["residency"] == "clean_unpinned"
    # still mapped, same generation; 3 empty blocks + this readable one can be allocated
    assert page.slot == slot and h.cache.tables["a", 0].resident[0].item() == slot
    assert h.cache.allocator.slots[slot].generation == generation
    assert h.cache.snapshot()["allocatable_device_blocks"] == 4
    h.attend("a", [0])
    assert h.row_stats()["misses"] == 0
    h.write("b", 12)  # empty blocks go first
    assert page.slot == slot and h.cache.storage.stats["unpinned_block_reuses"] == 0
    h.write("b", 1)  # none left: b's page 3 takes a's readable block
    assert page.slot is None and page.host_slot == host
    assert h.cache.tables["a", 0].resident[0].item() == -1
    assert h.cache.owners[slot] == ("b", 0, 3)
    assert h.cache.allocator.slots[slot].generation == generation + 1
    with pytest.raises(RuntimeError, match="stale"):
        h.cache.allocator.validate(slot, generation, page.key)
    h.attend("a", [0])
    assert h.row_stats()["misses"] == 1  # now loaded from the host mirror
    h.cache.assert_invariants()


def test_a_reader_keeps_a_reclaimable_block(device):
    h = cache_of(device)
    for name in "ab":
        h.cache.reserve(name, 64, 1)
    k, _ = h.write("a", 12)
    h.cache.storage.synchronize()
    h.cache.reclaim_history("a", 0)
    slot = h.page("a", 0).slot
    with h.cache.resolve("a", 0, positions(device, [0])) as lease:
        assert slot in h.cache.allocator.reclaimable and slot not in h.cache._available_blocks()
        if h.cache.storage.cuda:
            torch.cuda._sleep(2_000_000)
        read = h.cache.pool[slot, 0, 0].clone()
        h.write("b", 13)  # b must move its own history to its hot region instead
        assert h.page("a", 0).slot == slot and h.cache.tables["b", 0].blocks
        lease._validate()
    torch.testing.assert_close(read, k[0])
    assert slot in h.cache._available_blocks()
    h.cache.assert_invariants()


@pytest.mark.parametrize(
    "trigger,pages,window,watermark,first,second,free_after",
    [
        # a resident window of 3 pages: 2 pages written, then the third raises demand
        ("window", 12, 3, 0, 8, 4, 8),
        # 6 of 10 blocks used (4 free = watermark): the next allocation would cross it
        ("watermark", 10, 64, 4, 24, 4, 2),
    ],
)
def test_hot_region_triggers_before_any_eviction(device, trigger, pages, window, watermark, first, second,
                                                 free_after):
    h = cache_of(device, pages=pages, window=window, watermark=watermark)
    h.cache.reserve("a", 64, 1)
    h.write("a", first)
    tables = h.cache.tables["a", 0]
    assert not tables.hot_required and not tables.blocks
    h.write("a", second)
    assert tables.hot_required and tables.trigger == trigger and tables.blocks
    assert h.cache.storage.stats["evictions"] == 0
    assert len(h.cache.allocator.free) == free_after
    if trigger == "window":
        h.cache.storage.synchronize()
        h.cache.collect()
        assert h.cache.page_state(("a", 0, 0))["residency"] == "clean_unpinned" and h.resident("a", 0)
    h.cache.assert_invariants()


def test_demand_raised_during_a_lease_is_served_after_it(device):
    h = cache_of(device, pages=6)
    h.cache.reserve("a", 64, 1)
    h.write("a", 12)
    tables = h.cache.tables["a", 0]
    resident = tables.resident.clone()
    with h.cache.resolve("a", 0, positions(device, [0, 4, 8])):
        with pytest.raises(CapacityError, match="active row lease"):
            h.cache.transition_to_host("a", 0)
        assert tables.hot_required and not tables.blocks
        assert torch.equal(resident, tables.resident)  # residents kept
        h.cache.collect()
        assert not tables.blocks  # a busy layer is not transitioned
    h.cache.collect()
    assert tables.blocks
    h.cache.assert_invariants()


def test_both_active_tails_stay_resident_across_page_boundaries(device):
    assert ACTIVE_TAIL_PAGES == 2
    h = cache_of(device, pages=3, watermark=None)
    h.cache.reserve("a", 64, 1)
    h.write("a", 9)  # pages 0, 1 full, page 2 holds one row
    assert [h.resident("a", p) for p in range(3)] == [False, True, True]
    h.write("a", 3)  # page 2 seals; page 1 is still the tail before it
    assert h.resident("a", 1)
    h.write("a", 1)  # page 3 opens: page 1 leaves
    assert [h.resident("a", p) for p in (1, 2, 3)] == [False, True, True]
    h.cache.assert_invariants()
    small = cache_of(device, pages=2)
    with pytest.raises(CapacityError, match="credits"):
        small.cache.reserve("a", 64, 1)
    assert not small.cache.storage.requests and not small.cache.tables


def test_one_hot_block_serves_selections_that_always_miss(device):
    """H = U: no spare row, every selected row misses, zero hits protected, and the two
    tails never leave: 16 steps x 4 misses (reference known answer [0, 0, 64])."""
    h = cache_of(device, pages=3, watermark=None, seed=29)
    h.cache.reserve("a", 64, 1)
    h.write("a", 32)
    h.cache.reset_stats()
    for step in range(16):
        h.write("a", 1)
        chosen = ([0, 4, 8, 12], [1, 5, 9, 13])[step % 2]
        assert not any(h.resident("a", t // 4) for t in chosen)
        h.attend("a", chosen)
        tail = (len(h.kv("a")[0]) - 1) // 4
        assert h.resident("a", tail - 1) and h.resident("a", tail)
        h.cache.assert_invariants()
    assert h.cache.row_stats.tolist() == [0, 0, 64]
    assert h.cache.storage.requests["a"].lengths == [48]
    assert h.cache.storage.stats["peak_device_pages"] <= 3
    h.cache.release_request("a")
    h.cache.assert_invariants()


def test_a_page_with_a_pending_mirror_is_not_offered():
    h = cache_of("cpu", pages=6)
    h.cache.reserve("a", 64, 1)
    h.write("a", 12)
    page = h.page("a", 0)

    def never_wait():
        pytest.fail("a policy tick must not wait for a pending mirror")

    pending = FakeCompletion(on_wait=never_wait)
    page.host_ready, page.host_committed_version = pending, 0
    h.cache.pending_clean.add(page.key)
    h.cache.reclaim_history("a", 0)
    assert h.cache.page_state(page.key)["residency"] == "dirty"
    assert page.slot not in h.cache.allocator.reclaimable
    h.cache.collect()
    assert page.slot not in h.cache.allocator.reclaimable
    pending.done = True
    h.cache.collect()
    assert h.cache.page_state(page.key)["residency"] == "clean_unpinned"
    page.host_ready = None
    h.cache.release_request("a")
    h.cache.assert_invariants()


def test_pressure_waits_for_one_eligible_mirror():
    h = cache_of("cpu", pages=3, watermark=0)
    h.cache.reserve("a", 64, 1)
    h.write("a", 12)
    # every block is resident; a hot region plus a new tail need completed history
    doubles = []
    for index in (0, 1):
        page = h.page("a", index)
        doubles.append(FakeCompletion())
        page.host_ready, page.host_committed_version = doubles[-1], 0
        h.cache.pending_clean.add(page.key)
    real_wait = h.cache.storage.wait
    h.cache.storage.wait = lambda stream, event: None  # the doubles are not device events
    h.write("a", 1)
    assert sum(d.waits for d in doubles) >= 1
    assert h.cache.storage.stats["pressure_mirror_waits"] >= 1
    for key in list(h.cache.storage.pages):
        h.cache.storage.pages[key].host_ready = None
    h.cache.storage.wait = real_wait
    h.cache.release_request("a")
    h.cache.assert_invariants()


@pytest.mark.gpu
def test_device_mirror_still_running_keeps_the_page_pinned():
    """The host mirror of a write is part of its append launch on the compute stream:
    queued behind a long kernel, the page stays dirty (not reclaimable, no pressure
    wait) until that launch completes."""
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    h = cache_of("cuda:0", pages=8)
    h.cache.reserve("a", 64, 1)
    k, v = h.rows(12)
    h.cache.storage.synchronize()
    torch.cuda._sleep(100_000_000)  # on the compute stream, ahead of the write
    h.cache.write("a", 0, k, v)
    page = h.page("a", 0)
    h.cache.transition_to_host("a", 0)
    assert not page.host_ready.query()
    assert page.slot not in h.cache.allocator.reclaimable
    assert h.cache.storage.stats["pressure_mirror_waits"] == 0
    h.cache.storage.synchronize()
    h.cache.collect()
    assert h.cache.page_state(page.key)["residency"] == "clean_unpinned"
    h.cache.assert_invariants()
