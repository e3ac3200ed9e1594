"""Readable free pages, mirror publication and proactive hot admission,
re-expressed from the reference's tests/test_residency.py (CPU oracle backend
and GPU HIP backend)."""

import pytest
import torch

import oracle
from mini_hisparse_amd.attention import row_attention
from mini_hisparse_amd.config import CacheConfig, CapacityError
from mini_hisparse_amd.hybrid import ACTIVE_TAIL_PAGES, HotConfig
from mini_hisparse_amd.row_index import LogicalTopK
from tests.conftest import gpu_available
from tests.cpu_ops import make_cache


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    if request.param.startswith("cuda") and not gpu_available():
        pytest.skip("no ROCm GPU")
    torch.set_num_threads(1)
    return request.param


def make(device, pages=7, watermark=0, window=64):
    config = CacheConfig(gpu_pages=pages, host_pages=128, page_size=4, kv_heads=1, head_dim=8, device=device)
    return make_cache(config, HotConfig(4, 4, resident_window_pages=window, transition_watermark=watermark))


def spin_cycles(ms):
    """Cycle count for torch's spin kernel that keeps a stream busy for at least ``ms``.

    The spin counts shader clock cycles, whose rate follows the GPU's clock state:
    the fastest of three calibration spins sets the count, so that a later spin at a
    higher clock than during calibration still lasts ``ms``.
    """
    fastest = None
    for _ in range(3):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        torch.cuda._sleep(10_000_000)
        end.record()
        end.synchronize()
        elapsed = max(start.elapsed_time(end), 1e-3)
        fastest = elapsed if fastest is None else min(fastest, elapsed)
    return int(10_000_000 * ms / fastest)


def write(cache, name, count):
    k, v = [torch.randn(count, 1, 8, device=cache.device) for _ in range(2)]
    cache.write(name, 0, k, v)
    return k, v


def select(cache, positions):
    return LogicalTopK(torch.tensor(positions, dtype=torch.int32, device=cache.device))


def dense(q, k, v):
    return torch.from_numpy(oracle.dense_attention(q.cpu(), k.cpu(), v.cpu())).to(q.dtype).to(q.device)


def test_unpinned_page_still_hits_until_actual_block_reuse(device):
    cache = make(device)
    for name in ("a", "b"):
        cache.reserve(name, 64, 1)
    k, v = write(cache, "a", 12)
    cache.storage.synchronize()
    page = cache.storage.pages["a", 0, 0]
    slot, host = page.slot, page.host_slot
    generation = cache.allocator.slots[slot].generation
    cache.reclaim_history("a", 0)
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    assert page.slot == slot and cache.tables["a", 0].resident[0].item() == slot
    assert cache.allocator.slots[slot].generation == generation
    assert cache.snapshot()["allocatable_device_blocks"] == 4  # 3 empty + 1 readable

    q = torch.randn(2, 8, device=device)
    torch.testing.assert_close(row_attention(q, cache, "a", 0, select(cache, [0])), dense(q, k[:1], v[:1]))
    assert cache.snapshot()["row_stats"]["misses"] == 0
    write(cache, "b", 12)  # empty blocks are taken before readable clean KV
    assert page.slot == slot and cache.storage.stats["unpinned_block_reuses"] == 0
    write(cache, "b", 1)  # no empties left: A's old block is reused now
    assert page.slot is None and page.host_slot == host
    assert cache.tables["a", 0].resident[0].item() == -1
    assert cache.owners[slot] == ("b", 0, 3)
    assert cache.allocator.slots[slot].generation == generation + 1
    with pytest.raises(RuntimeError, match="stale"):
        cache.allocator.validate(slot, generation, page.key)
    torch.testing.assert_close(row_attention(q, cache, "a", 0, select(cache, [0])), dense(q, k[:1], v[:1]))
    assert cache.snapshot()["row_stats"]["misses"] == 1
    cache.assert_invariants()


def test_consumer_lease_temporarily_protects_a_readable_free_block(device):
    cache = make(device)
    for name in ("a", "b"):
        cache.reserve(name, 64, 1)
    k, _ = write(cache, "a", 12)
    cache.storage.synchronize()
    cache.reclaim_history("a", 0)
    page = cache.storage.pages["a", 0, 0]
    slot = page.slot
    with cache.resolve("a", 0, select(cache, [0])) as lease:
        assert slot in cache.allocator.reclaimable
        assert slot not in cache._available_blocks()
        if cache.storage.cuda:
            torch.cuda._sleep(2_000_000)
        observed = cache.pool[slot, 0, 0].clone()
        write(cache, "b", 13)  # B must reclaim its own history instead
        assert page.slot == slot
        assert cache.tables["b", 0].blocks
        lease._validate()
    torch.testing.assert_close(observed, k[0])
    assert slot in cache._available_blocks()
    cache.assert_invariants()


def test_window_triggers_hot_without_memory_exhaustion(device):
    cache = make(device, pages=12, window=3)
    cache.reserve("a", 64, 1)
    write(cache, "a", 8)
    assert not cache.tables["a", 0].hot_required
    write(cache, "a", 4)
    tables = cache.tables["a", 0]
    assert tables.hot_required and tables.trigger == "window" and tables.blocks
    assert cache.storage.stats["evictions"] == 0
    assert len(cache.allocator.free) == 8
    cache.storage.synchronize()
    cache.collect()
    assert cache.page_state(("a", 0, 0))["residency"] == "clean_unpinned"
    assert cache.storage.pages["a", 0, 0].slot is not None
    cache.assert_invariants()


def test_watermark_uses_projected_capacity_before_the_last_block(device):
    cache = make(device, pages=10, watermark=4)
    cache.reserve("a", 64, 1)
    write(cache, "a", 24)
    assert len(cache.allocator.free) == 4 and not cache.tables["a", 0].blocks
    write(cache, "a", 4)
    assert cache.tables["a", 0].trigger == "watermark"
    assert cache.tables["a", 0].blocks
    assert len(cache.allocator.free) == 2 and cache.storage.stats["evictions"] == 0
    cache.assert_invariants()


def test_hot_demand_survives_a_busy_layer_without_revoking_residents(device):
    cache = make(device, pages=6)
    cache.reserve("a", 64, 1)
    write(cache, "a", 12)
    before = cache.tables["a", 0].resident.clone()
    with cache.resolve("a", 0, select(cache, [0, 4, 8])):
        with pytest.raises(CapacityError, match="active row lease"):
            cache.transition_to_host("a", 0)
        assert cache.tables["a", 0].hot_required
        assert not cache.tables["a", 0].blocks
        torch.testing.assert_close(before, cache.tables["a", 0].resident)
        cache.collect()
        assert not cache.tables["a", 0].blocks
    cache.collect()
    assert cache.tables["a", 0].blocks
    cache.assert_invariants()


def test_two_active_tails_survive_full_and_partial_page_boundaries(device):
    assert ACTIVE_TAIL_PAGES == 2
    cache = make(device, pages=3, watermark=None)
    cache.reserve("a", 64, 1)
    write(cache, "a", 9)
    pages = cache.storage.pages
    assert pages["a", 0, 0].slot is None
    assert pages["a", 0, 1].slot is not None and pages["a", 0, 2].slot is not None
    write(cache, "a", 3)  # the last page seals; the full page before it is still a tail
    assert pages["a", 0, 1].slot is not None
    write(cache, "a", 1)
    assert pages["a", 0, 1].slot is None
    assert pages["a", 0, 2].slot is not None and pages["a", 0, 3].slot is not None
    cache.assert_invariants()
    small = make(device, pages=2)
    with pytest.raises(CapacityError, match="credits"):
        small.reserve("a", 64, 1)
    assert not small.storage.requests and not small.tables


def test_minimum_hot_capacity_progresses_when_every_selected_row_misses(device):
    """H = U needs no spare row: protect zero hits, replace every slot, cross the tails."""
    torch.manual_seed(29)
    cache = make(device, pages=3, watermark=None)  # one hot block + two tails
    cache.reserve("a", 64, 1)
    k, v = write(cache, "a", 32)
    cache.reset_stats()
    choices = ([0, 4, 8, 12], [1, 5, 9, 13])
    for step in range(16):
        new_k, new_v = write(cache, "a", 1)
        k, v = torch.cat((k, new_k)), torch.cat((v, new_v))
        positions = choices[step % 2]
        assert all(cache.storage.pages["a", 0, t // 4].slot is None for t in positions)
        q = torch.randn(2, 8, device=device)
        actual = row_attention(q, cache, "a", 0, select(cache, positions))
        torch.testing.assert_close(actual, dense(q, k[positions], v[positions]), atol=3e-6, rtol=3e-5)
        tail = (len(k) - 1) // 4
        assert all(cache.storage.pages["a", 0, p].slot is not None for p in (tail - 1, tail))
        cache.assert_invariants()
    assert cache.row_stats.tolist() == [0, 0, 64]
    assert cache.storage.requests["a"].lengths == [48]
    assert cache.storage.stats["peak_device_pages"] <= 3
    cache.release_request("a")
    cache.assert_invariants()


class Completion:
    """Host-side stand-in for a device event (query/synchronize)."""

    def __init__(self, fail_on_wait=False):
        self.done, self.waits, self.fail_on_wait = False, 0, fail_on_wait

    def query(self):
        return self.done

    def synchronize(self):
        if self.fail_on_wait:
            pytest.fail("a normal policy tick must not wait for pending mirrors")
        self.done = True
        self.waits += 1


def test_pending_mirror_is_not_clean_and_policy_tick_does_not_wait():
    cache = make("cpu", pages=6)
    cache.reserve("a", 64, 1)
    write(cache, "a", 12)
    page = cache.storage.pages["a", 0, 0]
    completion = Completion(fail_on_wait=True)
    page.host_ready, page.host_committed_version = completion, 0
    cache.pending_clean.add(page.key)
    cache.reclaim_history("a", 0)
    assert cache.page_state(page.key)["residency"] == "dirty"
    assert page.slot not in cache.allocator.reclaimable
    cache.collect()
    assert page.slot not in cache.allocator.reclaimable
    completion.done = True
    cache.collect()
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    page.host_ready = None
    cache.release_request("a")
    cache.assert_invariants()


@pytest.mark.gpu
def test_gpu_page_is_not_unpinned_before_its_d2h_event_completes():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    # the same writes once on a scratch cache, so first-launch code loading of
    # every kernel on this path is done before the timed stall below
    warm = make("cuda:0", pages=8)
    warm.reserve("w", 64, 1)
    write(warm, "w", 12)
    warm.transition_to_host("w", 0)
    warm.storage.synchronize()
    cache = make("cuda:0", pages=8)
    cache.reserve("a", 64, 1)
    k, v = [torch.randn(12, 1, 8, device=cache.device) for _ in range(2)]
    cache.storage.synchronize()
    with torch.cuda.stream(cache.storage.transfer):
        torch.cuda._sleep(spin_cycles(1000.0))  # the transfer stream stays busy for ~1 s
    cache.write("a", 0, k, v)
    page = cache.storage.pages["a", 0, 0]
    cache.transition_to_host("a", 0)
    assert not page.host_ready.query()
    assert page.slot not in cache.allocator.reclaimable
    assert cache.storage.stats["pressure_mirror_waits"] == 0
    cache.storage.synchronize()
    cache.collect()
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    cache.assert_invariants()


def test_pressure_waits_only_for_an_eligible_mirror_event():
    cache = make("cpu", pages=3, watermark=0)
    cache.reserve("a", 64, 1)
    write(cache, "a", 12)
    # every block resident: a hot region and a new tail need completed history
    completions = []
    for index in (0, 1):
        page = cache.storage.pages["a", 0, index]
        event = Completion()
        page.host_ready, page.host_committed_version = event, 0
        cache.pending_clean.add(page.key)
        completions.append(event)
    original_wait = cache.storage.wait
    cache.storage.wait = lambda stream, event: None  # CPU completion stand-in only
    write(cache, "a", 1)
    assert sum(e.waits for e in completions) >= 1
    assert cache.storage.stats["pressure_mirror_waits"] >= 1
    for page in cache.storage.pages.values():
        page.host_ready = None
    cache.storage.wait = original_wait
    cache.release_request("a")
    cache.assert_invariants()
