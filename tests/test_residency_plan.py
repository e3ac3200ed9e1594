"""The incremental placement of the batched engine (``PlacementPlan``) against the
policy itself (``HybridKVCache`` on the CPU): random write sequences -- prompts of
random lengths written layer by layer, then single-token decode writes in request
or layer order -- under tight and loose slabs, small windows and watermarks.  After
every write, every page's block, every hot region, the hot demand and its trigger,
the reclaim queue and the policy counters are equal, and so is every refusal."""

import re

import numpy as np
import pytest
import torch

from mini_hisparse_amd.config import CacheConfig, CapacityError
from mini_hisparse_amd.hybrid import HotConfig
from mini_hisparse_amd.residency import PlacementPlan
from tests.cpu_ops import make_cache

COUNTERS = ("hot_trigger_window", "hot_trigger_watermark", "hot_trigger_pressure", "hot_trigger_explicit",
            "hot_region_allocations", "clean_page_unpins", "unpinned_block_reuses", "evictions",
            "resident_hits", "append_resident_hits")


def compare(cache, plan):
    assert cache.allocator.reclaim_queue().tolist() == list(plan.queue)
    for key, tables in cache.tables.items():
        g = plan.group(key)
        lp = cache.storage.layer_pages(*key)
        n = lp.materialized
        np.testing.assert_array_equal(lp.slot[:n], g.slot[:n], err_msg=str(key))
        assert (g.slot[n:] < 0).all()
        assert list(tables.blocks) == g.hot, key
        assert (tables.hot_required, tables.trigger) == (g.required, g.trigger), key
    for name in COUNTERS:
        assert cache.storage.stats[name] == plan.stats[name], name


def run_case(seed, pressure=False):
    """One random sequence; ``pressure``: a window no layer reaches and no watermark, so
    blocks run out while no layer offers history (the pressure route)."""
    rng = np.random.default_rng(seed)
    P = int(rng.choice([2, 4]))
    requests, layers = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    hot_rows = P * int(rng.integers(1, 4))
    window = 64 if pressure else int(rng.integers(2, 9))
    watermark = 0 if pressure else [None, 0, int(rng.integers(1, 6))][int(rng.integers(0, 3))]
    lengths = [int(rng.integers(1, 14 * P)) for _ in range(requests)]
    decode = int(rng.integers(0, 3 * P))
    need = sum(layers * (-(-(n + decode) // P)) for n in lengths)
    blocks = max(layers * (hot_rows // P + 2), int(rng.integers(need // 4 + 1, need + requests * layers * 4 + 2)))
    host_pages = need + 8
    config = CacheConfig(gpu_pages=blocks, host_pages=host_pages, page_size=P, kv_heads=1, head_dim=8, device="cpu")
    cache = make_cache(config, HotConfig(hot_rows, hot_rows, resident_window_pages=window,
                                         transition_watermark=watermark))
    plan = PlacementPlan(blocks, P, hot_rows, window=window, watermark=watermark)
    gen = torch.Generator().manual_seed(seed)

    def both(real, mine):
        try:
            real()
        except CapacityError as error:
            with pytest.raises(CapacityError, match=re.escape(str(error)[:20])):
                mine()
            return False
        mine()
        return True

    admitted = []
    for r in range(requests):
        if not both(lambda: cache.reserve(r, lengths[r] + decode, layers), lambda: plan.reserve(r, lengths[r] + decode,
                                                                                                   layers)):
            continue
        admitted.append(r)
        compare(cache, plan)
        for layer in range(layers):
            k = torch.randn(lengths[r], 1, 8, generator=gen)
            if not both(lambda: cache.write(r, layer, k, k), lambda: plan.write((r, layer), lengths[r])):
                return
            compare(cache, plan)
    request_major = bool(rng.integers(0, 2))
    for _ in range(decode):
        order = [(r, l) for r in admitted for l in range(layers)] if request_major else \
            [(r, l) for l in range(layers) for r in admitted]
        if plan.append_within(order):  # the plan's shortcut for a step that places nothing
            for r, layer in order:
                k = torch.randn(1, 1, 8, generator=gen)
                cache.write(r, layer, k, k)
            compare(cache, plan)
            continue
        for r, layer in order:
            k = torch.randn(1, 1, 8, generator=gen)
            if not both(lambda: cache.write(r, layer, k, k), lambda: plan.write((r, layer), 1)):
                return
            compare(cache, plan)


@pytest.mark.parametrize("seed", range(40))
def test_placement_plan_takes_the_policys_decisions(seed):
    run_case(seed)


@pytest.mark.parametrize("seed", range(20))
def test_placement_plan_under_pressure(seed):
    run_case(1000 + seed, pressure=True)


def test_a_long_prefill_takes_the_window_route_and_queues_history_tail_first():
    """One request, one layer, 40 pages, window 4: the fourth page's tick requires the
    hot region, which comes from the empty blocks; the history (pages 0-1 then) joins
    the queue nearest the tail first, and later pages take empty blocks while any
    remain, then the oldest queued block."""
    P, blocks = 4, 24
    plan = PlacementPlan(blocks, P, hot_rows=8, window=4, watermark=0)
    plan.reserve("a", 40 * P, 1)
    plan.write(("a", 0), 40 * P)
    g = plan.group(("a", 0))
    assert g.trigger == "window" and len(g.hot) == 2
    assert g.hot == [4, 5]  # pages 0-3 took blocks 0-3, the region the next two
    pages, held = plan.resident_pages(("a", 0))
    assert held.size == blocks - 2  # every other block ends up holding a page
    assert pages[-1] == 39 and pages[-2] == 38


def run_churn_case(seed):
    """Requests admitted, decoded, released and replaced: after every release the freed
    hot blocks and resident pages are empty blocks again (queued ones leave the reclaim
    queue), and later admissions and writes take them lowest first -- the same blocks,
    regions, queue and counters as ``HybridKVCache.release_request``."""
    rng = np.random.default_rng(seed)
    P = int(rng.choice([2, 4]))
    layers = int(rng.integers(1, 4))
    hot_rows = P * int(rng.integers(1, 4))
    window = int(rng.integers(2, 9))
    watermark = [None, 0, int(rng.integers(1, 6))][int(rng.integers(0, 3))]
    max_len, decode = 10 * P, 2 * P
    per_request = layers * (-(-(max_len + decode) // P))
    blocks = max(layers * (hot_rows // P + 2) * 2, int(rng.integers(per_request // 2 + 1, 2 * per_request + 2)))
    config = CacheConfig(gpu_pages=blocks, host_pages=8 * per_request, page_size=P, kv_heads=1, head_dim=8,
                         device="cpu")
    cache = make_cache(config, HotConfig(hot_rows, hot_rows, resident_window_pages=window,
                                         transition_watermark=watermark))
    plan = PlacementPlan(blocks, P, hot_rows, window=window, watermark=watermark)
    gen = torch.Generator().manual_seed(seed)
    live, next_id, budget = [], 0, {}
    for _ in range(6):
        # admit up to two requests (a refused one is dropped, as the engine would defer it)
        for _ in range(int(rng.integers(1, 3))):
            r, n = next_id, int(rng.integers(1, max_len))
            next_id += 1
            try:
                cache.reserve(r, n + decode, layers)
            except CapacityError as error:
                with pytest.raises(CapacityError, match=re.escape(str(error)[:20])):
                    plan.reserve(r, n + decode, layers)
                continue
            plan.reserve(r, n + decode, layers)
            for layer in range(layers):
                k = torch.randn(n, 1, 8, generator=gen)
                try:
                    cache.write(r, layer, k, k)
                except CapacityError:
                    with pytest.raises(CapacityError):
                        plan.write((r, layer), n)
                    return
                plan.write((r, layer), n)
                compare(cache, plan)
            live.append(r)
            budget[r] = decode
        # a few decode steps, request by request, within each request's reservation
        for _ in range(int(rng.integers(0, decode // 2 + 1))):
            for r in live:
                if budget[r] == 0:
                    continue
                budget[r] -= 1
                for layer in range(layers):
                    k = torch.randn(1, 1, 8, generator=gen)
                    try:
                        cache.write(r, layer, k, k)
                    except CapacityError:
                        with pytest.raises(CapacityError):
                            plan.write((r, layer), 1)
                        return
                    plan.write((r, layer), 1)
            compare(cache, plan)
        # release one or two requests
        for _ in range(min(len(live), int(rng.integers(1, 3)))):
            r = live.pop(int(rng.integers(0, len(live))))
            cache.release_request(r)
            plan.release(r)
            compare(cache, plan)
    return next_id


@pytest.mark.parametrize("seed", range(30))
def test_placement_plan_releases_like_the_policy(seed):
    run_churn_case(2000 + seed)


def test_release_returns_every_block():
    """One request fills the slab (hot region, history queued); after its release every
    block is empty again and the next request's pages take them from the lowest."""
    P, blocks = 4, 24
    plan = PlacementPlan(blocks, P, hot_rows=8, window=4, watermark=0)
    plan.reserve("a", 40 * P, 1)
    plan.write(("a", 0), 40 * P)
    assert plan.available() < blocks
    plan.release("a")
    assert plan.available() == blocks and plan.queue == []
    plan.reserve("b", 3 * P, 1)
    assert [block for _, block in plan.write(("b", 0), 3 * P)] == [0, 1, 2]
    with pytest.raises(KeyError):
        plan.release("a")
