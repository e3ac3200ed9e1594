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
