"""The optional page layout (PagedKVCache, paged_attention), re-expressed from the
reference's tests/test_cache.py, tests/test_resources.py and the window case of
tests/test_selection.py.

Tests run on CPU (numpy oracle window kernel injected) and, where marked, on the GPU
with the product's hs_attend_window; the known answers are the reference's.
"""

from dataclasses import replace

import pytest
import torch

import oracle
from mini_hisparse_amd.config import CapacityError
from mini_hisparse_amd.engine import Engine
from mini_hisparse_amd.model import MiniModel, ModelConfig
from mini_hisparse_amd.paged import PagedConfig, paged_attention
from mini_hisparse_amd.selection import Selection, select_pages
from mini_hisparse_amd.storage import Location
from tests.conftest import gpu_available
from tests.cpu_ops import make_paged


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    if request.param.startswith("cuda") and not gpu_available():
        pytest.skip("no ROCm GPU")
    torch.set_num_threads(1)
    return request.param


def dense(q, k, v):
    return torch.from_numpy(oracle.dense_attention(q.cpu(), k.cpu(), v.cpu())).to(q.dtype).to(q.device)


def paged(device, **changes):
    """Two KV heads of 8 dims, pages of 4 tokens, windows of 2 pages (test_cache.py:22-34)."""
    base = PagedConfig(gpu_pages=3, host_pages=48, page_size=4, kv_heads=2, head_dim=8, chunk_pages=2, device=device)
    return make_paged(replace(base, **changes))


def small(**changes):
    """One KV head of 4 dims on the CPU (test_resources.py:15-19)."""
    base = PagedConfig(gpu_pages=3, host_pages=32, page_size=4, kv_heads=1, head_dim=4, device="cpu")
    return make_paged(replace(base, **changes))


def write(cache, name, count, layer=0):
    shape = (count, cache.config.kv_heads, cache.config.head_dim)
    k, v = [torch.randn(shape, device=cache.device, dtype=cache.config.dtype) for _ in range(2)]
    cache.write(name, layer, k, v)
    return k, v


def test_config_checks():
    with pytest.raises(ValueError, match="chunk_pages"):
        PagedConfig(chunk_pages=0, device="cpu")
    with pytest.raises(ValueError, match="eviction policy"):
        PagedConfig(eviction_policy="mru", device="cpu")


# ------------------------------------------------------------ test_cache.py
@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("budget", [1, 2, 5])
def test_partial_residency_append_and_sparse_oracle(device, overlap, budget):
    torch.manual_seed(17)
    cache = paged(device, gpu_pages=budget, overlap=overlap)
    cache.reserve("a", 35, 1)
    k, v = [torch.randn(19, 2, 8, device=device) for _ in range(2)]
    cache.write("a", 0, k, v)
    pointer = cache.pool.data_ptr()
    for _ in range(10):
        new_k, new_v = [torch.randn(1, 2, 8, device=device) for _ in range(2)]
        cache.write("a", 0, new_k, new_v)
        k, v = torch.cat((k, new_k)), torch.cat((v, new_v))
        q = torch.randn(4, 8, device=device)
        # a page listed twice is read once: duplicates do not change token multiplicity
        pages = [0, (len(k) - 1) // 4, 1, 0]
        tokens = [t for p in dict.fromkeys(pages) for t in range(4 * p, min(4 * p + 4, len(k)))]
        got = paged_attention(q, cache, "a", 0, pages)
        torch.testing.assert_close(got, dense(q, k[tokens], v[tokens]), atol=3e-6, rtol=3e-5)
        cache.assert_invariants()
    host_k, host_v = cache.storage.host_kv("a", 0)
    torch.testing.assert_close(host_k, k.cpu())
    torch.testing.assert_close(host_v, v.cpu())
    assert cache.pool.data_ptr() == pointer  # the slab is never reallocated
    assert cache.storage.stats["peak_device_pages"] <= budget
    assert cache.storage.stats["evictions"] > 0
    if budget < 3:
        assert cache.storage.stats["misses"] > 0


def test_acquire_protects_later_hits_and_rejects_overcommit(device):
    cache = paged(device, gpu_pages=2)
    cache.reserve("a", 12, 1)
    write(cache, "a", 12)
    # page 0 is on the host, pages 1 and 2 resident: page 1 is pinned before page 0
    # is placed, although it is older than page 2
    before = cache.storage.pages[("a", 0, 1)].slot
    lease = cache.acquire([("a", 0, 0), ("a", 0, 1)])
    assert cache.storage.pages[("a", 0, 1)].slot == before
    owners = list(cache.owners)
    with pytest.raises(CapacityError):
        cache.acquire([("a", 0, 2)])
    assert cache.owners == owners
    with pytest.raises(RuntimeError):
        cache.release_request("a")
    lease.wait()
    lease.release()
    cache.release_request("a")
    cache.assert_invariants()
    assert len(cache.storage.free_host) == cache.config.host_pages


def test_hot_reuse_no_reload_then_dynamic_pressure(device):
    cache = paged(device, gpu_pages=5)
    cache.reserve("a", 28, 1)
    k, v = write(cache, "a", 28)
    q = torch.randn(4, 8, device=device)
    paged_attention(q, cache, "a", 0, [0])
    assert cache.storage.pages[("a", 0, 0)].location == Location.HOT
    misses = cache.storage.stats["misses"]
    paged_attention(q, cache, "a", 0, [0])
    assert cache.storage.stats["misses"] == misses
    cache.set_budget(1)
    torch.testing.assert_close(paged_attention(q, cache, "a", 0), dense(q, k, v), atol=3e-6, rtol=3e-5)
    cache.set_budget(5)
    cache.assert_invariants()


def test_resident_hits_never_fetch(device):
    cache = paged(device, gpu_pages=5)
    cache.reserve("a", 16, 1)
    write(cache, "a", 13)
    paged_attention(torch.randn(4, 8, device=device), cache, "a", 0)
    assert cache.storage.stats["misses"] == cache.storage.stats["h2d_bytes"] == 0
    assert cache.storage.stats["resident_hits"] == 4


def test_host_admission_is_atomic_and_ids_are_reusable(device):
    cache = paged(device, host_pages=4)
    cache.reserve("a", 8, 2)
    with pytest.raises(CapacityError):
        cache.reserve("b", 1, 1)
    assert "b" not in cache.storage.requests
    cache.release_request("a")
    cache.reserve("a", 16, 1)
    cache.assert_invariants()


def test_indexer_tail_and_invalid_selections(device):
    cache = paged(device)
    cache.reserve("a", 20, 1)
    write(cache, "a", 20)
    q = torch.randn(4, 8, device=device)
    assert select_pages(cache, "a", 0, q, 1) == [4]
    chosen = select_pages(cache, "a", 0, q, 3)
    assert 0 in chosen and 4 in chosen and len(chosen) == 3
    for invalid in ([], [-1], [5]):
        with pytest.raises(ValueError):
            paged_attention(q, cache, "a", 0, invalid)
    with pytest.raises(ValueError):
        paged_attention(q, cache, "a", 0, [0], backend="cuda")
    cache.assert_invariants()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_and_non_power_of_two_page(gpu, dtype):
    cache = paged(gpu, page_size=7, head_dim=24, dtype=dtype)
    cache.reserve("a", 33, 1)
    k, v = [torch.randn(33, 2, 24, device=gpu, dtype=dtype) for _ in range(2)]
    q = torch.randn(6, 24, device=gpu, dtype=dtype)
    cache.write("a", 0, k, v)
    torch.testing.assert_close(paged_attention(q, cache, "a", 0), dense(q, k, v), atol=0.003, rtol=0.015)


@pytest.mark.gpu
def test_delayed_compute_cannot_be_overwritten_by_next_copy(gpu):
    cache = paged(gpu, gpu_pages=1)
    cache.reserve("a", 8, 1)
    k, v = [torch.randn(8, 2, 8, device=gpu) for _ in range(2)]
    cache.write("a", 0, k, v)
    for _ in range(16):
        with cache.acquire([("a", 0, 0)]) as lease:
            torch.cuda._sleep(100000)  # the read below is queued behind a busy kernel
            observed = cache.pool[lease.pages[0].slot, 0].clone()
        with cache.acquire([("a", 0, 1)]):  # loads page 1 into the same (only) slot
            pass
        torch.testing.assert_close(observed, k[:4])
    cache.assert_invariants()


def test_randomized_multi_request_eviction_and_reclamation(device):
    rng = torch.Generator().manual_seed(19)
    cache = paged(device, gpu_pages=3, host_pages=128)
    histories = {}
    for name in "abc":
        cache.reserve(name, 40, 2)
        for layer in range(2):
            k, v = [torch.randn(13, 2, 8, generator=rng).to(device) for _ in range(2)]
            cache.write(name, layer, k, v)
            histories[(name, layer)] = (k, v)
    for step in range(30):
        name, layer = "abc"[step % 3], (step // 3) % 2
        k, v = histories[(name, layer)]
        new_k, new_v = [torch.randn(1, 2, 8, generator=rng).to(device) for _ in range(2)]
        cache.write(name, layer, new_k, new_v)
        k, v = torch.cat((k, new_k)), torch.cat((v, new_v))
        histories[(name, layer)] = (k, v)
        q = torch.randn(4, 8, generator=rng).to(device)
        cache.set_budget(1 + step % 3)
        torch.testing.assert_close(paged_attention(q, cache, name, layer), dense(q, k, v), atol=3e-6, rtol=3e-5)
        cache.assert_invariants()
    for name in "bac":
        cache.release_request(name)
        cache.assert_invariants()


# -------------------------------------------------------- test_resources.py
@pytest.mark.parametrize("policy,keeps_hot", [("legacy", False), ("lru", True), ("fair_lru", True)])
def test_recent_hot_contents_survive_cold_resident(policy, keeps_hot):
    cache = small(gpu_pages=2, eviction_policy=policy)
    cache.reserve("a", 12, 1)
    write(cache, "a", 12)
    with cache.acquire([("a", 0, 0)]):
        pass
    with cache.acquire([("a", 0, 1)]):
        pass
    assert (cache.storage.pages[("a", 0, 0)].slot is not None) == keeps_hot
    cache.assert_invariants()


def test_soft_fair_share_and_borrowing_idle_capacity():
    cache = small(gpu_pages=4)
    cache.reserve("a", 24, 1)
    cache.reserve("b", 8, 1)
    write(cache, "b", 4)  # the oldest page belongs to the under-share request
    write(cache, "a", 12)
    write(cache, "b", 4)
    assert cache.allocator.occupancy == {"a": 2, "b": 2}
    assert cache.storage.pages[("b", 0, 0)].slot is not None
    cache.release_request("b")
    write(cache, "a", 12)
    assert cache.allocator.occupancy["a"] == 4
    cache.assert_invariants()


def test_sink_soft_protection_expires_when_access_pattern_changes():
    cache = small(gpu_pages=2)
    cache.reserve("a", 12, 1)
    write(cache, "a", 12)
    q = torch.randn(2, 4)
    paged_attention(q, cache, "a", 0, [0])
    for page in (1, 2, 1, 2):
        paged_attention(q, cache, "a", 0, [page])
    assert cache.storage.pages[("a", 0, 0)].slot is None
    cache.assert_invariants()


def test_lookahead_preserves_future_hit_and_window_respects_other_leases():
    cache = small()
    cache.reserve("a", 16, 1)
    k, v = write(cache, "a", 16)
    q = torch.randn(2, 4)
    before = cache.storage.stats["attention_misses"]
    got = paged_attention(q, cache, "a", 0, [0, 1, 3])
    assert cache.storage.stats["attention_misses"] - before == 1
    rows = [*range(8), *range(12, 16)]
    torch.testing.assert_close(got, dense(q, k[rows], v[rows]))
    cache.reserve("b", 4, 1)
    write(cache, "b", 4)
    with cache.acquire([("b", 0, 0)]):
        plan = cache.plan([("a", 0, i) for i in range(4)])
        assert plan.pinned_outside == 1 and plan.live_slot_limit <= 2
        torch.testing.assert_close(paged_attention(q, cache, "a", 0), dense(q, k, v))
    cache.assert_invariants()


def test_lazy_materialization_and_index_admission_are_atomic():
    cache = small(host_pages=20, index_budget_bytes=960)
    cache.reserve("a", 40, 2)
    assert len(cache.storage.pages) == 0 and len(cache.storage.free_host) == 20
    assert cache.storage.available_host_credits == 0
    write(cache, "a", 1)
    assert len(cache.storage.pages) == 1 and cache.storage.requests["a"].host_credits == 19
    cache.assert_invariants()
    cache.release_request("a")
    assert len(cache.storage.free_host) == 20
    cache = small(host_pages=20, index_budget_bytes=959)
    with pytest.raises(CapacityError, match="index budget"):
        cache.reserve("a", 40, 2)
    assert not cache.storage.requests and len(cache.storage.free_host) == 20


def test_bfloat16_bounds_are_exact_and_index_budget_counts_actual_bytes():
    cache = small(dtype=torch.bfloat16)
    cache.reserve("a", 12, 1)
    k = torch.randn(7, 1, 4).bfloat16()
    cache.write("a", 0, k, k)
    request = cache.storage.requests["a"]
    assert request.minimum.dtype == torch.bfloat16
    torch.testing.assert_close(request.minimum[0, 0], k[:4].amin(0))
    assert cache.index_bytes == cache.index_reservation_bytes(12, 1) == 3 * 1 * 4 * 8


def test_shrink_rejects_active_slot_atomically_and_versions_track_tail():
    cache = small(gpu_pages=3)
    cache.reserve("a", 12, 1)
    write(cache, "a", 9)
    owner = cache.owners[2]
    with cache.acquire([owner]):
        with pytest.raises(CapacityError):
            cache.set_budget(1)
        assert cache.budget == 3
    cache.set_budget(1)
    write(cache, "a", 3)
    state = cache.storage.page_state(("a", 0, 2))
    assert state["sealed"] and state["content_version"] == 2
    assert state["host_committed_version"] == 2
    cache.assert_invariants()


def test_attention_can_share_fully_leased_resident_pages():
    cache = small(gpu_pages=2)
    cache.reserve("a", 8, 1)
    k, v = write(cache, "a", 8)
    q = torch.randn(2, 4)
    with cache.acquire([("a", 0, 0), ("a", 0, 1)]):
        torch.testing.assert_close(paged_attention(q, cache, "a", 0), dense(q, k, v))
    cache.assert_invariants()


@pytest.mark.gpu
def test_deferred_reclaim_protects_host_bytes_and_slot_generation(gpu):
    cache = make_paged(PagedConfig(gpu_pages=1, host_pages=1, page_size=4, kv_heads=1, head_dim=4, device=gpu))
    cache.reserve("a", 4, 1)
    old_generation = cache.storage.requests["a"].generation
    old, _ = write(cache, "a", 4)
    with cache.acquire([("a", 0, 0)]) as lease:
        handle = lease.handles[0]
        torch.cuda._sleep(100_000_000)
        observed = cache.pool[0, 0].clone()
    cache.release_request("a", wait=False)
    # no device-wide synchronisation: the host slot stays owned by the retirement event
    assert cache.storage.retired and not cache.storage.free_host
    with pytest.raises(CapacityError):
        cache.reserve("a", 4, 1)
    cache.collect(wait=True)
    cache.reserve("a", 4, 1)
    assert cache.storage.requests["a"].generation > old_generation
    new, _ = write(cache, "a", 4)
    with pytest.raises(RuntimeError, match="generation"):
        cache.allocator.validate(*handle)
    torch.testing.assert_close(observed, old)
    torch.testing.assert_close(cache.storage.host_kv("a", 0)[0], new.cpu())
    cache.assert_invariants()


def test_cancellation_reclaims_only_cancelled_request():
    model = MiniModel(
        ModelConfig(hidden_size=16, intermediate_size=32, num_hidden_layers=1, num_attention_heads=4,
                    num_key_value_heads=1)
    ).eval()
    cache = small(gpu_pages=1)
    engine = Engine(model, cache)
    engine.add_request("a", [1] * 5, 5)
    engine.add_request("b", [2] * 7, 4)
    engine.add_request("c", [3] * 9, 4)
    engine.cancel("b")
    engine.step()
    engine.cancel("a")
    engine.run()
    assert engine.requests["a"].cancelled and engine.requests["b"].cancelled
    assert len(engine.requests["c"].generated) == 4
    assert not cache.storage.requests and not cache.storage.retired
    cache.assert_invariants()


# ------------------------------------------------------- test_selection.py
@pytest.mark.parametrize("budget", [1, 3])
def test_exact_tokens_head_masks_and_empty_windows(device, budget):
    torch.manual_seed(91)
    cache = make_paged(PagedConfig(gpu_pages=budget, host_pages=16, page_size=4, kv_heads=2, head_dim=8,
                                   device=device))
    cache.reserve("r", 19, 1)
    k, v = [torch.randn(19, 2, 8, device=device) for _ in range(2)]
    q = torch.randn(4, 8, device=device)
    cache.write("r", 0, k, v)
    # head 0 reads token 0 once (duplicates and -1 dropped); some windows are empty for some heads
    selection = Selection.from_tokens([[0, 0, -1], [18], [5, 6], [12, 18]], 19, 4, 4)
    expected = torch.from_numpy(oracle.selection_oracle(q.cpu(), k.cpu(), v.cpu(), selection.positions)).to(device)
    got = paged_attention(q, cache, "r", 0, selection=selection)
    torch.testing.assert_close(got, expected.to(got.dtype), rtol=2e-5, atol=2e-6)
    cache.assert_invariants()


# ------------------------------------------------------- CLI bench (page layout)
def _bench(device, ops=None):
    from mini_hisparse_amd.cli import build_parser, run

    args = build_parser().parse_args(["bench", "--device", device, "--tokens", "200", "--steps", "3",
                                      "--requests", "2", "--selected-pages", "5", "--gpu-pages", "4"])
    return run(args, ops=ops)


def test_layout_bench_on_cpu():
    """The CLI bench (experiments/benchmark.py): three arrangements, checked after timing."""
    from tests.cpu_ops import CpuOracleOps

    report = _bench("cpu", CpuOracleOps())
    modes = [r["mode"] for r in report["results"]]
    assert modes == ["resident", "pressured_serial", "pressured_overlap"]
    resident, serial, overlap = report["results"]
    assert "misses" not in resident["stats"] and serial["stats"]["misses"] > 0
    assert overlap["stats"]["prefetch_windows"] > 0 and "prefetch_windows" not in serial["stats"]
    assert max(r["max_abs_error"] for r in report["results"]) < 1e-5


@pytest.mark.gpu
def test_layout_bench_on_gpu(gpu):
    report = _bench(gpu)
    assert report["workload"]["gpu"]
    assert [r["mode"] for r in report["results"]] == ["resident", "pressured_serial", "pressured_overlap"]
    assert max(r["max_abs_error"] for r in report["results"]) < 3e-5


@pytest.mark.parametrize("policy", ["fair_lru", "legacy"])
def test_layout_bench_counters_match_the_reference(policy):
    """The CLI bench at its default settings (1024 tokens, 20 steps, 3 requests, 8 pages,
    8 slots): every cache counter of every arrangement equals the reference's
    (tests/golden/layout_bench_counters.json, reference CPU path)."""
    import json
    import os

    from mini_hisparse_amd.cli import build_parser, run
    from tests.cpu_ops import CpuOracleOps

    with open(os.path.join(os.path.dirname(__file__), "golden", "layout_bench_counters.json")) as f:
        case = next(c for c in json.load(f)["cases"] if c["eviction_policy"] == policy)
    torch.set_num_threads(1)
    args = build_parser().parse_args(["bench", "--device", "cpu", "--eviction-policy", policy])
    report = run(args, ops=CpuOracleOps())
    for got, want in zip(report["results"], case["results"]):
        assert got["mode"] == want["mode"]
        assert got["stats"] == want["stats"]
        assert got["budget_pages"] == want["budget_pages"]
