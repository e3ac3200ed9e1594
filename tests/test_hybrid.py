"""The hybrid row cache end to end: scenarios whose known answers come from the
reference's hybrid tests (mini-hisparse tests/test_hybrid.py) -- row statistics,
protection of late hits, hot-block fragmentation, admission, leases, graph capture
and the engine -- checked on the CPU (oracle kernels) and on the GPU (HIP).

Every attention is compared with dense attention over its selected tokens."""

import pytest
import torch

import oracle
from mini_hisparse_amd.config import CacheConfig, CapacityError
from mini_hisparse_amd.engine import Engine
from mini_hisparse_amd.hybrid import HotConfig
from mini_hisparse_amd.model import MiniModel, ModelConfig
from mini_hisparse_amd.row_index import LogicalTopK
from mini_hisparse_amd.selection import Selection
from tests.cache_harness import F32, LOW, Harness
from tests.conftest import gpu_available
from tests.cpu_ops import make_cache


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    if request.param.startswith("cuda") and not gpu_available():
        pytest.skip("no ROCm GPU")
    torch.set_num_threads(1)
    return request.param


def cuda_only():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    return "cuda:0"


# ------------------------------------------------------------------ row statistics
ROW_CASES = {
    # name: (gpu pages, tokens written, selections in order, expected (resident, hot, miss))
    "two_reads_of_four_rows": (3, 32, [[0, 7, 17, 31]] * 2, (2, 3, 3)),
    "all_resident": (8, 20, [[1, 7, 17, 19]], (4, 0, 0)),
}


@pytest.mark.parametrize("case", sorted(ROW_CASES))
def test_row_statistics_known_answers(device, case):
    pages, tokens, selections, (res, hot, miss) = ROW_CASES[case]
    h = Harness.hybrid(device, gpu_pages=pages)
    h.cache.reserve("a", 40, 1)
    h.write("a", tokens)
    pool = h.cache.pool.data_ptr()
    for positions in selections:
        h.attend("a", positions)
    stats = h.row_stats()
    assert (stats["resident_hits"], stats["hot_hits"], stats["misses"]) == (res, hot, miss)
    assert stats["h2d_bytes"] == 64 * miss  # a row is 2 planes x 8 float32: 192 bytes for three misses
    assert h.cache.pool.data_ptr() == pool == h.cache.allocator.storage.data_ptr()
    if case == "all_resident":
        assert not h.cache.tables["a", 0].blocks  # no hot region was needed
    h.cache.assert_invariants()


def test_hits_of_the_same_selection_are_protected_from_replacement(device):
    """Three selections over four hot rows; rows hit again must survive the misses of
    the same selection, and duplicates / -1 read each token once: 5 misses in all."""
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    h.write("a", 32)
    for positions in ([0, 4, 8, 12], [16, 4, 8, 12], [4, 4, -1, 12]):
        h.attend("a", positions)
    assert h.row_stats()["misses"] == 5
    first_row_tag = h.page("a", 0).host_slot * 4
    assert first_row_tag not in h.cache.tables["a", 0].tags.tolist()  # the LRU row went first
    h.cache.assert_invariants()


def test_per_head_selections_over_fragmented_hot_blocks(device):
    """Interleaved writes of two requests fragment the slab; request a's hot region is
    then blocks [7, 0], and per-head token selections read through it."""
    config = CacheConfig(gpu_pages=8, host_pages=64, page_size=3, kv_heads=2, head_dim=8, device=device)
    h = Harness(make_cache(config, HotConfig(6, 6, transition_watermark=0)))
    h.cache.reserve("a", 40, 1)
    h.cache.reserve("b", 40, 1)
    for _ in range(3):
        h.write("a", 3)
        h.write("b", 3)
    h.write("b", 3)
    h.cache.storage.synchronize()
    h.cache.transition_to_host("a", 0)
    assert h.cache.tables["a", 0].blocks == [7, 0]
    h.write("a", 18)
    q = h.query(4)
    selection = Selection.from_tokens([[0, 7], [2], [7, 11], [19, 0]], 27, 3, 4)
    out = h.cache.attention(q, "a", 0, selection=selection)
    k, v = h.cache.storage.host_kv("a", 0)
    expected = oracle.selection_oracle(q.cpu(), k, v, selection.positions)
    torch.testing.assert_close(out.double().cpu(), torch.from_numpy(expected), **F32)
    h.cache.assert_invariants()


# ---------------------------------------------------------------------- admission
def test_admission_and_oversized_selections_change_nothing(device):
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    index_before = h.cache.index_bytes
    with pytest.raises(CapacityError, match="credits"):
        h.cache.reserve("b", 40, 1)
    assert "b" not in h.cache.storage.requests and h.cache.index_bytes == index_before
    h.write("a", 32)
    tags = h.cache.tables["a", 0].tags.clone()
    five = LogicalTopK(torch.tensor([0, 1, 2, 3, 4], dtype=torch.int32, device=device))
    with pytest.raises(ValueError, match="max_union_rows"):
        h.cache.resolve("a", 0, five)
    assert torch.equal(tags, h.cache.tables["a", 0].tags)
    with pytest.raises(ValueError):
        HotConfig(8, 4)  # the hot region must cover the union bound
    h.cache.assert_invariants()


@pytest.mark.parametrize("slack", [-1, 0])
def test_index_budget_counts_tables_exactly(device, slack):
    needed = Harness.hybrid(device).cache.index_reservation_bytes(40, 1)
    h = Harness.hybrid(device, index_budget_bytes=needed + slack)
    if slack < 0:
        with pytest.raises(CapacityError, match="index budget"):
            h.cache.reserve("a", 40, 1)
        assert not h.cache.storage.requests and not h.cache.tables
        return
    h.cache.reserve("a", 40, 1)
    assert h.cache.index_bytes == needed
    h.cache.release_request("a")
    assert h.cache.index_bytes == 0


# ------------------------------------------------------------------------ leases
def test_row_lease_excludes_writes_and_release_and_tails_stay(device):
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    h.write("a", 32)
    selected = LogicalTopK(torch.tensor([0, 4, 8, 31], dtype=torch.int32, device=device))
    lease = h.cache.resolve("a", 0, selected)
    lease.wait()
    with pytest.raises(RuntimeError, match="already leased"):
        h.cache.resolve("a", 0, LogicalTopK(torch.tensor([1], dtype=torch.int32, device=device)))
    with pytest.raises(RuntimeError, match="active row"):
        h.cache.release_request("a")
    with pytest.raises(RuntimeError, match="append"):
        h.write("a", 1)
    lease.release()
    h.write("a", 1)  # token 32 opens page 8
    assert [h.resident("a", p) for p in (6, 7, 8)] == [False, True, True]
    h.cache.assert_invariants()
    h.cache.release_request("a")
    with pytest.raises(RuntimeError, match="released"):
        lease.wait()


def test_row_lease_notices_a_block_rebound_under_it(device):
    """A row lease holds its blocks' owners and generations: a block released and bound
    again to the same owner (a new generation) fails the lease's next check."""
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    h.write("a", 32)
    h.cache.transition_to_host("a", 0)
    lease = h.cache.resolve("a", 0, LogicalTopK(torch.tensor([0, 4, 31], dtype=torch.int32, device=device)))
    lease.wait()
    table = h.cache.allocator
    block = int(lease.handles[0][0])
    owner = table.owner_key(block)
    table.release(block, None)
    with pytest.raises(RuntimeError, match="stale device-slot"):
        lease.wait()
    table.bind(block, owner)
    with pytest.raises(RuntimeError, match="stale device-slot"):
        lease.release()


def test_invalid_or_padding_only_selection_reads_nothing(device):
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    h.write("a", 32)
    out = h.attend("a", [-1, -2, 100, 32])
    assert torch.count_nonzero(out) == 0
    assert h.row_stats()["misses"] == 0


def test_random_appends_and_row_replacement_over_two_requests(device):
    torch.manual_seed(17)
    h = Harness.hybrid(device, gpu_pages=12, host_pages=256, seed=17)
    for name in ("a", "b"):
        h.cache.reserve(name, 64, 2)
        for layer in range(2):
            h.write(name, 19, layer)
    rng = torch.Generator().manual_seed(18)
    for step in range(32):
        name, layer = "ab"[step % 2], (step // 2) % 2
        h.write(name, 1, layer)
        length = len(h.kv(name, layer)[0])
        selected = torch.randperm(length - 1, generator=rng)[:3].tolist() + [length - 1]
        h.attend(name, selected, layer)
        h.cache.assert_invariants()
    for name in ("a", "b"):
        h.cache.release_request(name)
    h.cache.assert_invariants()


# ----------------------------------------------------------------------------- engine
def test_engine_waits_for_hot_credits_and_prefills_once(device):
    torch.manual_seed(9)
    config = ModelConfig(hidden_size=16, intermediate_size=32, num_hidden_layers=2, num_attention_heads=2,
                         num_key_value_heads=1, vocab_size=32)
    model = MiniModel(config).eval().to(device)
    cache = make_cache(CacheConfig(gpu_pages=8, host_pages=64, page_size=4, kv_heads=1, head_dim=8, device=device),
                       HotConfig(8, 8))
    engine = Engine(model, cache, top_k=2)
    for name in "ab":
        engine.add_request(name, list(range(1, 22)), 5)
    engine.step()
    assert len(engine.waiting) == 1  # the second request waits for hot-region credits
    outputs = engine.run()
    assert all(len(tokens) == 5 for tokens in outputs.values())
    assert all((r.prefill_count, r.decode_count) == (1, 4) for r in engine.requests.values())
    assert not cache.storage.requests and not cache.tables and not any(cache.owners)
    cache.assert_invariants()


# -------------------------------------------------------------------------- GPU only
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_rows_on_a_seven_row_page(dtype):
    h = Harness.hybrid(cuda_only(), dtype=dtype, page_size=7, head_dim=24, kv_heads=2)
    h.cache.reserve("a", 100, 1)
    h.write("a", 80)
    h.attend("a", [0, 13, 39, 79], heads=6, tol=LOW)


@pytest.mark.gpu
def test_resolver_replays_from_a_captured_graph():
    from mini_hisparse_amd.row_index import resolve_rows

    device = cuda_only()
    h = Harness.hybrid(device)
    h.cache.reserve("a", 40, 1)
    h.write("a", 32)
    t = h.cache.tables["a", 0]
    logical = LogicalTopK(torch.tensor([0, 4, 8, 31], dtype=torch.int32, device=device))
    run = lambda: resolve_rows(logical, t.source, t.resident, t.hot, t.tags, t.lru, 32, 4)  # noqa: E731
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    logical.positions.copy_(torch.tensor([1, 5, 9, 31], dtype=torch.int32, device=device))
    graph.replay()
    assert captured.counts.tolist() == [1, 0, 3]


@pytest.mark.gpu
def test_released_request_keeps_its_bytes_until_readers_finish():
    device = cuda_only()
    h = Harness.hybrid(device)
    h.cache.reserve("same", 40, 1)
    k, _ = h.write("same", 32)
    with h.cache.resolve("same", 0, LogicalTopK(torch.tensor([0, 4, 8, 31], dtype=torch.int32,
                                                             device=device))) as lease:
        torch.cuda._sleep(2_000_000)
        row = lease.plan.physical_rows[0]
        read = h.cache.pool[row // 4, 0, row % 4].clone()
    old_slots = {p.host_slot for p in h.cache.storage.pages.values()}
    h.cache.release_request("same", wait=False)
    h.cache.reserve("same", 40, 1)
    h.history.clear()
    h.write("same", 32)
    if h.cache.storage.retired:  # host slots of a retiring request are not reused
        assert old_slots.isdisjoint({p.host_slot for p in h.cache.storage.pages.values()})
    torch.testing.assert_close(read, k[0])
    h.cache.release_request("same")
    h.cache.assert_invariants()


# ------------------------------------------------------------------ no CPU fallback
def test_a_cache_off_rocm_needs_explicit_ops():
    """The product has no CPU kernels: a cache on the CPU without an ops object fails at
    construction instead of falling back to anything."""
    from mini_hisparse_amd.hybrid import HybridKVCache
    from mini_hisparse_amd.paged import PagedKVCache

    config = CacheConfig(gpu_pages=4, host_pages=4, page_size=4, kv_heads=1, head_dim=8, device="cpu",
                         dtype=torch.float32)
    with pytest.raises(ValueError, match="ROCm"):
        HybridKVCache(config, HotConfig(max_union_rows=8))
    with pytest.raises(ValueError, match="ROCm"):
        PagedKVCache(config)


@pytest.mark.parametrize("backend", ["torch", "triton", "cpu"])
def test_row_attention_rejects_the_reference_backends(backend):
    """The reference's torch and Triton attention paths do not exist here (attention.py:7-9)."""
    from mini_hisparse_amd.attention import row_attention

    config = CacheConfig(gpu_pages=4, host_pages=4, page_size=4, kv_heads=1, head_dim=8, device="cpu",
                         dtype=torch.float32)
    cache = make_cache(config, HotConfig(max_union_rows=8))
    topk = LogicalTopK(torch.tensor([0], dtype=torch.int32))
    with pytest.raises(ValueError, match="invalid attention backend"):
        row_attention(torch.zeros(2, 8), cache, "r", 0, topk, backend=backend)


def test_product_refuses_a_non_rocm_cache_without_explicit_ops():
    """No CPU fallback in the product: a cache on the CPU needs an explicit ops backend
    (the tests' oracle backend), and the attention takes no backend but the HIP one."""
    from mini_hisparse_amd.attention import row_attention
    from mini_hisparse_amd.hybrid import HybridKVCache

    cfg = CacheConfig(gpu_pages=8, host_pages=8, page_size=4, kv_heads=1, head_dim=8, device="cpu",
                      dtype=torch.float32)
    with pytest.raises(ValueError, match="ROCm"):
        HybridKVCache(cfg, HotConfig(max_union_rows=4))
    for backend in ("torch", "triton", "cpu"):
        with pytest.raises(ValueError, match="invalid attention backend"):
            row_attention(torch.zeros(1, 8), None, 0, 0, None, backend=backend)
