"""The optional page layout (``PagedKVCache`` + ``paged_attention``): whole-page leases
read in bounded windows.  Scenarios and known answers follow the reference's page
layout tests (tests/test_cache.py, tests/test_resources.py and the window case of
tests/test_selection.py of mini-hisparse); on the CPU the window kernel is the
oracle's, on the GPU ``hs_attend_window``."""

import pytest
import torch

import oracle
from mini_hisparse_amd.config import CapacityError
from mini_hisparse_amd.engine import Engine
from mini_hisparse_amd.model import MiniModel, ModelConfig
from mini_hisparse_amd.paged import PagedConfig, paged_attention
from mini_hisparse_amd.selection import Selection, select_pages
from mini_hisparse_amd.storage import Location
from tests.cache_harness import F32, Harness
from tests.conftest import gpu_available


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    if request.param.startswith("cuda") and not gpu_available():
        pytest.skip("no ROCm GPU")
    torch.set_num_threads(1)
    return request.param


def narrow(**config):
    """One KV head of 4 dims, three slots, on the CPU (the resource tests' shape)."""
    values = dict(gpu_pages=3, host_pages=32, page_size=4, kv_heads=1, head_dim=4, device="cpu")
    values.update(config)
    return Harness.paged(**values)


def check(h, out, query, request, tokens, layer=0, tol=F32):
    torch.testing.assert_close(out.double().cpu(), h.expected(query, request, tokens, layer), **tol)


def all_tokens(h, request, layer=0):
    return list(range(len(h.kv(request, layer)[0])))


def test_config_is_validated():
    with pytest.raises(ValueError, match="chunk_pages"):
        PagedConfig(chunk_pages=0, device="cpu")
    with pytest.raises(ValueError, match="eviction policy"):
        PagedConfig(eviction_policy="mru", device="cpu")


# ---------------------------------------------------------- windows over partial residency
@pytest.mark.parametrize("budget,overlap", [(1, False), (1, True), (2, False), (2, True), (5, False), (5, True)])
def test_windows_read_every_selected_page_once(device, budget, overlap):
    """Reordered, duplicated page lists read each page's tokens once, with the decode
    appends mirrored to the host pool, whatever the slot budget."""
    h = Harness.paged(device, gpu_pages=budget, overlap=overlap, seed=17)
    h.cache.reserve("a", 35, 1)
    h.write("a", 19)
    pool = h.cache.pool.data_ptr()
    for _ in range(10):
        h.write("a", 1)
        length = len(h.kv("a")[0])
        pages = [0, (length - 1) // 4, 1, 0]
        tokens = [t for p in dict.fromkeys(pages) for t in range(4 * p, min(4 * p + 4, length))]
        q = h.query(4)
        check(h, paged_attention(q, h.cache, "a", 0, pages), q, "a", tokens)
        h.cache.assert_invariants()
    host_k, host_v = h.cache.storage.host_kv("a", 0)
    torch.testing.assert_close(host_k, h.kv("a")[0].cpu())
    torch.testing.assert_close(host_v, h.kv("a")[1].cpu())
    stats = h.cache.storage.stats
    assert h.cache.pool.data_ptr() == pool and stats["peak_device_pages"] <= budget and stats["evictions"] > 0
    assert budget >= 3 or stats["misses"] > 0


def test_resident_pages_are_read_without_copies(device):
    h = Harness.paged(device, gpu_pages=5)
    h.cache.reserve("a", 16, 1)
    h.write("a", 13)
    paged_attention(h.query(4), h.cache, "a", 0)
    stats = h.cache.storage.stats
    assert stats["misses"] == stats["h2d_bytes"] == 0 and stats["resident_hits"] == 4


def test_loaded_page_is_reused_then_one_slot_still_reads_everything(device):
    h = Harness.paged(device, gpu_pages=5)
    h.cache.reserve("a", 28, 1)
    h.write("a", 28)
    q = h.query(4)
    paged_attention(q, h.cache, "a", 0, [0])
    assert h.page("a", 0).location == Location.HOT
    misses = h.cache.storage.stats["misses"]
    paged_attention(q, h.cache, "a", 0, [0])
    assert h.cache.storage.stats["misses"] == misses  # no reload
    h.cache.set_budget(1)
    check(h, paged_attention(q, h.cache, "a", 0), q, "a", all_tokens(h, "a"))
    h.cache.set_budget(5)
    h.cache.assert_invariants()


@pytest.mark.parametrize("budget", [1, 3])
def test_per_head_token_masks_and_heads_with_empty_windows(device, budget):
    h = Harness.paged(device, gpu_pages=budget, host_pages=16, seed=91)
    h.cache.reserve("r", 19, 1)
    h.write("r", 19)
    q = h.query(4)
    selection = Selection.from_tokens([[0, 0, -1], [18], [5, 6], [12, 18]], 19, 4, 4)
    out = paged_attention(q, h.cache, "r", 0, selection=selection)
    k, v = h.kv("r")
    expected = oracle.selection_oracle(q.cpu(), k.cpu(), v.cpu(), selection.positions)
    torch.testing.assert_close(out.double().cpu(), torch.from_numpy(expected), **F32)
    h.cache.assert_invariants()


def test_quest_over_the_layouts_bounds_picks_the_reference_pages():
    """Known answer: Quest takes pages [0, 2], where mean-K scoring would take page 1;
    the bounds are the exact extrema of each page, also across two writes."""
    h = Harness.paged("cpu", gpu_pages=1, host_pages=4, page_size=2, kv_heads=1, head_dim=2)
    h.cache.reserve("r", 8, 1)
    k = torch.tensor([[[10.0, 0.0]], [[-10.0, 0.0]], [[1.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]])
    h.cache.write("r", 0, k[:4], k[:4])
    h.cache.write("r", 0, k[4:], k[4:])
    request = h.cache.storage.requests["r"]
    # the cache's kernel backend: the oracle's on the CPU (quest_selection itself is HIP-only)
    selection = h.cache.ops.quest_selection(torch.tensor([[1.0, 0.0]]), request.minimum[0], request.maximum[0], 5,
                                            2, 2, keep_sink=False)
    assert selection.pages == [0, 2]
    torch.testing.assert_close(request.minimum[0, 0], k[:2].amin(0))
    torch.testing.assert_close(request.maximum[0, 0], k[:2].amax(0))


def test_mean_selector_keeps_the_tail_and_rejects_bad_pages(device):
    h = Harness.paged(device)
    h.cache.reserve("a", 20, 1)
    h.write("a", 20)
    q = h.query(4)
    assert select_pages(h.cache, "a", 0, q, 1) == [4]
    chosen = select_pages(h.cache, "a", 0, q, 3)
    assert 0 in chosen and 4 in chosen and len(chosen) == 3
    for bad in ([], [-1], [5]):
        with pytest.raises(ValueError):
            paged_attention(q, h.cache, "a", 0, bad)
    h.cache.assert_invariants()


# --------------------------------------------------------------------------- victim policy
@pytest.mark.parametrize("policy,kept", [("legacy", False), ("lru", True), ("fair_lru", True)])
def test_which_page_a_new_copy_replaces(policy, kept):
    """Two slots: after leasing page 0 (loaded) then page 1, legacy drops the loaded copy
    first, the LRU policies the older written page."""
    h = narrow(gpu_pages=2, eviction_policy=policy)
    h.cache.reserve("a", 12, 1)
    h.write("a", 12)
    for page in (0, 1):
        with h.cache.acquire([("a", 0, page)]):
            pass
    assert h.resident("a", 0) == kept
    h.cache.assert_invariants()


def test_fair_share_is_soft_and_idle_slots_are_borrowed():
    h = narrow(gpu_pages=4)
    h.cache.reserve("a", 24, 1)
    h.cache.reserve("b", 8, 1)
    h.write("b", 4)  # the oldest page belongs to the request under its share
    h.write("a", 12)
    h.write("b", 4)
    assert h.cache.allocator.occupancy == {"a": 2, "b": 2}
    assert h.resident("b", 0)
    h.cache.release_request("b")
    h.write("a", 12)
    assert h.cache.allocator.occupancy["a"] == 4  # alone, a borrows every slot
    h.cache.assert_invariants()


def test_sink_protection_expires_when_it_is_no_longer_read():
    h = narrow(gpu_pages=2)
    h.cache.reserve("a", 12, 1)
    h.write("a", 12)
    q = h.query(2)
    paged_attention(q, h.cache, "a", 0, [0])
    for page in (1, 2, 1, 2):
        paged_attention(q, h.cache, "a", 0, [page])
    assert not h.resident("a", 0)
    h.cache.assert_invariants()


def test_lookahead_keeps_a_future_hit_and_windows_leave_room_for_other_leases():
    h = narrow()
    h.cache.reserve("a", 16, 1)
    h.write("a", 16)
    q = h.query(2)
    before = h.cache.storage.stats["attention_misses"]
    out = paged_attention(q, h.cache, "a", 0, [0, 1, 3])
    assert h.cache.storage.stats["attention_misses"] - before == 1
    check(h, out, q, "a", [*range(8), *range(12, 16)])
    h.cache.reserve("b", 4, 1)
    h.write("b", 4)
    with h.cache.acquire([("b", 0, 0)]):
        plan = h.cache.plan([("a", 0, i) for i in range(4)])
        assert plan.pinned_outside == 1 and plan.live_slot_limit <= 2
        check(h, paged_attention(q, h.cache, "a", 0), q, "a", all_tokens(h, "a"))
    h.cache.assert_invariants()


# --------------------------------------------------------------------- admission, budgets
def test_host_admission_is_atomic_and_ids_come_back(device):
    h = Harness.paged(device, host_pages=4)
    h.cache.reserve("a", 8, 2)
    with pytest.raises(CapacityError):
        h.cache.reserve("b", 1, 1)
    assert "b" not in h.cache.storage.requests
    h.cache.release_request("a")
    h.cache.reserve("a", 16, 1)
    h.cache.assert_invariants()


@pytest.mark.parametrize("budget", [960, 959])
def test_pages_materialize_lazily_and_the_index_budget_is_exact(budget):
    h = narrow(host_pages=20, index_budget_bytes=budget)
    if budget == 959:
        with pytest.raises(CapacityError, match="index budget"):
            h.cache.reserve("a", 40, 2)
        assert not h.cache.storage.requests and len(h.cache.storage.free_host) == 20
        return
    h.cache.reserve("a", 40, 2)
    store = h.cache.storage
    assert len(store.pages) == 0 and len(store.free_host) == 20 and store.available_host_credits == 0
    h.write("a", 1)
    assert len(store.pages) == 1 and store.requests["a"].host_credits == 19
    h.cache.assert_invariants()
    h.cache.release_request("a")
    assert len(store.free_host) == 20


def test_bfloat16_bounds_are_exact_and_charged_by_their_bytes():
    h = narrow(dtype=torch.bfloat16)
    h.cache.reserve("a", 12, 1)
    k = torch.randn(7, 1, 4).bfloat16()
    h.cache.write("a", 0, k, k)
    request = h.cache.storage.requests["a"]
    assert request.minimum.dtype == torch.bfloat16
    torch.testing.assert_close(request.minimum[0, 0], k[:4].amin(0))
    # 3 pages x 1 head x 4 dims x (4-byte mean + two 2-byte bounds)
    assert h.cache.index_bytes == h.cache.index_reservation_bytes(12, 1) == 3 * 1 * 4 * 8


def test_shrinking_over_a_lease_fails_whole_and_versions_follow_the_tail():
    h = narrow(gpu_pages=3)
    h.cache.reserve("a", 12, 1)
    h.write("a", 9)
    owner = h.cache.owners[2]
    with h.cache.acquire([owner]):
        with pytest.raises(CapacityError):
            h.cache.set_budget(1)
        assert h.cache.budget == 3
    h.cache.set_budget(1)
    h.write("a", 3)
    state = h.cache.storage.page_state(("a", 0, 2))
    assert state["sealed"] and state["content_version"] == 2 and state["host_committed_version"] == 2
    h.cache.assert_invariants()


# ----------------------------------------------------------------------------- leases
def test_hits_are_pinned_before_a_miss_is_placed(device):
    h = Harness.paged(device, gpu_pages=2)
    h.cache.reserve("a", 12, 1)
    h.write("a", 12)  # page 0 is on the host only; pages 1 and 2 are resident
    slot = h.page("a", 1).slot
    lease = h.cache.acquire([("a", 0, 0), ("a", 0, 1)])
    assert h.page("a", 1).slot == slot
    owners = list(h.cache.owners)
    with pytest.raises(CapacityError):
        h.cache.acquire([("a", 0, 2)])
    assert h.cache.owners == owners  # nothing changed
    with pytest.raises(RuntimeError):
        h.cache.release_request("a")
    lease.wait()
    lease.release()
    h.cache.release_request("a")
    h.cache.assert_invariants()
    assert len(h.cache.storage.free_host) == h.cache.config.host_pages


def test_an_attention_shares_pages_another_lease_holds():
    h = narrow(gpu_pages=2)
    h.cache.reserve("a", 8, 1)
    h.write("a", 8)
    q = h.query(2)
    with h.cache.acquire([("a", 0, 0), ("a", 0, 1)]):
        check(h, paged_attention(q, h.cache, "a", 0), q, "a", all_tokens(h, "a"))
    h.cache.assert_invariants()


def test_random_requests_layers_and_budgets(device):
    h = Harness.paged(device, gpu_pages=3, host_pages=128, seed=19)
    names = "abc"
    for name in names:
        h.cache.reserve(name, 40, 2)
        for layer in range(2):
            h.write(name, 13, layer)
    for step in range(30):
        name, layer = names[step % 3], (step // 3) % 2
        h.write(name, 1, layer)
        q = h.query(4)
        h.cache.set_budget(1 + step % 3)
        check(h, paged_attention(q, h.cache, name, layer), q, name, all_tokens(h, name, layer), layer)
        h.cache.assert_invariants()
    for name in "bac":
        h.cache.release_request(name)
        h.cache.assert_invariants()


# ------------------------------------------------------------------------------ engine
def _tiny_model(device, **config):
    values = dict(hidden_size=16, intermediate_size=32, num_hidden_layers=1, num_attention_heads=2,
                  num_key_value_heads=1)
    values.update(config)
    return MiniModel(ModelConfig(**values)).eval().to(device)


@pytest.mark.parametrize("top_k", [None, 2])
def test_decode_through_two_slots_equals_decode_with_everything_resident(device, top_k):
    torch.manual_seed(31)
    model = _tiny_model(device, hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=4,
                        num_key_value_heads=2, vocab_size=64)
    prompts = {"a": list(range(1, 18)), "b": list(range(8, 30))}
    outputs = []
    for budget in (64, 2):
        h = Harness.paged(device, gpu_pages=budget, host_pages=64, chunk_pages=4)
        engine = Engine(model, h.cache, top_k=top_k)
        engine.add_request("a", prompts["a"], 8)
        engine.add_request("b", prompts["b"], 6)
        outputs.append(engine.run())
        assert all(r.prefill_count == 1 and r.decode_count == r.max_new_tokens - 1 for r in engine.requests.values())
        assert not h.cache.storage.requests and not any(h.cache.owners)
        h.cache.assert_invariants()
        assert budget > 2 or h.cache.storage.stats["misses"] > 0
    assert outputs[0] == outputs[1]
    if top_k is None:  # full attention: every token is the prefill's greedy next token
        for name, prompt in prompts.items():
            history = list(prompt)
            for token in outputs[0][name]:
                assert model.prefill(history).argmax().item() == token
                history.append(token)


def test_host_backpressure_admits_waiters_in_turn():
    torch.manual_seed(4)
    model = _tiny_model("cpu")
    h = narrow(gpu_pages=1, host_pages=4, head_dim=8)
    engine = Engine(model, h.cache)
    for i in range(3):
        engine.add_request(str(i), [1] * 10, 5)
    engine.step()
    assert len(engine.waiting) == 2
    engine.run()
    assert all(len(r.generated) == 5 and r.prefill_count == 1 for r in engine.requests.values())


def test_cancelling_frees_only_the_cancelled_request():
    model = _tiny_model("cpu", num_attention_heads=4)
    h = narrow(gpu_pages=1)
    engine = Engine(model, h.cache)
    engine.add_request("a", [1] * 5, 5)
    engine.add_request("b", [2] * 7, 4)
    engine.add_request("c", [3] * 9, 4)
    engine.cancel("b")
    engine.step()
    engine.cancel("a")
    engine.run()
    assert engine.requests["a"].cancelled and engine.requests["b"].cancelled
    assert len(engine.requests["c"].generated) == 4
    assert not h.cache.storage.requests and not h.cache.storage.retired
    h.cache.assert_invariants()


# ---------------------------------------------------------------------------- GPU only
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_window_kernel_in_low_precision_on_seven_row_pages(dtype):
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    h = Harness.paged("cuda:0", page_size=7, head_dim=24, dtype=dtype)
    h.cache.reserve("a", 33, 1)
    h.write("a", 33)
    q = h.query(6)
    check(h, paged_attention(q, h.cache, "a", 0), q, "a", all_tokens(h, "a"), tol=dict(atol=0.003, rtol=0.015))


@pytest.mark.gpu
def test_a_slow_reader_finishes_before_its_slot_is_refilled():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    h = Harness.paged("cuda:0", gpu_pages=1)
    h.cache.reserve("a", 8, 1)
    k, _ = h.write("a", 8)
    for _ in range(16):
        with h.cache.acquire([("a", 0, 0)]) as lease:
            torch.cuda._sleep(100000)
            read = h.cache.pool[lease.pages[0].slot, 0].clone()
        with h.cache.acquire([("a", 0, 1)]):
            pass
        torch.testing.assert_close(read, k[:4])
    h.cache.assert_invariants()


@pytest.mark.gpu
def test_retired_host_bytes_and_slot_generations_outlive_a_slow_reader():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    h = Harness.paged("cuda:0", gpu_pages=1, host_pages=1, kv_heads=1, head_dim=4)
    h.cache.reserve("a", 4, 1)
    generation = h.cache.storage.requests["a"].generation
    old, _ = h.write("a", 4)
    with h.cache.acquire([("a", 0, 0)]) as lease:
        handle = lease.handles[0]
        torch.cuda._sleep(100_000_000)
        read = h.cache.pool[0, 0].clone()
    h.cache.release_request("a", wait=False)
    # no device synchronisation: the host slot belongs to the retirement event
    assert h.cache.storage.retired and not h.cache.storage.free_host
    with pytest.raises(CapacityError):
        h.cache.reserve("a", 4, 1)
    h.cache.collect(wait=True)
    h.cache.reserve("a", 4, 1)
    assert h.cache.storage.requests["a"].generation > generation
    h.history.clear()
    new, _ = h.write("a", 4)
    with pytest.raises(RuntimeError, match="generation"):
        h.cache.allocator.validate(*handle)
    torch.testing.assert_close(read, old)
    torch.testing.assert_close(h.cache.storage.host_kv("a", 0)[0], new.cpu())
    h.cache.assert_invariants()
