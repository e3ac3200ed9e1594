"""The reference Engine API over the layer-major batched decode (LayerMajorEngine).

* The CLI ``demo`` goldens recorded from the reference (BASELINE configs[0] and its
  65-token sibling) come out of the batched engine token for token, with the
  reference's prefill/decode counts and the same number of selected rows.
* Requests are admitted one per step between decode turns, finish on their last
  token or the end-of-sequence token, are cancelled mid-run, and their slots and
  blocks are taken by later admissions; every layer of every decode turn equals the
  oracle (Quest pages over the exact bounds of the history read back from the host
  pool, sparse attention over the selected tokens).
"""

import json
import os
from math import ceil

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "demo_outputs.json")
with open(GOLDEN) as f:
    CASES = json.load(f)["cases"]


@pytest.mark.parametrize("case", CASES, ids=[" ".join(c["argv"][3:7]) for c in CASES])
def test_layer_major_engine_reproduces_the_demo_goldens(gpu, case):
    """The CLI demo's model, prompts and cache configuration (cli.py, with the CLI's own
    defaults), decoded by the layer-major engine through the Engine API: the reference's
    tokens, schedule counts and number of selected rows.  (Where requests decode side
    by side, a step's policy writes all precede its layer-major reads, so a row another
    request's write took away is loaded from host memory instead of read in place: the
    split between resident, hot and missed rows may differ, their total may not.)"""
    from mini_hisparse_amd.cli import _model_and_prompts, build_parser, union_rows_bound
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.hybrid import HotConfig
    from mini_hisparse_amd.serving import LayerMajorCache, LayerMajorEngine

    argv = list(case["argv"])
    argv[argv.index("--device") + 1] = gpu
    args = build_parser().parse_args(argv)
    print(f"[case] demo through the layer-major engine: {' '.join(argv)}", flush=True)
    torch.manual_seed(42)
    model, prompts, _ = _model_and_prompts(args, torch.float32, None)
    cfg = model.config
    longest = max(map(len, prompts))
    bound = union_rows_bound(longest, args.max_new_tokens, args.top_k, cfg.num_attention_heads, args.page_size)
    hot = HotConfig(bound, args.hot_rows, resident_window_pages=args.resident_window_pages,
                    transition_watermark=args.hot_watermark)
    blocks = args.gpu_pages or hot.admission_blocks(args.page_size, cfg.num_hidden_layers)
    config = CacheConfig(gpu_pages=blocks, host_pages=args.host_pages, page_size=args.page_size,
                         kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, device=gpu, dtype=torch.float32,
                         index_budget_bytes=args.index_budget_mib << 20)
    cache = LayerMajorCache(config, hot, cfg.num_hidden_layers, max_requests=len(prompts),
                            max_tokens=longest + args.max_new_tokens)
    engine = LayerMajorEngine(model, cache, args.top_k)
    for i, prompt in enumerate(prompts):
        engine.add_request(str(i), prompt, args.max_new_tokens)
    outputs = engine.run()
    assert outputs == case["outputs"]
    assert {name: {"prefill_count": r.prefill_count, "decode_count": r.decode_count,
                   "generated_tokens": len(r.generated)} for name, r in engine.requests.items()} == case["requests"]
    rows = cache.snapshot()["row_stats"]
    expected = case["row_stats"]
    assert rows["resident_hits"] + rows["hot_hits"] + rows["misses"] == (
        expected["resident_hits"] + expected["hot_hits"] + expected["misses"])
    if len(prompts) == 1:  # one request: the reference's order exactly, every row in the same place
        assert rows == expected
    assert cache.free_slots == list(range(len(prompts)))  # every request released its slot
    assert cache.plan.available() == blocks  # ... and its blocks


def tiny_model(gpu):
    from mini_hisparse_amd.batched_engine import DecodeWorkload, random_model

    wl = DecodeWorkload(name="tiny", layers=2, hidden=256, heads=8, kv_heads=2, head_dim=32, ffn=512, vocab=300,
                        batch=3, context=0, steps=0, top_pages=6, resident_fraction=0.0, hot_rows=0)
    return wl, random_model(wl, gpu, seed=1)


def test_admission_finish_and_cancel_mid_run_match_the_oracle(gpu):
    """Three slots, five requests of different lengths: one admission per step, a
    request cancelled while it decodes and one while it waits, finishes on the last
    token and on an end-of-sequence token; freed slots and blocks go to later
    admissions.  Every decode turn is checked layer by layer against the oracle."""
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.hybrid import HotConfig
    from mini_hisparse_amd.selection import union_bound
    from mini_hisparse_amd.serving import LayerMajorCache, LayerMajorEngine

    print("[case] layer-major engine: 3 slots, 5 requests, cancel and EOS mid-run", flush=True)
    wl, model = tiny_model(gpu)
    P, L, Hkv, D = 16, wl.layers, wl.kv_heads, wl.head_dim
    max_tokens = 24 * P
    bound = union_bound(max_tokens, P, wl.top_pages, wl.heads)
    hot = HotConfig(bound, 2 * bound, resident_window_pages=8)
    blocks = 3 * hot.admission_blocks(P, L) + 40
    config = CacheConfig(gpu_pages=blocks, host_pages=3 * L * 24, page_size=P, kv_heads=Hkv, head_dim=D,
                         device=gpu, dtype=torch.bfloat16)
    cache = LayerMajorCache(config, hot, L, max_requests=3, max_tokens=max_tokens)
    gen = torch.Generator().manual_seed(5)
    lengths = {"a": 9 * P + 3, "b": 5 * P, "c": 12 * P + 11, "d": 7 * P + 1, "e": 3 * P + 9}
    new_tokens = {"a": 6, "b": 9, "c": 5, "d": 7, "e": 4}
    prompts = {name: torch.randint(0, wl.vocab, (n,), generator=gen).tolist() for name, n in lengths.items()}
    eos = None
    engine = LayerMajorEngine(model, cache, wl.top_pages, eos_token_id=eos)
    for name in lengths:
        engine.add_request(name, prompts[name], new_tokens[name])
    state = cache.state
    B, C = state.batch, state.pages
    records = []

    def observe(layer, q, k, v, out):
        slots, dec = engine.batched.current_group
        records.append((layer, list(slots), q.clone(), out.clone(), dec.pages.clone(), dec.union_count.clone()))

    checked, step, slots_used = 0, 0, set()
    while engine.waiting or engine.running:
        records.clear()
        if step == 4:
            engine.cancel("b")  # decoding
        if step == 5:
            engine.cancel("e")  # waiting
        emitted = engine.step(observe)
        torch.cuda.synchronize()
        slots_used.update(cache.slot_of.values())
        for layer, slots, q, out, layer_pages, union_count in records:
            for i, b in enumerate(slots):
                length = state.lengths[b]
                count = ceil(length / P)
                kv = state.host[layer].view(B, C, 2, P, Hkv, D)[b, :count].float()
                keys = kv[:, 0].reshape(count * P, Hkv, D)[:length]
                vals = kv[:, 1].reshape(count * P, Hkv, D)[:length]
                lo = torch.stack([keys[p * P : (p + 1) * P].amin(0) for p in range(count)])
                hi = torch.stack([keys[p * P : (p + 1) * P].amax(0) for p in range(count)])
                torch.testing.assert_close(state.minimum[layer, b, :count].float().cpu(), lo, rtol=0, atol=0)
                torch.testing.assert_close(state.maximum[layer, b, :count].float().cpu(), hi, rtol=0, atol=0)
                pages = oracle.quest_pages(q[i].cpu(), lo, hi, length, P, wl.top_pages)
                np.testing.assert_array_equal(layer_pages[i, :, : pages.shape[1]].cpu().numpy(), pages)
                positions = pages_to_positions(pages, length, P)
                assert int(union_count[i]) == len(set().union(*map(set, positions)))
                expected = oracle.selection_oracle(q[i].cpu(), keys, vals, positions)
                got = out[i].float().cpu().double().numpy()
                assert np.all(np.abs(got - expected) <= 2e-2 + 1e-2 * np.abs(expected)), np.abs(got - expected).max()
                checked += 1
        # one token per running request, plus the prefill token of the request admitted
        # this step, which also takes its first decode turn (engine.py:110-128)
        names = [name for name, _ in emitted]
        repeated = {name for name in names if names.count(name) > 1}
        assert len(repeated) <= 1 and all(names.count(name) == 2 and names[0] == name for name in repeated)
        step += 1
    engine.batched.check_status()
    r = engine.requests
    assert r["b"].cancelled and r["e"].cancelled and r["e"].prefill_count == 0
    for name in ("a", "c", "d"):
        assert len(r[name].generated) == new_tokens[name] and r[name].finished and not r[name].cancelled
        assert r[name].prefill_count == 1 and r[name].decode_count == new_tokens[name] - 1
    assert slots_used == {0, 1, 2} and checked > 30
    assert cache.free_slots == [0, 1, 2] and cache.slot_of == {}
    assert cache.plan.available() == blocks  # every block returned
    assert cache.snapshot()["stats"]["retired_requests"] == 4


def test_end_of_sequence_finishes_a_request(gpu):
    """A request whose next token is the end-of-sequence token finishes there, releases
    its slot, and the next waiting prompt takes it."""
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.hybrid import HotConfig
    from mini_hisparse_amd.selection import union_bound
    from mini_hisparse_amd.serving import LayerMajorCache, LayerMajorEngine

    wl, model = tiny_model(gpu)
    P, L = 16, wl.layers
    bound = union_bound(16 * P, P, wl.top_pages, wl.heads)
    hot = HotConfig(bound, 2 * bound)
    config = CacheConfig(gpu_pages=hot.admission_blocks(P, L) + 20, host_pages=L * 16, page_size=P,
                         kv_heads=wl.kv_heads, head_dim=wl.head_dim, device=gpu, dtype=torch.bfloat16)
    prompt = torch.randint(0, wl.vocab, (5 * P + 2,), generator=torch.Generator().manual_seed(9)).tolist()
    # the greedy continuation without an end-of-sequence token
    free = LayerMajorEngine(model, LayerMajorCache(config, hot, L, 1, 16 * P), wl.top_pages)
    free.add_request("x", prompt, 6)
    tokens = free.run()["x"]
    eos = tokens[2]
    cache = LayerMajorCache(config, hot, L, 1, 16 * P)
    engine = LayerMajorEngine(model, cache, wl.top_pages, eos_token_id=eos)
    engine.add_request("x", prompt, 6)
    engine.add_request("y", prompt, 2)
    out = engine.run()
    first = tokens.index(eos)
    assert out["x"] == tokens[: first + 1]
    # the same prompt in the freed slot decodes the same way, up to its own limit
    assert out["y"] == tokens[: min(2, first + 1)]
    assert engine.requests["y"].prefill_count == 1 and cache.free_slots == [0]
