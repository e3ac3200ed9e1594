"""Layer-major batched engine: every layer of a decode step against the oracle.

For each step and layer, the engine's own query is re-scored by the oracle
over the Quest bounds of the full history read back from the host pool (which
holds the mirrored appended rows), and its attention output is compared with
the oracle's sparse attention over the selected tokens."""

from math import ceil

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions
from tests.conftest import gpu_available


def tiny(**overrides):
    """Small workload; the hot region holds twice the union bound (the reference's default
    hot_rows = 2U, cli.py:141-151)."""
    from mini_hisparse_amd.batched_engine import DecodeWorkload
    from mini_hisparse_amd.selection import union_bound

    values = dict(name="tiny", layers=2, hidden=256, heads=8, kv_heads=2, head_dim=32, ffn=512, vocab=300,
                  batch=3, context=40 * 16 - 1, steps=24, top_pages=6, resident_fraction=0.3)
    values.update(overrides)
    end = values["context"] + values["steps"]
    values.setdefault("hot_rows", 2 * union_bound(end, 16, values["top_pages"], values["heads"]))
    return DecodeWorkload(**values)


def _engine_layers_match_oracle(gpu, wl, transfer_stream=False, steps=3, built=None, **engine_options):
    """Run `steps` decode steps and check every layer of every request against the oracle:
    the state's bounds are the exact extrema of the history read back from the host pool,
    the Quest pages equal the oracle's over those bounds, and the attention output is the
    oracle's sparse attention over the selected tokens.  With request groups the observer
    sees one group at a time (``engine.current_group``: its requests and decoder)."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    print(f"[case] {wl.name}: L={wl.layers} hidden={wl.hidden} heads={wl.heads}/{wl.kv_heads} "
          f"D={wl.head_dim} ffn={wl.ffn} batch={wl.batch} context={wl.context} {engine_options}", flush=True)
    if built is None:
        model, state, tokens = random_model(wl, gpu, seed=1), build_state(wl, gpu, seed=2), None
    else:
        model, state, tokens = built
    engine = BatchedDecodeEngine(model, state, wl.top_pages, transfer_stream=transfer_stream, **engine_options)
    L, B, C, P = wl.layers, wl.batch, state.pages, wl.page_size
    Hkv, D = wl.kv_heads, wl.head_dim
    records = []
    if tokens is None:
        tokens = torch.arange(1, B + 1, device=gpu)
    unions = 0

    entry_total = torch.zeros(1, dtype=torch.int64, device=gpu)
    engine.set_entry_stats(entry_total)  # the union launches total their entry counts here
    entries = []

    def observe(l, q, k, v, out):
        rows, dec = engine.current_group if engine.groups else (range(B), engine.decoder(l))
        records.append((l, rows, q.clone(), out.clone(), dec.pages.clone(), dec.union_count.clone()))
        entries.append(dec.entry_counts.sum())

    for step in range(steps):
        records.clear()
        tokens = engine.step(tokens, observe)
        torch.cuda.synchronize()
        length = state.lengths[0]
        count = ceil(length / P)
        assert sorted((r[0], r[1].start) for r in records) == sorted(
            (l, g.start) for l in range(L) for g in ([range(B)] if not engine.groups else [r for r, _ in engine.groups]))
        for l, rows, q, out, layer_pages, union_count in records:
            for i, b in enumerate(rows):
                kv = state.host[l].view(B, C, 2, P, Hkv, D)[b, :count].float()  # [count, 2, P, Hkv, D]
                keys = kv[:, 0].reshape(count * P, Hkv, D)[:length]
                vals = kv[:, 1].reshape(count * P, Hkv, D)[:length]
                # bounds of the state = exact extrema of the history (append + mirror)
                lo = torch.stack([keys[p * P : (p + 1) * P].amin(0) for p in range(count)])
                hi = torch.stack([keys[p * P : (p + 1) * P].amax(0) for p in range(count)])
                torch.testing.assert_close(state.minimum[l, b, :count].float().cpu(), lo, rtol=0, atol=0)
                torch.testing.assert_close(state.maximum[l, b, :count].float().cpu(), hi, rtol=0, atol=0)
                pages = oracle.quest_pages(q[i].cpu(), lo, hi, length, P, wl.top_pages)
                np.testing.assert_array_equal(layer_pages[i, :, : pages.shape[1]].cpu().numpy(), pages)
                positions = pages_to_positions(pages, length, P)
                expected = oracle.selection_oracle(q[i].cpu(), keys, vals, positions)
                got = out[i].float().cpu().double().numpy()
                assert np.all(np.abs(got - expected) <= 2e-2 + 1e-2 * np.abs(expected)), np.abs(got - expected).max()
                unions += int(union_count[i])
    engine.check_status()  # no union or entry list was truncated
    assert int(entry_total.item()) == int(sum(int(x) for x in entries))
    engine.set_entry_stats(None)
    stats = state.row_stats.tolist()
    assert sum(stats) == unions  # every selected row was a resident hit, a hot hit or a miss
    return stats


@pytest.mark.gpu
@pytest.mark.parametrize(
    "overrides,transfer_stream",
    [
        ({}, False),
        ({}, True),
        ({"heads": 16, "kv_heads": 2, "head_dim": 64, "hidden": 1024}, False),
        # more requests than one launch of the scorer, union builder, resolver and gather
        # (16) or of the append (32) takes: each entry point runs them in chunks
        ({"batch": 34}, False),
    ],
)
def test_batched_engine_layers_match_oracle(gpu, overrides, transfer_stream):
    stats = _engine_layers_match_oracle(gpu, tiny(**overrides), transfer_stream)
    assert stats[2] > 0 and stats[0] > 0 and stats[1] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("groups,gather_workgroups", [(2, 0), (3, 24)])
def test_pipelined_request_groups_match_oracle(gpu, groups, gather_workgroups):
    """Request groups pipelined across layers (one group's gather on the transfer stream
    while the compute stream serves the others): every layer of every request still
    equals the oracle, with uneven groups (5 requests in 3 groups) included."""
    stats = _engine_layers_match_oracle(gpu, tiny(batch=5), request_groups=groups,
                                        group_gather_workgroups=gather_workgroups)
    assert stats[2] > 0 and stats[0] > 0 and stats[1] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("resident_fraction", [0.3, 0.0])
def test_prefill_writes_history_bounds_and_residents_then_decodes(gpu, resident_fraction):
    """The engine's prefill runs the model over random prompts and writes every layer's
    K/V with the batched write kernel: the host pool holds exactly the model's K/V, the
    bounds are the exact extrema of each page (bit for bit), resident pages hold their
    host rows, the first tokens are the model's own prefill tokens; decoding then matches
    the oracle layer by layer."""
    from mini_hisparse_amd.batched_engine import empty_state, random_model, random_prompts

    wl = tiny(resident_fraction=resident_fraction, context=9 * 16 + 5)
    model = random_model(wl, gpu, seed=1)
    state = empty_state(wl, gpu)
    prompts = random_prompts(wl, gpu, seed=3)
    written = {}
    firsts = state.prefill(model, prompts, wl.resident_fraction, seed=4,
                           observer=lambda l, b, k, v: written.__setitem__((l, b), (k.clone(), v.clone())))
    torch.cuda.synchronize()
    B, C, P, Hkv, D = wl.batch, state.pages, wl.page_size, wl.kv_heads, wl.head_dim
    length = wl.context
    count = ceil(length / P)
    assert state.lengths == [length] * B
    for b in range(B):
        assert int(firsts[b]) == int(model.prefill(prompts[b].tolist()).argmax())
        for l in range(wl.layers):
            k, v = written[l, b]
            host = state.host[l].view(B, C, 2, P, Hkv, D)[b, :count]
            keys = host[:, 0].reshape(count * P, Hkv, D)[:length]
            vals = host[:, 1].reshape(count * P, Hkv, D)[:length]
            assert torch.equal(keys, k.cpu()) and torch.equal(vals, v.cpu())
            lo = torch.stack([keys[p * P : (p + 1) * P].amin(0) for p in range(count)])
            hi = torch.stack([keys[p * P : (p + 1) * P].amax(0) for p in range(count)])
            assert torch.equal(state.minimum[l, b, :count].cpu(), lo)
            assert torch.equal(state.maximum[l, b, :count].cpu(), hi)
            resident = state.resident[l, b, :count].cpu()
            assert resident[count - 1] >= 0  # the tail page is resident
            for p in torch.nonzero(resident >= 0).flatten().tolist():
                rows = min(P, length - p * P)
                assert torch.equal(state.pool[int(resident[p]), :, :rows].cpu(), host[p, :, :rows])
    _engine_layers_match_oracle(gpu, wl, built=(model, state, firsts))


@pytest.mark.gpu
def test_policy_residency_places_prefill_and_decode_pages_like_the_plan(gpu):
    """Residency by the hybrid policy: the prefill places every page and hot region as
    the placement plan decides (checked against HybridKVCache in
    tests/test_residency_plan.py), the slab holds each resident page's rows, hot regions
    and resident pages never share a block; a decode that opens pages (and takes queued
    blocks) keeps all of that and matches the oracle layer by layer."""
    from mini_hisparse_amd.batched_engine import empty_state, random_model, random_prompts

    wl = tiny(context=9 * 16 + 14, steps=6)
    model = random_model(wl, gpu, seed=1)
    state = empty_state(wl, gpu, residency="policy", window=4, watermark=0)
    firsts = state.prefill(model, random_prompts(wl, gpu, seed=3), wl.resident_fraction)
    plan = state.plan
    assert plan.stats["hot_trigger_window"] == wl.layers * wl.batch
    assert plan.stats["unpinned_block_reuses"] > 0  # the slab was too small for every page

    def check():
        torch.cuda.synchronize()
        B, C, P, Hkv, D = wl.batch, state.pages, wl.page_size, wl.kv_heads, wl.head_dim
        owners = {}
        for b in range(B):
            for l in range(wl.layers):
                g = plan.group((b, l))
                resident = state.resident[l, b].cpu().numpy()
                np.testing.assert_array_equal(resident, g.slot[:C])
                assert state.hot[l, b].tolist() == g.hot
                host = state.host[l].view(B, C, 2, P, Hkv, D)[b]
                length = state.lengths[b]
                for page in np.flatnonzero(resident >= 0).tolist():
                    rows = min(P, length - page * P)
                    assert torch.equal(state.pool[int(resident[page]), :, :rows].cpu(), host[page, :, :rows])
                    owners.setdefault(int(resident[page]), []).append(("page", b, l, page))
                for block in g.hot:
                    owners.setdefault(block, []).append(("hot", b, l))
        assert all(len(v) == 1 for v in owners.values()), "a block with two owners"

    check()
    opened = plan.stats["evictions"]
    _engine_layers_match_oracle(gpu, wl, steps=4, built=(model, state, firsts))
    assert state.lengths[0] == wl.context + 4  # crossed a page boundary: pages opened
    assert plan.stats["evictions"] > opened  # ... on queued blocks
    check()


def geometry(name, **overrides):
    """The real layer geometry of a BASELINE model workload (hidden, heads, head_dim,
    FFN, vocab, page budget, residency, hot rows) with two layers and the given batch
    and context, for oracle checks of whole engine steps."""
    from dataclasses import replace

    from mini_hisparse_amd.batched_engine import WORKLOADS
    from mini_hisparse_amd.selection import union_bound

    wl = replace(WORKLOADS[name], layers=2, steps=8, **overrides)
    bound = union_bound(wl.context + wl.steps, wl.page_size, wl.top_pages,
                        1 if wl.selector == "uniform" else wl.heads)
    return replace(wl, hot_rows=min(wl.hot_rows, 32768, max(2 * bound, bound)))


@pytest.mark.gpu
@pytest.mark.parametrize(
    "name,overrides",
    [
        # BASELINE configs[3] (north_star): hidden 3584, 28 q / 4 kv heads, head_dim 128,
        # FFN 18944, vocab 152064, top-64 pages, 15% resident; 4k-token histories
        ("qwen2.5-7b", {"batch": 4, "context": 4096 - 1}),
        # hidden 896, 14 q / 2 kv heads, head_dim 64, FFN 4864,
        # vocab 151936, top-32 pages, 25% resident; the full 32k-token histories
        ("qwen2.5-0.5b", {"batch": 4, "context": 32768 - 1}),
    ],
)
def test_engine_at_model_geometry_matches_oracle(gpu, name, overrides):
    stats = _engine_layers_match_oracle(gpu, geometry(name, **overrides))
    assert stats[0] > 0 and stats[2] > 0


@pytest.mark.gpu
def test_batched_engine_rejects_a_hot_region_below_the_union_bound(gpu):
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    wl = tiny(hot_rows=128)
    with pytest.raises(ValueError, match="below the union bound"):
        BatchedDecodeEngine(random_model(wl, gpu), build_state(wl, gpu), wl.top_pages)


def test_uniform_pages_draws_distinct_pages_with_the_tail():
    from mini_hisparse_amd.batched_engine import uniform_pages

    gen = torch.Generator().manual_seed(3)
    lengths = [40 * 16 - 1, 40 * 16 + 1, 5 * 16, 16 * 1000 + 7]
    pages = uniform_pages(lengths, 16, 6, 4, gen, "cpu")
    assert pages.shape == (4, 4, 6) and pages.dtype == torch.int32
    counts = [ceil(length / 16) for length in lengths]
    seen = set()
    for layer in range(4):
        for b, count in enumerate(counts):
            row = pages[layer, b, : min(6, count)].tolist()
            if count <= 6:
                assert row == list(range(count))
                continue
            assert row == sorted(set(row)) and row[-1] == count - 1 and 0 <= row[0]
            seen.update(row[:-1])
    # the draws cover the history (not a fixed subset): 4 layers x 3 requests x 5 draws
    assert len(seen) > 30
    again = uniform_pages(lengths, 16, 6, 4, torch.Generator().manual_seed(3), "cpu")
    assert torch.equal(pages, again)


def _uniform_engine_matches_oracle(gpu, wl, prefetch, steps=3):
    """The miss-heavy stress path: pages resampled every step and shared by every head,
    then union, resolver, gather and attention as for Quest selections.  With
    ``prefetch`` every layer's select, resolve and gather run at step start on the
    transfer stream (one decoder per layer), overlapping the dense layers."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    print(f"[case] {wl.name} uniform: L={wl.layers} hidden={wl.hidden} heads={wl.heads}/{wl.kv_heads} "
          f"batch={wl.batch} context={wl.context} prefetch={prefetch}", flush=True)
    model = random_model(wl, gpu, seed=1)
    state = build_state(wl, gpu, seed=2)
    engine = BatchedDecodeEngine(model, state, wl.top_pages, selector="uniform", seed=4, prefetch=prefetch)
    assert engine.dec.capacity == wl.top_pages * wl.page_size  # one head's selection bounds the union
    if prefetch:
        assert len({id(engine.decoder(l)) for l in range(wl.layers)}) == wl.layers
        assert all(engine.decoder(l).attend_ws is engine.dec.attend_ws for l in range(wl.layers))
    L, B, C, P = wl.layers, wl.batch, state.pages, wl.page_size
    Hkv, D = wl.kv_heads, wl.head_dim
    records = []
    tokens = torch.arange(1, B + 1, device=gpu)
    unions, drawn = 0, set()
    for step in range(steps):
        records.clear()
        tokens = engine.step(
            tokens,
            lambda l, q, k, v, out: records.append(
                (l, q.clone(), out.clone(), engine.decoder(l).pages.clone(), engine.decoder(l).union_count.clone())
            ),
        )
        torch.cuda.synchronize()
        length = state.lengths[0]
        count = ceil(length / P)
        for l, q, out, layer_pages, union_count in records:
            for b in range(B):
                pages = layer_pages[b].cpu().numpy()
                assert (pages == pages[0]).all()  # every head reads the same pages
                row = pages[0].tolist()
                assert row == sorted(set(row)) and row[-1] == count - 1
                drawn.update((l, b, p) for p in row[:-1])
                kv = state.host[l].view(B, C, 2, P, Hkv, D)[b, :count].float()
                keys = kv[:, 0].reshape(count * P, Hkv, D)[:length]
                vals = kv[:, 1].reshape(count * P, Hkv, D)[:length]
                positions = pages_to_positions(pages, length, P)
                assert int(union_count[b]) == len(positions[0])
                expected = oracle.selection_oracle(q[b].cpu(), keys, vals, positions)
                got = out[b].float().cpu().double().numpy()
                assert np.all(np.abs(got - expected) <= 2e-2 + 1e-2 * np.abs(expected)), np.abs(got - expected).max()
                unions += int(union_count[b])
    stats = state.row_stats.tolist()
    assert sum(stats) == unions
    assert stats[2] > stats[1]  # resampling every step: misses outnumber hot hits
    return stats, drawn


@pytest.mark.gpu
@pytest.mark.parametrize("prefetch", [False, True])
def test_batched_engine_uniform_selection_matches_oracle(gpu, prefetch):
    from mini_hisparse_amd.selection import union_bound

    wl = tiny(selector="uniform", hot_rows=2 * union_bound(40 * 16 + 23, 16, 6, 1), resident_fraction=0.4)
    _, drawn = _uniform_engine_matches_oracle(gpu, wl, prefetch)
    # fresh draws each step (5 per step; about 13 distinct expected per (layer, request))
    assert len(drawn) >= 8 * wl.layers * wl.batch


@pytest.mark.gpu
def test_engine_at_stress_geometry_matches_oracle(gpu):
    """BASELINE configs[4]'s layer geometry (hidden 5120, 40 q / 8 kv heads, head_dim 128,
    FFN 27648, vocab 152064, 64 uniformly resampled pages shared by every head, 40%
    resident, hot_rows 2048) with two layers, batch 2 and 8k-token histories, prefetched
    as the bench runs it: about 60% of the selected rows miss."""
    stats, _ = _uniform_engine_matches_oracle(gpu, geometry("qwen2.5-32b-stress", batch=2, context=8192), True)
    assert stats[2] > 0.4 * sum(stats)


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", [False, True])
def test_prefetched_uniform_steps_equal_in_order_steps(gpu, graphs):
    """Prefetching every layer's select/resolve/gather at step start changes only the
    launch order across streams: tokens, attention outputs, the resolver's row
    statistics and every hot region's tags and LRU equal the in-order engine's bit for bit
    (also with the dense layer boundaries replayed from HIP graphs between the waits)."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model
    from mini_hisparse_amd.selection import union_bound

    wl = tiny(selector="uniform", hot_rows=2 * union_bound(40 * 16 + 23, 16, 6, 1), resident_fraction=0.4)
    runs = []
    for prefetch in (False, True):
        model = random_model(wl, gpu, seed=1)
        state = build_state(wl, gpu, seed=2)
        engine = BatchedDecodeEngine(model, state, wl.top_pages, selector="uniform", seed=4, prefetch=prefetch,
                                     graphs=graphs, projections="kernel" if graphs else "auto")
        assert engine.use_graphs == graphs
        outs, toks = [], []
        tokens = torch.tensor([1, 2, 3], device=gpu)
        for step in range(4):  # with graphs: step 0 eager, captured after it, replayed from step 1
            tokens = engine.step(tokens, lambda l, q, k, v, out: outs.append(out.clone()))
            toks.append(tokens.clone())
        torch.cuda.synchronize()
        runs.append((outs, toks, state.row_stats.clone(), (state.tags.clone(), state.lru.clone())))
    (eo, et, es, etab), (po, pt, ps, ptab) = runs
    assert len(eo) == len(po) == 4 * wl.layers
    assert all(torch.equal(a, b) for a, b in zip(eo, po))
    assert all(torch.equal(a, b) for a, b in zip(et, pt))
    assert torch.equal(es, ps)
    assert torch.equal(etab[0], ptab[0]) and torch.equal(etab[1], ptab[1])


def test_prefetch_needs_the_uniform_selector():
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine

    with pytest.raises(ValueError, match="uniform"):
        BatchedDecodeEngine(None, None, 4, prefetch=True)


@pytest.mark.gpu
def test_graph_replayed_dense_layers_match_eager_launches(gpu):
    """The dense launches replayed from HIP graphs give bit-identical tokens and attention
    outputs to the same launches made eagerly, step after step (the sparse stages run
    eagerly in between)."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    wl = tiny()
    runs = []
    for graphs in (False, True):
        model = random_model(wl, gpu, seed=1)
        state = build_state(wl, gpu, seed=2)
        engine = BatchedDecodeEngine(model, state, wl.top_pages, graphs=graphs, projections="kernel")
        assert engine.use_graphs == graphs
        outs, toks = [], []
        tokens = torch.tensor([1, 2, 3], device=gpu)
        for step in range(5):  # step 0 eager; the graphs are captured after it and replayed from step 1
            tokens = engine.step(tokens, lambda l, q, k, v, out: outs.append((q.clone(), out.clone())))
            toks.append(tokens.clone())
        torch.cuda.synchronize()
        if graphs:
            assert engine._graphs is not None and len(engine._graphs) == wl.layers + 1
        runs.append((outs, toks, state.row_stats.clone()))
    (eo, et, es), (go, gt, gs) = runs
    assert len(eo) == len(go) == 5 * wl.layers
    for (q0, o0), (q1, o1) in zip(eo, go):
        assert torch.equal(q0, q1) and torch.equal(o0, o1)
    for t0, t1 in zip(et, gt):
        assert torch.equal(t0, t1)
    assert torch.equal(es, gs)


@pytest.mark.gpu
def test_full_7b_step_matches_oracle_on_every_layer(gpu):
    """The whole BASELINE configs[3] step at its full size for one request: 28 layers,
    131,072-token history (synthetic), top-64 pages, 32,768 hot rows (the resolver's split
    front), two decode steps.  Every layer of each step is checked against the oracle: the bounds equal the exact extrema of the history read back from the host
    pool, the Quest pages equal the oracle's, the attention equals the oracle's sparse
    attention over the selected tokens; every layer's rows are resident, hot or missed."""
    from dataclasses import replace

    from mini_hisparse_amd.batched_engine import WORKLOADS, BatchedDecodeEngine, build_state, random_model

    wl = replace(WORKLOADS["qwen2.5-7b"], batch=1, context=131072 - 1, steps=4)
    print(f"[case] full 7B step: L={wl.layers} context={wl.context} hot_rows={wl.hot_rows}", flush=True)
    model, state = random_model(wl, gpu, seed=1), build_state(wl, gpu, seed=2)
    engine = BatchedDecodeEngine(model, state, wl.top_pages)
    P, Hkv, D, C = wl.page_size, wl.kv_heads, wl.head_dim, state.pages
    sampled = tuple(range(wl.layers))
    records = []

    def observe(l, q, k, v, out):
        if l in sampled:
            dec = engine.decoder(l)
            records.append((l, q.clone(), out.clone(), dec.pages.clone(), dec.union_count.clone()))

    tokens = torch.tensor([7], device=gpu)
    stats0 = state.row_stats.clone()
    for step in range(2):
        records.clear()
        tokens = engine.step(tokens, observe)
        torch.cuda.synchronize()
        length = state.lengths[0]
        count = ceil(length / P)
        assert [r[0] for r in records] == list(sampled)
        for l, q, out, layer_pages, union_count in records:
            kv = state.host[l].view(1, C, 2, P, Hkv, D)[0, :count].float()
            keys = kv[:, 0].reshape(count * P, Hkv, D)[:length]
            vals = kv[:, 1].reshape(count * P, Hkv, D)[:length]
            padded = torch.cat([keys, keys[-1:].expand(count * P - length, Hkv, D)]).view(count, P, Hkv, D)
            lo, hi = padded.amin(1), padded.amax(1)  # the last page's padding repeats its last row
            torch.testing.assert_close(state.minimum[l, 0, :count].float().cpu(), lo, rtol=0, atol=0)
            torch.testing.assert_close(state.maximum[l, 0, :count].float().cpu(), hi, rtol=0, atol=0)
            pages = oracle.quest_pages(q[0].cpu(), lo, hi, length, P, wl.top_pages)
            np.testing.assert_array_equal(layer_pages[0, :, : pages.shape[1]].cpu().numpy(), pages,
                                          err_msg=f"step {step} layer {l}")
            positions = pages_to_positions(pages, length, P)
            assert int(union_count[0]) == len(set().union(*map(set, positions)))
            # each head over its selected tokens (the request's host rows are its tokens)
            width = max(len(p) for p in positions)
            rows = np.full((len(positions), width), -1, np.int64)
            for h, p in enumerate(positions):
                rows[h, : len(p)] = p
            expected = oracle.row_attention_rows(q[0].cpu(), state.host[l].view(C, 2, P, Hkv, D), rows, P)
            got = out[0].float().cpu().double().numpy()
            assert np.all(np.abs(got - expected) <= 2e-2 + 1e-2 * np.abs(expected)), (step, l)
    engine.check_status()
    rows = (state.row_stats - stats0).tolist()
    assert rows[0] > 0 and rows[1] + rows[2] > 0  # resident, hot and missed rows all occur


@pytest.mark.gpu
def test_fused_rotary_append_equals_the_separate_launches(gpu):
    """hs_rotary_split_append (the engine's default) against hs_rotary_split followed by
    hs_append_rows: over four steps (one crossing a page boundary) the tokens, the pool,
    the host mirror and the Quest bounds are bit-identical."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    wl = tiny(context=40 * 16 - 2)
    print(f"[case] fused rotary+append: {wl}", flush=True)
    runs = []
    for fused in (True, False):
        model, state = random_model(wl, gpu, seed=1), build_state(wl, gpu, seed=2)
        engine = BatchedDecodeEngine(model, state, wl.top_pages, fuse_rotary_append=fused)
        tokens = torch.arange(1, wl.batch + 1, device=gpu)
        seq = []
        for _ in range(4):
            tokens = engine.step(tokens)
            seq.append(tokens.clone())
        torch.cuda.synchronize()
        runs.append((seq, state))
    (seq_a, a), (seq_b, b) = runs
    assert all(torch.equal(x, y) for x, y in zip(seq_a, seq_b))
    # the rows the four appends wrote, in the pool (the tail blocks, placed alike) and in
    # the host mirror; the bounds of every page
    P, C, B = wl.page_size, a.pages, wl.batch
    for l in range(wl.layers):
        assert a.tail_block[l] == b.tail_block[l]
        pool_a, pool_b = a.pool.view(-1, 2, P, wl.kv_heads, wl.head_dim), b.pool.view(-1, 2, P, wl.kv_heads, wl.head_dim)
        host_a = a.host[l].view(-1, 2, P, wl.kv_heads, wl.head_dim)
        host_b = b.host[l].view(-1, 2, P, wl.kv_heads, wl.head_dim)
        for r in range(B):
            for pos in range(wl.context, wl.context + 4):
                page, off = divmod(pos, P)
                hb = r * C + page
                assert torch.equal(host_a[hb, :, off].view(torch.int16).cpu(), host_b[hb, :, off].view(torch.int16).cpu())
            blk = a.tail_block[l][r]
            for pos in range((wl.context + 3) // P * P, wl.context + 4):  # the current tail page's new rows
                off = pos % P
                assert torch.equal(pool_a[blk, :, off].view(torch.int16), pool_b[blk, :, off].view(torch.int16))
    assert torch.equal(a.minimum.view(torch.int16), b.minimum.view(torch.int16))
    assert torch.equal(a.maximum.view(torch.int16), b.maximum.view(torch.int16))


@pytest.mark.gpu
def test_a_step_past_the_history_capacity_is_refused_on_the_host(gpu):
    """A state sized for 641 tokens (41 pages of 16: room up to token 655) decodes from
    637 tokens until full; the next step raises before it launches anything (the new
    page would index past the state's tables), and the state is left as it was."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model

    wl = tiny(context=40 * 16 - 3, steps=4)
    model, state = random_model(wl, gpu, seed=1), build_state(wl, gpu, seed=2)
    engine = BatchedDecodeEngine(model, state, wl.top_pages)
    capacity = state.pages * wl.page_size
    assert capacity == 656
    tokens = torch.arange(1, wl.batch + 1, device=gpu)
    while state.lengths[0] < capacity:
        tokens = engine.step(tokens)
    torch.cuda.synchronize()
    lengths = list(state.lengths)
    with pytest.raises(RuntimeError, match="history full"):
        engine.step(tokens)
    torch.cuda.synchronize()
    assert state.lengths == lengths
