"""Every stage of one batched decode layer at the per-(request, layer) shapes of
BASELINE configs[2] (Qwen2.5-0.5B) and configs[4] (Qwen2.5-32B miss-heavy stress),
against the CPU oracle, over several steps that carry the hot tags and LRU.

Per step and request: the chosen pages (Quest: equal to the oracle's; uniform:
the drawn pages, identical for every head), the union and head columns, every
resolver output (physical rows, miss plan, counts, the updated tags and LRU)
bit for bit, the whole device pool after the gather byte for byte (the oracle
applies the same plan to a host copy), and the attention output within the
north_star tolerance (2e-2 abs / 1e-2 rel, bf16 in, fp32 accumulate).  The
reference pattern is its multi-step hybrid test (tests/test_hybrid.py:273-296):
the hot region's state after one step is the next step's input.
"""

from __future__ import annotations

from math import ceil

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions
from oracle.union import from_selection as oracle_union
from tests.kernel_cases import make_pool

pytestmark = pytest.mark.gpu


def _bounds(host_req, length, P):
    """Exact per-page K extrema of one request's host pages ([pages, 2, P, Hkv, D])."""
    count = ceil(length / P)
    keys = host_req[:count, 0].float()  # [count, P, Hkv, D]
    lo = keys.amin(1)
    hi = keys.amax(1)
    tail = length - (count - 1) * P
    lo[count - 1] = keys[count - 1, :tail].amin(0)
    hi[count - 1] = keys[count - 1, :tail].amax(0)
    pages = host_req.shape[0]
    full_lo = torch.full((pages, *lo.shape[1:]), float("inf"))
    full_hi = torch.full((pages, *hi.shape[1:]), float("-inf"))
    full_lo[:count], full_hi[:count] = lo, hi
    return full_lo.to(host_req.dtype), full_hi.to(host_req.dtype)


def _run_layer(gpu, *, B, Hkv, g, D, pages, length, top, hot_rows, resident_frac, selector, steps, seed):
    from mini_hisparse_amd.batched import BatchedSparseDecode, LayerTablesView
    from mini_hisparse_amd.batched_engine import uniform_pages
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import MappedHost

    P, heads, dtype = 16, Hkv * g, torch.bfloat16
    dev = torch.device(gpu)
    print(f"[case] B={B} heads={heads}/{Hkv} D={D} pages={pages} length={length} top={top} "
          f"S={hot_rows} selector={selector}", flush=True)
    host = make_pool(B * pages, P, Hkv, D, dtype, seed=seed, outliers=True).pin_memory()
    count = ceil(length / P)
    rng = np.random.default_rng(seed)
    hot_blocks = ceil(hot_rows / P)
    resident_sets = []
    for b in range(B):
        chosen = rng.permutation(count - 1)[: round(resident_frac * count)]
        resident_sets.append(np.unique(np.append(chosen, count - 1)))  # the tail page is resident
    n_resident = sum(len(r) for r in resident_sets)
    blocks = n_resident + B * hot_blocks
    pool_cpu = torch.zeros(blocks, 2, P, Hkv, D, dtype=dtype)
    tables_np, next_block = [], 0
    for b in range(B):
        resident = np.full(pages, -1, np.int32)
        res = resident_sets[b]
        resident[res] = np.arange(next_block, next_block + len(res), dtype=np.int32)
        pool_cpu[next_block : next_block + len(res)] = host[b * pages + torch.from_numpy(res).long()]
        next_block += len(res)
        source = np.arange(b * pages, (b + 1) * pages, dtype=np.int32)
        hot = (n_resident + b * hot_blocks + rng.permutation(hot_blocks)).astype(np.int32)  # fragmented
        tags = np.full(hot_rows, -1, np.int32)
        lru = rng.permutation(hot_rows).astype(np.int64)
        tables_np.append(dict(source=source, resident=resident, hot=hot, tags=tags, lru=lru))
    bounds = [_bounds(host[b * pages : (b + 1) * pages], length, P) for b in range(B)]
    cfg = CacheConfig(gpu_pages=blocks, host_pages=B * pages, page_size=P, kv_heads=Hkv, head_dim=D,
                      device=gpu, dtype=dtype)
    dec = BatchedSparseDecode(cfg, heads, top, [length] * B, device=dev, shared_selection=selector == "uniform",
                              head_rows=True)
    assert hot_rows >= dec.capacity, "the hot region must cover the union bound"
    tables = [LayerTablesView(*[torch.from_numpy(t[k]).to(dev) for k in ("source", "resident", "hot", "tags", "lru")])
              for t in tables_np]
    lo_d = [lo.to(dev) for lo, _ in bounds]
    hi_d = [hi.to(dev) for _, hi in bounds]
    pool = pool_cpu.to(dev)
    alias = MappedHost(host)
    row_stats = torch.zeros(3, dtype=torch.int64, device=dev)
    expected_stats = np.zeros(3, np.int64)
    sampler = torch.Generator(device=dev).manual_seed(seed + 1)
    totals = np.zeros(3, np.int64)
    for step in range(steps):
        q = torch.randn(B, heads, D, generator=torch.Generator().manual_seed(seed * 100 + step)).to(dtype)
        if selector == "quest":
            dec.select(q.to(dev), lo_d, hi_d)
        else:
            drawn = uniform_pages([length] * B, P, top, 1, sampler, dev)[0]
            dec.select_pages(drawn)
        dec.resolve(tables, row_stats=row_stats)
        dec.gather(alias, pool, torch.cuda.current_stream(dev))
        out = dec.attend(q.to(dev), pool)
        torch.cuda.synchronize()
        dec.check_status()  # no union or entry capacity overflow
        for b in range(B):
            t = tables_np[b]
            if selector == "quest":
                pages_o = oracle.quest_pages(q[b], bounds[b][0], bounds[b][1], length, P, top)
                np.testing.assert_array_equal(dec.pages[b, :, : pages_o.shape[1]].cpu().numpy(), pages_o)
            else:
                got = dec.pages[b].cpu().numpy()
                assert (got == got[0]).all(), "a shared selection reads the same pages in every head"
                row = got[0, : min(top, count)].tolist()
                assert row == sorted(set(row)) and row[-1] == count - 1 and row[0] >= 0
                pages_o = got[:, : min(top, count)].astype(np.int64)
            union, cols = oracle_union(pages_to_positions(pages_o, length, P))
            n = len(union)
            assert int(dec.union_count[b]) == n
            marked = np.zeros(dec.page_bits_stride * 32, bool)
            marked[np.unique(pages_o[pages_o >= 0])] = True  # the union's pages
            words = np.packbits(marked.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").reshape(-1)
            got_bits = dec.page_bits[b].cpu().numpy().view(np.uint32)
            nw = (count + 31) // 32
            np.testing.assert_array_equal(got_bits[:nw], words[:nw].astype(np.uint32))
            np.testing.assert_array_equal(dec.positions[b, :n].cpu().numpy(), union)
            np.testing.assert_array_equal(dec.head_columns[b, :, : cols.shape[1]].cpu().numpy(), cols)
            phys, mh, md, counts, tags1, lru1 = oracle.resolve_rows(
                union, t["source"], t["resident"], t["hot"], t["tags"], t["lru"], length, P, head_columns=cols)
            np.testing.assert_array_equal(dec.physical[b, :, : phys.shape[1]].cpu().numpy(), phys)
            m = int(counts[2])  # the decoder writes the plan's compact prefix only
            assert (mh[m:] == -1).all() and (md[m:] == -1).all()
            np.testing.assert_array_equal(dec.miss_host[b, :m].cpu().numpy(), mh[:m])
            np.testing.assert_array_equal(dec.miss_device[b, :m].cpu().numpy(), md[:m])
            np.testing.assert_array_equal(dec.row_counts[b].cpu().numpy(), counts)
            np.testing.assert_array_equal(tables[b].tags.cpu().numpy(), tags1)
            np.testing.assert_array_equal(tables[b].lru.cpu().numpy(), lru1)
            t["tags"], t["lru"] = tags1.astype(np.int32), lru1
            expected_stats += counts
            totals += counts
            oracle.gather_rows(host, pool_cpu, mh, md, P)
        assert torch.equal(pool.cpu(), pool_cpu), f"step {step}: pool differs from the oracle's gather"
        for b in range(B):
            expected = oracle.row_attention_rows(q[b], pool_cpu, dec.physical[b].cpu(), P)
            err = np.abs(out[b].float().cpu().double().numpy() - expected)
            assert (err <= 2e-2 + 1e-2 * np.abs(expected)).all(), f"step {step} request {b}: {err.max():.3g}"
        assert row_stats.cpu().numpy().tolist() == expected_stats.tolist()
    return totals


def test_qwen05b_layer_shape_matches_oracle(gpu):
    """configs[2] per (request, layer): 14 q / 2 kv heads, head_dim 64, 2,048 pages of
    32k-token history (+1 decoded token), Quest top-32, 25% of pages resident,
    hot_rows = 2U = 13,504, batch 4; three steps with fresh queries."""
    totals = _run_layer(gpu, B=4, Hkv=2, g=7, D=64, pages=2056, length=32769, top=32, hot_rows=13504,
                        resident_frac=0.25, selector="quest", steps=3, seed=61)
    assert totals[0] > 0 and totals[2] > 0 and totals[1] > 0  # resident hits, misses, and hot hits by step 3


def test_qwen32b_stress_layer_shape_matches_oracle(gpu):
    """configs[4] per (request, layer): 40 q / 8 kv heads, head_dim 128, 4,096 pages of
    64k-token history (+1), 64 pages resampled uniformly per step and shared by every
    head, 40% of pages resident, hot_rows 2048 (2U of one shared selection), batch 2;
    about 60% of the selected rows miss to pinned host memory."""
    totals = _run_layer(gpu, B=2, Hkv=8, g=5, D=128, pages=4104, length=65537, top=64, hot_rows=2048,
                        resident_frac=0.4, selector="uniform", steps=3, seed=71)
    selected = totals.sum()
    assert 0.45 < totals[2] / selected < 0.75, totals  # the miss-heavy regime


def test_pipelined_groups_with_split_front_match_one_batch(gpu, monkeypatch):
    """``PipelinedSparseDecode`` (two request groups, transfer stream, split resolver
    front forced on) against one ``BatchedSparseDecode`` of the whole batch with the
    single-workgroup front, from identical tables, pool and queries, over two steps
    that carry the tags and LRU: the same miss plans, tags, LRU and pool bit for bit,
    and the same attention output within the bf16 tolerance (2e-2 abs / 1e-2 rel; the
    groups' split-K schedules may differ from the whole batch's)."""
    from mini_hisparse_amd.batched import BatchedSparseDecode, LayerTablesView, PipelinedSparseDecode
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import MappedHost

    monkeypatch.setenv("HS_RESOLVE_SPLIT", "1")
    B, Hkv, g, D, P, pages, length, top, hot_rows = 4, 2, 7, 64, 16, 1032, 16385, 32, 7168
    heads, dtype, dev = Hkv * g, torch.bfloat16, torch.device(gpu)
    print(f"[case] pipelined split front: B={B} length={length} S={hot_rows}", flush=True)
    host = make_pool(B * pages, P, Hkv, D, dtype, seed=5, outliers=True).pin_memory()
    rng = np.random.default_rng(5)
    count, hot_blocks = ceil(length / P), ceil(hot_rows / P)
    res_sets = [np.unique(np.append(rng.permutation(count - 1)[: count // 4], count - 1)) for _ in range(B)]
    n_res = sum(len(r) for r in res_sets)
    pool0 = torch.zeros(n_res + B * hot_blocks, 2, P, Hkv, D, dtype=dtype)
    tables_np, nb = [], 0
    for b in range(B):
        resident = np.full(pages, -1, np.int32)
        resident[res_sets[b]] = np.arange(nb, nb + len(res_sets[b]), dtype=np.int32)
        pool0[nb : nb + len(res_sets[b])] = host[b * pages + torch.from_numpy(res_sets[b]).long()]
        nb += len(res_sets[b])
        tables_np.append(dict(source=np.arange(b * pages, (b + 1) * pages, dtype=np.int32), resident=resident,
                              hot=(n_res + b * hot_blocks + rng.permutation(hot_blocks)).astype(np.int32),
                              tags=np.full(hot_rows, -1, np.int32), lru=rng.permutation(hot_rows).astype(np.int16)))
    bounds = [_bounds(host[b * pages : (b + 1) * pages], length, P) for b in range(B)]
    lo = [x.to(dev) for x, _ in bounds]
    hi = [x.to(dev) for _, x in bounds]
    cfg = CacheConfig(gpu_pages=pool0.shape[0], host_pages=B * pages, page_size=P, kv_heads=Hkv, head_dim=D,
                      device=gpu, dtype=dtype)
    runs = {}
    for name in ("pipelined", "batch"):
        if name == "pipelined":
            dec = PipelinedSparseDecode(cfg, heads, top, [length] * B, parts=2, device=dev, split_front=True)
            transfer = torch.cuda.Stream(dev)
            assert all(part.split_front for part in dec.parts)
            assert hot_rows >= dec.parts[0].capacity, "the hot region must cover the union bound"
        else:
            dec = BatchedSparseDecode(cfg, heads, top, [length] * B, device=dev, split_front=False)
            transfer = torch.cuda.current_stream(dev)
        tables = [LayerTablesView(*[torch.from_numpy(t[k]).to(dev) for k in ("source", "resident", "hot", "tags", "lru")])
                  for t in tables_np]
        pool, alias, outs = pool0.to(dev), MappedHost(host), []
        for step in range(2):
            q = torch.randn(B, heads, D, generator=torch.Generator().manual_seed(50 + step)).to(dtype).to(dev)
            if name == "pipelined":
                out, _ = dec.step(q, lo, hi, tables, pool, alias, transfer)
            else:
                out = dec.step(q, lo, hi, tables, pool, alias, transfer)[0]
            torch.cuda.synchronize()
            outs.append(out.float().cpu())
        runs[name] = (outs, [(t.tags.cpu(), t.lru.cpu()) for t in tables], pool.cpu())
    (outs_p, tl_p, pool_p), (outs_b, tl_b, pool_b) = runs["pipelined"], runs["batch"]
    for (tp, lp), (tb, lb) in zip(tl_p, tl_b):
        assert torch.equal(tp, tb) and torch.equal(lp, lb)
    assert torch.equal(pool_p, pool_b)
    for a, b in zip(outs_p, outs_b):
        assert ((a - b).abs() <= 2e-2 + 1e-2 * b.abs()).all()
