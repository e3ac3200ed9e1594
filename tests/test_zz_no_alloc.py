"""hs_resolve_rows_noalloc (the resolver with its scratch in a fixed device array of the
library, for callers that cannot allocate) against hs_resolve_rows_batched with a
caller workspace: identical outputs, including the in-place tags and LRU, on two
calls in a row whose second batch is smaller -- so leftovers of the first call in
the shared scratch would show -- and a batch above the scratch size is rejected
before anything is launched."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.kernel_cases import random_positions, resolver_tables

pytestmark = pytest.mark.gpu


def _batch(gpu, cases):
    """Descriptors over fresh device copies of each case's tables, and their outputs."""
    from mini_hisparse_amd import _lib

    descs = (_lib.ResolveDesc * len(cases))()
    keep = []
    for d, (length, P, tables, positions) in zip(descs, cases):
        t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
        pos = torch.from_numpy(positions).to(gpu)
        n = pos.numel()
        out = {name: torch.full((n,), -7, dtype=torch.int64, device=gpu) for name in ("phys", "uphys", "mh", "md")}
        out["counts"] = torch.full((3,), -7, dtype=torch.int64, device=gpu)
        d.positions, d.n, d.positions_i64 = pos.data_ptr(), n, 1
        d.source, d.resident, d.n_pages = t["source"].data_ptr(), t["resident"].data_ptr(), t["source"].numel()
        d.hot, d.hot_blocks = t["hot"].data_ptr(), t["hot"].numel()
        d.tags, d.lru, d.hot_rows = t["tags"].data_ptr(), t["lru"].data_ptr(), t["tags"].numel()
        d.length, d.page_size = length, P
        d.physical, d.union_physical = out["phys"].data_ptr(), out["uphys"].data_ptr()
        d.miss_host_rows, d.miss_device_rows = out["mh"].data_ptr(), out["md"].data_ptr()
        d.counts = out["counts"].data_ptr()
        keep.append((t, pos, out))
    return descs, keep


def _cases(seed, shapes):
    cases = []
    for i, (length, P, S, n) in enumerate(shapes):
        tables = resolver_tables(seed + i, length, P, S, resident_frac=0.1 * (i % 6), tag_frac=0.4)
        cases.append((length, P, tables, random_positions(seed + 100 + i, n, length)))
    return cases


def _run_both(gpu, cases):
    from mini_hisparse_amd import _lib

    lib = _lib.load()
    stream = _lib.stream_handle(torch.device(gpu))
    ref_descs, ref = _batch(gpu, cases)
    need = sum(lib.hs_resolve_workspace_bytes(d.n, d.length, d.n_pages, d.hot_rows) for d in ref_descs)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    _lib.check(lib.hs_resolve_rows_batched(ref_descs, len(cases), ws.data_ptr(), need, stream),
               "hs_resolve_rows_batched")
    na_descs, na = _batch(gpu, cases)
    _lib.check(lib.hs_resolve_rows_noalloc(na_descs, len(cases), stream), "hs_resolve_rows_noalloc")
    torch.cuda.synchronize()
    for (t0, _, o0), (t1, _, o1) in zip(ref, na):
        for name in ("phys", "uphys", "mh", "md", "counts"):
            assert torch.equal(o0[name], o1[name]), name
        assert torch.equal(t0["tags"], t1["tags"]) and torch.equal(t0["lru"], t1["lru"])
    return need


def test_noalloc_resolver_equals_the_workspace_resolver_twice(gpu):
    print("[case] noalloc: 18 descriptors (two launches of 16 + 2), then 3 smaller ones", flush=True)
    big = _cases(300, [(131072, 16, 32768, 27808), (4096, 16, 2048, 1500), (1000, 16, 512, 300),
                       (97, 4, 64, 40), (300, 7, 128, 100), (65536, 16, 32768, 20000)] * 3)
    first = _run_both(gpu, big)
    small = _cases(400, [(1000, 16, 512, 300), (97, 4, 64, 40), (50, 3, 30, 30)])
    second = _run_both(gpu, small)
    assert second < first


def test_noalloc_resolver_rejects_a_batch_above_its_scratch(gpu):
    from mini_hisparse_amd import _lib

    lib = _lib.load()
    limit = lib.hs_resolve_noalloc_max_bytes()
    assert limit == 32 << 20
    cases = _cases(500, [(131072, 16, 32768, 100)])
    descs1, keep = _batch(gpu, cases)
    per = lib.hs_resolve_workspace_bytes(descs1[0].n, descs1[0].length, descs1[0].n_pages, descs1[0].hot_rows)
    count = limit // per + 1  # one descriptor more than fits
    descs = (_lib.ResolveDesc * count)(*([descs1[0]] * count))
    tags_before = keep[0][0]["tags"].clone()
    status = lib.hs_resolve_rows_noalloc(descs, count, _lib.stream_handle(torch.device(gpu)))
    assert status == -1
    assert b"scratch" in lib.hs_last_error()
    torch.cuda.synchronize()
    assert torch.equal(keep[0][0]["tags"], tags_before)  # nothing ran
    assert int(keep[0][2]["counts"][0]) == -7


def test_noalloc_resolver_replays_from_a_captured_graph(gpu):
    """After one uncaptured call (the scratch address lookup), the call is captured into a
    HIP graph; each replay must equal a fresh eager hs_resolve_rows_batched on tables that
    went through the same steps (the in-place tags and LRU carry hits between steps)."""
    from mini_hisparse_amd import _lib

    print("[case] noalloc under graph capture: 3 descriptors, 3 replays", flush=True)
    lib = _lib.load()
    cases = _cases(600, [(4096, 16, 2048, 1500), (97, 4, 64, 40), (65536, 16, 32768, 20000)])
    warm, _ = _batch(gpu, cases)
    _lib.check(lib.hs_resolve_rows_noalloc(warm, len(cases), _lib.stream_handle(torch.device(gpu))), "warm-up")
    torch.cuda.synchronize()
    ref_descs, ref = _batch(gpu, cases)
    need = sum(lib.hs_resolve_workspace_bytes(d.n, d.length, d.n_pages, d.hot_rows) for d in ref_descs)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    g_descs, cap = _batch(gpu, cases)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.hs_resolve_rows_noalloc(g_descs, len(cases), torch.cuda.current_stream().cuda_stream)
    assert status == 0, lib.hs_last_error()
    for step in range(3):
        _lib.check(lib.hs_resolve_rows_batched(ref_descs, len(cases), ws.data_ptr(), need,
                                               _lib.stream_handle(torch.device(gpu))), "hs_resolve_rows_batched")
        graph.replay()
        torch.cuda.synchronize()
        for (t0, _, o0), (t1, _, o1) in zip(ref, cap):
            for name in ("phys", "uphys", "mh", "md", "counts"):
                assert torch.equal(o0[name], o1[name]), (step, name)
            assert torch.equal(t0["tags"], t1["tags"]) and torch.equal(t0["lru"], t1["lru"]), step
    assert int(cap[0][2]["counts"][1]) > 0  # later steps hit the rows the first one loaded
