"""Parity of the gfx950 kernels with the CPU oracle on identical seeded inputs.

Integer outputs (resolver, Quest pages, union builder, gather) must be
bit-exact; attention must match the float64 oracle within the north-star
tolerance (2e-2 abs / 1e-2 rel in bf16/fp16, fp32 accumulate) and the
reference's own test tolerances (fp32: 2e-6 / 2e-5, low precision 0.004 / 0.02,
tests/test_hybrid.py:59, :187-189).
"""

from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions
from oracle.union import from_selection as oracle_union, group_entries
from tests.kernel_cases import (
    cfg,
    make_pool,
    quest_bounds,
    random_positions,
    random_rows,
    resolver_tables,
)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _close(actual, expected, atol, rtol):
    actual = actual.detach().cpu().double().numpy()
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    assert (err <= bound).all(), f"max err {err.max():.3g}, worst excess {(err - bound).max():.3g}"


TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2), torch.float32: (2e-6, 2e-5)}


# ----------------------------------------------------------------- attention
@pytest.mark.parametrize(
    "dtype,P,kv,g,D,W,blocks",
    [
        (torch.bfloat16, 16, 8, 8, 128, 300, 64),  # microbench head shape
        (torch.bfloat16, 16, 4, 7, 128, 200, 40),  # Qwen2.5-7B head shape
        (torch.bfloat16, 16, 2, 7, 64, 130, 40),   # Qwen2.5-0.5B head shape
        (torch.float16, 7, 2, 3, 24, 45, 30),      # non-power-of-two page and head_dim
        (torch.bfloat16, 4, 1, 2, 8, 9, 10),
        (torch.float32, 4, 1, 2, 8, 9, 10),        # reference test shape
        (torch.float32, 16, 2, 7, 64, 70, 20),
        (torch.bfloat16, 16, 1, 20, 32, 40, 20),   # more than 16 heads per KV head
    ],
)
def test_attend_rows_matches_oracle(gpu, dtype, P, kv, g, D, W, blocks):
    from mini_hisparse_amd.row_kernels import attend_rows

    heads = kv * g
    pool = make_pool(blocks, P, kv, D, dtype, seed=1, outliers=True)
    q = torch.randn(heads, D, generator=torch.Generator().manual_seed(2)).to(dtype)
    rows = random_rows(heads, W, blocks * P, seed=3)
    expected = oracle.row_attention_rows(q, pool, rows, P)
    actual = attend_rows(q.to(gpu), pool.to(gpu), rows.to(gpu), cfg(P, kv, D))
    assert actual.dtype == dtype and actual.shape == (heads, D)
    _close(actual, expected, *TOL[dtype])
    if dtype != torch.float32:
        _close(actual, expected, 0.004, 0.02)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attend_shared_rows_masks_and_empty_heads(gpu, dtype):
    from mini_hisparse_amd.row_kernels import attend_rows

    P, kv, D, heads, blocks = 16, 2, 64, 8, 12
    pool = make_pool(blocks, P, kv, D, dtype, seed=5)
    q = torch.randn(heads, D, generator=torch.Generator().manual_seed(6)).to(dtype)
    shared = torch.tensor([5, -1, 17, 17, 190, -1, 3])  # duplicate rows count twice, like the reference
    expected = oracle.row_attention_rows(q, pool, shared, P)
    actual = attend_rows(q.to(gpu), pool.to(gpu), shared.to(gpu), cfg(P, kv, D))
    _close(actual, expected, *TOL[dtype])
    masked = torch.full((heads, 5), -1)
    masked[1, 2] = 7
    out = attend_rows(q.to(gpu), pool.to(gpu), masked.to(gpu), cfg(P, kv, D)).cpu()
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2:]) == 0
    _close(out[1:2], oracle.row_attention_rows(q, pool, masked, P)[1:2], *TOL[dtype])


def test_attend_batched_matches_single(gpu):
    from mini_hisparse_amd.row_kernels import attend_rows

    P, kv, g, D, blocks, W = 16, 4, 7, 128, 50, 260
    heads = kv * g
    pool = make_pool(blocks, P, kv, D, torch.bfloat16, seed=8).to(gpu)
    qs = torch.randn(3, heads, D, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(gpu)
    rows = torch.stack([random_rows(heads, W, blocks * P, seed=10 + b) for b in range(3)]).to(gpu)
    batched = attend_rows(qs, pool, rows, cfg(P, kv, D))
    for b in range(3):
        single = attend_rows(qs[b], pool, rows[b], cfg(P, kv, D))
        torch.testing.assert_close(batched[b], single, atol=1e-2, rtol=1e-2)


# ------------------------------------------------------------------ resolver
def _resolve_gpu(gpu, tables, positions, length, page_size, head_columns=None):
    from mini_hisparse_amd.row_index import LogicalTopK, resolve_rows

    t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
    cols = None if head_columns is None else torch.from_numpy(head_columns).to(gpu)
    topk = LogicalTopK(torch.from_numpy(positions).to(gpu), cols)
    plan = resolve_rows(topk, t["source"], t["resident"], t["hot"], t["tags"], t["lru"], length, page_size)
    return plan, t["tags"].cpu().numpy(), t["lru"].cpu().numpy()


def _assert_plan(plan, tags, lru, expected):
    phys, mh, md, counts, tags_after, lru_after = expected
    np.testing.assert_array_equal(plan.physical_rows.cpu().numpy(), phys)
    np.testing.assert_array_equal(plan.miss_host_rows.cpu().numpy(), mh)
    np.testing.assert_array_equal(plan.miss_device_rows.cpu().numpy(), md)
    np.testing.assert_array_equal(plan.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(tags, tags_after)
    np.testing.assert_array_equal(lru, lru_after)


def test_resolver_walkthrough_known_answer(gpu):
    with open(os.path.join(GOLDEN, "index_walkthrough.json")) as f:
        w = json.load(f)
    tables = dict(
        source=np.asarray(w["source_table"], np.int32),
        resident=np.asarray(w["resident_table"], np.int32),
        hot=np.asarray(w["hot_block_table"], np.int32),
        tags=np.asarray(w["tags_before"], np.int32),
        lru=np.asarray([0, 1, 2, 3, 4, 6, 7, 5], np.int64),
    )
    positions = np.asarray(w["logical_tokens"], np.int64)
    plan, tags, lru = _resolve_gpu(gpu, tables, positions, 16, w["page_size"])
    assert plan.physical_rows.tolist() == w["physical_rows"]
    assert plan.miss_host_rows.tolist() == w["miss_host_rows"]
    assert plan.miss_device_rows.tolist() == w["miss_device_rows"]
    c = w["counts"]
    assert plan.counts.tolist() == [c["resident_hits"], c["hot_hits"], c["misses"]]
    assert tags.tolist() == w["tags_after"]
    expected = oracle.resolve_rows(positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], 16, 4)
    _assert_plan(plan, tags, lru, expected)


@pytest.mark.parametrize(
    "seed,length,P,S,n,res_frac",
    [
        (0, 97, 4, 64, 40, 0.5),
        (1, 1000, 16, 512, 300, 0.3),
        (2, 4096, 16, 2048, 1500, 0.5),
        (3, 65536, 16, 32768, 20000, 0.5),
        (4, 131072, 16, 32768, 27808, 0.15),
        (5, 50, 3, 30, 30, 0.0),
        (6, 300, 7, 128, 100, 1.0),
    ],
)
def test_resolver_random_matches_oracle(gpu, seed, length, P, S, n, res_frac):
    tables = resolver_tables(seed, length, P, S, resident_frac=res_frac)
    positions = random_positions(seed + 100, n, length)
    expected = oracle.resolve_rows(positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], length, P)
    plan, tags, lru = _resolve_gpu(gpu, tables, positions, length, P)
    _assert_plan(plan, tags, lru, expected)
    # int32 positions give the same answer
    plan32, tags32, lru32 = _resolve_gpu(gpu, tables, positions.astype(np.int32), length, P)
    _assert_plan(plan32, tags32, lru32, expected)


@pytest.mark.parametrize(
    "seed,length,P,S,n,res_frac,base",
    [
        (30, 97, 4, 64, 40, 0.5, 0),
        (31, 4096, 16, 2048, 1500, 0.5, 1000),
        (32, 131072, 16, 32768, 27808, 0.15, 3 * 8193),  # 7B shape: the fourth request's host slots
        (33, 300, 7, 128, 100, 0.0, 5),
    ],
)
def test_resolver_affine_source_matches_oracle(gpu, seed, length, P, S, n, res_frac, base):
    """Source tables of contiguous host slots (host block = base + page, a few host-less
    pages) take the resolver's subtraction path; tags of other requests' host rows never hit."""
    tables = resolver_tables(seed, length, P, S, resident_frac=res_frac, affine_base=base, foreign_tags=40)
    positions = random_positions(seed + 100, n, length)
    expected = oracle.resolve_rows(positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], length, P)
    plan, tags, lru = _resolve_gpu(gpu, tables, positions, length, P)
    _assert_plan(plan, tags, lru, expected)


@pytest.mark.parametrize("lru_dtype", [torch.int64, torch.int16])
def test_resolver_batched_descriptors_match_oracle(gpu, lru_dtype):
    """hs_resolve_rows_batched over 17 (request, layer) descriptors of different sizes: one
    launch of 16 descriptors and one of 1; every output of every request equals the oracle.
    The LRU in the reference's int64 and in int16 (the batched engine's tables), up to the
    full 32768 hot rows (slot 32767, the largest int16)."""
    from mini_hisparse_amd import _lib

    lib = _lib.load()
    cases = []
    shapes = [(1000, 16, 512, 300), (4096, 16, 2048, 1500), (97, 4, 64, 40), (300, 7, 128, 100),
              (40000, 16, 32768, 9000)]
    for i in range(17):
        length, P, S, n = shapes[i % len(shapes)]
        tables = resolver_tables(50 + i, length, P, S, resident_frac=0.1 * (i % 6))
        positions = random_positions(150 + i, n, length)
        cases.append((length, P, tables, positions))
    descs = (_lib.ResolveDesc * len(cases))()
    keep, total = [], 0
    for d, (length, P, tables, positions) in zip(descs, cases):
        t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
        t["lru"] = t["lru"].to(lru_dtype)
        pos = torch.from_numpy(positions).to(gpu)
        n = pos.numel()
        out = {name: torch.full((n,), -7, dtype=torch.int64, device=gpu) for name in ("phys", "uphys", "mh", "md")}
        out["counts"] = torch.empty(3, dtype=torch.int64, device=gpu)
        d.positions, d.n, d.positions_i64 = pos.data_ptr(), n, 1
        d.source, d.resident, d.n_pages = t["source"].data_ptr(), t["resident"].data_ptr(), t["source"].numel()
        d.hot, d.hot_blocks = t["hot"].data_ptr(), t["hot"].numel()
        d.tags, d.lru, d.hot_rows = t["tags"].data_ptr(), t["lru"].data_ptr(), t["tags"].numel()
        d.lru_i16 = int(lru_dtype == torch.int16)
        d.miss_prefix_only = len(keep) % 2  # every other descriptor: the plan's prefix only
        d.length, d.page_size = length, P
        d.physical, d.union_physical = out["phys"].data_ptr(), out["uphys"].data_ptr()
        d.miss_host_rows, d.miss_device_rows = out["mh"].data_ptr(), out["md"].data_ptr()
        d.counts = out["counts"].data_ptr()
        total += lib.hs_resolve_workspace_bytes(n, length, d.n_pages, d.hot_rows)
        keep.append((t, pos, out))
    ws = torch.empty(total, dtype=torch.uint8, device=gpu)
    _lib.check(lib.hs_resolve_rows_batched(descs, len(cases), ws.data_ptr(), total,
                                           _lib.stream_handle(torch.device(gpu))), "hs_resolve_rows_batched")
    torch.cuda.synchronize()
    for i, ((length, P, tables, positions), (t, _, out)) in enumerate(zip(cases, keep)):
        phys, mh, md, counts, tags_after, lru_after = oracle.resolve_rows(
            positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], length, P)
        case = f"descriptor {i}: length {length}, page {P}, hot rows {tables['tags'].size}"
        np.testing.assert_array_equal(out["phys"].cpu().numpy(), phys, err_msg=case)
        if i % 2:  # miss_prefix_only: the compact prefix, and the -1 tail left unwritten
            m = int(counts[2])
            np.testing.assert_array_equal(out["mh"][:m].cpu().numpy(), mh[:m], err_msg=case)
            np.testing.assert_array_equal(out["md"][:m].cpu().numpy(), md[:m], err_msg=case)
            assert (out["mh"][m:] == -7).all() and (out["md"][m:] == -7).all(), case
        else:
            np.testing.assert_array_equal(out["mh"].cpu().numpy(), mh, err_msg=case)
            np.testing.assert_array_equal(out["md"].cpu().numpy(), md, err_msg=case)
        np.testing.assert_array_equal(out["counts"].cpu().numpy(), counts, err_msg=case)
        np.testing.assert_array_equal(t["tags"].cpu().numpy(), tags_after, err_msg=case)
        np.testing.assert_array_equal(t["lru"].cpu().numpy(), lru_after, err_msg=case)


@pytest.mark.parametrize("affine", [False, True])
def test_resolver_page_bits_matches_oracle(gpu, affine):
    """Positions that are the tokens of a page set (the union builder's output, padded with
    -1 to a capacity) resolved from the page bitmap (hs_resolve_desc.page_bits, no position
    read in the front) and from the positions: both equal the oracle, int16 LRU."""
    from mini_hisparse_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(31)
    for length, P, S, sel in [(5000, 16, 2048, 60), (131072, 16, 32768, 1700), (999, 7, 512, 40), (64, 4, 64, 16)]:
        count = -(-length // P)
        tables = resolver_tables(int(rng.integers(1 << 30)), length, P, S, resident_frac=0.3,
                                 affine_base=1000 if affine else None)
        pages = np.unique(np.append(rng.choice(count, size=min(sel, count), replace=False), count - 1))
        union = np.asarray(pages_to_positions(pages[None, :], length, P)[0], np.int32)
        cap = len(union) + 37
        positions = np.full(cap, -1, np.int32)
        positions[: len(union)] = union
        words = -(-count // 32)
        marked = np.zeros(words * 32, bool)
        marked[pages] = True
        bits = np.packbits(marked.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").reshape(-1).astype(np.uint32)
        expected = oracle.resolve_rows(positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")],
                                       length, P)
        for use_bits in (True, False):
            t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
            t["lru"] = t["lru"].to(torch.int16)
            pos = torch.from_numpy(positions).to(gpu)
            bits_d = torch.from_numpy(bits.view(np.int32)).to(gpu)
            out = {name: torch.empty(cap, dtype=torch.int64, device=gpu) for name in ("phys", "mh", "md")}
            out["counts"] = torch.empty(3, dtype=torch.int64, device=gpu)
            d = _lib.ResolveDesc()
            d.positions, d.n, d.positions_i64 = pos.data_ptr(), cap, 0
            d.page_bits = bits_d.data_ptr() if use_bits else None
            d.source, d.resident, d.n_pages = t["source"].data_ptr(), t["resident"].data_ptr(), t["source"].numel()
            d.hot, d.hot_blocks = t["hot"].data_ptr(), t["hot"].numel()
            d.tags, d.lru, d.hot_rows, d.lru_i16 = t["tags"].data_ptr(), t["lru"].data_ptr(), S, 1
            d.length, d.page_size = length, P
            d.physical = d.union_physical = out["phys"].data_ptr()
            d.miss_host_rows, d.miss_device_rows = out["mh"].data_ptr(), out["md"].data_ptr()
            d.counts = out["counts"].data_ptr()
            need = lib.hs_resolve_workspace_bytes(cap, length, d.n_pages, S)
            ws = torch.empty(need, dtype=torch.uint8, device=gpu)
            _lib.check(lib.hs_resolve_rows(d, ws.data_ptr(), need, _lib.stream_handle(torch.device(gpu))),
                       "hs_resolve_rows")
            torch.cuda.synchronize()
            case = f"length {length}, page {P}, hot rows {S}, page bits {use_bits}"
            for got, want in ((out["phys"], expected[0]), (out["mh"], expected[1]), (out["md"], expected[2]),
                              (out["counts"], expected[3]), (t["tags"], expected[4]), (t["lru"], expected[5])):
                np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=case)


def test_resolver_head_columns_and_multistep_trajectory(gpu):
    from mini_hisparse_amd.row_index import LogicalTopK, resolve_rows

    length, P, S = 3000, 16, 1024
    tables = resolver_tables(11, length, P, S, resident_frac=0.4, tag_frac=0.3)
    gpu_t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
    cpu_tags, cpu_lru = tables["tags"].copy(), tables["lru"].copy()
    rng = np.random.default_rng(12)
    for step in range(6):
        heads, width = 6, 64
        sel = [sorted(set(rng.integers(0, length, size=width).tolist())) for _ in range(heads)]
        union, columns = oracle_union(sel)
        expected = oracle.resolve_rows(union, tables["source"], tables["resident"], tables["hot"], cpu_tags, cpu_lru, length, P, head_columns=columns)
        topk = LogicalTopK(torch.from_numpy(union.astype(np.int32)).to(gpu), torch.from_numpy(columns).to(gpu))
        plan = resolve_rows(topk, gpu_t["source"], gpu_t["resident"], gpu_t["hot"], gpu_t["tags"], gpu_t["lru"], length, P)
        _assert_plan(plan, gpu_t["tags"].cpu().numpy(), gpu_t["lru"].cpu().numpy(), expected)
        cpu_tags, cpu_lru = expected[4], expected[5]


def test_resolver_row_stats_accumulate(gpu):
    from mini_hisparse_amd.row_index import LogicalTopK, resolve_rows

    tables = resolver_tables(21, 500, 4, 200)
    positions = random_positions(22, 120, 500)
    expected = oracle.resolve_rows(positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], 500, 4)
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
    stats = torch.tensor([10, 20, 30], dtype=torch.int64, device=gpu)
    resolve_rows(LogicalTopK(torch.from_numpy(positions).to(gpu)), t["source"], t["resident"], t["hot"], t["tags"], t["lru"], 500, 4, row_stats=stats)
    assert stats.tolist() == [10 + int(expected[3][0]), 20 + int(expected[3][1]), 30 + int(expected[3][2])]


# --------------------------------------------------------------------- Quest
@pytest.mark.parametrize(
    "dtype,pages,P,kv,g,D,top,sink,length",
    [
        (torch.bfloat16, 300, 16, 2, 4, 64, 16, True, None),
        (torch.bfloat16, 4096, 16, 8, 8, 128, 64, True, None),  # microbench shape
        (torch.bfloat16, 8193, 16, 4, 7, 128, 64, True, 131073),  # 7B shape at 128k (+1 decoded token)
        (torch.bfloat16, 1000, 16, 4, 7, 128, 64, False, 15990),
        (torch.float16, 77, 7, 2, 3, 24, 5, True, 535),
        (torch.float32, 90, 4, 1, 2, 8, 7, True, 357),
        (torch.bfloat16, 10, 16, 2, 2, 32, 12, True, 150),  # top >= count: every page
        (torch.bfloat16, 50, 16, 2, 2, 32, 1, True, None),  # top == 1: tail only
        (torch.bfloat16, 40, 16, 2, 3, 20, 6, True, None),  # D not a multiple of 8: strided scorer
        (torch.bfloat16, 64, 16, 16, 1, 256, 8, True, None),  # query tile above the LDS limit
        (torch.bfloat16, 120, 16, 1, 12, 64, 9, True, None),  # two head chunks per KV head
        (torch.float16, 20000, 16, 1, 2, 32, 64, True, None),  # keys beyond the LDS key buffer
    ],
)
def test_quest_pages_match_oracle(gpu, dtype, pages, P, kv, g, D, top, sink, length):
    from mini_hisparse_amd.selection import quest_selection

    length = length or pages * P
    lo, hi = quest_bounds(7, pages, P, kv, D, dtype, length)
    q = torch.randn(kv * g, D, generator=torch.Generator().manual_seed(8)).to(dtype)
    expected = oracle.quest_pages(q, lo, hi, length, P, top, keep_sink=sink)
    sel = quest_selection(q.to(gpu), lo.to(gpu), hi.to(gpu), length, P, top, keep_sink=sink)
    k = expected.shape[1]
    np.testing.assert_array_equal(sel.device_pages[:, :k].cpu().numpy(), expected)
    assert sel.positions == pages_to_positions(expected, length, P)


@pytest.mark.parametrize(
    "q_dtype,counts,kv,g,D",
    [
        (torch.bfloat16, [4096, 4000], 8, 8, 128),  # microbench geometry, a ragged second request
        (torch.bfloat16, [8193], 4, 7, 128),  # 7B geometry: 28 q heads, 4 KV heads
        (torch.float32, [1000, 129], 4, 7, 128),  # fp32 queries: multiply, then add
        (torch.bfloat16, [2048, 300, 77], 2, 7, 64),  # 0.5B geometry
        (torch.float32, [300], 1, 12, 64),  # two head chunks per KV head
        (torch.bfloat16, [130], 3, 5, 40),  # D = 40: five 16-byte units per row
    ],
)
def test_quest_scores_bit_exact(gpu, q_dtype, counts, kv, g, D):
    """Every page score in the scorer's workspace equals the oracle's float32 sum bit for bit
    (bf16 bounds), with exact zeros and -0 among the query values."""
    from mini_hisparse_amd import _lib

    lib = _lib.load()
    P, B, heads = 16, len(counts), kv * g
    bounds = [quest_bounds(11 + i, c, P, kv, D, torch.bfloat16) for i, c in enumerate(counts)]
    q = torch.randn(B, heads, D, generator=torch.Generator().manual_seed(12)).to(q_dtype)
    q[:, :, 3] = 0.0
    q[:, :, 5] = -0.0
    lo = [b[0].to(gpu) for b in bounds]
    hi = [b[1].to(gpu) for b in bounds]
    qg = q.to(gpu)
    ws_bytes = lib.hs_quest_workspace_bytes(B, heads, max(counts))
    ws = torch.full((ws_bytes // 4,), float("nan"), dtype=torch.float32, device=gpu)
    pages = torch.empty((B, heads, 1), dtype=torch.int32, device=gpu)
    ptrs = ctypes.c_void_p * B
    status = lib.hs_quest_topk(
        qg.data_ptr(), qg.stride(0), qg.stride(1), _lib.dtype_code(q_dtype),
        ptrs(*[t.data_ptr() for t in lo]), ptrs(*[t.data_ptr() for t in hi]), _lib.dtype_code(torch.bfloat16),
        (ctypes.c_int64 * B)(*counts), B, heads, kv, D, 1, 1, pages.data_ptr(), pages.stride(0),
        ws.data_ptr(), ws_bytes, _lib.stream_handle(gpu))
    _lib.check(status, "hs_quest_topk")
    scores = ws[: B * heads * max(counts)].view(B, heads, max(counts)).cpu().numpy()
    for i, c in enumerate(counts):
        expected = oracle.quest_scores(q[i], bounds[i][0], bounds[i][1], c)
        np.testing.assert_array_equal(scores[i, :, :c].view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("pages,top,sink", [(2049, 32, True), (4096, 64, True), (300, 300 - 1, False), (65, 64, True),
                                             (4097, 32, True), (2048, 1, True), (1000, 7, False),
                                             (16384, 64, True), (16385, 64, False), (3000, 65, True)])
def test_quest_topk_with_many_ties_matches_oracle(gpu, pages, top, sink):
    """Bounds and queries of small integers, so that many pages score exactly alike: the
    radix select's pages equal the oracle's, ties taken from the lowest page (16384 pages
    keep the keys in LDS; one more reads them from the scores)."""
    from mini_hisparse_amd.selection import quest_selection

    P, kv, g, D = 16, 2, 7, 64
    length = pages * P
    gen = torch.Generator().manual_seed(pages + top)
    lo = torch.randint(-2, 1, (pages, kv, D), generator=gen).to(torch.bfloat16)
    hi = lo + torch.randint(0, 2, (pages, kv, D), generator=gen).to(torch.bfloat16)
    q = torch.randint(-1, 2, (kv * g, D), generator=gen).to(torch.bfloat16)
    expected = oracle.quest_pages(q, lo, hi, length, P, top, keep_sink=sink)
    sel = quest_selection(q.to(gpu), lo.to(gpu), hi.to(gpu), length, P, top, keep_sink=sink)
    np.testing.assert_array_equal(sel.device_pages[:, : expected.shape[1]].cpu().numpy(), expected)


def test_quest_reference_known_answer(gpu):
    """tests/test_selection.py:33-47 of the reference: pages [0, 2], not the mean's page 1."""
    from mini_hisparse_amd.selection import quest_selection

    k = torch.tensor([[[10.0, 0.0]], [[-10.0, 0.0]], [[1.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]])
    lo = torch.stack([k[0:2].amin(0), k[2:4].amin(0), k[4:5].amin(0)])
    hi = torch.stack([k[0:2].amax(0), k[2:4].amax(0), k[4:5].amax(0)])
    sel = quest_selection(torch.tensor([[1.0, 0.0]], device=gpu), lo.to(gpu), hi.to(gpu), 5, 2, 2, keep_sink=False)
    assert sel.pages == [0, 2]


# -------------------------------------------------------------- union builder
@pytest.mark.parametrize(
    "pages,P,kv,g,top,length",
    [
        (300, 16, 2, 4, 16, None),
        (77, 7, 2, 3, 5, 535),
        (10, 16, 2, 2, 12, 150),
        (4096, 16, 8, 8, 64, None),
        (2000, 16, 1, 8, 600, None),  # a group selects > 4096 pages: head masks by binary search
        (30000, 16, 2, 2, 8, None),  # history beyond the LDS rank -> page map: per-page writes
    ],
)
def test_union_builder_matches_host_adapter(gpu, pages, P, kv, g, top, length):
    from mini_hisparse_amd.selection import quest_selection

    length = length or pages * P
    lo, hi = quest_bounds(17, pages, P, kv, 32, torch.bfloat16, length)
    q = torch.randn(kv * g, 32, generator=torch.Generator().manual_seed(18)).to(torch.bfloat16)
    sel = quest_selection(q.to(gpu), lo.to(gpu), hi.to(gpu), length, P, top)
    topk = sel.logical_topk(torch.device(gpu))
    union, columns = oracle_union(sel.positions)
    n = int(topk.union_count.item())
    assert n == len(union)
    pos = topk.positions.cpu().numpy()
    np.testing.assert_array_equal(pos[:n], union)
    assert (pos[n:] == -1).all()
    hc = topk.head_columns.cpu().numpy()
    np.testing.assert_array_equal(hc[:, : columns.shape[1]], columns)
    assert (hc[:, columns.shape[1] :] == -1).all()
    groups = group_entries(columns, kv)
    counts = topk.entries.counts.cpu().numpy()
    for k, (cols, masks) in enumerate(groups):
        assert counts[k] == len(cols)
        np.testing.assert_array_equal(topk.entries.columns[k, : len(cols)].cpu().numpy(), cols)
        np.testing.assert_array_equal(topk.entries.masks[k, : len(cols)].cpu().numpy().astype(np.int64), masks)


# --------------------------------------------------------------------- gather
# rows of 2 KB and 1 KB (one row plane per wave instruction), 256, 128 and 8 bytes (a wave
# instruction reads one plane of 4, 8 and 64 consecutive entries), 32 bytes (2 units) and 96
# bytes (6 units, not a divisor of the wave: per-row mapping)
@pytest.mark.parametrize("dtype,P,kv,D", [(torch.bfloat16, 16, 8, 128), (torch.float32, 4, 1, 8), (torch.float16, 7, 2, 24),
                                          (torch.bfloat16, 16, 4, 128), (torch.bfloat16, 16, 2, 64),
                                          (torch.bfloat16, 16, 1, 64), (torch.float16, 3, 1, 4)])
def test_gather_copies_planned_rows(gpu, dtype, P, kv, D):
    from mini_hisparse_amd.row_index import RowPlan
    from mini_hisparse_amd.row_kernels import MappedHost, gather_rows

    host_blocks, dev_blocks = 40, 30
    host = make_pool(host_blocks, P, kv, D, dtype, seed=31).pin_memory()
    pool_cpu = make_pool(dev_blocks, P, kv, D, dtype, seed=32)
    rng = np.random.default_rng(33)
    m = 57
    hrows = rng.choice(host_blocks * P, size=m, replace=False)
    drows = rng.choice(dev_blocks * P, size=m, replace=False)
    hplan = np.full(m + 20, -1, np.int64)
    dplan = np.full(m + 20, -1, np.int64)
    hplan[:m], dplan[:m] = hrows, drows
    expected = pool_cpu.clone()
    oracle.gather_rows(host, expected, hplan, dplan, P)
    pool = pool_cpu.to(gpu)
    plan = RowPlan(None, torch.from_numpy(hplan).to(gpu), torch.from_numpy(dplan).to(gpu), None)
    gather_rows(MappedHost(host), pool, plan, cfg(P, kv, D))
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu(), expected)


def test_gather_full_size_rows_equal_host_rows(gpu):
    """BASELINE configs[1] scale (one request: 4096 host pages of 4 KB rows, ~8k misses): every
    planned device row holds its host row afterwards and no other device row changes."""
    from mini_hisparse_amd.row_index import RowPlan
    from mini_hisparse_amd.row_kernels import MappedHost, gather_rows

    P, kv, D = 16, 8, 128
    host_blocks, dev_blocks, m = 4096, 1024, 8000
    gen = torch.Generator(device=gpu).manual_seed(5)
    host_dev = torch.randn((host_blocks, 2, P, kv, D), generator=gen, device=gpu).to(torch.bfloat16)
    host = torch.empty(host_dev.shape, dtype=torch.bfloat16, pin_memory=True)
    host.copy_(host_dev)
    pool = torch.randn((dev_blocks, 2, P, kv, D), generator=gen, device=gpu).to(torch.bfloat16)
    before = pool.clone()
    rng = np.random.default_rng(6)
    hrows = torch.from_numpy(rng.choice(host_blocks * P, size=m, replace=False)).to(gpu)
    drows = torch.from_numpy(rng.choice(dev_blocks * P, size=m, replace=False)).to(gpu)
    pad = torch.full((100,), -1, dtype=torch.int64, device=gpu)
    plan = RowPlan(None, torch.cat((hrows, pad)), torch.cat((drows, pad)), None)
    gather_rows(MappedHost(host), pool, plan, cfg(P, kv, D))
    torch.cuda.synchronize()
    got = pool[drows // P, :, drows % P]
    want = host_dev[hrows // P, :, hrows % P]
    assert torch.equal(got, want)
    untouched = torch.ones(dev_blocks * P, dtype=torch.bool, device=gpu)
    untouched[drows] = False
    rows = torch.nonzero(untouched).flatten()
    assert torch.equal(pool[rows // P, :, rows % P], before[rows // P, :, rows % P])


# ---------------------------------------------- group attention = row attention
@pytest.mark.parametrize(
    "P,kv,g,D,pages,top",
    [
        (16, 8, 8, 128, 512, 64),
        (16, 4, 7, 128, 300, 32),
        (7, 2, 3, 24, 60, 6),
        (16, 8, 8, 128, 4096, 64),  # one request of the microbench
        (16, 4, 7, 128, 8192, 64),  # one (request, layer) of the 7B shape at 128k
    ],
)
def test_group_attention_matches_per_head_rows(gpu, P, kv, g, D, pages, top):
    from mini_hisparse_amd.row_index import resolve_rows
    from mini_hisparse_amd.row_kernels import attend_groups, attend_rows
    from mini_hisparse_amd.selection import quest_selection

    length = pages * P - 3
    heads = kv * g
    lo, hi = quest_bounds(41, pages, P, kv, D, torch.bfloat16, length)
    q = torch.randn(heads, D, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16).to(gpu)
    sel = quest_selection(q, lo.to(gpu), hi.to(gpu), length, P, top)
    topk = sel.logical_topk(torch.device(gpu))
    # every page resident at block = page, so physical rows are the logical tokens
    resident = torch.arange(pages, dtype=torch.int32, device=gpu)
    source = torch.arange(pages, dtype=torch.int32, device=gpu)
    hot = torch.zeros(1, dtype=torch.int32, device=gpu)
    tags = torch.full((P,), -1, dtype=torch.int32, device=gpu)
    lru = torch.arange(P, dtype=torch.int64, device=gpu)
    plan = resolve_rows(topk, source, resident, hot, tags, lru, length, P)
    pool = make_pool(pages, P, kv, D, torch.bfloat16, seed=43, outliers=True).to(gpu)
    c = cfg(P, kv, D)
    by_rows = attend_rows(q, pool, plan.physical_rows, c)
    by_groups = attend_groups(q, pool, plan.union_physical, topk.entries, c)
    expected = oracle.row_attention_rows(q.cpu(), pool.cpu(), plan.physical_rows.cpu(), P)
    _close(by_rows, expected, 2e-2, 1e-2)
    _close(by_groups, expected, 2e-2, 1e-2)


def _group_rows_oracle(union_physical, cols, masks, counts, capacity, kv, g):
    """Per-head physical row lists [B, Hq, W] (-1 padded) that the entry lists
    encode: head kv*g + i reads entry e < clamp(count, 0, capacity) when bit i of
    its mask is set and its column is valid."""
    B = counts.shape[0]
    n = np.clip(counts, 0, capacity)
    lists = [[[] for _ in range(kv * g)] for _ in range(B)]
    for b in range(B):
        for k in range(kv):
            c = cols[b, k, : n[b, k]]
            m = masks[b, k, : n[b, k]].astype(np.uint32)
            ok = c >= 0
            phys = np.where(ok, union_physical[b, np.clip(c, 0, None)], -1)
            for i in range(g):
                sel = ok & ((m >> np.uint32(i)) & 1).astype(bool)
                lists[b][k * g + i] = phys[sel]
    W = max(1, max(len(r) for req in lists for r in req))
    rows = np.full((B, kv * g, W), -1, np.int64)
    for b in range(B):
        for h, r in enumerate(lists[b]):
            rows[b, h, : len(r)] = r
    return rows


@pytest.mark.parametrize(
    "name,B,kv,g,D,capacity,counts",
    [
        # ragged lists: empty, one entry, around the 32-entry tile and the chunk sizes,
        # above the capacity (clamped) and negative (empty)
        ("ragged", 5, 3, 5, 128, 5000,
         [0, 1, 31, 32, 33, 127, 128, 129, 500, 2047, 2048, 2049, 5007, -3, 3000]),
        ("two-head-chunks", 3, 2, 20, 64, 3000, [2999, 17, 1500, 0, 2200, 800]),
        ("several-rounds", 40, 8, 2, 32, 2100, None),  # > 256 workgroups of ACH entries
        ("all-empty", 2, 4, 8, 128, 64, [0] * 8),
        ("many-groups", 520, 8, 1, 32, 40, None),  # > 4096 groups: always the split schedule
    ],
)
@pytest.mark.parametrize("merge", ["in-kernel", "launch"])
@pytest.mark.parametrize("schedule", ["split", "balanced"])
def test_group_attention_schedule_matches_oracle(gpu, monkeypatch, schedule, merge, name, B, kv, g, D, capacity,
                                                 counts):
    """hs_attend_groups over synthetic entry lists of very different lengths, with
    the default split schedule and the device-derived balanced one (HS_ATTEND_SCHED=1),
    each with the last workgroup's merge and with the merge launch
    (HS_ATTEND_FUSED_MERGE=1 / 0; both read per call), against the per-head oracle."""
    monkeypatch.setenv("HS_ATTEND_SCHED", "1" if schedule == "balanced" else "0")
    monkeypatch.setenv("HS_ATTEND_FUSED_MERGE", "1" if merge == "in-kernel" else "0")
    from mini_hisparse_amd.row_index import GroupEntries
    from mini_hisparse_amd.row_kernels import attend_groups

    P, blocks, U = 16, 96, 700
    rng = np.random.default_rng(B * 1000 + g)
    if counts is None:
        low = 1500 if name == "several-rounds" else 0
        counts = rng.integers(low, capacity + 1, size=B * kv)
    counts = np.asarray(counts, np.int64).reshape(B, kv)
    union_physical = rng.integers(0, blocks * P, size=(B, U))
    union_physical[rng.random((B, U)) < 0.05] = -1
    cols = rng.integers(0, U, size=(B, kv, capacity)).astype(np.int32)
    cols[rng.random(cols.shape) < 0.03] = -1
    masks = rng.integers(0, 1 << g, size=(B, kv, capacity)).astype(np.int64)
    masks[rng.random(masks.shape) < 0.02] = 0
    masks = masks.astype(np.uint32).view(np.int32)
    pool = make_pool(blocks, P, kv, D, torch.bfloat16, seed=B + g, outliers=True)
    q = torch.randn(B, kv * g, D, generator=torch.Generator().manual_seed(g)).to(torch.bfloat16)
    entries = GroupEntries(
        torch.from_numpy(cols).to(gpu), torch.from_numpy(masks).to(gpu),
        torch.from_numpy(counts.astype(np.int32)).to(gpu), capacity,
    )
    got = attend_groups(q.to(gpu), pool.to(gpu), torch.from_numpy(union_physical).to(gpu), entries, cfg(P, kv, D))
    rows = _group_rows_oracle(union_physical, cols, masks.view(np.uint32), counts, capacity, kv, g)
    for b in range(B):
        expected = oracle.row_attention_rows(q[b], pool, rows[b], P)
        _close(got[b], expected, 2e-2, 1e-2)
    if name == "all-empty":
        assert not got.any()


def _group_case(gpu, B=6, kv=4, g=7, D=128, capacity=3000, seed=11):
    from mini_hisparse_amd.row_index import GroupEntries

    P, blocks, U = 16, 96, 900
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, capacity + 1, size=(B, kv))
    union_physical = rng.integers(0, blocks * P, size=(B, U))
    cols = rng.integers(0, U, size=(B, kv, capacity)).astype(np.int32)
    masks = rng.integers(1, 1 << g, size=(B, kv, capacity)).astype(np.uint32).view(np.int32)
    pool = make_pool(blocks, P, kv, D, torch.bfloat16, seed=seed, outliers=True).to(gpu)
    q = torch.randn(B, kv * g, D, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(gpu)
    entries = GroupEntries(torch.from_numpy(cols).to(gpu), torch.from_numpy(masks).to(gpu),
                           torch.from_numpy(counts.astype(np.int32)).to(gpu), capacity)
    return q, pool, torch.from_numpy(union_physical).to(gpu), entries, cfg(P, kv, D)


def test_in_kernel_merge_starts_from_any_workspace_contents(gpu, monkeypatch):
    """The arrival counters live in the caller's workspace, which may hold anything
    (uninitialised memory, another launch's counters): every launch gives the same
    output as the merge launch, whatever the workspace held before it."""
    from mini_hisparse_amd import row_kernels
    from mini_hisparse_amd.row_kernels import attend_groups

    case = _group_case(gpu)
    monkeypatch.setenv("HS_ATTEND_FUSED_MERGE", "0")
    want = attend_groups(*case)
    monkeypatch.setenv("HS_ATTEND_FUSED_MERGE", "1")
    gen = torch.Generator(device=gpu).manual_seed(3)
    for fill in ("random", "ones", "zeros", "same"):
        ws = row_kernels._ATTEND_WS[(torch.device(gpu), torch.cuda.current_stream(gpu).cuda_stream)]
        if fill == "random":
            ws.copy_(torch.randint(0, 256, ws.shape, generator=gen, device=gpu, dtype=torch.int32).to(torch.uint8))
        elif fill == "ones":
            ws.fill_(0xFF)
        elif fill == "zeros":
            ws.zero_()
        got = attend_groups(*case)
        torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_in_kernel_merge_replays_from_a_captured_graph(gpu, monkeypatch):
    """A captured attention replays with the epoch (and partial-word tag) of its
    capture: the last workgroup clears its group's counter and the partial words it
    merged, so every replay (with eager launches of other epochs between them, and a
    new query each time) merges this replay's partials exactly once per group."""
    from mini_hisparse_amd.row_kernels import attend_groups

    monkeypatch.setenv("HS_ATTEND_FUSED_MERGE", "1")
    case = _group_case(gpu)
    q = case[0]
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        attend_groups(*case)  # workspace of the capture stream
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = attend_groups(*case)
    gen = torch.Generator().manual_seed(99)
    for _ in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))  # the graph reads q in place
        eager = attend_groups(*case)  # another workspace, another epoch
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, eager, rtol=0, atol=0)


# ------------------------------------------------------- page-window attention
@pytest.mark.parametrize(
    "dtype,P,kv,g,D,n_pages,masked",
    [
        (torch.bfloat16, 16, 8, 8, 128, 4, True),   # microbench head shape
        (torch.bfloat16, 16, 4, 7, 128, 64, False),  # Qwen2.5-7B head shape, a wide window
        (torch.float16, 7, 2, 3, 24, 5, True),      # non-power-of-two page and head_dim
        (torch.bfloat16, 16, 1, 20, 32, 3, True),   # more than 16 heads per KV head
        (torch.float32, 4, 2, 2, 8, 2, True),       # reference test shape (VALU kernel)
        (torch.float32, 16, 2, 7, 64, 9, False),
    ],
)
def test_attend_window_matches_oracle(gpu, dtype, P, kv, g, D, n_pages, masked):
    from mini_hisparse_amd.row_kernels import attend_window

    heads, blocks = kv * g, 3 * n_pages + 2
    pool = make_pool(blocks, P, kv, D, dtype, seed=n_pages, outliers=True)
    q = torch.randn(heads, D, generator=torch.Generator().manual_seed(D)).to(dtype)
    gen = torch.Generator().manual_seed(P * 7 + g)
    slots = torch.randperm(blocks, generator=gen)[:n_pages].to(torch.int32)
    lengths = torch.full((n_pages,), P, dtype=torch.int32)
    lengths[-1] = max(1, P // 3)  # a partial tail page
    mask = None
    if masked:
        mask = torch.rand((heads, n_pages, P), generator=gen) < 0.5
        mask[0] = False  # a head that reads nothing: (-inf, 0, 0)
    m, l, acc = attend_window(q.to(gpu), pool.to(gpu), slots.to(gpu), lengths.to(gpu),
                              None if mask is None else mask.to(gpu), cfg(P, kv, D))
    em, el, eacc = oracle.window_state(q, pool, slots, lengths, mask, P)
    got_m, got_l, got_acc = (x.cpu().double().numpy() for x in (m, l, acc))
    reads = np.isfinite(em)
    assert (np.isfinite(got_m) == reads).all()
    assert (got_l[~reads] == 0).all() and (got_acc[~reads] == 0).all()
    # the state's scale is free (exp(s - m)); compare the normalised output and m
    atol, rtol = TOL[dtype]
    np.testing.assert_allclose(got_m[reads], em[reads], rtol=1e-3 if dtype != torch.float32 else 1e-6, atol=1e-3)
    out = got_acc[reads] / got_l[reads][:, None]
    want = eacc[reads] / el[reads][:, None]
    err = np.abs(out - want)
    assert (err <= atol + rtol * np.abs(want)).all(), err.max()


# --------------------------------------------------------------------- append
def _bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_append_rows_match_oracle_and_torch_bounds(gpu, dtype):
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import MappedHost, append_rows

    P, Hkv, D, B = 16, 4, 64, 5
    cfg = CacheConfig(gpu_pages=12, host_pages=20, page_size=P, kv_heads=Hkv, head_dim=D, device=gpu, dtype=dtype)
    g = torch.Generator().manual_seed(21)
    pool = torch.randn(12, 2, P, Hkv, D, generator=g).to(dtype)
    host = torch.randn(20, 2, P, Hkv, D, generator=g).to(dtype).pin_memory()
    k = torch.randn(B, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, D, generator=g).to(dtype)
    lo = torch.randn(B, Hkv, D, generator=g).to(dtype)
    hi = lo + torch.rand(B, Hkv, D, generator=g).to(dtype)
    # NaNs and equal signed zeros on both sides
    k[0, 0, :4] = float("nan")
    lo[1, 0, :4] = float("nan")
    hi[1, 1, :4] = float("nan")
    k[2, 0, :8] = -0.0
    lo[2, 0, :8] = 0.0
    hi[2, 0, :8] = 0.0
    k[3, 1, :8] = 0.0
    lo[3, 1, :8] = -0.0
    hi[3, 1, :8] = -0.0
    device_rows, host_rows = [0 * P + 3, 5 * P + 15, 7 * P, 11 * P + 8, 2 * P + 1], [19 * P + 2, -1, 4 * P + 9, 0, 13 * P]
    # expected in bit space: rows are copied; a bound keeps its bits or takes the new
    # element's bits where the oracle's torch.minimum/maximum rule picks the new one
    exp_pool, exp_host = _bits(pool).copy(), _bits(host).copy()
    kb, vb, lob, hib = _bits(k), _bits(v), _bits(lo).copy(), _bits(hi).copy()
    for b in range(B):
        db, do = divmod(device_rows[b], P)
        exp_pool[db, 0, do], exp_pool[db, 1, do] = kb[b], vb[b]
        if host_rows[b] >= 0:
            hb, ho = divmod(host_rows[b], P)
            exp_host[hb, 0, ho], exp_host[hb, 1, ho] = kb[b], vb[b]
        kf, bits = k[b].float().numpy(), 8 * k.element_size()
        lob[b] = np.where(oracle.takes_new_min(lo[b].float().numpy(), kf, bits), kb[b], lob[b])
        hib[b] = np.where(oracle.takes_new_max(hi[b].float().numpy(), kf, bits), kb[b], hib[b])
    torch_lo, torch_hi = torch.minimum(lo.to(gpu), k.to(gpu)), torch.maximum(hi.to(gpu), k.to(gpu))
    dpool, dlo, dhi = pool.to(gpu), lo.to(gpu), hi.to(gpu)
    append_rows(k.to(gpu), v.to(gpu), dpool, device_rows, list(dlo), list(dhi), cfg, host=MappedHost(host), host_rows=host_rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(dpool), exp_pool)
    np.testing.assert_array_equal(_bits(host), exp_host)
    np.testing.assert_array_equal(_bits(dlo), lob)
    np.testing.assert_array_equal(_bits(dhi), hib)
    # the reference's own device ops, bit for bit (NaN payloads and zero signs included)
    np.testing.assert_array_equal(_bits(dlo), _bits(torch_lo))
    np.testing.assert_array_equal(_bits(dhi), _bits(torch_hi))


def test_append_fills_a_page_to_its_extrema(gpu):
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import append_rows

    P, Hkv, D = 16, 8, 128
    cfg = CacheConfig(gpu_pages=4, host_pages=4, page_size=P, kv_heads=Hkv, head_dim=D, device=gpu, dtype=torch.bfloat16)
    keys = torch.randn(P, Hkv, D, device=gpu).to(torch.bfloat16)
    vals = torch.randn(P, Hkv, D, device=gpu).to(torch.bfloat16)
    pool = torch.zeros(4, 2, P, Hkv, D, dtype=torch.bfloat16, device=gpu)
    lo = torch.full((Hkv, D), float("inf"), dtype=torch.bfloat16, device=gpu)
    hi = torch.full((Hkv, D), float("-inf"), dtype=torch.bfloat16, device=gpu)
    for t in range(P):
        append_rows(keys[t : t + 1].contiguous(), vals[t : t + 1].contiguous(), pool, [3 * P + t], [lo], [hi], cfg)
    torch.testing.assert_close(lo, keys.amin(0), rtol=0, atol=0)
    torch.testing.assert_close(hi, keys.amax(0), rtol=0, atol=0)
    torch.testing.assert_close(pool[3, 0], keys, rtol=0, atol=0)
    torch.testing.assert_close(pool[3, 1], vals, rtol=0, atol=0)
    assert not pool[:3].any()


def test_append_rejects_rows_outside_the_pool(gpu):
    from mini_hisparse_amd._lib import HipLibraryError
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import append_rows

    cfg = CacheConfig(gpu_pages=2, host_pages=2, page_size=16, kv_heads=2, head_dim=64, device=gpu, dtype=torch.bfloat16)
    pool = torch.zeros(2, 2, 16, 2, 64, dtype=torch.bfloat16, device=gpu)
    kv = torch.zeros(1, 2, 64, dtype=torch.bfloat16, device=gpu)
    bound = torch.zeros(2, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(HipLibraryError, match="outside the pool"):
        append_rows(kv, kv, pool, [32], [bound], [bound], cfg)


def test_row_read_probe_covers_the_attention_entries(gpu):
    """The diagnostic read probe gets one K offset per group-attention entry, stays inside
    the pool and leaves it untouched."""
    from mini_hisparse_amd.batched import BatchedSparseDecode, LayerTablesView
    from mini_hisparse_amd.config import CacheConfig

    P, Hkv, g, D, pages, top = 16, 2, 4, 64, 64, 8
    cfg = CacheConfig(gpu_pages=pages, host_pages=pages, page_size=P, kv_heads=Hkv, head_dim=D, device=gpu, dtype=torch.bfloat16)
    L = pages * P
    k = torch.randn(pages, P, Hkv, D, device=gpu).to(torch.bfloat16)
    dec = BatchedSparseDecode(cfg, Hkv * g, top, [L], device=gpu)
    dec.select(torch.randn(1, Hkv * g, D, device=gpu).to(torch.bfloat16), [k.amin(1)], [k.amax(1)])
    pool = torch.randn(pages, 2, P, Hkv, D, device=gpu).to(torch.bfloat16)
    resident = torch.arange(pages, dtype=torch.int32, device=gpu)
    table = LayerTablesView(resident.clone(), resident, torch.zeros(1, dtype=torch.int32, device=gpu),
                            torch.full((P,), -1, dtype=torch.int32, device=gpu), torch.arange(P, device=gpu))
    dec.resolve([table])
    before = pool.clone()
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    offsets = dec.entry_offsets(pool)
    assert offsets.numel() == int(dec.entry_counts.sum()) > 0
    assert int(offsets.max()) + D * 2 + P * Hkv * D * 2 <= pool.numel() * 2
    dec.probe_reads(pool, offsets, sink)
    torch.cuda.synchronize()
    assert torch.equal(pool, before)


# ------------------------------------------------------------- batched write (append)
@pytest.mark.parametrize(
    "dtype,P,kv,D,start,tokens",
    [
        (torch.bfloat16, 16, 4, 128, 5, 1),       # a decode token in the middle of a page
        (torch.bfloat16, 16, 4, 128, 0, 16 * 70 + 3),  # a prefill of 71 pages: two launches of 64 pages
        (torch.bfloat16, 16, 2, 64, 13, 40),      # starts 3 rows before a page boundary
        (torch.float16, 7, 2, 24, 3, 30),         # 96-byte rows
        (torch.float32, 4, 1, 8, 2, 11),          # the reference tests' shape
        (torch.bfloat16, 3, 1, 6, 1, 9),          # 12-byte rows: the 2-byte copy path
    ],
)
def test_append_tokens_matches_oracle(gpu, dtype, P, kv, D, start, tokens):
    from mini_hisparse_amd.row_kernels import MappedHost, append_tokens

    pages_total = (start + tokens + P - 1) // P + 2
    first, within = divmod(start, P)
    write_pages = (within + tokens + P - 1) // P
    rng = np.random.default_rng(start * 1000 + tokens)
    blocks, host_blocks = write_pages + 5, pages_total + 9
    slots = rng.permutation(blocks)[:write_pages].astype(np.int64)
    slots[rng.random(write_pages) < 0.3] = -1  # pages the policy did not keep resident
    host_slots = rng.permutation(host_blocks)[:write_pages].astype(np.int64)
    if within:
        slots[0] = max(int(slots[0]), 0)  # an existing tail page is resident
    pool = make_pool(blocks, P, kv, D, dtype, seed=71)
    host = make_pool(host_blocks, P, kv, D, dtype, seed=72)
    if within:  # the tail's earlier rows sit in its block and in its host slot alike
        host[host_slots[0], :, :within] = pool[slots[0], :, :within]
    gen = torch.Generator().manual_seed(73)
    k = torch.randn(tokens, kv, D, generator=gen).to(dtype)
    v = torch.randn(tokens, kv, D, generator=gen).to(dtype)
    lo = torch.full((pages_total, kv, D), float("inf")).to(dtype)
    hi = torch.full((pages_total, kv, D), float("-inf")).to(dtype)
    if within:
        lo[first] = pool[slots[0], 0, :within].amin(0)
        hi[first] = pool[slots[0], 0, :within].amax(0)
    summ = torch.zeros(pages_total, kv, D)
    expected = [x.clone() for x in (pool, host, lo, hi, summ)]
    oracle.append_tokens(expected[0], expected[1], k, v, first, within, slots.tolist(), host_slots.tolist(),
                         expected[2], expected[3], expected[4], P, 32 if dtype == torch.float32 else 16)
    host_pinned = host.pin_memory()
    pool_d, lo_d, hi_d, summ_d = (x.to(gpu) for x in (pool, lo, hi, summ))
    append_tokens(k.to(gpu), v.to(gpu), first, within, slots.tolist(), host_slots.tolist(), pool_d,
                  MappedHost(host_pinned), lo_d, hi_d, summ_d, cfg(P, kv, D))
    torch.cuda.synchronize()
    assert torch.equal(pool_d.cpu(), expected[0])
    assert torch.equal(host_pinned, expected[1])
    assert torch.equal(lo_d.cpu(), expected[2]) and torch.equal(hi_d.cpu(), expected[3])
    assert torch.equal(summ_d.cpu(), expected[4])
