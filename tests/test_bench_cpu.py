"""CPU checks of bench.py's CPU legs (no GPU): the all-cores CPU baseline runs each
request of a step in its own spawned process on the numpy oracle and returns outputs
that match the sequential oracle's."""

import os
import sys
import types

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402
import oracle  # noqa: E402
from oracle.quest import pages_to_positions  # noqa: E402


def test_all_cores_cpu_baseline_matches_sequential_oracle():
    from mini_hisparse_amd.batched import LayerTablesView

    B, C, P, Hkv, g, D, top, hot_rows = 3, 40, 16, 2, 4, 64, 6, 256
    L = C * P - 5
    gen = torch.Generator().manual_seed(0)
    host = torch.randn(B * C, 2, P, Hkv, D, generator=gen).to(torch.bfloat16)
    blocks = 8 + B * (hot_rows // P)
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, Hkv * g, D, generator=gen).to(torch.bfloat16)
    kmin = [host[b * C : (b + 1) * C, 0].amin(1) for b in range(B)]
    kmax = [host[b * C : (b + 1) * C, 0].amax(1) for b in range(B)]
    tables = []
    for b in range(B):
        resident = torch.full((C,), -1, dtype=torch.int32)
        resident[C - 1] = b  # the tail page
        hot = torch.arange(8 + b * (hot_rows // P), 8 + (b + 1) * (hot_rows // P), dtype=torch.int32)
        tables.append(LayerTablesView(torch.arange(b * C, (b + 1) * C, dtype=torch.int32), resident, hot, None, None))
    tags0 = torch.full((B, hot_rows), -1, dtype=torch.int32)
    lru0 = torch.arange(hot_rows, dtype=torch.int64).repeat(B, 1)
    expected, sequential_pool = [], pool.clone()
    for b in range(B):
        pages = oracle.quest_pages(q[b], kmin[b], kmax[b], L, P, top)
        union, cols = oracle.from_selection(pages_to_positions(pages, L, P))
        t = tables[b]
        phys, mh, md, _, _, _ = oracle.resolve_rows(
            union, t.source.numpy(), t.resident.numpy(), t.hot.numpy(), tags0[b].numpy().copy(),
            lru0[b].numpy().copy(), L, P, head_columns=cols,
        )
        assert (mh >= 0).sum() > 0  # the step gathers rows
        oracle.gather_rows(host, sequential_pool, mh, md, P)
        expected.append(oracle.row_attention_rows(q[b], sequential_pool, phys, P))
    # the GPU output stands in as the oracle's own, rounded to bf16
    w = dict(
        shape=types.SimpleNamespace(page_size=P, top=top), dec=types.SimpleNamespace(batch=B), host=host,
        pool=pool, q=q, kmin=kmin, kmax=kmax, tables=tables, tags0=tags0, lru0=lru0,
        out=torch.from_numpy(np.stack(expected)).to(torch.bfloat16), length=L,
    )
    result = bench.cpu_baseline_all_cores(torch, w, max_workers=2)
    assert result["cores"] == 2 and result["value"] > 0
    assert result["sample"].endswith("True")
