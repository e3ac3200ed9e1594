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


def test_reference_cpu_path_of_one_request_layer():
    """The model workloads' CPU leg (oracle.cpu_path via bench._sparse_path): its Quest
    selection equals the numpy oracle's, its gather loop copies exactly the planned misses,
    and its row attention over the selected rows equals the float64 oracle's."""
    from oracle import cpu_path

    C, P, Hkv, g, D, top, hot_rows = 64, 16, 2, 4, 32, 8, 512
    L = C * P - 3
    gen = torch.Generator().manual_seed(3)
    host = torch.randn(C, 2, P, Hkv, D, generator=gen).to(torch.bfloat16)
    host[-1, :, L - (C - 1) * P:] = 0
    lo, hi = host[:, 0].amin(1), host[:, 0].amax(1)
    lo[-1], hi[-1] = host[-1, 0, : L - (C - 1) * P].amin(0), host[-1, 0, : L - (C - 1) * P].amax(0)
    q = torch.randn(Hkv * g, D, generator=gen).to(torch.bfloat16)
    positions = cpu_path.quest_select(q, lo, hi, L, P, top)
    assert list(positions) == list(pages_to_positions(oracle.quest_pages(q, lo, hi, L, P, top), L, P))
    resident = np.full(C, -1, np.int32)
    resident[::3] = np.arange(len(resident[::3]))
    i16 = lambda t: t.contiguous().view(torch.int16).numpy()
    x = {"q": i16(q), "lo": i16(lo), "hi": i16(hi), "source": np.arange(C, dtype=np.int64), "resident": resident,
         "tags": np.full(hot_rows, -1, np.int64), "lru": np.arange(hot_rows, dtype=np.int64), "host": i16(host),
         "meta": np.array([L, P, top, Hkv, D, Hkv * g, 0, hot_rows // P, 1], dtype=np.int64)}
    stages, misses = bench._sparse_path(x)
    assert set(stages) == {"select", "union", "resolve", "gather_loop", "attention"}
    union, _ = oracle.from_selection(positions)
    expected_misses = int((resident[union // P] < 0).sum())
    assert misses == expected_misses > 0
    rows = cpu_path.host_rows(positions, x["source"], P)
    out = cpu_path.row_attention(q, host, torch.from_numpy(rows), P, Hkv, D).double().numpy()
    ref = oracle.row_attention_rows(q, host, rows, P)
    np.testing.assert_allclose(out, ref, atol=2e-2, rtol=1e-2)
