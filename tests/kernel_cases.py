"""Seeded input generators shared by the kernel parity tests (CPU tensors)."""

from __future__ import annotations

from math import ceil
from types import SimpleNamespace

import numpy as np
import torch


def cfg(page_size, kv_heads, head_dim):
    return SimpleNamespace(page_size=page_size, kv_heads=kv_heads, head_dim=head_dim)


def make_pool(blocks, page_size, kv_heads, head_dim, dtype, seed, outliers=False):
    gen = torch.Generator().manual_seed(seed)
    pool = torch.randn(blocks, 2, page_size, kv_heads, head_dim, generator=gen)
    if outliers:
        # 2% of channels scaled x8 (the microbench's K/V shape)
        channels = max(1, round(0.02 * head_dim))
        idx = torch.randperm(head_dim, generator=gen)[:channels]
        pool[..., idx] *= 8
    return pool.to(dtype)


def random_rows(heads, width, max_row, seed, invalid=0.1):
    gen = torch.Generator().manual_seed(seed)
    rows = torch.randint(0, max_row, (heads, width), generator=gen)
    drop = torch.rand(heads, width, generator=gen) < invalid
    return torch.where(drop, torch.full_like(rows, -1), rows)


def resolver_tables(seed, length, page_size, hot_rows, resident_frac=0.5, tag_frac=0.6,
                    host_pages=None, affine_base=None, foreign_tags=0):
    """Consistent per-(request, layer) tables: injective source, fragmented hot
    blocks, unique tags that cache host rows of non-resident pages.

    ``affine_base``: the source table is ``base + page`` (a request's contiguous host
    slots) with a few host-less pages; ``foreign_tags``: that many empty tag slots
    then hold host rows of blocks outside the request's range (other requests' rows)."""
    rng = np.random.default_rng(seed)
    n_pages = ceil(length / page_size) + int(rng.integers(0, 3))
    host_pages = host_pages or (n_pages * 3 + 7)
    materialized = ceil(length / page_size)
    if affine_base is None:
        source = rng.permutation(host_pages)[:n_pages].astype(np.int32)
    else:
        source = (affine_base + np.arange(n_pages)).astype(np.int32)
        holes = rng.random(n_pages) < 0.03
        holes[0] = False
        source[holes] = -1
    source[materialized:] = -1
    blocks_total = n_pages + ceil(hot_rows / page_size) + 5
    block_perm = rng.permutation(blocks_total)
    resident = np.full(n_pages, -1, np.int32)
    is_res = rng.random(n_pages) < resident_frac
    is_res[materialized:] = False
    resident[is_res] = block_perm[: is_res.sum()]
    hot_blocks = ceil(hot_rows / page_size)
    hot = block_perm[is_res.sum() : is_res.sum() + hot_blocks].astype(np.int32)
    # tags: unique host rows of non-resident materialized pages
    candidates = [
        int(source[p]) * page_size + o
        for p in range(materialized)
        if resident[p] < 0
        for o in range(page_size)
        if p * page_size + o < length
    ]
    tags = np.full(hot_rows, -1, np.int32)
    k = min(len(candidates), int(tag_frac * hot_rows))
    if k:
        chosen = rng.choice(len(candidates), size=k, replace=False)
        slots = rng.choice(hot_rows, size=k, replace=False)
        tags[slots] = np.asarray(candidates, dtype=np.int64)[chosen]
    if foreign_tags:
        free = np.flatnonzero(tags < 0)[:foreign_tags]
        lo_block = int(source[source >= 0].min()) if (source >= 0).any() else 0
        hi_block = int(source.max()) + 1
        for j, slot in enumerate(free):  # blocks just below and just above the request's range
            step = j // page_size
            below = j % 2 == 0 and lo_block - 1 - step >= 0
            block = lo_block - 1 - step if below else hi_block + step
            tags[slot] = block * page_size + j % page_size
    lru = rng.permutation(hot_rows).astype(np.int64)
    return dict(source=source, resident=resident, hot=hot, tags=tags, lru=lru)


def random_positions(seed, n, length, dup=0.05, invalid=0.05):
    rng = np.random.default_rng(seed)
    pos = rng.integers(0, length, size=n)
    d = rng.random(n) < dup
    if d.any() and n > 1:
        pos[d] = pos[rng.integers(0, n, size=d.sum())]
    bad = rng.random(n) < invalid
    pos[bad] = rng.choice([-1, -2, length, length + 5], size=bad.sum())
    return pos.astype(np.int64)


def quest_bounds(seed, pages, page_size, kv_heads, head_dim, dtype, length=None):
    """K pages -> exact per-page min/max in the KV dtype ([pages, Hkv, D])."""
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(pages * page_size, kv_heads, head_dim, generator=gen)
    channels = max(1, round(0.02 * head_dim))
    idx = torch.randperm(head_dim, generator=gen)[:channels]
    k[..., idx] *= 8
    k = k.to(dtype)
    length = length or pages * page_size
    k = k[:length]
    mins, maxs = [], []
    for p in range(pages):
        chunk = k[p * page_size : min((p + 1) * page_size, length)]
        if len(chunk) == 0:
            mins.append(torch.full((kv_heads, head_dim), float("inf")).to(dtype))
            maxs.append(torch.full((kv_heads, head_dim), float("-inf")).to(dtype))
        else:
            mins.append(chunk.amin(0))
            maxs.append(chunk.amax(0))
    return torch.stack(mins), torch.stack(maxs)
