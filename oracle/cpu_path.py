"""The reference's CPU decode path for one (request, layer), as torch CPU ops -- BENCH
INFRASTRUCTURE ONLY.

``bench.py``'s ``cpu_baseline`` leg times this: what the reference runs for a
(request, layer) when its cache lives on the CPU (``device="cpu"``, torch backend).
It is never the product and never a checker of the product's kernels (the
numpy modules of this package are); its steps follow the reference's own calls:

* ``quest_select``  -- ``quest_selection`` (``mini_hisparse/selection.py:80-101``):
  the bound scores as the reference's torch expression over every page and
  channel at once, the forced sink/tail pages, ``topk``, then
  ``Selection.from_pages`` (``selection.py:43-60``): each head's tokens.
* ``union_columns`` -- ``LogicalTopK.from_selection`` (``row_index.py:20-31``),
  the Python union and head columns (``oracle.union.from_selection``).
* the resolver     -- ``oracle.resolve_rows`` (``row_index.py:59-137``).
* ``gather_loop``   -- the CPU branch of ``HybridKVCache.resolve``
  (``hybrid.py:466-472``): one ``copy_`` per missed row.
* ``row_attention`` -- the torch branch of ``row_attention``
  (``attention.py:26-35``) over the selected rows.
"""

from __future__ import annotations

from math import ceil

import numpy as np
import torch

from .resolver import resolve_rows
from .union import from_selection


def quest_select(query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
    """Per-head token tuples of the Quest selection (selection.py:80-101, 43-60)."""
    count = ceil(length / page_size)
    heads = query.shape[0]
    if top_pages >= count:
        chosen = [list(range(count))] * heads
    else:
        groups = heads // minimum.shape[1]
        low = minimum[:count].repeat_interleave(groups, 1).transpose(0, 1).float()
        high = maximum[:count].repeat_interleave(groups, 1).transpose(0, 1).float()
        scores = torch.maximum(query.float()[:, None] * low, query.float()[:, None] * high).sum(-1)
        required = [count - 1]
        if keep_sink and top_pages > 1 and count > 1:
            required.append(0)
        scores[:, required] = torch.inf
        chosen = scores.topk(top_pages, dim=-1).indices.tolist()
    positions = []
    for pages in chosen:
        tokens = set()
        for page in pages:
            tokens.update(range(page * page_size, min((page + 1) * page_size, length)))
        positions.append(tuple(sorted(tokens)))
    return positions


def union_columns(positions):
    """(union int64 [n], head columns int64 [H, W]) of LogicalTopK.from_selection."""
    return from_selection(positions)


def resolve(union, columns, source, resident, hot, tags, lru, length, page_size):
    """RowPlan of row_index.py:59-137 (tags and lru updated in place)."""
    phys, miss_host, miss_dev, counts, tags1, lru1 = resolve_rows(
        union, source, resident, hot, tags, lru, length, page_size, head_columns=columns)
    tags[:] = tags1
    lru[:] = lru1
    return phys, miss_host, miss_dev, counts


def gather_loop(host, pool, miss_host, miss_dev, page_size):
    """The reference's CPU gather: one row copy per planned miss (hybrid.py:466-472).
    Returns the rows copied."""
    copied = 0
    for h, d in zip(miss_host.tolist(), miss_dev.tolist()):
        if h >= 0:
            hb, ho = divmod(h, page_size)
            db, do = divmod(d, page_size)
            pool[db, :, do].copy_(host[hb, :, ho])
            copied += 1
    return copied


def row_attention(query, pool, rows, page_size, kv_heads, head_dim):
    """The torch branch of row_attention (attention.py:26-35) over physical rows [Hq, W]."""
    rows = torch.as_tensor(rows)
    if rows.ndim == 1:
        rows = rows[None, :].expand(query.shape[0], -1)
    safe = rows.clamp(min=0)
    blocks, offsets = safe // page_size, safe % page_size
    head = torch.arange(query.shape[0])
    kv_head = head // (query.shape[0] // kv_heads)
    k = pool[blocks, 0, offsets, kv_head[:, None]].float()
    v = pool[blocks, 1, offsets, kv_head[:, None]].float()
    v = torch.where((rows >= 0)[..., None], v, 0.0)
    scores = (k * query.float()[:, None]).sum(-1) * head_dim**-0.5
    weights = scores.masked_fill(rows < 0, -torch.inf).softmax(-1).nan_to_num()
    return (weights[..., None] * v).sum(1).to(query.dtype)


def host_rows(positions, source, page_size):
    """Host rows [H, W] (-1 padded) of each head's selected tokens: where the K/V of a
    selected token lives in the host pool (``source[page] * P + offset``)."""
    width = max(len(p) for p in positions)
    rows = np.full((len(positions), width), -1, dtype=np.int64)
    for h, p in enumerate(positions):
        t = np.asarray(p, dtype=np.int64)
        rows[h, : t.size] = source[t // page_size].astype(np.int64) * page_size + t % page_size
    return rows
