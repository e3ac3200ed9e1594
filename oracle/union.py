"""Selection -> (union positions, head columns) adapter (test infrastructure only).

Restates ``LogicalTopK.from_selection`` (``mini_hisparse/row_index.py:20-31``):
the ascending union of every head's tokens, and for each head the union
column of each of its tokens, padded with -1 to the widest head.
"""

from __future__ import annotations

import numpy as np


def from_selection(positions):
    """``positions``: per-head tuples of canonical tokens -> (union int64 [n], columns int64 [H, W])."""
    union = sorted({t for row in positions for t in row})
    column = {t: i for i, t in enumerate(union)}
    width = max(len(row) for row in positions)
    columns = np.full((len(positions), width), -1, dtype=np.int64)
    for h, row in enumerate(positions):
        columns[h, : len(row)] = [column[t] for t in row]
    return np.asarray(union, dtype=np.int64), columns


def group_entries(columns, kv_heads):
    """Per KV head, the union columns any of its query heads reads, ascending,
    with a bit mask of those heads (bit i = head ``kv*g + i``).  This is the
    deduplicated row set the group attention reads once per KV head."""
    columns = np.asarray(columns)
    heads = columns.shape[0]
    groups = heads // kv_heads
    result = []
    for kv in range(kv_heads):
        masks = {}
        for i in range(groups):
            for c in columns[kv * groups + i].tolist():
                if c >= 0:
                    masks[c] = masks.get(c, 0) | (1 << i)
        cols = sorted(masks)
        result.append((np.asarray(cols, dtype=np.int64), np.asarray([masks[c] for c in cols])))
    return result
