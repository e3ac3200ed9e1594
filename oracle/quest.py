"""numpy restatement of the Quest page scorer and per-head top-k (test infrastructure only).

Follows ``mini_hisparse/selection.py:80-101``.  Two orders that the reference
leaves to torch are fixed here, and the HIP kernel follows the same rules:

* the float32 score of (query head h, page p) is the sum over channels d in
  ascending order, ``s = s + max(q_d * lo_d, q_d * hi_d)``, one float32
  rounding per step (the reference's ``.sum(-1)`` order is torch's);
* the top-k keeps the ``top`` largest scores, ties broken by the lower page
  index (``torch.topk`` leaves ties unspecified).

For bf16 and fp16 inputs every product is exact in float32, so the score
differs from the reference's only by summation order; equal chosen sets are
expected whenever the k-th/(k+1)-th score margin exceeds that rounding.
"""

from __future__ import annotations

from math import ceil

import numpy as np


def _f32(x):
    """float32 view of a numpy array or a (CPU) torch tensor of any float dtype."""
    if hasattr(x, "detach"):
        x = x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float32)


def quest_scores(query, minimum, maximum, count):
    """``[Hq, count]`` float32 page upper bounds, sequential-channel order."""
    q = _f32(query)
    lo = _f32(minimum)[:count]
    hi = _f32(maximum)[:count]
    heads, dim = q.shape
    kv_heads = lo.shape[1]
    groups = heads // kv_heads
    kv_of = np.arange(heads) // groups
    lo_h = lo[:, kv_of, :].transpose(1, 0, 2)  # [Hq, C, D]
    hi_h = hi[:, kv_of, :].transpose(1, 0, 2)
    scores = np.zeros((heads, count), dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for d in range(dim):
            qd = q[:, d : d + 1]
            term = np.maximum(qd * lo_h[:, :, d], qd * hi_h[:, :, d])
            scores = (scores + term).astype(np.float32)
    return scores


def quest_pages(query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
    """Chosen logical pages per query head, each row ascending (``[Hq, k]`` int64).

    Mirrors selection.py:86-101: all pages when ``top >= count``; otherwise
    the tail page and (if ``keep_sink and top > 1 and count > 1``) page 0
    are forced with +inf scores.
    """
    count = ceil(length / page_size)
    heads = _f32(query).shape[0]
    kv_heads = _f32(minimum).shape[1]
    if top_pages < 1 or heads % kv_heads:
        raise ValueError("invalid page budget or GQA shape")
    if top_pages >= count:
        return np.tile(np.arange(count, dtype=np.int64), (heads, 1))
    scores = quest_scores(query, minimum, maximum, count)
    required = [count - 1]
    if keep_sink and top_pages > 1 and count > 1:
        required.append(0)
    scores[:, required] = np.inf
    index = np.arange(count)
    chosen = np.empty((heads, top_pages), dtype=np.int64)
    for h in range(heads):
        order = np.lexsort((index, -scores[h].astype(np.float64)))
        chosen[h] = np.sort(order[:top_pages])
    return chosen


def pages_to_positions(pages, length, page_size):
    """Selection.from_pages canonicalisation (selection.py:43-60, 30-39): per head, the
    sorted token set of its pages clipped to ``length``."""
    rows = []
    for row in pages.tolist() if hasattr(pages, "tolist") else pages:
        tokens = sorted(
            {t for p in row for t in range(p * page_size, min((p + 1) * page_size, length))}
        )
        rows.append(tuple(tokens))
    return tuple(rows)


def quest_selection_positions(
    query, minimum, maximum, length, page_size, top_pages, keep_sink=True
):
    """Per-head canonical token tuples, i.e. ``quest_selection(...).positions``."""
    pages = quest_pages(query, minimum, maximum, length, page_size, top_pages, keep_sink)
    return pages_to_positions(pages, length, page_size)
