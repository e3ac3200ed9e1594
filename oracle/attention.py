"""Physical-row GQA decode attention, float64 reference (test infrastructure only).

* ``row_attention_rows`` restates the torch branch of ``row_attention``
  (``mini_hisparse/attention.py:26-35``) and the masking rules of the Triton
  ``_attend`` (``row_kernels.py:90-113``): query head h reads KV head
  ``h // (Hq / Hkv)``; rows ``< 0`` are masked; ``s = (K . q) * D**-0.5``;
  softmax over the unmasked rows; output 0 when every row is masked.
* ``window_state`` restates the page-window kernel of the reference's paged
  layout (``reference/kernels.py:12-68``, and ``_torch_chunk`` of
  ``reference/attention.py:21-37``): the unnormalised state (m, l, acc) of
  each head over the valid, unmasked tokens of a window of whole pages.
* ``dense_attention`` restates ``selection.py:158-163``.
* ``selection_oracle`` restates the sparse output of ``selection.py:104-126``.

Everything is computed in float64 from the stored values and returned as a
float64 numpy array; callers cast to the query dtype.
"""

from __future__ import annotations

import numpy as np


def _f64(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def _softmax_weighted(scores, valid, values):
    """scores [H, N], valid [H, N] bool, values [H, N, D] -> [H, D]; 0 where no row is valid."""
    s = np.where(valid, scores, -np.inf)
    top = s.max(axis=1, keepdims=True)
    top = np.where(np.isfinite(top), top, 0.0)
    w = np.where(valid, np.exp(s - top), 0.0)
    denom = w.sum(axis=1, keepdims=True)
    out = (w[..., None] * values).sum(axis=1)
    return np.where(denom > 0, out / np.where(denom > 0, denom, 1.0), 0.0)


def row_attention_rows(query, pool, rows, page_size):
    """query [Hq, D]; pool [blocks, 2, P, Hkv, D]; rows [Hq, W] or [W] (shared) -> [Hq, D] float64."""
    q = _f64(query)
    rows = np.asarray(rows.cpu() if hasattr(rows, "cpu") else rows, dtype=np.int64)
    heads, dim = q.shape
    kv_heads = pool.shape[3]
    if rows.ndim == 1:
        rows = np.broadcast_to(rows[None, :], (heads, rows.size))
    kv_of = np.arange(heads) // (heads // kv_heads)
    safe = np.clip(rows, 0, None)
    blocks, offsets = safe // page_size, safe % page_size
    if hasattr(pool, "detach"):  # gather in the storage dtype first, then widen
        import torch

        bi, oi, ki = (torch.from_numpy(np.array(x, dtype=np.int64)) for x in (blocks, offsets, np.broadcast_to(kv_of[:, None], blocks.shape)))
        k = _f64(pool[bi, 0, oi, ki])  # [Hq, W, D]
        v = _f64(pool[bi, 1, oi, ki])
    else:
        pool = np.asarray(pool, dtype=np.float64)
        k = pool[blocks, 0, offsets, kv_of[:, None]]
        v = pool[blocks, 1, offsets, kv_of[:, None]]
    scores = (k * q[:, None, :]).sum(-1) * dim**-0.5
    return _softmax_weighted(scores, rows >= 0, v)


def window_state(query, pool, slots, lengths, mask, page_size):
    """One window of whole pages (reference/kernels.py:12-68).

    query [Hq, D]; pool [blocks, 2, P, Hkv, D]; page i of the window is device
    slot ``slots[i]`` with ``lengths[i]`` valid tokens; ``mask`` [Hq, N, P]
    bool or None (every valid token).  Returns float64 (m [Hq], l [Hq],
    acc [Hq, D]): m = the largest valid score (-inf if none), l = sum of
    exp(s - m), acc = sum of exp(s - m) V (both 0 when the head reads nothing),
    with s = (K . q) * D**-0.5.
    """
    slots = np.asarray(slots.cpu() if hasattr(slots, "cpu") else slots, dtype=np.int64)
    lengths = np.asarray(lengths.cpu() if hasattr(lengths, "cpu") else lengths, dtype=np.int64)
    q = _f64(query)
    heads, dim = q.shape
    kv_heads = pool.shape[3]
    t = np.arange(page_size)
    rows = np.where(t[None, :] < lengths[:, None], slots[:, None] * page_size + t[None, :], -1).reshape(-1)
    valid = np.broadcast_to(rows >= 0, (heads, rows.size))
    if mask is not None:
        m = np.asarray(mask.cpu() if hasattr(mask, "cpu") else mask, dtype=bool).reshape(heads, -1)
        valid = valid & m
    kv_of = np.arange(heads) // (heads // kv_heads)
    safe = np.clip(rows, 0, None)
    blocks, offsets = safe // page_size, safe % page_size
    if hasattr(pool, "detach"):
        import torch

        bi = torch.from_numpy(np.broadcast_to(blocks[None, :], valid.shape).copy())
        oi = torch.from_numpy(np.broadcast_to(offsets[None, :], valid.shape).copy())
        ki = torch.from_numpy(np.broadcast_to(kv_of[:, None], valid.shape).copy())
        k, v = _f64(pool[bi, 0, oi, ki]), _f64(pool[bi, 1, oi, ki])  # [Hq, N*P, D]
    else:
        pool = np.asarray(pool, dtype=np.float64)
        k = pool[blocks[None, :], 0, offsets[None, :], kv_of[:, None]]
        v = pool[blocks[None, :], 1, offsets[None, :], kv_of[:, None]]
    scores = np.where(valid, (k * q[:, None, :]).sum(-1) * dim**-0.5, -np.inf)
    top = scores.max(axis=1)
    shift = np.where(np.isfinite(top), top, 0.0)
    w = np.where(valid, np.exp(scores - shift[:, None]), 0.0)
    return top, w.sum(axis=1), (w[..., None] * v).sum(axis=1)


def attend_rows(query, pool, rows, page_size):
    """Alias with the product's argument order (query, pool, rows)."""
    return row_attention_rows(query, pool, rows, page_size)


def dense_attention(query, k, v):
    """query [Hq, D], k/v [T, Hkv, D] -> [Hq, D] float64 softmax attention over all T."""
    q, k, v = _f64(query), _f64(k), _f64(v)
    heads, dim = q.shape
    groups = heads // k.shape[1]
    k = np.repeat(k, groups, axis=1).transpose(1, 0, 2)  # [Hq, T, D]
    v = np.repeat(v, groups, axis=1).transpose(1, 0, 2)
    scores = (k * q[:, None, :]).sum(-1) / np.sqrt(dim)
    return _softmax_weighted(scores, np.ones(scores.shape, dtype=bool), v)


def selection_oracle(query, k, v, positions):
    """Sparse attention of each head over its own token set ``positions[h]``."""
    q, k, v = _f64(query), _f64(k), _f64(v)
    heads, dim = q.shape
    groups = heads // k.shape[1]
    k = np.repeat(k, groups, axis=1).transpose(1, 0, 2)
    v = np.repeat(v, groups, axis=1).transpose(1, 0, 2)
    scores = (k * q[:, None, :]).sum(-1) / np.sqrt(dim)
    mask = np.zeros(scores.shape, dtype=bool)
    for h, row in enumerate(positions):
        mask[h, list(row)] = True
    return _softmax_weighted(scores, mask, v)
