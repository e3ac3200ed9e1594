"""One-token append (test infrastructure only).

Restates the single-token case of ``HostStore.append``
(``mini_hisparse/storage.py:246-319``) for a batch of (request, layer) pairs:

* the new K and V rows are written to pool row ``d`` (block ``d // P``,
  offset ``d % P``) of a ``[blocks, 2, P, Hkv, D]`` pool (``storage.py:287-288``);
* the tail page's bounds become ``torch.minimum(minimum, k)`` and
  ``torch.maximum(maximum, k)`` (``storage.py:291-297``; with one new row,
  ``amin``/``amax`` over the new rows is the row itself).  torch's element rule
  on the device (where the reference's cache lives) is restated exactly as
  measured on MI355X (``takes_new_min``); ``numpy.minimum`` differs from it on
  signed zeros, so it is not used;
* the rows are mirrored to host row ``h`` when ``h >= 0`` (``storage.py:301-308``).
"""

from __future__ import annotations

import numpy as np


def takes_new_min(old, new, dtype_bits=16):
    """Where torch.minimum(old, new) on the device returns the new element.

    Rule measured on MI355X (PyTorch-ROCm) for the cache dtypes: a NaN operand
    is returned (the existing bound first); otherwise, for 16-bit floats,
    ``old < new ? old : new`` (an equal compare -- including +0 vs -0 --
    returns the new element); for float32, IEEE minimum with -0 below +0.
    """
    old, new = np.asarray(old, np.float64), np.asarray(new, np.float64)
    if dtype_bits == 16:
        ordered = ~(old < new)
    else:
        ordered = (new < old) | ((new == old) & np.signbit(new) & ~np.signbit(old))
    return ~np.isnan(old) & (np.isnan(new) | ordered)


def takes_new_max(old, new, dtype_bits=16):
    """Where torch.maximum(old, new) on the device returns the new element (same rule,
    mirrored: 16-bit ``old > new ? old : new``; float32 IEEE maximum with +0 above -0)."""
    old, new = np.asarray(old, np.float64), np.asarray(new, np.float64)
    if dtype_bits == 16:
        ordered = ~(old > new)
    else:
        ordered = (new > old) | ((new == old) & ~np.signbit(new) & np.signbit(old))
    return ~np.isnan(old) & (np.isnan(new) | ordered)


def bound_min(old, new, dtype_bits=16):
    """torch.minimum(old, new) element rule (see ``takes_new_min``)."""
    return np.where(takes_new_min(old, new, dtype_bits), new, old)


def bound_max(old, new, dtype_bits=16):
    """torch.maximum(old, new) element rule (see ``takes_new_max``)."""
    return np.where(takes_new_max(old, new, dtype_bits), new, old)


def append_rows(pool, host, k, v, device_rows, host_rows, minimum, maximum, page_size, dtype_bits=16):
    """In place on float/uint views: pool/host [blocks, 2, P, Hkv, D]; k, v [B, Hkv, D];
    minimum/maximum: per pair, the tail page's [Hkv, D] bounds (lists of arrays);
    ``dtype_bits`` the cache dtype's width (16 or 32) for the bound rule."""
    for b, d in enumerate(device_rows):
        db, do = divmod(int(d), page_size)
        pool[db, 0, do] = k[b]
        pool[db, 1, do] = v[b]
        h = int(host_rows[b]) if host_rows is not None else -1
        if h >= 0:
            hb, ho = divmod(h, page_size)
            host[hb, 0, ho] = k[b]
            host[hb, 1, ho] = v[b]
        minimum[b][...] = bound_min(minimum[b], k[b], dtype_bits)
        maximum[b][...] = bound_max(maximum[b], k[b], dtype_bits)
    return pool, host, minimum, maximum


def append_tokens(pool, host, k, v, first_page, first_within, slots, host_slots, minimum, maximum, summaries,
                  page_size, dtype_bits=16):
    """A write of ``T`` consecutive tokens to one (request, layer) (the page loop of
    ``HostStore.append``, ``mini_hisparse/storage.py:273-318``), on CPU torch tensors.

    Token ``t`` goes to page ``first_page + j`` of the write's pages (the first page
    starts at row ``first_within``, the others at row 0); page ``j`` sits in device
    block ``slots[j]`` (``< 0``: not resident, no pool write) and host slot
    ``host_slots[j]``.  Per page:

    * K and V rows are written to the pool block (when resident) and to the host
      slot (the mirror, ``storage.py:300-308``);
    * the bounds fold the new K rows in order, ``b = rule(b, row)`` with torch's
      device ``minimum``/``maximum`` rule (``takes_new_min``): for rows without NaN
      or equal signed zeros this is ``min(old, amin(rows))`` of ``storage.py:291-297``;
    * the summary is the float32 mean of all the page's valid K rows (the rows
      before ``first_within`` are read back from the host slot), summed in row
      order then divided (``storage.py:290``).
    """
    import torch

    tokens, t = len(k), 0
    for j, (slot, hslot) in enumerate(zip(slots, host_slots)):
        index = first_page + j
        within = first_within if j == 0 else 0
        count = min(page_size - within, tokens - t)
        rows_k, rows_v = k[t : t + count], v[t : t + count]
        if slot >= 0:
            pool[slot, 0, within : within + count] = rows_k
            pool[slot, 1, within : within + count] = rows_v
        host[hslot, 0, within : within + count] = rows_k
        host[hslot, 1, within : within + count] = rows_v
        lo = minimum[index].float().numpy().astype(np.float64)
        hi = maximum[index].float().numpy().astype(np.float64)
        for r in range(count):
            row = rows_k[r].float().numpy().astype(np.float64)
            lo = bound_min(lo, row, dtype_bits)
            hi = bound_max(hi, row, dtype_bits)
        minimum[index] = torch.from_numpy(lo).to(minimum.dtype)
        maximum[index] = torch.from_numpy(hi).to(maximum.dtype)
        valid = within + count
        acc = np.zeros(host.shape[3:], np.float32)
        for r in range(valid):
            acc = (acc + host[hslot, 0, r].float().numpy()).astype(np.float32)
        summaries[index] = torch.from_numpy((acc / np.float32(valid)).astype(np.float32))
        t += count
