"""numpy restatement of the row resolver (test infrastructure only).

Follows ``mini_hisparse/row_index.py:59-137`` step by step.  Every quantity is
int64; the tables are copied, never mutated, and the updated ``tags`` / ``lru``
are returned.

Two places where the reference leaves the order open are fixed here and in the
HIP kernel alike:

* ``tags.sort()`` is unstable; it only matters for equal tags, and equal tags
  are either ``-1`` (never looked up) or forbidden by the cache invariant
  (``hybrid.py:595-596``).  The slot returned for a hit is the slot holding
  that tag.
* ``updates.scatter_`` with repeated indices: repeated destinations only occur
  when misses outnumber the replaceable slots (a caller precondition,
  ``row_index.py:41-42``).  The later miss in sorted-logical order wins, as a
  sequential scatter does.
"""

from __future__ import annotations

import numpy as np


def _i64(x):
    return np.ascontiguousarray(np.asarray(x), dtype=np.int64)


def resolve_rows(
    positions,
    source_table,
    resident_table,
    hot_table,
    tags,
    lru,
    length,
    page_size,
    head_columns=None,
):
    """Return ``(physical, miss_host, miss_device, counts, tags_after, lru_after)``.

    ``physical`` is in input order, or ``[H, W]`` when ``head_columns`` is
    given (row_index.py:127-131).  ``counts`` = (resident hits, hot hits,
    misses) over unique valid tokens (row_index.py:136).
    """
    raw = _i64(positions).reshape(-1)
    source_table = _i64(source_table).reshape(-1)
    resident_table = _i64(resident_table).reshape(-1)
    hot_table = _i64(hot_table).reshape(-1)
    tags = _i64(tags).reshape(-1)
    lru = _i64(lru).reshape(-1)
    n, size, pages = raw.size, tags.size, source_table.size
    if n < 1 or size < 1 or pages < 1:
        raise ValueError("resolver needs nonempty positions, tags and page tables")
    L, P = int(length), int(page_size)

    # 1. normalise, sort, deduplicate (row_index.py:66-71)
    valid_raw = (raw >= 0) & (raw < L)
    normalized = np.where(valid_raw, raw, L)
    logical = np.sort(normalized, kind="stable")
    unique = logical < L
    unique[1:] &= logical[1:] != logical[:-1]

    # 2. address translation and residency (row_index.py:72-80)
    page = np.minimum(logical // P, pages - 1)
    offset = logical % P
    source = source_table[page]
    resident = resident_table[page]
    host = source * P + offset
    valid = unique & (source >= 0)
    resident_hit = valid & (resident >= 0)
    needs_hot = valid & ~resident_hit
    wanted = np.where(needs_hot, host, -1)

    # 3. hot tag lookup (row_index.py:84-87): sort + left search
    tag_slots = np.argsort(tags, kind="stable")
    sorted_tags = tags[tag_slots]
    host32 = host.astype(np.int32).astype(np.int64)
    lookup = np.minimum(np.searchsorted(sorted_tags, host32, side="left"), size - 1)
    hot_hit = needs_hot & (sorted_tags[lookup] == host)
    existing = tag_slots[lookup]

    # 4. protection of every selected hit (row_index.py:88-90)
    sorted_wanted = np.sort(wanted, kind="stable")
    lookup_wanted = np.minimum(np.searchsorted(sorted_wanted, tags, side="left"), n - 1)
    protected = (tags >= 0) & (sorted_wanted[lookup_wanted] == tags)

    # 5. victims: unprotected slots first, each group in LRU order (row_index.py:94-95)
    rank = np.arange(size, dtype=np.int64)
    victims = lru[np.argsort(protected[lru].astype(np.int64) * size + rank, kind="stable")]

    # 6. miss ranks, slots and physical rows (row_index.py:96-103)
    miss = needs_hot & ~hot_hit
    miss_rank = np.cumsum(miss.astype(np.int64)) - 1
    assigned = victims[np.clip(miss_rank, 0, size - 1)]
    slots = np.where(hot_hit, existing, assigned)
    hot_physical = hot_table[slots // P] * P + slots % P
    physical = np.where(resident_hit, resident * P + offset, hot_physical)
    physical = np.where(valid, physical, -1)

    # 7. tag update through a sentinel slot (row_index.py:106-111); sequential
    #    scatter, so a repeated destination keeps the later value
    updates = np.full(size + 1, -1, dtype=np.int64)
    destinations = np.where(miss, assigned, size)
    values = np.where(miss, host32, -1)
    for dst, val in zip(destinations.tolist(), values.tolist()):
        updates[dst] = val
    inserted = updates[:size] >= 0
    tags_after = np.where(inserted, updates[:size], tags)

    # 8. LRU: stable reorder by category 0 untouched, 1 filled, 2 hit (row_index.py:112-113)
    category = inserted.astype(np.int64) + 2 * protected.astype(np.int64)
    lru_after = lru[np.argsort(category[lru] * size + rank, kind="stable")]

    # 9. compact miss plan (row_index.py:115-120)
    host_plan = np.full(n + 1, -1, dtype=np.int64)
    device_plan = np.full(n + 1, -1, dtype=np.int64)
    plan_dst = np.where(miss, miss_rank, n)
    host_plan[plan_dst[miss]] = host[miss]
    device_plan[plan_dst[miss]] = hot_physical[miss]

    # 10. back to input order, first occurrence wins (row_index.py:121-126)
    first = np.minimum(np.searchsorted(logical, normalized, side="left"), n - 1)
    input_rank = np.arange(n, dtype=np.int64)
    first_input = np.full(n, n, dtype=np.int64)
    np.minimum.at(first_input, first, input_rank)
    keep = valid_raw & (input_rank == first_input[first])
    result = np.where(keep, physical[first], -1)

    # 11. per-head remap (row_index.py:127-131)
    if head_columns is not None:
        columns = _i64(head_columns)
        inside = (columns >= 0) & (columns < n)
        result = np.where(inside, result[np.clip(columns, 0, n - 1)], -1)

    counts = np.array(
        [int(resident_hit.sum()), int(hot_hit.sum()), int(miss.sum())], dtype=np.int64
    )
    return result, host_plan[:n], device_plan[:n], counts, tags_after, lru_after
