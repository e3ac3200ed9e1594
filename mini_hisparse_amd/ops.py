"""Kernel backend of the cache: the gfx950 HIP library, and nothing else.

``HybridKVCache``, ``PagedKVCache`` and ``MiniModel.decode`` call their kernels
through an ops object.  The product has exactly one, :class:`HipOps`; a cache on a non-ROCm
device must be given an explicit ops object (the CPU restatement used by the
test-suite lives outside this package) and otherwise fails at construction.
"""

from __future__ import annotations

import torch

from . import _lib
from .row_index import resolve_rows
from .row_kernels import MappedHost, append_tokens, attend_groups, attend_rows, attend_window, gather_rows
from .selection import quest_selection


class HipOps:
    """Resolver, gather, attention and Quest selection on libhisparse_hip.so."""

    name = "hip"

    def __init__(self):
        _lib.load()  # raises when the library is missing: there is no fallback

    def host_source(self, host):
        """Device alias of the pinned host pool (MappedHost, row_kernels.py:10-32)."""
        return MappedHost(host)

    def append_tokens(self, k, v, first_page, first_within, slots, host_slots, pool, host_source, host,
                      minimum, maximum, summaries, config):
        """Rows, host mirror, bounds and summaries of one write (storage.py:273-318)."""
        append_tokens(k, v, first_page, first_within, slots, host_slots, pool, host_source, minimum, maximum,
                      summaries, config)

    def resolve_rows(self, topk, source, resident, hot, tags, lru, length, page_size, row_stats=None):
        return resolve_rows(topk, source, resident, hot, tags, lru, length, page_size, row_stats=row_stats)

    def gather_rows(self, host_source, pool, plan, config):
        gather_rows(host_source, pool, plan, config, miss_count=plan.counts[2:])

    def attend(self, query, pool, plan, topk, config):
        if topk.entries is not None and plan.union_physical is not None and topk.head_columns is not None:
            return attend_groups(query, pool, plan.union_physical, topk.entries, config)
        rows = plan.physical_rows
        return attend_rows(query, pool, rows, config)

    def attend_window(self, query, pool, slots, lengths, mask, config):
        """Unnormalised (m, l, acc) of one page window of the paged layout."""
        return attend_window(query, pool, slots, lengths, mask, config)

    def quest_selection(self, query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
        return quest_selection(query, minimum, maximum, length, page_size, top_pages, keep_sink)


def default_ops(device):
    if torch.device(device).type != "cuda":
        raise ValueError(
            "mini_hisparse_amd runs its kernels on ROCm devices only; a cache on "
            f"device {device!r} needs an explicit ops backend"
        )
    return HipOps()
