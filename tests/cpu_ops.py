"""CPU kernel backend for host-logic tests: the numpy oracle behind the cache's ops interface.

The product (``mini_hisparse_amd``) has only the HIP backend.  These tests
inject this object into ``HybridKVCache(..., ops=CpuOracleOps())`` to run the
reference's control-plane tests on CPU tensors; the same tests run on the GPU
with the default HIP backend.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle.quest import quest_selection_positions
from mini_hisparse_amd.row_index import RowPlan
from mini_hisparse_amd.selection import Selection


class CpuOracleOps:
    name = "cpu-oracle"

    def host_source(self, host):
        return host

    def resolve_rows(self, topk, source, resident, hot, tags, lru, length, page_size, row_stats=None):
        columns = None if topk.head_columns is None else topk.head_columns.numpy()
        phys, miss_host, miss_device, counts, tags_after, lru_after = oracle.resolve_rows(
            topk.positions.numpy(), source.numpy(), resident.numpy(), hot.numpy(), tags.numpy(), lru.numpy(),
            length, page_size, head_columns=columns,
        )
        tags.copy_(torch.from_numpy(tags_after.astype(np.int64)).to(tags.dtype))
        lru.copy_(torch.from_numpy(lru_after).to(lru.dtype))
        counts_t = torch.from_numpy(counts)
        if row_stats is not None:
            row_stats.add_(counts_t)
        return RowPlan(torch.from_numpy(phys), torch.from_numpy(miss_host), torch.from_numpy(miss_device), counts_t)

    def append_tokens(self, k, v, first_page, first_within, slots, host_slots, pool, host_source, host,
                      minimum, maximum, summaries, config):
        oracle.append_tokens(pool, host, k, v, first_page, first_within, slots, host_slots, minimum, maximum,
                             summaries, config.page_size, 32 if pool.dtype == torch.float32 else 16)

    def gather_rows(self, host_source, pool, plan, config):
        oracle.gather_rows(host_source, pool, plan.miss_host_rows.tolist(), plan.miss_device_rows.tolist(), config.page_size)

    def attend(self, query, pool, plan, topk, config):
        out = oracle.row_attention_rows(query, pool, plan.physical_rows, config.page_size)
        return torch.from_numpy(out).to(query.dtype)

    def attend_window(self, query, pool, slots, lengths, mask, config):
        m, l, acc = oracle.window_state(query, pool, slots, lengths, mask, config.page_size)
        return tuple(torch.from_numpy(x).to(torch.float32) for x in (m, l, acc))

    def quest_selection(self, query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
        positions = quest_selection_positions(query, minimum, maximum, length, page_size, top_pages, keep_sink)
        return Selection(positions, length, page_size, "quest")


def make_cache(config, hot):
    """HybridKVCache with the HIP backend on ROCm devices, the CPU oracle otherwise."""
    from mini_hisparse_amd.hybrid import HybridKVCache

    ops = CpuOracleOps() if torch.device(config.device).type == "cpu" else None
    return HybridKVCache(config, hot, ops=ops)


def make_paged(config):
    """PagedKVCache with the HIP backend on ROCm devices, the CPU oracle otherwise."""
    from mini_hisparse_amd.paged import PagedKVCache

    ops = CpuOracleOps() if torch.device(config.device).type == "cpu" else None
    return PagedKVCache(config, ops=ops)
