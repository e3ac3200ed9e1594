"""A cache under test together with the K/V history written to each (request, layer),
so that any attention can be checked against dense attention over the tokens it
selected (the CPU oracle).  CPU caches run the oracle kernels; ROCm caches the HIP
library."""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import torch

import oracle
from mini_hisparse_amd.config import CacheConfig
from mini_hisparse_amd.hybrid import HotConfig
from mini_hisparse_amd.paged import PagedConfig
from mini_hisparse_amd.row_index import LogicalTopK
from tests.cpu_ops import make_cache, make_paged

# float32 tolerances of the reference's tests (tests/test_hybrid.py:59 and :187-189)
F32 = dict(atol=3e-6, rtol=3e-5)
LOW = dict(atol=0.004, rtol=0.02)


class Harness:
    def __init__(self, cache, seed=0):
        self.cache = cache
        self.history: dict[tuple, tuple] = {}
        self.gen = torch.Generator().manual_seed(seed)

    # -- construction ----------------------------------------------------------------
    @classmethod
    def hybrid(cls, device, union=4, hot_rows=4, window=64, watermark=None, seed=0, **config):
        base = CacheConfig(gpu_pages=3, host_pages=64, page_size=4, kv_heads=1, head_dim=8, device=device)
        hot = HotConfig(union, hot_rows, resident_window_pages=window, transition_watermark=watermark)
        return cls(make_cache(replace(base, **config), hot), seed)

    @classmethod
    def paged(cls, device, seed=0, **config):
        base = PagedConfig(gpu_pages=3, host_pages=48, page_size=4, kv_heads=2, head_dim=8, chunk_pages=2,
                           device=device)
        return cls(make_paged(replace(base, **config)), seed)

    # -- data ------------------------------------------------------------------------------
    @property
    def device(self):
        return self.cache.device

    def rows(self, count):
        cfg = self.cache.config
        k, v = (torch.randn(count, cfg.kv_heads, cfg.head_dim, generator=self.gen) for _ in range(2))
        return k.to(self.device, cfg.dtype), v.to(self.device, cfg.dtype)

    def query(self, heads):
        cfg = self.cache.config
        return torch.randn(heads, cfg.head_dim, generator=self.gen).to(self.device, cfg.dtype)

    def write(self, request, count, layer=0):
        k, v = self.rows(count)
        self.cache.write(request, layer, k, v)
        old = self.history.get((request, layer))
        self.history[request, layer] = (k, v) if old is None else (torch.cat((old[0], k)), torch.cat((old[1], v)))
        return k, v

    def kv(self, request, layer=0):
        return self.history[request, layer]

    # -- checks ------------------------------------------------------------------------------
    def expected(self, query, request, tokens, layer=0):
        """Dense attention of every head over ``tokens`` (each counted once)."""
        k, v = self.kv(request, layer)
        tokens = sorted(set(tokens))
        return torch.from_numpy(oracle.dense_attention(query.cpu(), k[tokens].cpu(), v[tokens].cpu()))

    def attend(self, request, positions, layer=0, heads=2, query=None, tol=F32):
        """Row attention over ``positions`` (one list shared by every head, int32) checked
        against dense attention over its valid distinct tokens; returns the output."""
        from mini_hisparse_amd.attention import row_attention

        query = self.query(heads) if query is None else query
        topk = LogicalTopK(torch.tensor(positions, dtype=torch.int32, device=self.device))
        out = row_attention(query, self.cache, request, layer, topk)
        length = len(self.kv(request, layer)[0])
        valid = [t for t in positions if 0 <= t < length]
        if valid:
            got = out.float().cpu().double()
            torch.testing.assert_close(got, self.expected(query, request, valid, layer), **tol)
        return out

    def row_stats(self):
        return self.cache.snapshot()["row_stats"]

    def page(self, request, index, layer=0):
        return self.cache.storage.pages[request, layer, index]

    def resident(self, request, index, layer=0):
        return self.page(request, index, layer).slot is not None


def all_close_to_oracle(out, expected, tol=F32):
    got = out.float().cpu().double()
    np.testing.assert_allclose(got.numpy(), np.asarray(expected), rtol=tol["rtol"], atol=tol["atol"])
