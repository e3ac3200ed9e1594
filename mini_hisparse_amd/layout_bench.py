"""KV microbenchmark of the page layout (the CLI's ``bench``; experiments/benchmark.py
of the reference): per step, every request appends one token and attends over a
fixed rotating page selection (the live tail plus ``selected_pages - 1`` pages),
timed in three arrangements of the same data -- every page resident, a pressured
pool read window by window, and the pressured pool with overlapped windows.  It
measures cache mechanics, not LLM serving throughput.

Outputs are checked after timing against a float32 PyTorch softmax over the same
tokens (a self-check of the benchmark, never used to produce its results).
"""

from __future__ import annotations

from dataclasses import replace
from math import ceil
from statistics import median
from time import perf_counter

import torch

from .paged import PagedConfig, PagedKVCache, paged_attention


def _softmax_attention(q, k, v):
    """float32 softmax attention of q [Hq, D] over k, v [T, Hkv, D] (validation only)."""
    groups = q.shape[0] // k.shape[1]
    k = k.float().repeat_interleave(groups, 1).transpose(0, 1)
    v = v.float().repeat_interleave(groups, 1).transpose(0, 1)
    scores = (k @ q.float()[:, :, None])[..., 0] / q.shape[-1] ** 0.5
    return (scores.softmax(-1)[:, None, :] @ v)[:, 0]


def benchmark(config: PagedConfig, tokens=1024, steps=20, requests=3, selected_pages=8, backend="auto", ops=None):
    if min(tokens, steps, requests, selected_pages) < 1:
        raise ValueError("benchmark dimensions must be positive")
    torch.manual_seed(42)
    # the same CPU-generated histories, queries and selections for every arrangement
    histories = {
        str(i): [torch.randn(tokens + steps, config.kv_heads, config.head_dim, dtype=config.dtype) for _ in range(2)]
        for i in range(requests)
    }
    queries = torch.randn(steps, requests, config.kv_heads * 2, config.head_dim, dtype=config.dtype)
    total_pages = ceil((tokens + steps) / config.page_size) * requests
    rows = []
    for mode, slots, overlap in (
        ("resident", total_pages, False),
        ("pressured_serial", config.gpu_pages, False),
        ("pressured_overlap", config.gpu_pages, True),
    ):
        cfg = replace(config, gpu_pages=slots, host_pages=max(config.host_pages, total_pages), overlap=overlap)
        cache = PagedKVCache(cfg, ops=ops)
        for name, (k, v) in histories.items():
            cache.reserve(name, tokens + steps, 1)
            cache.write(name, 0, k[:tokens].to(cfg.device), v[:tokens].to(cfg.device))
        q_dev = queries.to(cfg.device)
        first = list(range(min(selected_pages, ceil(tokens / cfg.page_size))))
        for name in histories:  # warm the kernels and window widths outside the timer
            paged_attention(q_dev[0, int(name)], cache, name, 0, first, backend)
        cache.storage.synchronize()
        cache.storage.stats.clear()
        observed, durations = [], []
        for step in range(steps):
            incoming = {
                name: (k[tokens + step : tokens + step + 1].to(cfg.device), v[tokens + step : tokens + step + 1].to(cfg.device))
                for name, (k, v) in histories.items()
            }
            cache.storage.synchronize()
            start = perf_counter()
            for name, (k, v) in incoming.items():
                cache.write(name, 0, k, v)
                count = ceil((tokens + step + 1) / cfg.page_size)
                # a reproducible rotating access trace that always includes the live tail
                pages = list(dict.fromkeys([count - 1] + [(step * 3 + j) % count for j in range(selected_pages - 1)]))
                observed.append((step, name, pages, paged_attention(q_dev[step, int(name)], cache, name, 0, pages, backend)))
            cache.storage.synchronize()
            durations.append((perf_counter() - start) * 1000)
        max_error = 0.0
        atol, rtol = (3e-5, 3e-4) if cfg.dtype == torch.float32 else (0.006, 0.03)
        for step, name, pages, out in observed:
            idx = [t for p in pages for t in range(p * cfg.page_size, min((p + 1) * cfg.page_size, tokens + step + 1))]
            k, v = histories[name]
            want = _softmax_attention(queries[step, int(name)], k[idx], v[idx])
            err = (out.cpu().float() - want).abs()
            max_error = max(max_error, err.max().item())
            if (err > atol + rtol * want.abs()).any():
                raise AssertionError(f"{mode}: attention differs from the softmax check by {err.max().item():.3g}")
        cache.assert_invariants()
        ordered = sorted(durations)
        rows.append({
            "mode": mode,
            "median_step_ms": median(durations),
            "p95_step_ms": ordered[min(len(ordered) - 1, ceil(0.95 * len(ordered)) - 1)],
            "request_steps_per_second": steps * requests / (sum(durations) / 1000),
            "max_abs_error": max_error,
            **cache.snapshot(),
        })
        for name in histories:
            cache.release_request(name)
    device = str(config.device)
    return {
        "workload": {
            "tokens": tokens, "steps": steps, "requests": requests, "selected_pages": selected_pages,
            "page_size": config.page_size, "chunk_pages": config.chunk_pages, "backend": backend,
            "dtype": str(config.dtype), "device": device,
            "gpu": torch.cuda.get_device_name(config.device) if device.startswith("cuda") else None,
            "torch": torch.__version__, "seed": 42,
            "timing": "append + fixed-selection attention; validation and input preparation excluded",
        },
        "results": rows,
    }
