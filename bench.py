#!/usr/bin/env python
"""Sparse decode benchmark on one MI355X.

Default workload ("qwen2.5-7b", BASELINE configs[3], the north_star shape): greedy
decode of a random-init Qwen2.5-7B-shape model (28 layers, hidden 3584, 28 q / 4 kv
heads, head_dim 128, FFN 18944, bf16) with the layer-major batched engine after a
prefill of 131,072-token uniformly random prompts through the same model (causal
SDPA, untimed; every layer's K/V, Quest bounds and resident pages written by
hs_append_tokens), Quest top-64 pages per query head, 15% of pages resident,
hot_rows 32768.  A step is one decode step of every request through all
28 layers: dense layers, append (rows, Quest bounds, host mirror), Quest scorer +
top-k, device union, resolver, pinned-host -> hot-row gather, group attention.
`value` = decode tokens/s = batch x steps / wall time of the timed steps.  The
batch is cut to what the box's pinned host memory holds (16 histories need 112 GiB;
the GPU boxes here pin at most 64 GiB), and the line says so.  `roofline` is the
group attention kernel (hs_attend_groups) over the timed steps: algorithmic bytes
of every launch / its duration from HIP events on the compute stream.

The default run also carries the isolated kernel microbench
as the key "microbench" (--no-microbench skips it).  Workload "microbench": one
layer, 8 KV heads x 64 query heads (GQA group 8), head_dim 128, page_size 16, 4096
logical pages (65,536 tokens) per request, batch 8, bf16; K/V ~ N(0,1) with 2% of
channels scaled x8; Quest top-64 pages per query head (sink and tail forced); of
the selected union rows 50% sit in resident pages, 30% in hot slots and 20% miss
to pinned host memory.  A microbench step restores the hot tags/LRU to the step's
starting state (so every step sees the same 20% misses) and runs Quest, union,
resolver, gather and group attention for the 8 requests.

Workload "qwen2.5-7b-layer": the microbench step at the north_star layer shape
(28 q / 4 kv heads, 8192 pages per request, batch 16).  "qwen2.5-0.5b" and
"qwen2.5-32b-stress" run BASELINE configs[2] and configs[4] end to end.
Inputs are seeded and synthetic; they live in HBM / pinned host memory before timing.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from dataclasses import dataclass
from math import ceil

import numpy as np

METRIC = "decode tokens/s at 1 MI355X; sparse-attn HBM GB/s as % of peak"
# request groups pipelined across layers by default, per model workload
DEFAULT_REQUEST_GROUPS = {"qwen2.5-7b": 2}
# gather workgroups per request with request groups: enough host reads in flight for the
# link while leaving the fabric to the compute stream (7B, batch 8, two groups: 8 -> 68.8
# ms per step, 16 -> 57.4, 24 -> 56.4, 32 -> 61.3, the library default 128 -> 74.1)
DEFAULT_GROUP_GATHER_WORKGROUPS = {"qwen2.5-7b": 24}
HBM_PEAK_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", default="qwen2.5-7b",
                   choices=["microbench", "qwen2.5-7b-layer", "qwen2.5-0.5b-layer", "qwen2.5-0.5b", "qwen2.5-7b",
                            "qwen2.5-32b-stress"],
                   help="qwen2.5-7b = BASELINE configs[3] end to end (default, the north_star shape); "
                        "microbench = configs[1]; qwen2.5-7b-layer = the microbench step at the north_star "
                        "layer shape (7B heads, 128k histories, batch 16); qwen2.5-0.5b-layer = the same at "
                        "the configs[2] layer shape; qwen2.5-0.5b and qwen2.5-32b-stress "
                        "run configs[2] and configs[4] end to end")
    p.add_argument("--no-microbench", action="store_true",
                   help="default workload: skip the configs[1] microbench figures carried as extra keys")
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--batch", type=int, default=None, help="requests (default: the workload's)")
    p.add_argument("--host-budget-gib", type=float, default=60.0,
                   help="pinned host memory for the model workloads' histories; the batch is cut to "
                        "what fits (the GPU boxes here pin at most 64 GiB)")
    p.add_argument("--seed", type=int, default=2024)
    p.add_argument("--parts", type=int, default=1,
                   help="request groups of the microbench step: group g gathers while g+1 resolves "
                        "and g-1 attends (1 = no overlap; on MI355X the host reads of a running "
                        "gather stall concurrent HBM kernels, so overlap does not pay)")
    p.add_argument("--transfer-stream", action="store_true",
                   help="gather on a separate stream ordered by events (the reference's arrangement); "
                        "by default a single request group runs every stage on the compute stream")
    p.add_argument("--no-prefetch", action="store_true",
                   help="uniform-selector model workloads: run select, resolve and gather in layer order "
                        "on the compute stream instead of prefetching every layer's at step start on a "
                        "transfer stream (overlapping the dense layers)")
    p.add_argument("--projections", choices=["auto", "kernel", "torch"], default="auto",
                   help="model workloads: the decode projections on hs_skinny_gemm or PyTorch's GEMM, or the faster "
                        "of the two timed at start (auto; a kernel trace perturbs that timing, so the traces of "
                        "the model workloads name the choice the bench line made)")
    p.add_argument("--graphs", action="store_true",
                   help="model workloads: replay each dense layer boundary as a captured HIP graph")
    p.add_argument("--request-groups", type=int, default=None,
                   help="Quest model workloads: request groups pipelined across layers (one group's gather "
                        "overlaps the others' compute); default 2 for qwen2.5-7b, else 1")
    p.add_argument("--group-gather-workgroups", type=int, default=None,
                   help="gather workgroups per request with request groups (0 = the library's default; "
                        "default 24 for qwen2.5-7b)")
    p.add_argument("--residency", choices=["policy", "fraction"], default="policy",
                   help="model workloads with a prefill: the hybrid policy places pages and hot regions in a slab "
                        "of resident_fraction of the history plus every layer's promised hot region and tails "
                        "(default), or a seeded fixed fraction of each layer's pages is resident")
    p.add_argument("--resolver-front", choices=("split", "single"), default="split",
                   help="the resolver's front over several workgroups per request (split, the default) or one "
                        "(single)")
    p.add_argument("--direct", action="store_true",
                   help="model workloads: prefill every prompt first and time the engine's device-resident "
                        "token loop only, instead of admitting and decoding through the Engine API")
    p.add_argument("--synthetic-history", action="store_true",
                   help="model workloads: write synthetic K/V histories (N(0,1), 2%% of channels x8) directly "
                        "instead of prefilling random prompts through the model")
    p.add_argument("--context", type=int, default=None,
                   help="model workloads: prompt length (default: the workload's); the line then names it")
    p.add_argument("--engine", choices=("layer-major", "per-request"), default="layer-major",
                   help="model workloads: the layer-major engine (the default) or the reference-shaped "
                        "per-request Engine over HybridKVCache (each request's layers decoded in turn); the "
                        "latter prints its own line and no roofline")
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle leg")
    p.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU sample work")
    p.add_argument("--attention-sweep", action="store_true",
                   help="print the group attention's duration against its work (fixed cost and "
                        "incremental rate of both schedules) as a markdown table and exit")
    p.add_argument("--summarize-trace", metavar="TRACE_DIR",
                   help="summarise a rocprofv3 --kernel-trace run of this script (same --workload, --steps, "
                        "--warmup) over its timed steps into profiles/ and exit")
    p.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="summarise two rocprofv3 --pmc runs of this script (FETCH_SIZE, WRITE_SIZE) "
                        "into profiles/microbench_pmc.txt and exit")
    return p.parse_args()


@dataclass(frozen=True)
class Shape:
    """One layer of synthetic sparse-decode state (the microbench machinery)."""

    label: str
    batch: int
    kv_heads: int
    heads: int
    pages: int  # logical pages per request
    head_dim: int = 128
    page_size: int = 16
    top: int = 64
    hot_rows: int = 32768
    resident_frac: float = 0.5
    hot_frac_of_rest: float = 0.6  # 30% of all union rows


SHAPES = {
    # BASELINE configs[1]
    "microbench": Shape("microbench (BASELINE configs[1]): 1 layer, 64 q / 8 kv heads, head_dim 128, page 16, "
                        "4096 pages/request", batch=8, kv_heads=8, heads=64, pages=4096),
    # one layer of the north_star shape: Qwen2.5-7B heads, 128k-token histories, batch 16
    "qwen2.5-7b-layer": Shape("one layer of the Qwen2.5-7B shape (BASELINE configs[3] / north_star): 28 q / 4 kv "
                              "heads, head_dim 128, page 16, 8192 pages/request (131,072 tokens)",
                              batch=16, kv_heads=4, heads=28, pages=8192),
    # one layer of the Qwen2.5-0.5B shape: 32k-token histories, batch 4,
    # the end-to-end workload's top 32 pages and 13,504 hot rows
    "qwen2.5-0.5b-layer": Shape("one layer of the Qwen2.5-0.5B shape (BASELINE configs[2]): 14 q / 2 kv heads, "
                                "head_dim 64, page 16, 2048 pages/request (32,768 tokens), top 32",
                                batch=4, kv_heads=2, heads=14, pages=2048, head_dim=64, top=32, hot_rows=13504),
}


def build_workload(args, torch, device):
    """Seeded synthetic state of the microbench in HBM and pinned host memory."""
    from mini_hisparse_amd.batched import BatchedSparseDecode, LayerTablesView, PipelinedSparseDecode
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.row_kernels import MappedHost

    S = SHAPES[args.workload]
    B, P, C, Hkv, D = args.batch, S.page_size, S.pages, S.kv_heads, S.head_dim
    L = C * P
    gen = torch.Generator(device=device).manual_seed(args.seed)
    cpu_gen = torch.Generator().manual_seed(args.seed)
    scale = torch.ones(Hkv, D)
    outliers = max(1, round(0.02 * D))
    for kv in range(Hkv):
        scale[kv, torch.randperm(D, generator=cpu_gen)[:outliers]] = 8.0
    scale = scale.to(device)
    # KV in page layout [B, C, 2, P, Hkv, D]
    kv_pages = torch.empty((B, C, 2, P, Hkv, D), dtype=torch.bfloat16, device=device)
    for b in range(B):
        x = torch.randn((C, 2, P, Hkv, D), generator=gen, device=device)
        kv_pages[b] = (x * scale).to(torch.bfloat16)
        del x
    kmin = [kv_pages[b, :, 0].amin(1).contiguous() for b in range(B)]  # [C, Hkv, D]
    kmax = [kv_pages[b, :, 0].amax(1).contiguous() for b in range(B)]
    q = torch.randn((B, S.heads, D), generator=gen, device=device).to(torch.bfloat16)
    host = torch.empty((B * C, 2, P, Hkv, D), dtype=torch.bfloat16, pin_memory=True)
    host.copy_(kv_pages.view(B * C, 2, P, Hkv, D))
    torch.cuda.synchronize()

    cfg_probe = CacheConfig(gpu_pages=1, host_pages=1, page_size=P, kv_heads=Hkv, head_dim=D, device=device, dtype=torch.bfloat16)
    dec = BatchedSparseDecode(cfg_probe, S.heads, S.top, [L] * B, device=device)
    dec.select(q, kmin, kmax)
    torch.cuda.synchronize()
    positions = dec.positions.cpu().numpy()
    union_n = dec.union_count.cpu().numpy()

    HB = ceil(S.hot_rows / P)
    plan = []
    n_resident_blocks = 0
    for b in range(B):
        rng = np.random.default_rng(args.seed + 17 * b)
        union = positions[b, : union_n[b]].astype(np.int64)
        upages = np.unique(union // P)
        res = set(rng.choice(upages, size=int(round(S.resident_frac * len(upages))), replace=False).tolist())
        res.add(C - 1)  # the active tail page stays resident
        res = sorted(res)
        rest = union[~np.isin(union // P, res)]
        hot_tokens = np.sort(rng.choice(rest, size=int(round(S.hot_frac_of_rest * len(rest))), replace=False))
        plan.append((res, hot_tokens, rng))
        n_resident_blocks += len(res)
    blocks = n_resident_blocks + B * HB
    pool = torch.empty((blocks, 2, P, Hkv, D), dtype=torch.bfloat16, device=device)
    perm = np.random.default_rng(args.seed + 1).permutation(B * HB) + n_resident_blocks
    tags_all = torch.full((B, S.hot_rows), -1, dtype=torch.int32, device=device)
    lru_all = torch.empty((B, S.hot_rows), dtype=torch.int16, device=device)  # the engine's LRU dtype
    tables = []
    next_block = 0
    stats = {"union_rows": 0, "resident_rows": 0, "hot_rows": 0, "miss_rows": 0}
    for b, (res, hot_tokens, rng) in enumerate(plan):
        source = torch.arange(b * C, (b + 1) * C, dtype=torch.int32, device=device)
        resident = torch.full((C,), -1, dtype=torch.int32, device=device)
        res_blocks = torch.arange(next_block, next_block + len(res), device=device)
        res_idx = torch.tensor(res, device=device)
        resident[res_idx] = res_blocks.to(torch.int32)
        pool[res_blocks] = kv_pages[b, res_idx]
        next_block += len(res)
        hot = torch.from_numpy(perm[b * HB : (b + 1) * HB].astype(np.int32)).to(device)
        slots = rng.choice(S.hot_rows, size=len(hot_tokens), replace=False)
        host_rows = (b * C + hot_tokens // P) * P + hot_tokens % P
        tags = np.full(S.hot_rows, -1, np.int32)
        tags[slots] = host_rows
        tags_all[b] = torch.from_numpy(tags).to(device)
        lru_all[b] = torch.from_numpy(rng.permutation(S.hot_rows).astype(np.int16)).to(device)
        slot_t = torch.from_numpy(slots).to(device)
        phys = hot[slot_t // P].long() * P + slot_t % P
        tok = torch.from_numpy(hot_tokens).to(device)
        pool[phys // P, :, phys % P] = kv_pages[b, tok // P, :, tok % P]
        tables.append(LayerTablesView(source, resident, hot, tags_all[b], lru_all[b]))
        n = int(union_n[b])
        n_res = int(np.isin(positions[b, :n] // P, res).sum())
        stats["union_rows"] += n
        stats["resident_rows"] += n_res
        stats["hot_rows"] += len(hot_tokens)
        stats["miss_rows"] += n - n_res - len(hot_tokens)
    del kv_pages
    torch.cuda.synchronize()
    cfg = CacheConfig(gpu_pages=blocks, host_pages=B * C, page_size=P, kv_heads=Hkv, head_dim=D, device=device, dtype=torch.bfloat16)
    dec = BatchedSparseDecode(cfg, S.heads, S.top, [L] * B, device=device,
                              split_front=args.resolver_front == "split")  # request b's host pages: b C + page
    pipe = PipelinedSparseDecode(cfg, S.heads, S.top, [L] * B, parts=args.parts, device=device,
                                 split_front=args.resolver_front == "split")
    return dict(
        cfg=cfg, dec=dec, pipe=pipe, q=q, kmin=kmin, kmax=kmax, host=host, alias=MappedHost(host), pool=pool,
        tables=tables, tags_all=tags_all, lru_all=lru_all, tags0=tags_all.clone(), lru0=lru_all.clone(),
        stats=stats, length=L, shape=S,
    )


def run_steps(torch, w, steps, record):
    """`steps` decode steps; per-stage HIP events when `record`."""
    from mini_hisparse_amd.streams import independent_stream

    dec, device = w["dec"], w["pool"].device
    compute = torch.cuda.current_stream(device)
    if "transfer" not in w:
        w["transfer"] = independent_stream(device)
    transfer = w["transfer"]
    row_stats = w.setdefault("row_stats", torch.zeros(3, dtype=torch.int64, device=device))
    events = []
    last = w.get("last_use")
    out = None
    kernel = KernelTimer(torch, steps) if record else None
    w["attention_kernel"] = kernel
    for step in range(steps):
        ev = [torch.cuda.Event(enable_timing=record) for _ in range(8)]
        w["tags_all"].copy_(w["tags0"])
        w["lru_all"].copy_(w["lru0"])
        ev[0].record(compute)
        dec.select(w["q"], w["kmin"], w["kmax"])
        ev[1].record(compute)
        dec.resolve(w["tables"], row_stats=row_stats)
        ev[2].record(compute)
        transfer.wait_event(ev[2])
        if last is not None:
            transfer.wait_event(last)
        ev[3].record(transfer)
        dec.gather(w["alias"], w["pool"], transfer)
        ev[4].record(transfer)
        compute.wait_event(ev[4])
        ev[5].record(compute)
        if kernel is not None:
            kernel.arm(step)
        out = dec.attend(w["q"], w["pool"])
        ev[6].record(compute)
        last = ev[6]
        events.append(ev)
    w["last_use"] = last
    w["out"] = out
    return events


def run_pipelined(torch, w, steps):
    """`steps` decode steps of the whole batch as overlapped request groups."""
    from mini_hisparse_amd.streams import independent_stream

    pipe, device = w["pipe"], w["pool"].device
    if w["use_transfer_stream"] and "transfer" not in w:
        w["transfer"] = independent_stream(device)
    transfer = w["transfer"] if w["use_transfer_stream"] else None
    row_stats = w.setdefault("row_stats", torch.zeros(3, dtype=torch.int64, device=device))
    out = w.get("pipe_out")
    for _ in range(steps):
        w["tags_all"].copy_(w["tags0"])
        w["lru_all"].copy_(w["lru0"])
        out, done = pipe.step(w["q"], w["kmin"], w["kmax"], w["tables"], w["pool"], w["alias"], transfer,
                              row_stats=row_stats, out=out)
        if transfer is not None:
            # the next step restores the hot tables only after this step's readers
            transfer.wait_event(done)
    w["pipe_out"] = out
    return out


def stage_ms(events, kernel=None):
    """Per-stage milliseconds: the median over the recorded steps, so that a one-off host
    stall (the GPU idles inside one stage's event pair until the host launches) does not
    move it.  With ``kernel`` (the steps' KernelTimer), "attention" is the attention
    launch's own kernel duration and "attention_event_window" the stream events around it."""
    def avg(i, j):
        return float(np.median([e[i].elapsed_time(e[j]) for e in events]))

    out = {
        "quest_and_union": avg(0, 1),
        "resolve": avg(1, 2),
        "gather": avg(3, 4),
        "attention": avg(5, 6),
    }
    if kernel is not None:
        out["attention_event_window"] = out["attention"]
        out["attention"] = float(np.median([kernel.ms(i) for i in range(len(events))]))
    return out


def host_link_gbs(torch, device, nbytes=1 << 30):
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    return 3 * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9


def hbm_copy_gbs(torch, device, nbytes=1 << 30):
    """Plain device-to-device copy of known size (also the PMC calibration kernel)."""
    a = torch.empty(nbytes, dtype=torch.uint8, device=device)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    return 5 * 2 * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9


def attention_ceilings(torch, w, nbytes, reps=10):
    """The attention, a read-only pass over the same row segments (hs_probe_row_reads) and a
    contiguous read of as many bytes, in GB/s of the attention's algorithmic bytes:
    `warm` back to back (rows partly in the 256 MB Infinity Cache); `cold` after reading 1 GiB
    of other data (clean caches: HBM); `cold_dirty` after a 1 GiB copy, whose dirty lines the
    reads must write back (the state after the step's gather has written its rows)."""
    from mini_hisparse_amd import _lib

    dec, pool, q = w["dec"], w["pool"], w["q"]
    dev = pool.device
    sink = torch.empty(16, dtype=torch.int32, device=dev)
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    offsets = dec.entry_offsets(pool)
    n = nbytes // 512
    stream_buf = torch.empty(n * 512, dtype=torch.uint8, device=dev)
    stream_offsets = torch.arange(n, dtype=torch.int64, device=dev) * 512

    def stream_read():
        _lib.check(_lib.load().hs_probe_row_reads(
            stream_buf.data_ptr(), stream_buf.numel(), stream_offsets.data_ptr(), n, 256, 256, sink.data_ptr(),
            torch.cuda.current_stream(dev).cuda_stream), "hs_probe_row_reads")

    flushes = {"cold": lambda: src.view(torch.int64).sum(), "cold_dirty": lambda: dst.copy_(src)}
    runs = {"attention": lambda: dec.attend(q, pool), "probe": lambda: dec.probe_reads(pool, offsets, sink),
            "stream_read": stream_read}
    out = {}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, fn in runs.items():
        fn()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[f"{name}_warm_GBps"] = nbytes / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9
        for label, flush in flushes.items():
            times = []
            for _ in range(reps):
                flush()
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1))
            out[f"{name}_{label}_GBps"] = nbytes / (float(np.median(times)) * 1e-3) / 1e9
    return out


def attention_sweep(torch, device, reps=8):
    """Duration of hs_attend_groups against its work at the microbench head shape (B=8,
    8 KV heads of 8 query heads, head_dim 128, bf16): every group reads the same number of
    entries (random pages of a 1.5 GB pool), from 32 to 6144 per group; split and balanced
    schedules (HS_ATTEND_SCHED); warm (back to back) and cold (after reading 1 GiB of other
    data).  A long kernel runs before each timed launch so the host is ahead of the GPU and
    the events time the GPU only.  Fits duration = fixed + bytes / rate over the points of
    >= 1536 entries per group.  Prints a markdown table."""
    import os

    from mini_hisparse_amd.row_index import GroupEntries
    from mini_hisparse_amd.row_kernels import attend_groups

    P, Hkv, g, D, B, blocks, cap = 16, 8, 8, 128, 8, 24000, 8192
    cfg = type("Cfg", (), dict(page_size=P, kv_heads=Hkv, head_dim=D))
    gen = torch.Generator(device=device).manual_seed(5)
    pool = torch.randn((blocks, 2, P, Hkv, D), generator=gen, device=device).to(torch.bfloat16)
    q = torch.randn((B, Hkv * g, D), generator=gen, device=device).to(torch.bfloat16)
    other = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    rng = np.random.default_rng(5)
    counts_list = (32, 128, 512, 1024, 1536, 3072, 6144)
    union = np.empty((B, cap), np.int64)
    for b in range(B):
        pages = np.sort(rng.choice(blocks, cap // P, replace=False))
        union[b] = (pages[:, None] * P + np.arange(P)[None, :]).reshape(-1)
    union_t = torch.from_numpy(union).to(device)
    cols = torch.arange(cap, dtype=torch.int32, device=device).expand(B, Hkv, cap).contiguous()
    masks = torch.from_numpy(rng.integers(1, 1 << g, size=(B, Hkv, cap)).astype(np.int32)).to(device)
    results = {}
    saved = os.environ.get("HS_ATTEND_SCHED")
    try:
        for schedule, env in (("split", "0"), ("balanced", "1")):
            os.environ["HS_ATTEND_SCHED"] = env
            for c in counts_list:
                counts = torch.full((B, Hkv), c, dtype=torch.int32, device=device)
                entries = GroupEntries(cols, masks, counts, cap)
                run = lambda: attend_groups(q, pool, union_t, entries, cfg)
                run()
                for state in ("warm", "cold"):
                    times = []
                    for _ in range(reps):
                        if state == "cold":
                            other.view(torch.int64).sum()
                        else:
                            run()
                        torch.cuda._sleep(1_000_000)  # keeps the GPU busy while the host enqueues
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record()
                        run()
                        e1.record()
                        torch.cuda.synchronize()
                        times.append(e0.elapsed_time(e1) * 1e3)
                    results[(schedule, c, state)] = float(np.median(times))
    finally:
        if saved is None:
            os.environ.pop("HS_ATTEND_SCHED", None)
        else:
            os.environ["HS_ATTEND_SCHED"] = saved
    mb = {c: B * Hkv * c * 512 / 1e6 for c in counts_list}
    lines = ["| entries / group | MB | split warm µs | split cold µs | balanced warm µs | balanced cold µs |",
             "|---|---|---|---|---|---|"]
    for c in counts_list:
        r = [results[(s, c, st)] for s in ("split", "balanced") for st in ("warm", "cold")]
        lines.append(f"| {c} | {mb[c]:.1f} | " + " | ".join(f"{t:.1f}" for t in r) + " |")
    # The balanced schedule spreads any total over every workgroup, so its duration is
    # linear in the bytes; the split schedule's chunks are sized for the capacity (8192
    # entries), which leaves workgroups empty below it, so no line fits it.
    lines.append("")
    lines.append("| balanced schedule, fit over >= 1536 entries / group | fixed µs | incremental rate TB/s |")
    lines.append("|---|---|---|")
    big = [c for c in counts_list if c >= 1536]
    for st in ("warm", "cold"):
        x = np.array([mb[c] for c in big])
        y = np.array([results[("balanced", c, st)] for c in big])
        slope, fixed = np.polyfit(x, y, 1)
        lines.append(f"| {st} | {fixed:.1f} | {1.0 / slope:.2f} |")
    print("\n".join(lines))


def algorithmic_bytes(w, torch):
    """Per-launch algorithmic bytes of each kernel (per-unit formulas x units)."""
    S, dec = w["shape"], w["dec"]
    B, e, D = dec.batch, 2, S.head_dim
    entries = int(w["dec"].entry_counts.sum().item())
    per_head = int((w["dec"].head_physical() >= 0).sum().item())
    misses = int(w["dec"].row_counts[:, 2].sum().item())
    n_union = int(w["dec"].union_count.sum().item())
    W = dec.width
    attention = entries * 2 * D * e + 8 * S.heads * W * B + 2 * S.heads * D * e * B
    attention_per_head = per_head * 2 * D * e + 8 * S.heads * W * B + 2 * S.heads * D * e * B
    quest = B * (2 * S.pages * S.kv_heads * D * e + S.heads * D * e + S.heads * S.top * 4)
    # per request, over the n selected tokens and the C-entry position array (the union,
    # padded with -1 to the batch's capacity): positions read (4C), source + resident of
    # each selected token's page (8n), tags read and written (8S), LRU read and written
    # (2 x its element size x S), the miss plan (16C: the misses, then -1, as the reference's fixed-width plan)
    # and the union rows (8C) written, counts; with per-head rows also the head columns
    # read and the rows written (16 H W)
    head_rows = 16 * S.heads * W if dec.head_rows else 0
    C = dec.capacity
    lru_bytes = 2 * w["lru_all"].element_size() * S.hot_rows
    resolver = sum(
        4 * C + 8 * n + 8 * S.hot_rows + lru_bytes + 16 * C + 8 * C + head_rows + 24
        for n in w["dec"].union_count.tolist()
    )
    gather = misses * 2 * S.kv_heads * D * e
    return dict(
        attention=attention, attention_per_head=attention_per_head, quest=quest,
        resolver=resolver, gather=gather, entries=entries, misses=misses, union_rows=n_union,
    )


def cpu_baseline(torch, w, budget_s):
    """The numpy oracle on the host cores: whole requests of the same step."""
    import oracle
    from oracle.quest import pages_to_positions

    torch.set_num_threads(1)
    S, dec = w["shape"], w["dec"]
    P, L = S.page_size, w["length"]
    q = w["q"].cpu()
    pool = w["pool"].cpu()
    host = w["host"]
    tags0, lru0 = w["tags0"].cpu().numpy(), w["lru0"].cpu().numpy()
    gpu_pages = dec.pages.cpu().numpy()
    gpu_phys = dec.head_physical().cpu().numpy()
    gpu_out = w["out"].float().cpu()
    done = 0
    parity = {"pages_equal": True, "physical_equal": True, "max_abs_err": 0.0,
              "attention_within_tolerance": True, "tolerance": "abs 2e-2 + rel 1e-2 (north_star, bf16)"}
    t0 = time.perf_counter()
    for b in range(dec.batch):
        t = w["tables"][b]
        pages = oracle.quest_pages(q[b], w["kmin"][b].cpu(), w["kmax"][b].cpu(), L, P, S.top)
        positions = pages_to_positions(pages, L, P)
        union, cols = oracle.from_selection(positions)
        phys, mh, md, counts, _, _ = oracle.resolve_rows(
            union, t.source.cpu().numpy(), t.resident.cpu().numpy(), t.hot.cpu().numpy(),
            tags0[b], lru0[b], L, P, head_columns=cols,
        )
        oracle.gather_rows(host, pool, mh, md, P)
        out = oracle.row_attention_rows(q[b], pool, phys, P)
        done += 1
        parity["pages_equal"] &= bool((gpu_pages[b, :, : pages.shape[1]] == pages).all())
        parity["physical_equal"] &= bool((gpu_phys[b, :, : phys.shape[1]] == phys).all())
        err = np.abs(gpu_out[b].double().numpy() - out)
        parity["max_abs_err"] = max(parity["max_abs_err"], float(err.max()))
        parity["attention_within_tolerance"] &= bool((err <= 2e-2 + 1e-2 * np.abs(out)).all())
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0
    return {
        "value": done / elapsed,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{done} of {dec.batch} requests of one step (Quest scores+top-k, union, resolve, "
        f"row gather, attention), numpy oracle, 1 thread, {elapsed:.1f} s",
        "host": platform.processor() or platform.machine(),
        "host_cpus": os.cpu_count(),
    }, parity


def _cpu_request(job):
    """One request of the microbench step on the numpy oracle, in a worker process: the
    inputs are mapped from the files `cpu_baseline_all_cores` wrote (the pool
    copy-on-write, so this request's gather stays private).  Returns the attention
    output and the seconds the request took."""
    import torch

    import oracle
    from oracle.quest import pages_to_positions

    torch.set_num_threads(1)
    d, b, L, P, top = job
    load = lambda name, mode="r": np.load(os.path.join(d, name + ".npy"), mmap_mode=mode)
    bf16 = lambda a: torch.from_numpy(a).view(torch.bfloat16)
    t0 = time.perf_counter()
    q = bf16(np.array(load("q")[b]))
    host = bf16(load("host", "c"))
    pool = bf16(load("pool", "c"))
    pages = oracle.quest_pages(q, bf16(np.array(load("kmin")[b])), bf16(np.array(load("kmax")[b])), L, P, top)
    positions = pages_to_positions(pages, L, P)
    union, cols = oracle.from_selection(positions)
    phys, mh, md, _, _, _ = oracle.resolve_rows(
        union, load("source")[b], load("resident")[b], load("hot")[b], np.array(load("tags0")[b]),
        np.array(load("lru0")[b]), L, P, head_columns=cols,
    )
    oracle.gather_rows(host, pool, mh, md, P)
    out = oracle.row_attention_rows(q, pool, phys, P)
    return out, time.perf_counter() - t0


def _cpu_worker_ready(_):
    import torch  # noqa: F401

    import oracle  # noqa: F401

    return os.getpid()


def cpu_baseline_all_cores(torch, w, max_workers=16):
    """The step's B requests on the numpy oracle, one spawned worker process per request
    (at most `max_workers` -- the GPU box's CPU share -- and the host's CPU count), each
    timed from a warm worker; inputs go through files mapped by every worker."""
    import shutil
    import tempfile
    from concurrent.futures import ProcessPoolExecutor
    from multiprocessing import get_context

    S, dec = w["shape"], w["dec"]
    B = dec.batch
    workers = max(1, min(B, max_workers, os.cpu_count() or 1))
    d = tempfile.mkdtemp(prefix="hs_cpu_")
    try:
        i16 = lambda t: t.detach().cpu().contiguous().view(torch.int16).numpy()
        arrays = {
            "host": i16(w["host"]), "pool": i16(w["pool"]), "q": i16(w["q"]),
            "kmin": np.stack([i16(t) for t in w["kmin"]]), "kmax": np.stack([i16(t) for t in w["kmax"]]),
            "source": np.stack([t.source.cpu().numpy() for t in w["tables"]]),
            "resident": np.stack([t.resident.cpu().numpy() for t in w["tables"]]),
            "hot": np.stack([t.hot.cpu().numpy() for t in w["tables"]]),
            "tags0": w["tags0"].cpu().numpy(), "lru0": w["lru0"].cpu().numpy(),
        }
        for name, a in arrays.items():
            np.save(os.path.join(d, name + ".npy"), a)
        del arrays
        gpu_out = w["out"].float().cpu().double().numpy()
        with ProcessPoolExecutor(workers, mp_context=get_context("spawn")) as pool:
            list(pool.map(_cpu_worker_ready, range(workers)))
            t0 = time.perf_counter()
            results = list(pool.map(_cpu_request, [(d, b, w["length"], S.page_size, S.top) for b in range(B)]))
            elapsed = time.perf_counter() - t0
    finally:
        shutil.rmtree(d, ignore_errors=True)
    within = all(bool((np.abs(gpu_out[b] - out) <= 2e-2 + 1e-2 * np.abs(out)).all()) for b, (out, _) in enumerate(results))
    return {
        "value": B / elapsed,
        "unit": "tokens/s",
        "cores": workers,
        "sample": f"{B} of {B} requests of one step, one spawned process per request ({workers} at a time, "
        f"inputs memory-mapped), numpy oracle, {elapsed:.1f} s; slowest request "
        f"{max(t for _, t in results):.1f} s; outputs within the bf16 tolerance of the GPU's: {within}",
    }


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
PMC_SUMMARY = os.path.join(PROFILES, "microbench_pmc.txt")
# counter summaries per single-layer workload (the step the bench line times)
PMC_SUMMARIES = {
    "microbench": (PMC_SUMMARY, "microbench step (BASELINE configs[1]), batch 8, bf16"),
    "qwen2.5-7b": (os.path.join(PROFILES, "qwen2.5-7b_e2e_pmc.txt"),
                   "Qwen2.5-7B-shape end-to-end decode (BASELINE configs[3]), batch 8, bf16"),
    "qwen2.5-7b-layer": (os.path.join(PROFILES, "qwen2.5-7b_layer_pmc.txt"),
                         "one layer of the north_star step (Qwen2.5-7B heads, 128k histories), batch 16, bf16"),
}
# (batch, request groups) each counter summary was taken at: its per-launch traffic applies
# to that configuration only
PMC_CONFIG = {"microbench": (8, 1), "qwen2.5-7b": (8, 2), "qwen2.5-7b-layer": (16, 1)}
ROOFLINE_KERNELS = ("attend_mfma_kernel", "attend_merge_kernel")
ATTENTION_KERNELS = ("attend_mfma_kernel, its last workgroup per (request, KV head) merging the split partials "
                     "(attend_merge_kernel instead when a group has more than 16 splits)")
CALIBRATION_BYTES = 1 << 30  # hbm_copy_gbs: a plain device-to-device copy of 1 GiB


def summarize_pmc(fetch_dir, write_dir, workload="microbench"):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE of each hs:: kernel, scaled by what the
    same counters read for the 1 GiB device copy this script makes."""
    import csv
    import glob
    from collections import defaultdict

    def load(d, counter):
        (path,) = glob.glob(os.path.join(d, "*counter_collection.csv"))
        rows = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                rows[int(r["Dispatch_Id"])] = (r["Kernel_Name"], float(r["Counter_Value"]))
        return rows

    fetch, write = load(fetch_dir, "FETCH_SIZE"), load(write_dir, "WRITE_SIZE")
    kib = CALIBRATION_BYTES / 1024
    # the two runs need not number their dispatches alike: find the copy in each on its own
    calib_write = [v for name, v in write.values() if "copyBuffer" in name and abs(v - kib) < 0.01 * kib]
    calib_fetch = [v for name, v in fetch.values() if "copyBuffer" in name and abs(v - kib) < 0.6 * kib]
    if not calib_write or not calib_fetch:
        raise SystemExit("no 1 GiB device copy found in the counter runs")
    calib = calib_write
    fetch_scale = kib / float(np.mean(calib_fetch))
    write_scale = kib / float(np.mean(calib_write))
    per = defaultdict(lambda: [[], []])
    for i, (name, v) in fetch.items():
        if "hs::" in name:
            per[name.split("(")[0].replace("void ", "")][0].append(v)
    for i, (name, v) in write.items():
        if "hs::" in name:
            per[name.split("(")[0].replace("void ", "")][1].append(v)
    out_path, title = PMC_SUMMARIES[workload]
    flag = f" --workload {workload}" + (" --no-microbench" if workload == "qwen2.5-7b" else "")
    lines = [
        f"# rocprofv3 --pmc summary: {title}",
        "# FETCH_SIZE and WRITE_SIZE (KiB per dispatch) from two runs of",
        f"#   rocprofv3 --pmc FETCH_SIZE -f csv -d <dir> -o bench -- python bench.py{flag} --steps 3 --warmup 1 --no-cpu-baseline",
        f"#   rocprofv3 --pmc WRITE_SIZE -f csv -d <dir> -o bench -- python bench.py{flag} --steps 3 --warmup 1 --no-cpu-baseline",
        f"# summarised by: python bench.py{flag} --summarize-pmc <fetch dir> <write dir>",
        f"# calibration: the 1 GiB device-to-device copy of hbm_copy_gbs ({len(calib)} dispatches) reads "
        f"FETCH_SIZE x{fetch_scale:.3f}, WRITE_SIZE x{write_scale:.3f} of its true bytes",
        f"calibration fetch_scale {fetch_scale:.4f} write_scale {write_scale:.4f}",
        "# kernel  dispatches  fetch_bytes_per_dispatch  write_bytes_per_dispatch  (scaled)",
    ]
    for name in sorted(per):
        f, w = per[name]
        fb = float(np.mean(f)) * 1024 * fetch_scale if f else 0.0
        wb = float(np.mean(w)) * 1024 * write_scale if w else 0.0
        lines.append(f"kernel {name.replace('hs::', '').replace(' ', '')} {len(f)} {fb:.0f} {wb:.0f}")
    with open(out_path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


TRACE_SUMMARIES = {
    "qwen2.5-7b": os.path.join(PROFILES, "qwen2.5-7b_e2e_kernel_trace.md"),
    "qwen2.5-0.5b": os.path.join(PROFILES, "qwen2.5-0.5b_e2e_kernel_trace.md"),
    "qwen2.5-32b-stress": os.path.join(PROFILES, "qwen2.5-32b-stress_e2e_kernel_trace.md"),
    "microbench": os.path.join(PROFILES, "microbench_kernel_trace.md"),
    "qwen2.5-7b-layer": os.path.join(PROFILES, "qwen2.5-7b_layer_kernel_trace.md"),
    "qwen2.5-0.5b-layer": os.path.join(PROFILES, "qwen2.5-0.5b_layer_kernel_trace.md"),
}


def summarize_layer_trace(trace_dir, args):
    """Per-kernel dispatches and durations of the library's kernels in a kernel trace of a
    single-layer workload (microbench, qwen2.5-7b-layer): every step of the run (warmup,
    timed, profiled) with the attention ceilings' probes beside them, avg / min / max."""
    import csv
    import glob
    from collections import defaultdict

    (path,) = glob.glob(os.path.join(trace_dir, "*kernel_trace.csv"))
    per = defaultdict(list)
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    previous = ""
    for r in rows:
        name = r["Kernel_Name"].split("(")[0].replace("void ", "")
        if not name.startswith("hs::"):
            continue
        name = name.replace("hs::", "")
        duration = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        per[name].append(duration)
        if name.startswith("attend_mfma_kernel") and previous.startswith("gather_kernel"):
            per[name + " (in step: after the gather)"].append(duration)
        previous = name
    cmd = (f"rocprofv3 --kernel-trace --stats -f csv -d <dir> -o bench -- python3 bench.py --workload "
           f"{args.workload} --steps {args.steps} --warmup {args.warmup} --no-cpu-baseline")
    lines = [
        f"# Kernel trace: {SHAPES[args.workload].label}, batch {SHAPES[args.workload].batch}, bf16",
        "",
        f"Command: `{cmd}`",
        f"Summarised by: `python bench.py --workload {args.workload} --steps {args.steps} --warmup {args.warmup} "
        "--summarize-trace <dir>`",
        "",
        "Every dispatch of the library's kernels in the run: the warmup, timed and profiled steps and the "
        "measured ceilings' probes (`probe_row_reads_kernel`; the attention kernel's count includes the "
        "ceilings' launches).  Microseconds.",
        "",
        "| kernel | dispatches | avg us | min us | max us |",
        "|---|---|---|---|---|",
    ]
    for name, ds in sorted(per.items(), key=lambda x: -float(np.mean(x[1]))):
        lines.append(f"| `{name}` | {len(ds)} | {np.mean(ds):.1f} | {min(ds):.1f} | {max(ds):.1f} |")
    with open(TRACE_SUMMARIES[args.workload], "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def summarize_trace(trace_dir, args):
    """Per-kernel dispatches and durations over the timed steps of a model workload's
    kernel trace: the kernels between the first two spin kernels (``_time_steps``'s
    markers) after the first decode attention; they must be layers x steps x groups
    attention launches."""
    import csv
    import glob
    from collections import defaultdict

    from mini_hisparse_amd.batched_engine import WORKLOADS

    wl = WORKLOADS[args.workload]
    (path,) = glob.glob(os.path.join(trace_dir, "*kernel_trace.csv"))
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    first = next(i for i, r in enumerate(rows) if "attend_mfma_kernel" in r["Kernel_Name"])
    marks = [i for i, r in enumerate(rows) if i > first and "spin_kernel" in r["Kernel_Name"]]
    L = wl.layers
    if len(marks) < 2:
        raise SystemExit("the trace holds no marked timed region (spin kernels around it)")
    window = rows[marks[0] + 1 : marks[1]]
    groups = args.request_groups if args.request_groups is not None else DEFAULT_REQUEST_GROUPS.get(args.workload, 1)
    launches = sum("attend_mfma_kernel" in r["Kernel_Name"] for r in window)
    if launches != L * args.steps * groups:
        raise SystemExit(f"the timed region holds {launches} attention launches, expected {L * args.steps * groups}")
    agg = defaultdict(lambda: [0, 0])
    for r in window:
        name = r["Kernel_Name"].split("(")[0].replace("void ", "")
        agg[name][0] += 1
        agg[name][1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    span_ms = (int(window[-1]["End_Timestamp"]) - int(window[0]["Start_Timestamp"])) / 1e6
    path = " --direct" if args.direct else ""  # the engine driven directly, not through the Engine API
    cmd = f"rocprofv3 --kernel-trace --stats -f csv -d <dir> -o bench -- python3 bench.py --workload {args.workload}" \
          f"{path} --no-microbench --no-cpu-baseline --projections {args.projections} --steps {args.steps} " \
          f"--warmup {args.warmup}"
    att = [agg[k] for k in agg if k.startswith("hs::attend_mfma_kernel")]
    mrg = [agg[k] for k in agg if k.startswith("hs::attend_merge_kernel")]
    att_us = sum(d for _, d in att) / max(1, sum(c for c, _ in att)) / 1e3
    mrg_us = sum(d for _, d in mrg) / max(1, sum(c for c, _ in mrg)) / 1e3
    lines = [
        f"# Kernel trace: {wl.name} end to end, timed steps only",
        "",
        f"Command: `{cmd}`",
        f"Summarised by: `python bench.py --workload {args.workload}{path} --projections {args.projections} "
        f"--steps {args.steps} --warmup {args.warmup} --summarize-trace <dir>`",
        "",
        f"Timed region: {args.steps} steps x {L} layers x {groups} request group(s), {len(window)} dispatches "
        f"over {span_ms:.1f} ms "
        f"({span_ms / args.steps:.2f} ms per step under the profiler).",
        f"Attention (`hs_attend_groups`) per launch: attend_mfma_kernel {att_us:.2f} us"
        + (f" + attend_merge_kernel {mrg_us:.2f} us = {att_us + mrg_us:.2f} us (the bench line's HIP events around "
           "the call also hold the dispatch gap between the two kernels)." if mrg else
           " (the last workgroup of each group merges the partials: no merge launch)."),
        "",
        "| kernel | dispatches | total ms | avg us | ms per step |",
        "|---|---|---|---|---|",
    ]
    for name, (count, dur) in sorted(agg.items(), key=lambda x: -x[1][1]):
        lines.append(f"| `{name.replace('hs::', '')}` | {count} | {dur / 1e6:.2f} | {dur / count / 1e3:.2f} | "
                     f"{dur / 1e6 / args.steps:.3f} |")
    out = TRACE_SUMMARIES[args.workload]
    with open(out, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def pmc_traffic(kernels=ROOFLINE_KERNELS, path=PMC_SUMMARY):
    """HBM bytes per launch of `kernels` (sum of those the summary lists) from the committed
    counter summary, or None when it lacks the first (the attention kernel; the merge
    kernel runs only when the attention does not merge its own partials)."""
    if not os.path.exists(path):
        return None
    total, found = 0.0, set()
    for line in open(path):
        parts = line.split()
        if len(parts) == 5 and parts[0] == "kernel":
            for k in kernels:
                if parts[1].startswith(k):
                    total += float(parts[3]) + float(parts[4])
                    found.add(k)
    return total if kernels[0] in found else None


def _sparse_inputs(torch, engine, wl, request=0, layer=0):
    """One (request, layer) of the engine's state as host arrays: the reference CPU path's
    inputs (query drawn at random; bounds, tables and the layer's host pool as they are)."""
    st = engine.state
    P, Hkv, D, C = wl.page_size, wl.kv_heads, wl.head_dim, st.pages
    length = st.lengths[request]
    count = ceil(length / P)
    gen = torch.Generator().manual_seed(5 + 97 * request + layer)
    t = st.tables[layer][request]
    i16 = lambda x: x.detach().cpu().contiguous().view(torch.int16).numpy()
    host = st.host[layer].view(wl.batch, C, 2, P, Hkv, D)[request]
    source = t.source.cpu().numpy().astype(np.int64)
    source = source - int(source[0])  # this request's host pages, numbered from 0 in `host`
    return {
        "q": i16(torch.randn(wl.heads, D, generator=gen).to(wl.dtype)),
        "lo": i16(st.minimum[layer, request, :count]), "hi": i16(st.maximum[layer, request, :count]),
        "source": source, "resident": t.resident.cpu().numpy(),
        "tags": (t.tags.cpu().numpy().astype(np.int64) - int(t.source[0].item()) * P).clip(min=-1),
        "lru": t.lru.cpu().numpy().astype(np.int64), "host": i16(host),
        "meta": np.array([length, P, wl.top_pages, Hkv, D, wl.heads, 1 if wl.selector == "uniform" else 0,
                          t.hot.numel(), 5 + 97 * request + layer], dtype=np.int64),
    }


def _sparse_path(x):
    """The reference CPU path of one (request, layer) on host arrays (``_sparse_inputs``):
    Quest (or the uniform draw), union, resolver, the per-row gather loop into a CPU hot
    region, row attention over the selected rows.  Returns (seconds per stage, misses)."""
    import torch

    from oracle import cpu_path

    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)
    length, P, top, Hkv, D, heads, uniform, hot_blocks, seed = (int(v) for v in x["meta"])
    q, lo, hi, host = bf(x["q"]), bf(x["lo"]), bf(x["hi"]), bf(x["host"])
    hot_pool = torch.empty((hot_blocks, 2, P, Hkv, D), dtype=torch.bfloat16)
    hot = np.arange(hot_blocks, dtype=np.int64)  # the layer's hot blocks, numbered in hot_pool
    tags, lru = np.array(x["tags"]), np.array(x["lru"])
    count = ceil(length / P)
    t = [time.perf_counter()]
    if uniform:  # the tail page and top - 1 uniform others, shared by every head
        rng = np.random.default_rng(seed)
        drawn = np.sort(np.append(rng.choice(count - 1, size=top - 1, replace=False), count - 1))
        tokens = tuple(int(tok) for pg in drawn for tok in range(pg * P, min((pg + 1) * P, length)))
        positions = [tokens] * heads
    else:
        positions = cpu_path.quest_select(q, lo, hi, length, P, top)
    t.append(time.perf_counter())
    union, cols = cpu_path.union_columns(positions)
    t.append(time.perf_counter())
    _, mh, md, counts = cpu_path.resolve(union, cols, x["source"], x["resident"], hot, tags, lru, length, P)
    t.append(time.perf_counter())
    misses = cpu_path.gather_loop(host, hot_pool, mh, md, P)
    t.append(time.perf_counter())
    # the K/V of every selected row, read where its values live in the host pool's layout
    rows = torch.from_numpy(cpu_path.host_rows(positions, x["source"], P))
    t.append(time.perf_counter())
    cpu_path.row_attention(q, host, rows, P, Hkv, D)
    t.append(time.perf_counter())
    stages = {"select": t[1] - t[0], "union": t[2] - t[1], "resolve": t[3] - t[2], "gather_loop": t[4] - t[3],
              "attention": t[6] - t[5]}
    return stages, misses


def _sparse_worker(job):
    """A worker process of the all-cores leg: map the inputs, wait for the start, run."""
    import torch

    torch.set_num_threads(1)
    d, start_at = job
    x = {f[:-4]: np.load(os.path.join(d, f), mmap_mode="r") for f in os.listdir(d) if f.endswith(".npy")}
    while time.time() < start_at:
        time.sleep(0.001)
    t0 = time.perf_counter()
    stages, misses = _sparse_path(x)
    return time.perf_counter() - t0, stages, misses


def _dense_seconds(torch, engine, wl, threads):
    """One dense layer for the batch's tokens plus the LM head, torch fp32 on the host cores
    (q/k/v, o_proj and the SwiGLU MLP; norms and rotary are a few vector ops and left out)."""
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(6)
    layer = engine.model.model.layers[0]
    w = {n: p.detach().float().cpu() for n, p in layer.named_parameters()}
    x = torch.randn(wl.batch, wl.hidden, generator=gen)
    lin = torch.nn.functional.linear
    t0 = time.perf_counter()
    for _ in range(2):
        hq = lin(x, w["self_attn.q_proj.weight"], w["self_attn.q_proj.bias"])
        lin(x, w["self_attn.k_proj.weight"], w["self_attn.k_proj.bias"])
        lin(x, w["self_attn.v_proj.weight"], w["self_attn.v_proj.bias"])
        y = x + lin(hq, w["self_attn.o_proj.weight"])
        g, u = lin(y, w["mlp.gate_proj.weight"]), lin(y, w["mlp.up_proj.weight"])
        y = y + lin(torch.nn.functional.silu(g) * u, w["mlp.down_proj.weight"])
    dense_s = (time.perf_counter() - t0) / 2
    head = engine.model.lm_head.weight.detach()[: wl.vocab // 8].float().cpu()
    t0 = time.perf_counter()
    lin(x, head)
    head_s = (time.perf_counter() - t0) * 8
    return dense_s, head_s


def model_cpu_baseline(torch, engine, wl, budget_s, max_workers=16):
    """The reference CPU path (BASELINE.md's plan), extrapolated to one decode step of the
    workload: per (request, layer) the sparse path of ``oracle.cpu_path`` -- the Quest
    scorer as the reference's torch expression over every page and channel, the Python
    union, the resolver, the per-row gather loop (hybrid.py:466-472) and row attention
    over the selected rows (attention.py:26-35) -- and per layer one dense layer, plus the
    LM head.  Two legs, each labelled with the threads it used:

    * one thread: sparse paths of sampled (request, layer) pairs one after another,
      dense math with ``torch.set_num_threads(1)`` (the reference CLI's setting);
    * all cores: ``workers`` processes (the host's CPU share, at most ``max_workers``)
      each run one sparse path at the same moment, so paths/s = workers / wall time;
      dense math with that many torch threads.

    Per step = layers x batch sparse paths + layers dense layers + LM head."""
    import shutil
    import tempfile
    from concurrent.futures import ProcessPoolExecutor
    from multiprocessing import get_context

    L, B = wl.layers, wl.batch
    workers = max(1, min(max_workers, os.cpu_count() or 1))
    pairs = [(b, l) for l in (0, L // 2, L - 1) for b in (0, B - 1)]
    # leg 1: one thread, sampled (request, layer) pairs within half the budget
    torch.set_num_threads(1)
    samples, stages_sum, misses_sum = [], {}, 0
    t_leg = time.perf_counter()
    for b, l in pairs:
        x = _sparse_inputs(torch, engine, wl, b, l)
        stages, misses = _sparse_path(x)
        samples.append(sum(stages.values()))
        misses_sum += misses
        for k, v in stages.items():
            stages_sum[k] = stages_sum.get(k, 0.0) + v
        if time.perf_counter() - t_leg > budget_s / 2:
            break
    n = len(samples)
    path_s = float(np.mean(samples))
    dense_s, head_s = _dense_seconds(torch, engine, wl, 1)
    step_1 = L * B * path_s + L * dense_s + head_s
    stage_txt = ", ".join(f"{k} {v / n * 1e3:.0f} ms" for k, v in stages_sum.items())
    single = {
        "value": B / step_1, "unit": "tokens/s", "cores": 1, "kind": "port",
        "sample": f"extrapolated from {n} (request, layer) sparse paths run one after another on 1 thread "
                  f"(mean {path_s:.2f} s: {stage_txt}; {misses_sum / n:.0f} rows copied by the gather loop "
                  f"per path) x {L * B} + one dense layer for {B} tokens ({dense_s:.2f} s, torch fp32, 1 thread) "
                  f"x {L} + LM head ({head_s:.2f} s) = {step_1:.1f} s per step",
    }
    # leg 2: all cores, one sparse path per worker process at the same moment
    d = tempfile.mkdtemp(prefix="hs_cpu_path_")
    try:
        for k, v in _sparse_inputs(torch, engine, wl, 0, 0).items():
            np.save(os.path.join(d, k + ".npy"), v)
        with ProcessPoolExecutor(workers, mp_context=get_context("spawn")) as pool:
            list(pool.map(_cpu_worker_ready, range(workers)))
            start_at = time.time() + 2.0
            results = list(pool.map(_sparse_worker, [(d, start_at)] * workers))
    finally:
        shutil.rmtree(d, ignore_errors=True)
    slowest = max(r[0] for r in results)
    paths_per_s = workers / slowest
    dense_all, head_all = _dense_seconds(torch, engine, wl, workers)
    step_all = L * B / paths_per_s + L * dense_all + head_all
    torch.set_num_threads(1)
    return {
        "value": B / step_all, "unit": "tokens/s", "cores": workers, "kind": "port",
        "sample": f"extrapolated: {workers} worker processes (1 thread each) ran the sparse path of (request 0, "
                  f"layer 0) at the same moment, the slowest in {slowest:.2f} s ({paths_per_s:.2f} paths/s: Quest "
                  "scores as the reference's torch expression, Python union, resolver, per-row gather loop, row "
                  f"attention over the selected rows) x {L * B} + one dense layer for {B} tokens ({dense_all:.2f} s, "
                  f"torch fp32, {workers} threads) x {L} + LM head ({head_all:.2f} s) = {step_all:.1f} s per step",
        "single_thread": single,
        "host": platform.processor() or platform.machine(),
        "host_cpus": os.cpu_count(),
    }


class KernelTimer:
    """Durations of attention launches from their own kernel dispatches: before a launch,
    ``arm(i)`` hands event pair i to ``hs_attend_time_next``, so the library launches the
    attention kernel with ``hipExtLaunchKernel`` and the pair is stamped by the dispatch
    itself (start of the attention kernel, end of the launch's last kernel).  That is the
    duration a kernel trace reports, without the queueing and dispatch gaps that events
    recorded on the stream include.  Events are created (by one record each) before the
    timed region."""

    def __init__(self, torch, launches):
        from mini_hisparse_amd import _lib

        self.lib = _lib.load()
        self.start = [torch.cuda.Event(enable_timing=True) for _ in range(launches)]
        self.stop = [torch.cuda.Event(enable_timing=True) for _ in range(launches)]
        for ev in self.start + self.stop:
            ev.record()  # creates the HIP event
        torch.cuda.synchronize()

    def arm(self, i):
        self.lib.hs_attend_time_next(self.start[i], self.stop[i])

    def ms(self, i):
        return self.start[i].elapsed_time(self.stop[i])


class AttendProbe:
    """Timing of every attention launch of the timed steps: its kernels' own duration
    (``KernelTimer``), and the launch's algorithmic bytes from the union launches' own
    entry total (``BatchedDecodeEngine.set_entry_stats``: the union builder adds its
    entry counts to a device counter, so the probe puts no copy into the step) plus
    the per-launch row lists, queries and outputs, known on the host."""

    def __init__(self, torch, device, launches, engine):
        self.torch = torch
        self.engine = engine
        self.kernel = KernelTimer(torch, launches)
        self.entries = torch.zeros(1, dtype=torch.int64, device=device)
        self.widths = []
        self.i = 0

    def __enter__(self):
        self.engine.set_entry_stats(self.entries)
        return self

    def __exit__(self, *exc):
        self.engine.set_entry_stats(None)

    def before_attend(self, layer, stream, dec):
        self.kernel.arm(self.i)

    def after_attend(self, layer, stream, dec):
        self.widths.append((dec.width, dec.batch))
        self.i += 1

    def totals(self, entry_bytes, launch_bytes):
        """(kernel ms, algorithmic bytes, launches) over the launches: ``entry_bytes`` per
        entry read, ``launch_bytes(width, batch)`` per launch."""
        n = self.i
        kernel_ms = sum(self.kernel.ms(i) for i in range(n))
        nbytes = int(self.entries.item()) * entry_bytes + sum(launch_bytes(w, b) for w, b in self.widths)
        return kernel_ms, nbytes, n


def _time_steps(torch, run, steps):
    """Wall time of ``steps`` calls of ``run`` between two device synchronisations.  A
    short spin kernel before and after the region (outside the timing) marks it in
    kernel traces (``summarize_trace``)."""
    torch.cuda._sleep(100)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    torch.cuda._sleep(100)
    return elapsed


def run_model_workload(args, torch, device):
    """End-to-end decode of a Qwen-shape random-init model with the layer-major engine.

    Default (the drop-in path): through the reference's Engine API (``LayerMajorEngine``).
    The batch's random prompts are added as requests and admitted one per step between
    decode turns (each prefilled through the model, its K/V written by hs_append_tokens and
    its pages placed by the hybrid policy); once all run, the timed steps are
    ``Engine.step()`` calls, each returning the step's (request, token) pairs (one read of
    the tokens per step).  The same state then runs as many steps on the engine's
    device-resident token loop (``BatchedDecodeEngine.step``, no read-back per step):
    ``device_loop``.  ``--direct``, ``--synthetic-history`` or ``--residency fraction``:
    every prompt prefilled (or the history written) first, then the device loop only."""
    from dataclasses import replace

    from mini_hisparse_amd.batched_engine import (
        WORKLOADS, BatchedDecodeEngine, build_state, empty_state, host_bytes_per_request, policy_blocks,
        random_model, random_prompts,
    )

    wl = WORKLOADS[args.workload]
    configured = wl.batch
    if args.batch is not None:
        wl = replace(wl, batch=args.batch)
    if args.context is not None:
        wl = replace(wl, context=args.context)
    per_request = host_bytes_per_request(wl)
    fits = int(args.host_budget_gib * 2**30 // per_request)
    if fits < 1:
        raise SystemExit("one request's history exceeds the pinned host budget")
    if wl.batch > fits:
        print(f"[bench] batch {wl.batch} needs {wl.batch * per_request / 2**30:.0f} GiB pinned; "
              f"running batch {fits}", file=sys.stderr, flush=True)
        wl = replace(wl, batch=fits)
    api = not (args.direct or args.synthetic_history or args.residency == "fraction")
    # decode steps a request takes in the run: admission turns, warmup, timed steps, two
    # in-order steps, the profiled step and the device-loop steps
    needed = wl.batch + args.warmup + 2 * args.steps + 4
    if needed > wl.steps:
        raise SystemExit(f"the run needs {needed} decode steps per request, above the workload's {wl.steps}")
    groups = args.request_groups
    if groups is None:
        groups = DEFAULT_REQUEST_GROUPS.get(args.workload, 1)
    options = dict(seed=args.seed, graphs=args.graphs, projections=args.projections,
                   resolver_split=args.resolver_front == "split",
                   prefetch=not args.no_prefetch and wl.selector == "uniform",
                   request_groups=groups if wl.selector == "quest" else 1,
                   group_gather_workgroups=args.group_gather_workgroups if args.group_gather_workgroups is not None
                   else DEFAULT_GROUP_GATHER_WORKGROUPS.get(args.workload, 0))
    t0 = time.perf_counter()
    print(f"[bench] {wl.name}: model + {'synthetic history' if args.synthetic_history else 'prefill'} "
          f"(batch {wl.batch}, {wl.context} tokens, {'Engine API' if api else 'direct'})", file=sys.stderr,
          flush=True)
    model = random_model(wl, device, seed=args.seed)
    prefill_s, admission = None, None
    if api:
        from mini_hisparse_amd.config import CacheConfig
        from mini_hisparse_amd.hybrid import HotConfig
        from mini_hisparse_amd.selection import union_bound
        from mini_hisparse_amd.serving import LayerMajorCache, LayerMajorEngine

        P = wl.page_size
        max_tokens = wl.context + wl.steps
        config = CacheConfig(gpu_pages=policy_blocks(wl), host_pages=wl.batch * wl.layers * ceil(max_tokens / P),
                             page_size=P, kv_heads=wl.kv_heads, head_dim=wl.head_dim, device=str(device),
                             dtype=wl.dtype, index_budget_bytes=1 << 40)
        heads = 1 if wl.selector == "uniform" else wl.heads
        hot = HotConfig(union_bound(max_tokens, P, wl.top_pages, heads), wl.hot_rows)
        cache = LayerMajorCache(config, hot, wl.layers, max_requests=wl.batch, max_tokens=max_tokens)
        api_engine = LayerMajorEngine(model, cache, wl.top_pages, selector=wl.selector, **options)
        engine, state = api_engine.batched, cache.state
        prompts = random_prompts(wl, device, seed=args.seed).cpu()
        for b in range(wl.batch):
            api_engine.add_request(str(b), prompts[b].tolist(), wl.steps)
        del prompts
        print(f"[bench] admitting {wl.batch} requests through Engine.step (one prefill per step)", file=sys.stderr,
              flush=True)
        t_prefill = time.perf_counter()
        admission = 0
        while api_engine.waiting:
            api_engine.step()
            admission += 1
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t_prefill
        step = lambda **kw: api_engine.step(**kw)  # noqa: E731
    else:
        if not args.synthetic_history:
            state = empty_state(wl, device, residency=args.residency)
            print(f"[bench] prefill of {wl.batch} random prompts", file=sys.stderr, flush=True)
            t_prefill = time.perf_counter()
            tokens = state.prefill(model, random_prompts(wl, device, seed=args.seed), wl.resident_fraction,
                                   seed=args.seed)
            prefill_s = time.perf_counter() - t_prefill
        else:
            state = build_state(wl, device, seed=args.seed)
            gen = torch.Generator(device=device).manual_seed(args.seed)
            tokens = torch.randint(0, wl.vocab, (wl.batch,), generator=gen, device=device)
        engine = BatchedDecodeEngine(model, state, wl.top_pages, selector=wl.selector, **options)
        loop = {"tokens": tokens}

        def step(**kw):
            loop["tokens"] = engine.step(loop["tokens"], **kw)

    setup_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        step()
    print("[bench] timing", file=sys.stderr, flush=True)
    stats0 = state.row_stats.clone()
    launches = args.steps * wl.layers * (len(engine.groups) if engine.groups else 1)
    with AttendProbe(torch, device, launches, engine) as probe:
        elapsed = _time_steps(torch, lambda: step(probe=probe), args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    rows = ((state.row_stats - stats0).double() / args.steps).tolist()
    in_order = None
    if engine.groups:
        # the same attention with the batch in one group and no gather running beside it:
        # two extra steps in layer order, outside the timed region
        groups_saved, engine.groups = engine.groups, None
        with AttendProbe(torch, device, 2 * wl.layers, engine) as in_order:
            for _ in range(2):
                step(probe=in_order)
            torch.cuda.synchronize()
        engine.groups = groups_saved
    timer = []
    step(timer=timer)  # profiled step, outside the timed region
    torch.cuda.synchronize()
    device_loop = None
    if api:
        # the same state on the engine's device-resident token loop (no read-back per step)
        loop_tokens = torch.zeros(wl.batch, dtype=torch.int64, device=device)
        for request in api_engine.running:
            loop_tokens[cache.slot_of[request.request_id]] = request.generated[-1]
        loop = {"tokens": loop_tokens}

        def device_step():
            loop["tokens"] = engine.step(loop["tokens"])

        loop_s = _time_steps(torch, device_step, args.steps)
        device_loop = {"value": wl.batch * args.steps / loop_s, "ms_per_step": loop_s * 1e3 / args.steps,
                       "how": "BatchedDecodeEngine.step on the same state after the timed Engine.step calls: "
                              "the tokens stay on the device (no per-step read-back or host-side scheduling)"}
    stage_ms = {}
    for _, marks, _, _ in timer:
        for stage, (start, end) in marks.items():
            stage_ms[stage] = stage_ms.get(stage, 0.0) + start.elapsed_time(end)
    misses = sum(int(m) for _, _, _, m in timer)
    e, D, Hq, B, L = 2, wl.head_dim, wl.heads, wl.batch, wl.layers

    def launch_bytes(width, batch):
        # beside the union-deduplicated K/V rows (2 D e per entry): the per-head row
        # lists, the queries and the outputs
        return 8 * Hq * width * batch + 2 * Hq * D * e * batch

    att_ms, att_bytes, launches = probe.totals(2 * D * e, launch_bytes)
    att_gbs = att_bytes / (att_ms * 1e-3) / 1e9
    solo_line = None
    if in_order is not None:
        solo_ms, solo_bytes, solo_n = in_order.totals(2 * D * e, launch_bytes)
        solo_gbs = solo_bytes / (solo_ms * 1e-3) / 1e9
        solo_line = {"achieved": solo_gbs, "frac": solo_gbs / HBM_PEAK_GBS, "launches": solo_n,
                     "bytes_per_launch": solo_bytes / solo_n, "us_per_launch": solo_ms * 1e3 / solo_n,
                     "how": "two extra steps after the timed region with the whole batch in one group, "
                            "in layer order (no gather running beside the attention); kernel duration "
                            "from dispatch-stamped events"}
    pmc_path = PMC_SUMMARIES.get(args.workload, (None,))[0]
    profiled = PMC_CONFIG.get(args.workload)
    traffic = pmc_traffic(ROOFLINE_KERNELS, pmc_path) if pmc_path and profiled == (
        wl.batch, len(engine.groups) if engine.groups else 1) and wl.context == WORKLOADS[args.workload].context \
        else None
    row_bytes = 2 * wl.kv_heads * D * e
    gather_bytes = misses * row_bytes
    link = host_link_gbs(torch, device)
    # the step's floor: the HBM bytes it must move (weights once per request group, the
    # Quest bounds of every page, the attention's rows, the gathered rows written) at
    # 8 TB/s, or the gathered rows at the measured host-link rate, whichever is longer
    embed = model.model.embed_tokens.weight
    tied = model.lm_head.weight.data_ptr() == embed.data_ptr()
    weight_bytes = sum(t.numel() * t.element_size() for t in model.parameters()
                       if tied or t.data_ptr() != embed.data_ptr())
    pages_read = sum(ceil(state.lengths[b] / wl.page_size) for b in range(wl.batch)) * wl.layers
    hbm_bytes = (weight_bytes * (len(engine.groups) if engine.groups else 1) + pages_read * 2 * wl.kv_heads * D * e
                 + att_bytes / args.steps + gather_bytes)
    hbm_ms, host_ms = hbm_bytes / (HBM_PEAK_GBS * 1e9) * 1e3, gather_bytes / (link * 1e9) * 1e3
    step_roofline = {"hbm_bytes": hbm_bytes, "host_link_bytes": gather_bytes, "hbm_ms": hbm_ms,
                     "host_link_ms": host_ms, "bound": "host link" if host_ms > hbm_ms else "hbm",
                     "frac": max(hbm_ms, host_ms) / ms_per_step,
                     "how": "max(HBM bytes / 8 TB/s, gathered bytes / measured pinned memcpy rate) / ms_per_step; "
                            "HBM bytes: weights (once per request group), every page's Quest bounds, the "
                            "attention's rows, the gathered rows written"}
    copy = hbm_copy_gbs(torch, device)  # also the counter runs' calibration kernel
    result = {
        "metric": METRIC,
        "value": wl.batch * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": (f"synthetic: random-init {wl.name} weights; {wl.context}-token uniformly random prompts "
                 "prefilled through the model (causal SDPA; K/V, bounds and resident pages written by "
                 "hs_append_tokens); greedy decode from the prefill's tokens" if not args.synthetic_history else
                 f"synthetic: random-init {wl.name} weights; {wl.context}-token K/V histories (N(0,1), 2% "
                 "channels x8) written directly instead of a prefill; greedy decode from random tokens"),
        "config": {
            "workload": f"{wl.name} end to end (layer-major batched engine"
            + (", through the Engine API: requests admitted one per step, timed Engine.step() calls" if api else "")
            + f"): {wl.layers} layers, hidden "
            f"{wl.hidden}, {wl.heads} q / {wl.kv_heads} kv heads, head_dim {wl.head_dim}, FFN {wl.ffn}, "
            f"batch {wl.batch}, {wl.context}-token histories, "
            + (f"Quest top-{wl.top_pages} pages, " if wl.selector == "quest" else
               f"{wl.top_pages} pages resampled uniformly each step (tail page forced), shared by every head, ")
            + (f"hybrid residency policy (window 64 pages, default watermark) over a slab of "
               f"{state.blocks} blocks = {wl.resident_fraction:.0%} of the history + every layer's hot region "
               f"and two tails, hot_rows {wl.hot_rows}" if state.plan is not None else
               f"{wl.resident_fraction:.0%} of pages resident, hot_rows {wl.hot_rows}")
            + ("; dense layer boundaries replayed as HIP graphs" if engine.use_graphs else "")
            + (f"; {len(engine.groups)} request groups pipelined across layers (a group's gather on a transfer "
               "stream overlaps the other groups' compute)" if engine.groups else "")
            + ("; every layer's select/resolve/gather prefetched on a transfer stream at step start "
               "(stage times of those overlap the dense layers)" if engine.prefetch else "")
            + (f"; batch cut from {configured}: {configured} histories need "
               f"{configured * per_request / 2**30:.0f} GiB of pinned host memory, the box pins at most "
               f"64 GiB (budget {args.host_budget_gib:g} GiB)" if wl.batch < configured else ""),
            "global_batch": wl.batch,
            "seq_len": wl.context,
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": att_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": att_gbs / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": f"{ATTENTION_KERNELS} (hs_attend_groups), every layer of the timed steps"
            + (" (one launch per request group, beside the other group's gather)" if engine.groups else ""),
            "timing": "each launch's own kernel duration: HIP events stamped by the dispatch "
                      "(hipExtLaunchKernel via hs_attend_time_next), the figure a kernel trace reports",
            "launches": launches,
            "bytes_per_launch": att_bytes / launches,
            "us_per_launch": att_ms * 1e3 / launches,
            "in_order": solo_line,
        },
        "step_roofline": step_roofline,
        "device_loop": device_loop,
        "stages_ms_per_step": stage_ms,
        "projections_on_hs_skinny_gemm": engine.projection_kernel,
        "projection_choice_ms": engine.projection_times,  # each side's device ms over the layers' weights
        "rows_per_step": {"resident_hits": rows[0], "hot_hits": rows[1], "misses": rows[2]},
        "gather": {"bytes_per_step": gather_bytes, "GBps": gather_bytes / (stage_ms["gather"] * 1e-3) / 1e9,
                   "host_link_memcpy_GBps": link,
                   "frac_host_link": gather_bytes / (stage_ms["gather"] * 1e-3) / 1e9 / link},
        "setup_s": setup_s,
        "prefill_s": prefill_s,
        "admission_steps": admission,
        "placement": None if state.plan is None else {
            "resident_pages_per_request": [
                sum(int((state.plan.group((b, l)).slot >= 0).sum()) for l in range(wl.layers))
                for b in range(wl.batch)],
            "policy_counters": {k: int(v) for k, v in state.plan.stats.items()}},
        "hbm_copy_GBps": copy,
    }
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline (extrapolated)", file=sys.stderr, flush=True)
        result["cpu_baseline"] = model_cpu_baseline(torch, engine, wl, args.cpu_budget)
    else:
        result["cpu_baseline"] = None
    return result


def run_per_request_engine(args, torch, device):
    """The same model workload through the reference-shaped per-request stack:
    ``Engine(model, HybridKVCache(...))`` (engine.py:36-146, hybrid.py), whose decode turn
    runs one request's layers in turn (append, Quest selection, resolve, gather and
    attention per (request, layer), each on the HIP library).  The batch's prompts are
    admitted one per step; the timed steps are ``Engine.step()`` calls once every request
    runs.  The slab, host pool, hot bound and hot rows are the layer-major leg's."""
    from dataclasses import replace

    from mini_hisparse_amd.batched_engine import WORKLOADS, policy_blocks, random_model, random_prompts
    from mini_hisparse_amd.cli import union_rows_bound
    from mini_hisparse_amd.config import CacheConfig
    from mini_hisparse_amd.engine import Engine
    from mini_hisparse_amd.hybrid import HotConfig, HybridKVCache

    wl = WORKLOADS[args.workload]
    if args.batch is not None:
        wl = replace(wl, batch=args.batch)
    if args.context is not None:
        wl = replace(wl, context=args.context)
    if wl.selector != "quest":
        raise SystemExit("the per-request Engine selects with Quest or page means; this workload samples uniformly")
    needed = wl.batch + args.warmup + args.steps
    if needed > wl.steps:
        raise SystemExit(f"the run needs {needed} decode steps per request, above the workload's {wl.steps}")
    P = wl.page_size
    model = random_model(wl, device, seed=args.seed)
    config = CacheConfig(gpu_pages=policy_blocks(wl), host_pages=wl.batch * wl.layers * ceil((wl.context + wl.steps) / P),
                         page_size=P, kv_heads=wl.kv_heads, head_dim=wl.head_dim, device=str(device), dtype=wl.dtype,
                         index_budget_bytes=1 << 40)
    hot = HotConfig(union_rows_bound(wl.context, wl.steps, wl.top_pages, wl.heads, P), wl.hot_rows)
    cache = HybridKVCache(config, hot)
    engine = Engine(model, cache, wl.top_pages, selector="quest")
    prompts = random_prompts(wl, device, seed=args.seed).cpu()
    for b in range(wl.batch):
        engine.add_request(str(b), prompts[b].tolist(), wl.steps)
    del prompts
    print(f"[bench] {wl.name}: per-request Engine over HybridKVCache, admitting {wl.batch} requests",
          file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    admission = 0
    while engine.waiting:
        engine.step()
        admission += 1
        print(f"[bench] admission step {admission}: {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        engine.step()
    print("[bench] timing", file=sys.stderr, flush=True)
    emitted = []
    elapsed = _time_steps(torch, lambda: emitted.extend(engine.step()), args.steps)
    if len(emitted) != wl.batch * args.steps:
        raise SystemExit(f"expected {wl.batch * args.steps} tokens from the timed steps, got {len(emitted)}")
    return {
        "metric": METRIC,
        "value": len(emitted) / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": (f"synthetic: random-init {wl.name} weights; {wl.context}-token uniformly random prompts "
                 "prefilled through the model; greedy decode"),
        "config": {
            "workload": f"{wl.name} end to end through the per-request Engine over HybridKVCache (every "
                        f"(request, layer) decoded in turn): {wl.layers} layers, batch {wl.batch}, "
                        f"{wl.context}-token histories, Quest top-{wl.top_pages} pages, slab of "
                        f"{config.gpu_pages} blocks, hot_rows {wl.hot_rows}",
            "global_batch": wl.batch,
            "seq_len": wl.context,
            "parallelism": "none (1 GPU)",
        },
        "roofline": None,
        "cpu_baseline": None,
        "why_no_roofline": "a comparison leg: the layer-major line of the same workload carries the roofline "
                           "and CPU baseline",
        "admission_steps": admission,
        "prefill_s": prefill_s,
        "row_stats": [int(v) for v in cache.row_stats.tolist()],
    }


def main():
    args = parse_args()
    if args.summarize_trace:
        if args.workload in SHAPES:
            summarize_layer_trace(args.summarize_trace, args)
        else:
            summarize_trace(args.summarize_trace, args)
        return
    if args.summarize_pmc:
        if args.workload not in PMC_SUMMARIES:
            raise SystemExit(f"counter summaries are kept for {sorted(PMC_SUMMARIES)}")
        summarize_pmc(*args.summarize_pmc, workload=args.workload)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus above 1 is not supported "
                          "(the decode path would shard by request, one GPU per request set)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    device = torch.device("cuda:0")
    if args.attention_sweep:
        attention_sweep(torch, device)
        return
    if args.engine == "per-request":
        if args.workload in SHAPES:
            raise SystemExit("--engine per-request runs a model workload")
        print(json.dumps(run_per_request_engine(args, torch, device)))
        return
    if args.workload not in SHAPES:
        result = run_model_workload(args, torch, device)
        if args.workload == "qwen2.5-7b" and not args.no_microbench:
            import gc

            gc.collect()  # frees the 7B histories' pinned memory before the microbench pins its own
            torch.cuda.empty_cache()
            mb_args = argparse.Namespace(**vars(args))
            mb_args.workload, mb_args.batch = "microbench", None
            mb = run_microbench(mb_args, torch, device)
            result["microbench"] = {k: mb[k] for k in ("value", "unit", "ms_per_step", "config", "roofline",
                                                       "kernels", "rows", "cpu_baseline", "parity") if k in mb}
        print(json.dumps(result))
        return
    print(json.dumps(run_microbench(args, torch, device)))


def run_microbench(args, torch, device):
    """The isolated kernel microbench (configs[1], or the same step at the 7B layer shape)."""
    shape = SHAPES[args.workload]
    if args.batch is None:
        args.batch = shape.batch
    print(f"[bench] building workload (batch {args.batch})", file=sys.stderr, flush=True)
    w = build_workload(args, torch, device)
    w["use_transfer_stream"] = args.transfer_stream or args.parts > 1
    run_pipelined(torch, w, args.warmup)
    torch.cuda.synchronize()
    print("[bench] timing", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    run_pipelined(torch, w, args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    # per-stage times, the roofline and the CPU parity check from the same step run
    # without the overlap (every stage of the whole batch timed on its own stream)
    run_steps(torch, w, 2, record=False)
    events = run_steps(torch, w, args.steps, record=True)
    torch.cuda.synchronize()
    stages = stage_ms(events, w["attention_kernel"])
    sequential_ms = float(np.mean([e[0].elapsed_time(e[6]) for e in events]))
    diff = (w["pipe_out"].float() - w["out"].float()).abs().max().item()
    bytes_ = algorithmic_bytes(w, torch)
    link = host_link_gbs(torch, device)
    copy = hbm_copy_gbs(torch, device)
    ceilings = attention_ceilings(torch, w, bytes_["attention"])
    att_gbs = bytes_["attention"] / (stages["attention"] * 1e-3) / 1e9
    # the committed counter summary of this workload, when its shape is the one profiled
    pmc_path = PMC_SUMMARIES[args.workload][0] if args.workload in PMC_SUMMARIES else None
    counters_apply = pmc_path is not None and args.batch == shape.batch

    def hbm_line(stage, nbytes, pmc_kernels, **extra):
        """A stage's algorithmic-byte rate and, from the committed counter summary, the HBM
        bytes its kernels move per launch and the rate those give (the counter evidence)."""
        ms = stages[stage]
        gbs = nbytes / (ms * 1e-3) / 1e9
        traffic = pmc_traffic(pmc_kernels, pmc_path) if counters_apply else None
        line = {"ms": ms, "bytes": nbytes, "GBps": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
                "hbm_traffic_bytes": traffic,
                "hbm_traffic_GBps": None if traffic is None else traffic / (ms * 1e-3) / 1e9,
                "kernels": list(pmc_kernels)}
        line.update(extra)
        return line

    kernels = {
        "attention": hbm_line("attention", bytes_["attention"], ROOFLINE_KERNELS,
                              per_head_bytes=bytes_["attention_per_head"],
                              timing="the launch's own kernel duration (dispatch-stamped HIP events, "
                                     "hs_attend_time_next); median over the recorded steps",
                              event_window_ms=stages["attention_event_window"]),
        "quest_and_union": hbm_line("quest_and_union", bytes_["quest"],
                                    ("quest_score", "quest_topk_kernel", "build_union_kernel")),
        # the split front's three launches at these lengths (above 40,000 tokens), else the one front launch
        "resolve": hbm_line("resolve", bytes_["resolver"],
                            ("resolve_split", "resolve_outputs_kernel") if args.resolver_front == "split"
                            else ("resolve_front_kernel", "resolve_outputs_kernel")),
        "gather": {"ms": stages["gather"], "bytes": bytes_["gather"],
                   "GBps": bytes_["gather"] / (stages["gather"] * 1e-3) / 1e9,
                   "host_link_memcpy_GBps": link,
                   "frac_host_link": bytes_["gather"] / (stages["gather"] * 1e-3) / 1e9 / link},
    }
    result = {
        "metric": METRIC,
        "value": args.batch / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded K/V ~ N(0,1), 2% channels x8; random-init tables)",
        "config": {
            "workload": f"{shape.label}, batch {args.batch}, Quest top-{shape.top}, "
            "50% resident / 30% hot / 20% miss; "
            + (f"{args.parts} request groups overlapped" if args.parts > 1 else
               "gather on a transfer stream ordered by events" if args.transfer_stream else
               "every stage on one stream"),
            "global_batch": args.batch,
            "seq_len": w["length"],
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": att_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": att_gbs / HBM_PEAK_GBS,
            "traffic": pmc_traffic(ROOFLINE_KERNELS, pmc_path) if counters_apply else None,
            "kernel": f"{ATTENTION_KERNELS} (hs_attend_groups)",
            "measured_ceilings": ceilings,
        },
        "kernels": kernels,
        "rows": {**w["stats"], "misses_per_step": bytes_["misses"], "attention_entries": bytes_["entries"]},
        "step_without_overlap_ms": sequential_ms,
        "overlapped_vs_sequential_max_abs_diff": diff,
        "hbm_copy_GBps": copy,
    }
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base, parity = cpu_baseline(torch, w, args.cpu_budget)
        print("[bench] cpu baseline, all cores", file=sys.stderr, flush=True)
        try:
            base["all_cores"] = cpu_baseline_all_cores(torch, w)
        except OSError as exc:  # no room for the mapped inputs on this host
            base["all_cores"] = {"value": None, "error": str(exc)}
        result["cpu_baseline"] = base
        result["parity"] = parity
    else:
        result["cpu_baseline"] = None
    return result


if __name__ == "__main__":
    main()
