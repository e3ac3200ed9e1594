"""Write golden vectors from the reference implementation (run in the build container only).

    python tests/golden/make_golden.py /path/to/reference

Imports the reference package (mini_hisparse 0.2.0, CPU path, torch ops) and
records, as small JSON fixtures next to this script:

* resolver_trajectories.json -- multi-step ``resolve_rows`` runs on seeded
  tables (tags and LRU carried between steps), every output of every step;
* quest_selections.npz       -- ``quest_selection`` chosen pages on seeded
  bf16 / fp32 bounds, with the reference's own fp32 scores' k-th/(k+1)-th
  margin per head;
* demo_outputs.json          -- the reference CLI ``demo`` (CPU, fp32):
  generated tokens, row statistics and counters for a few settings.
* paged_demo_outputs.json    -- the same CLI with the optional page layout
  (``--cache-layout pages``, reference/cache.py): tokens, counters and page
  locations under each eviction policy, with and without window overlap.

These are the functions no reference test or closed form pins.  The fixtures
are data; nothing under tests/ or the product reads the reference at run time.
"""

from __future__ import annotations

import contextlib
import io
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def resolver_trajectories(reference_row_index):
    LogicalTopK, resolve_rows = reference_row_index.LogicalTopK, reference_row_index.resolve_rows
    cases = []
    for seed, (length, P, S, steps, n, heads) in enumerate(
        [(97, 4, 64, 6, 30, None), (300, 7, 128, 5, 60, 3), (1000, 16, 256, 6, 120, 4), (50, 3, 30, 8, 25, None)]
    ):
        rng = np.random.default_rng(1000 + seed)
        pages = -(-length // P)
        source = rng.permutation(pages * 3)[:pages].astype(np.int32)
        resident = np.full(pages, -1, np.int32)
        is_res = rng.random(pages) < 0.4
        resident[is_res] = rng.permutation(pages * 2)[: is_res.sum()]
        hot = (rng.permutation(64) + pages * 2)[: -(-S // P)].astype(np.int32)
        tags = torch.full((S,), -1, dtype=torch.int32)
        lru = torch.from_numpy(rng.permutation(S).astype(np.int64))
        case = {"length": length, "page_size": P, "source": source.tolist(), "resident": resident.tolist(),
                "hot": hot.tolist(), "tags0": tags.tolist(), "lru0": lru.tolist(), "steps": []}
        for _ in range(steps):
            if heads is None:
                positions = rng.integers(-2, length + 3, size=n)
                dup = rng.random(n) < 0.1
                positions[dup] = positions[rng.integers(0, n, size=dup.sum())]
                topk = LogicalTopK(torch.tensor(positions, dtype=torch.int64))
                columns = None
            else:
                rows = [sorted(set(rng.integers(0, length, size=n // heads).tolist())) for _ in range(heads)]
                union = sorted({t for r in rows for t in r})
                col = {t: i for i, t in enumerate(union)}
                width = max(map(len, rows))
                columns = [[col[t] for t in r] + [-1] * (width - len(r)) for r in rows]
                positions = np.asarray(union)
                topk = LogicalTopK(torch.tensor(union, dtype=torch.int32), torch.tensor(columns, dtype=torch.int64))
            plan = resolve_rows(topk, torch.from_numpy(source), torch.from_numpy(resident), torch.from_numpy(hot),
                                tags, lru, length, P)
            case["steps"].append({
                "positions": positions.tolist(), "head_columns": columns,
                "physical": plan.physical_rows.tolist(), "miss_host": plan.miss_host_rows.tolist(),
                "miss_device": plan.miss_device_rows.tolist(), "counts": plan.counts.tolist(),
                "tags": tags.tolist(), "lru": lru.tolist(),
            })
        cases.append(case)
    return cases


def quest_selections(reference_selection):
    quest = reference_selection.quest_selection
    cases = []
    for seed, (pages, P, kv, g, D, top, sink, dtype, tail) in enumerate(
        [(160, 16, 2, 4, 64, 16, True, "bfloat16", 16), (100, 16, 2, 7, 64, 24, True, "bfloat16", 5),
         (120, 4, 1, 2, 8, 7, True, "float32", 3), (64, 16, 2, 3, 32, 10, False, "bfloat16", 16)]
    ):
        gen = torch.Generator().manual_seed(2000 + seed)
        dt = getattr(torch, dtype)
        length = (pages - 1) * P + tail
        k = torch.randn(pages * P, kv, D, generator=gen)
        k[..., torch.randperm(D, generator=gen)[: max(1, D // 50)]] *= 8
        k = k.to(dt)[:length]
        lo = torch.stack([k[p * P : (p + 1) * P].amin(0) for p in range(pages)])
        hi = torch.stack([k[p * P : (p + 1) * P].amax(0) for p in range(pages)])
        q = torch.randn(kv * g, D, generator=gen).to(dt)
        selection = quest(q, lo, hi, length, P, top, keep_sink=sink)
        chosen = [sorted({t // P for t in row}) for row in selection.positions]
        # the reference's own fp32 scores (selection.py:92-95), for the tie margin
        groups = g
        low = lo.repeat_interleave(groups, 1).transpose(0, 1).float()
        high = hi.repeat_interleave(groups, 1).transpose(0, 1).float()
        scores = torch.maximum(q.float()[:, None] * low, q.float()[:, None] * high).sum(-1)
        scores[:, [pages - 1] + ([0] if sink and top > 1 else [])] = torch.inf
        ordered = scores.sort(-1, descending=True).values
        margin = (ordered[:, top - 1] - ordered[:, top]).tolist()
        cases.append({"pages": pages, "page_size": P, "kv_heads": kv, "groups": g, "head_dim": D, "top": top,
                      "keep_sink": sink, "dtype": dtype, "length": length,
                      "query": q.float().numpy(), "minimum": lo.float().numpy(), "maximum": hi.float().numpy(),
                      "chosen": np.asarray(chosen, dtype=np.int32), "margin": np.asarray(margin, dtype=np.float32)})
    return cases


def save_quest(cases, path):
    arrays = {}
    for i, case in enumerate(cases):
        for key, value in case.items():
            arrays[f"{i}/{key}"] = np.asarray(value)
    np.savez_compressed(path, **arrays)


def demo_outputs(reference_cli):
    settings = [
        ["demo", "--device", "cpu", "--top-k", "2", "--prompt-tokens", "257", "--gpu-pages", "12",
         "--requests", "1", "--max-new-tokens", "17"],
        ["demo", "--device", "cpu", "--top-k", "2", "--prompt-tokens", "65", "--gpu-pages", "12",
         "--requests", "1", "--max-new-tokens", "3"],  # reference tests/test_runtime_boundary.py
        ["demo", "--device", "cpu", "--top-k", "4", "--prompt-tokens", "90", "--requests", "3",
         "--max-new-tokens", "9"],  # Quest scoring with default admission-sized pool
        ["demo", "--device", "cpu", "--top-k", "3", "--prompt-tokens", "120", "--requests", "2",
         "--max-new-tokens", "8", "--gpu-pages", "60", "--resident-window-pages", "4"],  # window-triggered hot regions
    ]
    results = []
    for argv in settings:
        sys.argv = ["mini-hisparse", *argv]
        out = io.StringIO()
        with contextlib.redirect_stdout(out):
            reference_cli.main()
        report = json.loads(out.getvalue())
        results.append({"argv": argv, "outputs": report["outputs"], "requests": report["requests"],
                        "row_stats": report["row_stats"], "stats": report["stats"],
                        "locations": report["locations"], "final_timeline": report["timeline"][-1]})
    return results


def paged_demo_outputs(reference_cli):
    base = ["demo", "--device", "cpu", "--cache-layout", "pages", "--prompt-tokens", "70", "--requests", "2",
            "--max-new-tokens", "6"]
    settings = [
        base + ["--top-k", "3", "--gpu-pages", "6"],  # fair_lru, overlapping windows of 2 pages
        base + ["--top-k", "3", "--gpu-pages", "6", "--eviction-policy", "lru", "--no-overlap"],
        base + ["--top-k", "4", "--gpu-pages", "5", "--eviction-policy", "legacy", "--chunk-pages", "3"],
        base + ["--gpu-pages", "4"],  # every page, windows under pressure
    ]
    results = []
    for argv in settings:
        sys.argv = ["mini-hisparse", *argv]
        out = io.StringIO()
        with contextlib.redirect_stdout(out):
            reference_cli.main()
        report = json.loads(out.getvalue())
        results.append({"argv": argv, "outputs": report["outputs"], "requests": report["requests"],
                        "stats": report["stats"], "locations": report["locations"],
                        "final_timeline": report["timeline"][-1]})
    return results


def main():
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    only = set(sys.argv[2:])  # optional fixture names: write only these
    sys.path.insert(0, reference)
    torch.set_num_threads(1)
    from mini_hisparse import cli, row_index, selection  # the reference package

    if not only or "quest_selections.npz" in only:
        save_quest(quest_selections(selection), os.path.join(HERE, "quest_selections.npz"))
        print("quest_selections.npz", os.path.getsize(os.path.join(HERE, "quest_selections.npz")), "bytes")
    makers = {
        "resolver_trajectories.json": lambda: resolver_trajectories(row_index),
        "demo_outputs.json": lambda: demo_outputs(cli),
        "paged_demo_outputs.json": lambda: paged_demo_outputs(cli),
    }
    fixtures = {name: make() for name, make in makers.items() if not only or name in only}
    for name, data in fixtures.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump({"generated_by": "tests/golden/make_golden.py from mini-hisparse 0.2.0 (CPU)", "cases": data}, f)
        print(name, os.path.getsize(os.path.join(HERE, name)), "bytes")


if __name__ == "__main__":
    main()
