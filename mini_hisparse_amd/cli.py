"""Command line: ``demo`` (tiny random decoder), ``generate`` (local Qwen2 checkpoint) and
``bench`` (KV microbenchmark of the page layout).

Flags and the JSON report follow the reference CLI (cli.py:24-214).  The
kernels run on the ROCm device; ``--backend`` accepts ``auto`` or ``hip``.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch

from .attention import BACKENDS
from .config import CacheConfig
from .engine import Engine
from .hybrid import HotConfig, HybridKVCache
from .model import MiniModel


def _top_k(value):
    if value == "all":
        return None
    result = int(value)
    if result < 1:
        raise argparse.ArgumentTypeError("top-k must be 'all' or a positive page count")
    return result


def build_parser():
    parser = argparse.ArgumentParser(description="Mini-HiSparse on MI355X: decode through partial KV residency")
    sub = parser.add_subparsers(dest="command", required=True)
    for name in ("demo", "generate", "bench"):
        command = sub.add_parser(name)
        command.add_argument("--device", default="cuda:0")
        command.add_argument("--gpu-pages", type=int)
        command.add_argument("--host-pages", type=int, default=4096)
        command.add_argument("--page-size", type=int, default=16)
        command.add_argument("--backend", choices=list(BACKENDS), default="auto")
        command.add_argument("--dtype", choices=["float32", "float16", "bfloat16"], default="float32")
        command.add_argument("--output", type=Path)
        command.add_argument("--index-budget-mib", type=int, default=64)
        command.add_argument("--chunk-pages", type=int, default=2, help="pages layout only")
        command.add_argument("--eviction-policy", choices=["legacy", "lru", "fair_lru"], default="fair_lru",
                             help="pages layout only; hybrid uses request/layer-local row LRU")
        if name == "bench":  # experiments/benchmark.py of the reference, on the page layout
            command.add_argument("--tokens", type=int, default=1024)
            command.add_argument("--steps", type=int, default=20)
            command.add_argument("--requests", type=int, default=3)
            command.add_argument("--selected-pages", type=int, default=8)
            continue
        command.add_argument("--max-union-rows", type=int)
        command.add_argument("--hot-rows", type=int)
        command.add_argument("--resident-window-pages", type=int, default=64)
        command.add_argument("--hot-watermark", type=int)
        command.add_argument("--top-k", type=_top_k, default=None, help="page count, or all (default)")
        command.add_argument("--max-new-tokens", type=int, default=12)
        command.add_argument("--selector", choices=["quest", "mean"], default="quest")
        command.add_argument("--cache-layout", choices=["hybrid", "pages"], default="hybrid")
        command.add_argument("--no-overlap", action="store_true", help="pages layout only")
        if name == "generate":
            command.add_argument("--model", required=True, help="local Qwen2/2.5 directory")
            command.add_argument("--prompt", default="Explain how a KV cache works.")
            command.add_argument("--chat", action="store_true", help="apply the tokenizer's chat template")
        else:
            command.add_argument("--requests", type=int, default=3)
            command.add_argument("--prompt-tokens", type=int, default=65)
    return parser


def union_rows_bound(prompt_length, max_new_tokens, top_k, heads, page_size):
    """Hot union bound U (cli.py:136-143): sink/tail pages shared, the rest per head."""
    maximum = prompt_length + max_new_tokens
    if top_k is not None:
        forced = min(2, top_k)
        maximum = min(maximum, (forced + (top_k - forced) * heads) * page_size)
    return maximum


def run(args, parser=None, ops=None):
    torch.manual_seed(42)
    dtype = getattr(torch, args.dtype)
    if args.command == "bench":
        from .layout_bench import benchmark
        from .paged import PagedConfig

        config = PagedConfig(
            gpu_pages=args.gpu_pages if args.gpu_pages is not None else 8,
            host_pages=args.host_pages,
            page_size=args.page_size,
            device=args.device,
            dtype=dtype,
            index_budget_bytes=args.index_budget_mib * 1024 * 1024,
            chunk_pages=args.chunk_pages,
            eviction_policy=args.eviction_policy,
        )
        return benchmark(config, args.tokens, args.steps, args.requests, args.selected_pages, args.backend, ops=ops)
    tokenizer = None
    if args.command == "generate":
        from transformers import AutoTokenizer

        model = MiniModel.from_pretrained(args.model, args.device, dtype)
        tokenizer = AutoTokenizer.from_pretrained(args.model)
        if args.chat:
            prompt = tokenizer.apply_chat_template(
                [{"role": "user", "content": args.prompt}], tokenize=True, add_generation_prompt=True, return_dict=False
            )
        else:
            prompt = tokenizer.encode(args.prompt)
        prompts = [prompt]
    else:
        if args.requests < 1 or args.prompt_tokens < 1:
            (parser.error if parser else ValueError)("requests and prompt-tokens must be positive")
        model = MiniModel().eval().to(device=args.device, dtype=dtype)
        prompts = [
            torch.randint(0, model.config.vocab_size, (args.prompt_tokens + i * 7,)).tolist()
            for i in range(args.requests)
        ]
    cfg = model.config
    common = dict(
        host_pages=args.host_pages,
        page_size=args.page_size,
        kv_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim,
        device=args.device,
        dtype=dtype,
        index_budget_bytes=args.index_budget_mib * 1024 * 1024,
    )
    if args.cache_layout == "pages":  # whole-page windows (cli.py:155-165)
        from .paged import PagedConfig, PagedKVCache

        paged_cfg = PagedConfig(
            gpu_pages=args.gpu_pages if args.gpu_pages is not None else 8,
            chunk_pages=args.chunk_pages,
            overlap=not args.no_overlap,
            eviction_policy=args.eviction_policy,
            **common,
        )
        cache = PagedKVCache(paged_cfg, ops=ops)
    else:
        heads = cfg.num_attention_heads if args.selector == "quest" else 1
        bound = union_rows_bound(max(map(len, prompts)), args.max_new_tokens, args.top_k, heads, args.page_size)
        hot = HotConfig(
            bound if args.max_union_rows is None else args.max_union_rows,
            args.hot_rows,
            resident_window_pages=args.resident_window_pages,
            transition_watermark=args.hot_watermark,
        )
        gpu_pages = args.gpu_pages if args.gpu_pages is not None else hot.admission_blocks(args.page_size, cfg.num_hidden_layers)
        cache = HybridKVCache(CacheConfig(gpu_pages=gpu_pages, **common), hot, ops=ops)
    engine = Engine(model, cache, args.top_k, args.backend, tokenizer.eos_token_id if tokenizer else None,
                    selector=args.selector)
    for i, prompt in enumerate(prompts):
        engine.add_request(str(i), prompt, args.max_new_tokens)
    timeline = []
    while engine.waiting or engine.running:
        engine.step()
        timeline.append(
            {
                "active": len(engine.running),
                "waiting": len(engine.waiting),
                "locations": cache.snapshot()["locations"],
                "generated": {name: len(r.generated) for name, r in engine.requests.items()},
            }
        )
    outputs = {name: r.generated for name, r in engine.requests.items()}
    cache.collect(wait=True)
    result = {
        "model": args.model if tokenizer else "tiny random decoder (mechanics demo)",
        "selection": "full attention" if args.top_k is None
        else f"{args.selector}: approximate top-{args.top_k} pages per selection head",
        "outputs": {
            name: tokenizer.decode(tokens, skip_special_tokens=True) if tokenizer else tokens
            for name, tokens in outputs.items()
        },
        "requests": {
            name: {"prefill_count": r.prefill_count, "decode_count": r.decode_count, "generated_tokens": len(r.generated)}
            for name, r in engine.requests.items()
        },
        "timeline": timeline,
        **cache.snapshot(),
    }
    cache.assert_invariants()
    return result


def main(argv=None):
    parser = build_parser()
    args = parser.parse_args(argv)
    torch.set_num_threads(1)
    result = run(args, parser)
    serialized = json.dumps(result, indent=2, ensure_ascii=False)
    print(serialized)
    if args.output:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(serialized + "\n")


if __name__ == "__main__":
    main()
