"""Command line: ``demo`` (tiny random decoder) and ``generate`` (local Qwen2 checkpoint).

The flags and the JSON report are the reference CLI's interface
(``mini_hisparse/cli.py:24-214``); the kernels run on the ROCm device and
``--backend`` accepts ``auto`` or ``hip``.  The reference's ``bench`` subcommand
times its optional page layout in ``experiments/benchmark.py``, outside the
sparse decode path this package replaces, and is not provided; ``bench.py`` at
the repository root measures the decode path.
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


# (flag, keyword arguments) shared by both commands, then per command
_COMMON = [
    ("--device", dict(default="cuda:0")),
    ("--gpu-pages", dict(type=int)),
    ("--host-pages", dict(type=int, default=4096)),
    ("--page-size", dict(type=int, default=16)),
    ("--backend", dict(choices=list(BACKENDS), default="auto")),
    ("--dtype", dict(choices=["float32", "float16", "bfloat16"], default="float32")),
    ("--output", dict(type=Path)),
    ("--index-budget-mib", dict(type=int, default=64)),
    ("--chunk-pages", dict(type=int, default=2, help="pages layout only")),
    ("--eviction-policy", dict(choices=["legacy", "lru", "fair_lru"], default="fair_lru",
                               help="pages layout only; hybrid uses request/layer-local row LRU")),
    ("--max-union-rows", dict(type=int)),
    ("--hot-rows", dict(type=int)),
    ("--resident-window-pages", dict(type=int, default=64)),
    ("--hot-watermark", dict(type=int)),
    ("--top-k", dict(type=_top_k, default=None, help="page count, or all (default)")),
    ("--max-new-tokens", dict(type=int, default=12)),
    ("--selector", dict(choices=["quest", "mean"], default="quest")),
    ("--cache-layout", dict(choices=["hybrid", "pages"], default="hybrid")),
    ("--no-overlap", dict(action="store_true", help="pages layout only")),
]
_COMMANDS = {
    "demo": [
        ("--requests", dict(type=int, default=3)),
        ("--prompt-tokens", dict(type=int, default=65)),
    ],
    "generate": [
        ("--model", dict(required=True, help="local Qwen2/2.5 directory")),
        ("--prompt", dict(default="Explain how a KV cache works.")),
        ("--chat", dict(action="store_true", help="apply the tokenizer's chat template")),
    ],
}


def build_parser():
    parser = argparse.ArgumentParser(description="Mini-HiSparse on MI355X: decode through partial KV residency")
    sub = parser.add_subparsers(dest="command", required=True)
    for command, options in _COMMANDS.items():
        p = sub.add_parser(command)
        for flag, kwargs in _COMMON + options:
            p.add_argument(flag, **kwargs)
    return parser


def union_rows_bound(prompt_length, max_new_tokens, top_k, heads, page_size):
    """The hot union bound U: with a page budget, the sink and tail pages are shared by
    every head and the other ``top_k - 2`` may differ per head (the reference's bound,
    cli.py:136-143), never more than the whole history."""
    rows = prompt_length + max_new_tokens
    if top_k is None:
        return rows
    shared = min(2, top_k)
    return min(rows, (shared + (top_k - shared) * heads) * page_size)


def _model_and_prompts(args, dtype, fail):
    """The decoder and the prompts: a checkpoint and its tokenizer, or the seeded tiny
    random decoder with random prompts of ``prompt_tokens + 7 i`` tokens."""
    if args.command == "generate":
        from transformers import AutoTokenizer

        model = MiniModel.from_pretrained(args.model, args.device, dtype)
        tokenizer = AutoTokenizer.from_pretrained(args.model)
        if args.chat:
            prompt = tokenizer.apply_chat_template([{"role": "user", "content": args.prompt}], tokenize=True,
                                                   add_generation_prompt=True, return_dict=False)
        else:
            prompt = tokenizer.encode(args.prompt)
        return model, [prompt], tokenizer
    if args.requests < 1 or args.prompt_tokens < 1:
        fail("requests and prompt-tokens must be positive")
    model = MiniModel().eval().to(device=args.device, dtype=dtype)  # draws first from the seed
    vocab = model.config.vocab_size
    prompts = [torch.randint(0, vocab, (args.prompt_tokens + 7 * i,)).tolist() for i in range(args.requests)]
    return model, prompts, None


def _cache(args, model, prompts, dtype, ops):
    cfg = model.config
    common = dict(host_pages=args.host_pages, page_size=args.page_size, kv_heads=cfg.num_key_value_heads,
                  head_dim=cfg.head_dim, device=args.device, dtype=dtype,
                  index_budget_bytes=args.index_budget_mib * 1024 * 1024)
    if args.cache_layout == "pages":
        from .paged import PagedConfig, PagedKVCache

        paged = PagedConfig(gpu_pages=8 if args.gpu_pages is None else args.gpu_pages, chunk_pages=args.chunk_pages,
                            overlap=not args.no_overlap, eviction_policy=args.eviction_policy, **common)
        return PagedKVCache(paged, ops=ops)
    selection_heads = cfg.num_attention_heads if args.selector == "quest" else 1
    bound = union_rows_bound(max(map(len, prompts)), args.max_new_tokens, args.top_k, selection_heads,
                             args.page_size)
    hot = HotConfig(bound if args.max_union_rows is None else args.max_union_rows, args.hot_rows,
                    resident_window_pages=args.resident_window_pages, transition_watermark=args.hot_watermark)
    blocks = args.gpu_pages
    if blocks is None:  # exactly one request's credits
        blocks = hot.admission_blocks(args.page_size, cfg.num_hidden_layers)
    return HybridKVCache(CacheConfig(gpu_pages=blocks, **common), hot, ops=ops)


def run(args, parser=None, ops=None):
    """Run a ``demo`` or ``generate`` command and return its report."""
    torch.manual_seed(42)
    dtype = getattr(torch, args.dtype)

    def fail(message):
        if parser is None:
            raise ValueError(message)
        parser.error(message)

    model, prompts, tokenizer = _model_and_prompts(args, dtype, fail)
    cache = _cache(args, model, prompts, dtype, ops)
    engine = Engine(model, cache, args.top_k, args.backend, tokenizer.eos_token_id if tokenizer else None,
                    selector=args.selector)
    for i, prompt in enumerate(prompts):
        engine.add_request(str(i), prompt, args.max_new_tokens)
    timeline = []
    while engine.waiting or engine.running:
        engine.step()
        timeline.append({
            "active": len(engine.running),
            "waiting": len(engine.waiting),
            "locations": cache.snapshot()["locations"],
            "generated": {name: len(r.generated) for name, r in engine.requests.items()},
        })
    cache.collect(wait=True)
    decode = (lambda tokens: tokenizer.decode(tokens, skip_special_tokens=True)) if tokenizer else (lambda t: t)
    report = {
        "model": args.model if tokenizer else "tiny random decoder (mechanics demo)",
        "selection": "full attention" if args.top_k is None
        else f"{args.selector}: approximate top-{args.top_k} pages per selection head",
        "outputs": {name: decode(r.generated) for name, r in engine.requests.items()},
        "requests": {
            name: {"prefill_count": r.prefill_count, "decode_count": r.decode_count,
                   "generated_tokens": len(r.generated)}
            for name, r in engine.requests.items()
        },
        "timeline": timeline,
        **cache.snapshot(),
    }
    cache.assert_invariants()
    return report


def main(argv=None):
    parser = build_parser()
    args = parser.parse_args(argv)
    torch.set_num_threads(1)
    text = json.dumps(run(args, parser), indent=2, ensure_ascii=False)
    print(text)
    if args.output:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(text + "\n")


if __name__ == "__main__":
    main()
