"""Layer-major batched sparse decode: B requests per launch, every layer of a step.

The reference decodes one request at a time, and inside a request one layer
at a time (engine.py:115-128, model.py:199-225), with a Python control plane
that keeps one object per page (hybrid.py, storage.py).  At the Qwen2.5-7B
shape with 16 requests of 128k tokens that is 3.67 M pages and 448
(request, layer) pairs per step.  This engine keeps the same per-(request,
layer) state -- the host page of every logical page, the resident block of the
resident ones, the hot region (blocks, tags, LRU) and the Quest bounds -- as
stacked device tensors, and runs a decode step layer by layer over all B
requests:

    dense   RMSNorm, q|k|v projection, rotary + split              (HIP)
    append  hs_append_rows: tail rows, Quest bounds, host mirror   (HIP)
    select  hs_quest_topk + hs_build_union                         (HIP)
            (or pages resampled uniformly per step, shared by all heads,
            + hs_build_union: the miss-heavy stress shape)
    resolve hs_resolve_rows_batched, row statistics fused          (HIP, compute stream)
    gather  hs_gather_rows_batched, host -> hot rows               (HIP, transfer stream)
    attend  hs_attend_groups                                       (HIP)
    dense   o_proj, residual + RMSNorm, gate|up, SiLU, down        (HIP)

and the next tokens (greedy) stay on the device: a step never reads back to
the host.  The per-(request, layer) semantics are the reference's: the new
token is appended before selection, Quest picks pages over bounds that include
it, the resolver is bit-exact ``resolve_rows`` and attention covers the
selected tokens; hot rows follow the resolver's LRU exactly.  Residency is
either the reference's hybrid policy (hybrid.py:204-392: every page and hot
region placed by :class:`PlacementPlan` as the prefill and the decode write, in
the reference engine's request-by-request order) or a seeded fixed fraction of
each layer's pages (plus every tail page), chosen when the history is written.
With the policy, placements follow the reference's decisions for that write
order; the layer-major step then reads a layer's tables after every request's
write of the step, where the reference reads each request's before the next
request writes.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from math import ceil

import numpy as np
import torch
from torch.nn import functional as F

from . import _lib
from .streams import independent_stream
from .batched import BatchedSparseDecode, LayerTablesView
from .dense import (
    add_rms_norm, argmax_workspace_bytes, gemm_workspace_bytes, linear_argmax_tiled, linear_supported,
    linear_swiglu_tiled, linear_tiled, prepare_add_rms_norm,
    prepare_linear_swiglu_tiled, prepare_linear_tiled, prepare_rotary_split, prepare_silu_mul, rotary_split, silu_mul,
    tile_gate_up, tile_weight,
)
from .config import CacheConfig
from .model import MiniModel, ModelConfig
from .row_kernels import MappedHost, pinned_empty


@dataclass(frozen=True)
class DecodeWorkload:
    """A decode configuration: model shape, batch, history, selection and residency."""

    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    batch: int
    context: int
    steps: int
    top_pages: int
    resident_fraction: float
    hot_rows: int
    page_size: int = 16
    dtype: torch.dtype = torch.bfloat16
    selector: str = "quest"  # "quest", or "uniform": pages resampled every step, shared by all heads

    def model_config(self):
        return ModelConfig(
            vocab_size=self.vocab, hidden_size=self.hidden, intermediate_size=self.ffn,
            num_hidden_layers=self.layers, num_attention_heads=self.heads,
            num_key_value_heads=self.kv_heads,
        )


# BASELINE configs[2], configs[3] and configs[4] (hot rows: 2U for the 0.5B shape;
# the reference's cap of 32768 for the 7B shape, hybrid.py:34; 2U of one shared
# 64-page selection for the 32B stress shape, whose 40% resident pages and
# uniformly resampled selection make about 60% of the selected rows miss)
WORKLOADS = {
    "qwen2.5-0.5b": DecodeWorkload(
        "qwen2.5-0.5b", layers=24, hidden=896, heads=14, kv_heads=2, head_dim=64, ffn=4864,
        vocab=151936, batch=4, context=32768, steps=128, top_pages=32, resident_fraction=0.25,
        hot_rows=13504,
    ),
    "qwen2.5-7b": DecodeWorkload(
        "qwen2.5-7b", layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, ffn=18944,
        vocab=152064, batch=16, context=131072, steps=256, top_pages=64, resident_fraction=0.15,
        hot_rows=32768,
    ),
    "qwen2.5-32b-stress": DecodeWorkload(
        "qwen2.5-32b-stress", layers=64, hidden=5120, heads=40, kv_heads=8, head_dim=128, ffn=27648,
        vocab=152064, batch=32, context=65536, steps=128, top_pages=64, resident_fraction=0.4,
        hot_rows=2048, selector="uniform",
    ),
}


def uniform_pages(lengths, page_size, top_pages, layers, generator, device):
    """Per (layer, request) the tail page plus ``top_pages - 1`` other pages drawn
    uniformly without replacement: int32 [layers, B, top_pages], ascending.  A
    request with at most ``top_pages`` pages selects all of them (the first
    ``count`` entries; the rest are never read)."""
    B = len(lengths)
    counts = [ceil(length / page_size) for length in lengths]
    span = max(max(counts) - 1, top_pages - 1, 1)
    keys = torch.rand((layers, B, span), generator=generator, device=device)
    for b, count in enumerate(counts):
        keys[:, b, max(count - 1, 0):] = -1.0  # the tail page and pages past the history
    drawn = keys.topk(top_pages - 1, dim=-1).indices.to(torch.int32) if top_pages > 1 else keys[..., :0].int()
    tails = torch.tensor([count - 1 for count in counts], dtype=torch.int32, device=device)
    pages = torch.cat((drawn, tails.view(1, B, 1).expand(layers, B, 1)), -1).sort(-1).values
    for b, count in enumerate(counts):
        if count <= top_pages:
            pages[:, b, :count] = torch.arange(count, dtype=torch.int32, device=device)
    return pages


def uniform_pages_device(seed, step, lengths, page_size, top_pages, layers, heads, device="cuda", out=None,
                         stream=None):
    """:func:`uniform_pages`'s rule drawn on the device by ``hs_uniform_pages``: per (layer,
    request) the tail page plus ``top_pages - 1`` others uniformly without replacement,
    ascending, for every head: int32 [layers, B, heads, top_pages] (-1 past a short
    history's pages).  A counter-based generator: (seed, step) fixes the draw."""
    B = len(lengths)
    counts = (ctypes.c_int64 * B)(*[ceil(length / page_size) for length in lengths])
    if out is None:
        out = torch.empty((layers, B, heads, top_pages), dtype=torch.int32, device=device)
    if out.dtype != torch.int32 or tuple(out.shape) != (layers, B, heads, top_pages) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous int32 [{layers}, {B}, {heads}, {top_pages}]")
    handle = stream if stream is not None else _lib.stream_handle(out.device)
    _lib.check(_lib.load().hs_uniform_pages(seed & (2**64 - 1), step & (2**64 - 1), counts, B, layers, top_pages,
                                            heads, out.data_ptr(), handle), "hs_uniform_pages")
    return out


def rotary_at(tensor, positions, theta):
    """Rotary embedding of [B, heads, head_dim] at one position per row; the same
    arithmetic as the model's prefill/decode rotary (model.py)."""
    dim = tensor.shape[-1]
    inv = theta ** (-torch.arange(0, dim, 2, device=tensor.device).float() / dim)
    angles = positions.float()[:, None] * inv[None, :]
    angles = torch.cat((angles, angles), -1)[:, None, :]
    cosine, sine = angles.cos().to(tensor.dtype), angles.sin().to(tensor.dtype)
    first, second = tensor.chunk(2, -1)
    return tensor * cosine + torch.cat((-second, first), -1) * sine


class SparseKVState:
    """Per-(layer, request) KV state as stacked tensors.

    host      per layer a pinned [B * C, 2, P, Hkv, D] pool (one allocation per layer:
              pinned allocations are size-limited); logical page p of (l, b) lives
              in host block b * C + p of layer l's pool (the ``source`` table)
    pool      device [blocks, 2, P, Hkv, D]: resident pages, hot regions, spare
              blocks for the tail pages the decode opens
    source    int32 [L, B, C]    resident int32 [L, B, C] (-1 = host only)
    hot       int32 [L, B, S/P]  tags int32 [L, B, S]  lru int16 [L, B, S]
    minimum / maximum  [L, B, C, Hkv, D] Quest bounds (+inf / -inf when empty)
    """

    def __init__(self, layers, batch, max_tokens, config: CacheConfig, hot_rows, resident_pages, spare_blocks,
                 policy_blocks=None, policy_window=64, policy_watermark=None):
        """``resident_pages`` / ``spare_blocks`` size the slab of the fixed residency
        (resident blocks, then every hot region, then blocks for the tails the decode
        opens).  ``policy_blocks`` instead makes the slab that many blocks, placed by
        the hybrid policy (:class:`PlacementPlan`: pages, hot regions and reuse) with
        the resident window and watermark of :class:`HotConfig`."""
        P, Hkv, D, dev = config.page_size, config.kv_heads, config.head_dim, torch.device(config.device)
        self.layers, self.batch, self.config, self.device = layers, batch, config, dev
        self.pages = ceil(max_tokens / P)
        self.hot_rows = hot_rows
        C, L, B = self.pages, layers, batch
        hot_blocks = ceil(hot_rows / P)
        self.plan = None
        if policy_blocks is not None:
            from .residency import PlacementPlan

            self.plan = PlacementPlan(policy_blocks, P, hot_rows, window=policy_window, watermark=policy_watermark)
            resident_pages, spare_blocks = policy_blocks - L * B * hot_blocks, 0
        self.blocks = resident_pages + L * B * hot_blocks + spare_blocks
        self.pool = torch.empty((self.blocks, 2, P, Hkv, D), dtype=config.dtype, device=dev)
        self.host = [pinned_empty((B * C, 2, P, Hkv, D), config.dtype) for _ in range(L)]
        self.alias = [MappedHost(h) for h in self.host]
        self.source = torch.arange(B * C, dtype=torch.int32, device=dev).view(1, B, C).repeat(L, 1, 1)
        self.resident = torch.full((L, B, C), -1, dtype=torch.int32, device=dev)
        self.first_hot = resident_pages  # resident blocks are [0, first_hot)
        self.hot = (torch.arange(L * B * hot_blocks, dtype=torch.int32, device=dev) + self.first_hot).view(L, B, hot_blocks)
        self.tags = torch.full((L, B, hot_rows), -1, dtype=torch.int32, device=dev)
        self.lru = torch.arange(hot_rows, dtype=torch.int16, device=dev).repeat(L * B).view(L, B, hot_rows)
        self.minimum = torch.full((L, B, C, Hkv, D), float("inf"), dtype=config.dtype, device=dev)
        self.maximum = torch.full((L, B, C, Hkv, D), float("-inf"), dtype=config.dtype, device=dev)
        self.next_resident = 0
        self.next_spare = resident_pages + L * B * hot_blocks
        self.lengths = [0] * B
        self.tail_block = [[-1] * B for _ in range(L)]  # device block of each (l, b) tail page
        self._append_arrays = {}  # layer -> the ctypes arrays of its whole-batch hs_append_rows call
        self.tables = [
            [LayerTablesView(self.source[l, b], self.resident[l, b], self.hot[l, b], self.tags[l, b], self.lru[l, b])
             for b in range(B)]
            for l in range(L)
        ]
        self.bounds = [([self.minimum[l, b] for b in range(B)], [self.maximum[l, b] for b in range(B)]) for l in range(L)]
        self.row_stats = torch.zeros(3, dtype=torch.int64, device=dev)

    # -- history -------------------------------------------------------------
    @torch.inference_mode()
    def build_history(self, length, resident_fraction, seed=0, outlier_fraction=0.02, outlier_scale=8.0):
        """Synthetic history of `length` tokens for every (layer, request): K, V ~ N(0, 1)
        with a seeded 2% of channels per KV head scaled x8, written to the host pool;
        exact Quest bounds per page; a seeded `resident_fraction` of each (l, b)'s pages
        plus its tail page copied into resident blocks."""
        cfg, L, B, C, dev = self.config, self.layers, self.batch, self.pages, self.device
        P, Hkv, D = cfg.page_size, cfg.kv_heads, cfg.head_dim
        used = ceil(length / P)
        tail_valid = length - (used - 1) * P
        gen = torch.Generator(device=dev).manual_seed(seed)
        cpu_gen = torch.Generator().manual_seed(seed)
        for l in range(L):
            host = self.host[l].view(B, C, 2, P, Hkv, D)
            scale = torch.ones(B, 1, 1, Hkv, D)
            n_out = max(1, round(outlier_fraction * D))
            for b in range(B):
                for kv in range(Hkv):
                    scale[b, 0, 0, kv, torch.randperm(D, generator=cpu_gen)[:n_out]] = outlier_scale
            scale = scale.to(dev)
            kv_pages = torch.empty((B, used, 2, P, Hkv, D), dtype=cfg.dtype, device=dev)
            for b in range(B):  # one request at a time bounds the float32 scratch
                x = torch.randn((used, 2, P, Hkv, D), generator=gen, device=dev)
                kv_pages[b] = (x * scale[b]).to(cfg.dtype)
                del x
            kv_pages[:, -1, :, tail_valid:] = 0  # rows past the history
            keys = kv_pages[:, :, 0]
            self.minimum[l, :, :used] = keys.amin(2)
            self.maximum[l, :, :used] = keys.amax(2)
            self.minimum[l, :, used - 1] = keys[:, -1, :tail_valid].amin(1)
            self.maximum[l, :, used - 1] = keys[:, -1, :tail_valid].amax(1)
            host[:, :used].copy_(kv_pages)
            for b in range(B):
                pages, blocks = self._place_residents(l, b, used, resident_fraction, seed)
                self.pool[torch.from_numpy(blocks).to(dev)] = kv_pages[b, torch.from_numpy(pages).to(dev)]
            del kv_pages, keys
        torch.cuda.synchronize(dev)
        self.lengths = [length] * B

    def _place_residents(self, layer, b, used, resident_fraction, seed):
        """A seeded ``resident_fraction`` of the ``used`` pages of (layer, b), plus its tail
        page, get resident blocks; returns (pages, blocks) as int64 arrays."""
        rng = torch.Generator().manual_seed(seed * 1000003 + layer * 65537 + b)
        chosen = torch.randperm(max(used - 1, 0), generator=rng)[: round(resident_fraction * used)]
        pages = torch.cat((chosen, torch.tensor([used - 1]))).unique().numpy().astype(np.int64)
        if self.next_resident + len(pages) > self.first_hot:
            raise ValueError("resident pages exceed the reserved resident blocks")
        blocks = np.arange(self.next_resident, self.next_resident + len(pages), dtype=np.int64)
        self.next_resident += len(pages)
        self.resident[layer, b, torch.from_numpy(pages).to(self.device)] = torch.from_numpy(blocks).to(
            self.device, torch.int32)
        self.tail_block[layer][b] = int(blocks[-1])
        return pages, blocks

    def write_prompt(self, layer, b, k, v, slots):
        """The K/V rows ``[T, Hkv, D]`` of request b's prompt at layer ``layer``: every row
        to its host page, the rows of resident pages (``slots[p] >= 0``) to their blocks,
        and the exact Quest bounds of every page (``hs_append_tokens``)."""
        from .row_kernels import append_tokens

        C = self.pages
        used = len(slots)
        append_tokens(k, v, 0, 0, [int(x) for x in slots], [b * C + p for p in range(used)], self.pool,
                      self.alias[layer], self.minimum[layer, b], self.maximum[layer, b], None, self.config)

    @torch.inference_mode()
    def prefill(self, model, prompts, resident_fraction, seed=0, observer=None):
        """Run the model over each request's prompt (PyTorch-ROCm causal SDPA, one request
        at a time) and write every layer's K/V into the state: host pool, a seeded
        ``resident_fraction`` of the pages plus the tail page in resident blocks, exact
        Quest bounds.  Returns the greedy first tokens [B] (the prefill's logits).
        ``observer(layer, b, k, v)`` sees each layer's prompt K/V."""
        if len(prompts) != self.batch:
            raise ValueError(f"expected {self.batch} prompts")
        firsts = []
        for b, prompt in enumerate(prompts):
            if self.plan is not None:
                self.plan.reserve(b, self.pages * self.config.page_size, self.layers)
            firsts.append(self._prefill_request(model, b, prompt, resident_fraction, seed, observer))
        torch.cuda.synchronize(self.device)
        if self.plan is not None:
            self._tables_from_plan()
        return torch.stack(firsts)

    @torch.inference_mode()
    def prefill_slot(self, model, b, prompt, observer=None):
        """Admit one prompt into the empty slot ``b`` (its policy groups already reserved,
        the engine's admission): the prefill of ``prefill`` for that request, its pages
        placed by the policy, then its tables from the plan (and the resident entries of
        other slots whose blocks this prefill reclaimed).  Returns the first token
        (device scalar)."""
        if self.plan is None:
            raise ValueError("slot admission needs the policy residency")
        first = self._prefill_request(model, b, prompt, 0.0, 0, observer)
        self._tables_from_plan(slots=[b])
        return first

    def _prefill_request(self, model, b, prompt, resident_fraction, seed, observer):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        cfg = model.config
        groups = cfg.num_attention_heads // cfg.num_key_value_heads
        P = self.config.page_size
        tokens = torch.as_tensor(prompt, device=self.device)
        used = ceil(len(tokens) / P)
        if len(tokens) > self.pages * P:
            raise ValueError("prompt longer than the state's capacity")
        slots = []
        if self.plan is None:
            for l in range(self.layers):
                pages, blocks = self._place_residents(l, b, used, resident_fraction, seed)
                row = np.full(used, -1, np.int64)
                row[pages] = blocks
                slots.append(row)

        def attend(index, q, k, v):
            if self.plan is not None:  # the policy places this layer's pages as it writes them
                self.plan.write((b, index), len(k))
                slots.append(self.plan.group((b, index)).slot[:used].copy())
            self.write_prompt(index, b, k, v, slots[index])
            if observer is not None:
                observer(index, b, k, v)
            # [1, heads, tokens, dim]: the fused kernels take 4-D operands only
            heads_first = lambda t: t.transpose(0, 1).unsqueeze(0).contiguous()  # noqa: E731
            grouped = lambda t: heads_first(t.repeat_interleave(groups, 1))  # noqa: E731
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                out = F.scaled_dot_product_attention(heads_first(q), grouped(k), grouped(v), is_causal=True)
            return out[0].transpose(0, 1)

        hidden = model._layers(tokens, 0, attend)
        self.lengths[b] = len(tokens)
        return model._logits(hidden[-1]).argmax()

    def reset_slot(self, b):
        """Slot ``b`` empty again (a released request's): no resident page, no hot tag,
        the LRU in slot order, empty Quest bounds, no history."""
        self.resident[:, b] = -1
        self.tags[:, b] = -1
        self.lru[:, b] = torch.arange(self.hot_rows, dtype=self.lru.dtype, device=self.device)
        self.minimum[:, b] = float("inf")
        self.maximum[:, b] = float("-inf")
        self.lengths[b] = 0
        for l in range(self.layers):
            self.tail_block[l][b] = -1

    def _tables_from_plan(self, slots=None):
        """Resident pages, hot regions and tail blocks of every (l, b) of ``slots``
        (default: every slot) as the policy left them (pages it detached again hold -1),
        and the resident entries of other slots' pages it detached meanwhile.  A
        (request, layer) whose prefill raised no hot demand (fewer pages than the window,
        the watermark never crossed) takes its region now, request by request (the
        policy's explicit transition): the decode serves every row it selects outside the
        resident pages from it."""
        L, C = self.layers, self.pages
        slots = list(range(self.batch)) if slots is None else list(slots)
        for b in slots:
            for l in range(L):
                if not self.plan.group((b, l)).hot:
                    self.plan.transition(self.plan.group((b, l)))
        resident = np.full((L, len(slots), C), -1, np.int32)
        hot = np.empty((L, len(slots), self.hot.shape[2]), np.int32)
        for i, b in enumerate(slots):
            for l in range(L):
                g = self.plan.group((b, l))
                held = min(C, len(g.slot))  # the group spans the request's own reservation
                resident[l, i, :held] = g.slot[:held]
                hot[l, i] = g.hot
                self.tail_block[l][b] = int(g.slot[(g.length - 1) // self.config.page_size])
        index = torch.tensor(slots, device=self.device)
        self.resident.index_copy_(1, index, torch.from_numpy(resident).to(self.device))
        self.hot.index_copy_(1, index, torch.from_numpy(hot).to(self.device))
        others = [(key, page) for key, page in self.plan.detached if key[0] not in slots]
        if others:
            rows = torch.tensor([(l, b, page) for (b, l), page in others], dtype=torch.int64).T.to(self.device)
            self.resident[rows[0], rows[1], rows[2]] = -1
        self.plan.detached.clear()

    # -- decode-step bookkeeping ---------------------------------------------------
    def open_tail_pages(self, positions, order=None):
        """Give every (l, b) whose next token starts a page a resident tail block, for the
        requests in ``order`` (default: every slot, in slot order; the policy places the
        writes in that order)."""
        rows = list(range(self.batch)) if order is None else list(order)
        # every step calls this before its first launch: a token past the capacity is
        # refused here, on the host, since its page would index past the tables that
        # the uploads below and the step's launches write
        full = [b for b in rows if positions[b] >= self.pages * self.config.page_size]
        if full:
            raise RuntimeError(f"slot(s) {full}: history full ({self.pages * self.config.page_size} tokens)")
        if self.plan is not None:
            self._plan_decode_writes(positions, rows)
            return
        P, L = self.config.page_size, self.layers
        starts = [b for b in rows if positions[b] % P == 0]
        if not starts:
            return
        if self.next_spare + L * len(starts) > self.blocks:
            raise RuntimeError("no spare device blocks left for new tail pages")
        ls, bs, ps, blocks = [], [], [], []
        for l in range(L):
            for b in starts:
                blk = self.next_spare
                self.next_spare += 1
                self.tail_block[l][b] = blk
                ls.append(l), bs.append(b), ps.append(positions[b] // P), blocks.append(blk)
        # one pinned upload, queued on the current stream (no host synchronisation)
        rows = torch.tensor([ls, bs, ps, blocks], dtype=torch.int64, pin_memory=True).to(self.device, non_blocking=True)
        self.resident[rows[0], rows[1], rows[2]] = rows[3].to(torch.int32)

    def _plan_decode_writes(self, positions, rows):
        """The step's one-token writes through the policy, request by request (``rows``,
        in the engine's turn order) and layer by layer (the reference engine's order,
        engine.py:115-128).  A write into a page that has rows changes no placement for a
        layer whose hot region is served, so such steps only count the rows; a step that
        opens pages places them, and every page the policy detaches or binds updates the
        resident table (one pinned upload queued on the current stream)."""
        L, plan = self.layers, self.plan
        if plan.append_within([(b, l) for b in rows for l in range(L)]):
            return
        ls, bs, ps, blocks = [], [], [], []
        for b in rows:
            for l in range(L):
                for page, block in plan.write((b, l), 1):
                    self.tail_block[l][b] = int(block)
                    ls.append(l), bs.append(b), ps.append(page), blocks.append(block)
        for (b, l), page in plan.detached:
            ls.append(l), bs.append(b), ps.append(page), blocks.append(-1)
        plan.detached.clear()
        if ls:  # no entry repeats: a page opened this step is a tail, never detached in it
            rows = torch.tensor([ls, bs, ps, blocks], dtype=torch.int64, pin_memory=True)
            rows = rows.to(self.device, non_blocking=True)
            self.resident[rows[0], rows[1], rows[2]] = rows[3].to(torch.int32)

    def append_args(self, layer, positions, rows=None):
        """ctypes arrays of one layer's hs_append_rows call for the requests in ``rows``
        (a range; default every request).  Every request's call reuses one set of arrays
        per layer, filled in place (the previous call's launch has read them: ctypes
        passes them to the library, which copies them into the launch's arguments)."""
        P, B, C = self.config.page_size, self.batch, self.pages
        Hkv, D = self.config.kv_heads, self.config.head_dim
        esz = self.minimum.element_size()
        page_elems = Hkv * D
        rows = range(B) if rows is None else rows
        n = len(rows)
        if n == B:
            arrays = self._append_arrays.get(layer)
            if arrays is None:
                arrays = self._append_arrays[layer] = (
                    (ctypes.c_int64 * B)(), (ctypes.c_int64 * B)(), (ctypes.c_void_p * B)(), (ctypes.c_void_p * B)())
            dev_rows, host_rows, lo, hi = arrays
        else:
            dev_rows = (ctypes.c_int64 * n)()
            host_rows = (ctypes.c_int64 * n)()
            lo = (ctypes.c_void_p * n)()
            hi = (ctypes.c_void_p * n)()
        base_lo, base_hi = self.minimum.data_ptr(), self.maximum.data_ptr()
        for i, b in enumerate(rows):
            page, off = divmod(positions[b], P)
            dev_rows[i] = self.tail_block[layer][b] * P + off
            host_rows[i] = (b * C + page) * P + off
            at = ((layer * B + b) * C + page) * page_elems * esz
            lo[i], hi[i] = base_lo + at, base_hi + at
        return dev_rows, host_rows, lo, hi


def _graph_time(calls, stream, replays=3):
    """Device milliseconds of ``calls`` in order (launches on the current stream), as
    the median of ``replays`` replays of a HIP graph captured from them on ``stream``
    after one eager pass there."""
    device = stream.device
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for call in calls:
            call()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for call in calls:
            call()
    times = []
    for _ in range(replays + 1):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
    del graph
    return sorted(times[1:])[replays // 2]


class BatchedDecodeEngine:
    """Greedy decode of B requests, layer-major, over a :class:`SparseKVState`."""

    PREFETCH_AHEAD = 4  # layers the prefetched transfers are issued ahead of the compute
    # workgroups of a prefetched gather (all requests together): enough host reads in
    # flight for the link while it overlaps the dense layers, few enough that its waiting
    # waves leave the projections most CUs (32B stress shape, batch 3: 48 -> 22.5 ms per
    # step, 96 -> 24.4, the unbounded ~430 -> 26.2)
    PREFETCH_GATHER_WORKGROUPS = 48

    def __init__(self, model: MiniModel, state: SparseKVState, top_pages, *, max_tokens=None, keep_sink=True,
                 selector="quest", seed=0, graphs=False, projections="auto", transfer_stream=False,
                 prefetch=None, request_groups=1, group_gather_workgroups=0, resolver_split=True,
                 fuse_rotary_append=True):
        """``selector``: "quest" (per-head Quest pages over the bounds) or "uniform"
        (:func:`uniform_pages_device`, shared by every head, resampled each step).  ``graphs``:
        replay the dense part of each layer boundary as a HIP graph (when every per-layer
        projection runs on hs_skinny_gemm; captured after the first step): it cuts the host
        time of a boundary from ~80 to ~22 us, which pays only where the host, not the GPU,
        paces the step.  ``projections``: "auto" (timed choice per projection), "kernel"
        (hs_skinny_gemm wherever it applies) or "torch".  ``transfer_stream``: gather on a
        separate stream ordered by events (the reference's arrangement, hybrid.py:443-477);
        the default gathers on the compute stream, because overlap does not pay on MI355X
        (host reads slow the kernels beside them) and each cross-stream hand-off costs
        ~20 us of GPU time.  ``prefetch`` (uniform selector only, on by default there): select, resolve and
        gather every layer at the start of the step on a transfer stream, one decoder
        (buffer set) per layer, so that the host reads overlap the dense layers; layer
        l's attention waits for layer l's gather only, and the step's first transfer
        waits for the previous step's last attention (the last reader of the hot rows).
        ``request_groups`` (Quest selector): split the batch into that many request groups
        and pipeline them across the layers -- while one group's gather reads host memory
        on the transfer stream, the compute stream runs the other groups' attention, dense
        layers, append, selection and resolve (each request's own sequence of stages is
        unchanged, so every output is the same); ``group_gather_workgroups`` sets the
        gather's workgroups per request there (0: the library's default).
        ``resolver_split``: the resolver's front over several workgroups per request
        (``hs_resolve_desc.split_front``; the state's source tables are affine by
        construction), else one workgroup per request.  ``fuse_rotary_append``: each
        layer's rotary embedding and the append of its new K/V rows in one launch
        (``hs_rotary_split_append``) where the dense launches are not graph-replayed."""
        if prefetch is None:
            prefetch = selector == "uniform"
        if prefetch and selector != "uniform":
            raise ValueError("prefetch needs the uniform selector (Quest pages depend on the layer's query)")
        if projections not in ("auto", "kernel", "torch"):
            raise ValueError(f"unknown projections {projections!r}")
        if selector not in ("quest", "uniform"):
            raise ValueError(f"unknown selector {selector!r}")
        cfg = model.config
        if (cfg.num_key_value_heads, cfg.head_dim) != (state.config.kv_heads, state.config.head_dim):
            raise ValueError("model/cache head dimensions differ")
        if model.dtype != state.config.dtype:
            raise ValueError("model/cache dtype differ")
        self.model, self.state = model, state
        self.device = state.device
        caps = [max_tokens or state.pages * state.config.page_size] * state.batch
        decoder = lambda donor=None: BatchedSparseDecode(
            state.config, cfg.num_attention_heads, top_pages, [max(1, l) for l in state.lengths],
            keep_sink=keep_sink, device=self.device, capacity_lengths=caps,
            shared_selection=selector == "uniform", workspaces_from=donor, split_front=resolver_split,
        )
        self.dec = decoder()
        self.prefetch = prefetch
        self.decs = [self.dec] + [decoder(self.dec) for _ in range(state.layers - 1)] if prefetch else None
        self.selector = selector
        self._sample_seed, self._sample_step = seed, 0  # the uniform selector's draws: (seed, step)
        if state.hot_rows < self.dec.capacity:
            # the resolver's precondition (row_index.py:41-42, hybrid.py:34): every
            # selected row must fit the hot region, or misses would share victim slots
            raise ValueError(
                f"hot_rows {state.hot_rows} below the union bound {self.dec.capacity} of "
                f"{cfg.num_attention_heads} heads x {top_pages} pages"
            )
        self.groups = None
        if request_groups > 1:
            if selector != "quest" or prefetch or graphs:
                raise ValueError("request groups pipeline the Quest path (no prefetch, no graphs)")
            count = min(request_groups, state.batch)
            edges = [round(i * state.batch / count) for i in range(count + 1)]
            self.groups = []
            for a, b in zip(edges, edges[1:]):
                group = BatchedSparseDecode(
                    state.config, cfg.num_attention_heads, top_pages, [max(1, l) for l in state.lengths[a:b]],
                    keep_sink=keep_sink, device=self.device, capacity_lengths=caps[a:b],
                    split_front=resolver_split,
                )
                self.groups.append((range(a, b), group))
            # per (layer, group): resolved (compute -> transfer) and gathered (transfer -> compute)
            self._group_events = [[(torch.cuda.Event(), torch.cuda.Event()) for _ in self.groups]
                                  for _ in range(state.layers)]
            self.group_gather_workgroups = group_gather_workgroups
        # its own hardware queue, or the transfers would run in the compute stream's order
        self.transfer = independent_stream(self.device) if transfer_stream or prefetch or self.groups else None
        self._pack_projections()
        self._choose_projections(projections)
        self._host_alias = [(ctypes.c_void_p * state.batch)(*([a.data_ptr()] * state.batch)) for a in state.alias]
        self.positions = torch.tensor(state.lengths, dtype=torch.int64, device=self.device)
        # per layer: resolved (compute -> transfer) and gathered (transfer -> compute)
        self._handoff = [(torch.cuda.Event(), torch.cuda.Event()) for _ in range(state.layers)]
        self._step_start = torch.cuda.Event()
        self._subsets = {}  # sorted slots of a partial batch -> its decoder and buffers
        self._keep_sink, self._top_pages, self._caps = keep_sink, top_pages, caps
        self.fuse_rotary_append = fuse_rotary_append
        self._pages_bufs = {}  # per running-set size: the uniform pages copied to every head
        self._resolver_split = resolver_split
        self.current_group = None  # (requests, decoder) the observer's arguments belong to
        self._static_buffers()
        self.use_graphs = graphs and all(self.projection_kernel[n] for n in ("qkv", "o_proj", "gate_up", "down"))
        self._graphs = None
        self._prepared = None  # per layer boundary, its bound dense launches (built on first use)

    def decoder(self, layer):
        """The decoder (selection, resolver and attention buffers) that serves `layer`."""
        return self.decs[layer] if self.decs is not None else self.dec

    def _draw_pages(self, lengths):
        """The step's uniform pages, [L, n, heads, top] for the ``n`` decoding requests'
        ``lengths``, drawn on the device (``hs_uniform_pages``, one launch) into a buffer
        reused every step; each layer's union build reads its slice in place.  The step's
        last attention waits for every layer's gather, so every read of the buffer precedes
        the next step's draw on the compute stream."""
        L, n = self.state.layers, len(lengths)
        Hq = self.model.config.num_attention_heads
        buf = self._pages_bufs.get(n)
        if buf is None:
            buf = self._pages_bufs[n] = torch.empty((L, n, Hq, self.dec.top), dtype=torch.int32,
                                                    device=self.device)
        uniform_pages_device(self._sample_seed, self._sample_step, lengths, self.state.config.page_size,
                             self.dec.top, L, Hq, out=buf)
        self._sample_step += 1
        return buf

    def _prefetch(self, index, sampled, transfer, mark):
        """Layer `index`'s select, resolve and gather on `transfer`; returns its stage
        marks.  The transfer stream was ordered (at step start) after everything then
        queued on the compute stream: the step's tail-page table updates and page draws,
        and the previous step's attention, the last reader of the hot rows the gathers
        overwrite.  Layers are issued in order, a few ahead of the compute stream's."""
        st, dec = self.state, self.decs[index]
        with torch.cuda.stream(transfer):
            m = {"select": [mark(transfer)]}
            dec.select_pages(sampled[index], validate=False)  # uniform_pages: ascending, tail last
            m["select"].append(mark(transfer))
            m["resolve"] = [m["select"][1]]
            dec.resolve(st.tables[index], row_stats=st.row_stats)
            m["resolve"].append(mark(transfer))
            m["gather"] = [m["resolve"][1]]
            dec.gather(st.alias[index], st.pool, transfer, grid_x=ceil(self.PREFETCH_GATHER_WORKGROUPS / st.batch))
            m["gather"].append(mark(transfer))
            self._handoff[index][1].record(transfer)
        return m

    def _static_buffers(self):
        """Fixed buffers of the dense stages, so that their launches can be replayed."""
        cfg, B, dev, dt = self.model.config, self.state.batch, self.device, self.model.dtype
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        new = lambda *shape: torch.empty(shape, dtype=dt, device=dev)
        self._x, self._h, self._o, self._delta = (new(B, cfg.hidden_size) for _ in range(4))
        self._qkv = new(B, (Hq + 2 * Hkv) * D)
        self._q, self._k, self._v = new(B, Hq, D), new(B, Hkv, D), new(B, Hkv, D)
        self._attn_out = new(B, Hq, D)
        self._gate_up = new(B, 2 * cfg.intermediate_size)
        self._act = new(B, cfg.intermediate_size)

    # -- dense stages (the same launches eagerly and inside the graphs) ---------
    def _dense_in(self, index, first, rows=slice(None)):
        """Residual add of the previous MLP + input RMSNorm, q|k|v, rotary + split, for the
        requests in ``rows`` (a slice of the batch)."""
        cfg = self.model.config
        layer = self.model.model.layers[index]
        qkv_w, qkv_b, _ = self._packed[index]
        h = add_rms_norm(self._x[rows], None if first else self._delta[rows], layer.input_layernorm.weight,
                         cfg.rms_norm_eps, out=self._h[rows])
        rotary_split(self._project("qkv", h, qkv_w, qkv_b, out=self._qkv[rows]), self.positions[rows],
                     cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rope_theta,
                     out=(self._q[rows], self._k[rows], self._v[rows]))

    def _dense_out(self, index, rows=slice(None)):
        """o_proj + residual + post-attention RMSNorm, gate|up, SiLU gate, down (-> delta),
        for the requests in ``rows``."""
        cfg = self.model.config
        layer = self.model.model.layers[index]
        _, _, gate_up_w = self._packed[index]
        attn = self._attn_out[rows]
        o = self._project("o_proj", attn.view(attn.shape[0], -1), layer.self_attn.o_proj.weight, out=self._o[rows])
        h = add_rms_norm(self._x[rows], o, layer.post_attention_layernorm.weight, cfg.rms_norm_eps,
                         out=self._h[rows])
        if self.projection_kernel["gate_up"]:  # gate|up and the SiLU gate in one launch
            act = linear_swiglu_tiled(h, self._tiles[gate_up_w.data_ptr()], cfg.intermediate_size,
                                      out=self._act[rows])
        else:  # PyTorch's GEMM, then the SiLU gate
            act = silu_mul(self._project("gate_up", h, gate_up_w, out=self._gate_up[rows]), out=self._act[rows])
        self._project("down", act, layer.mlp.down_proj.weight, out=self._delta[rows])

    def _boundary(self, index):
        """Dense launches between the sparse stages of layer index - 1 and index
        (index = layers: after the last layer)."""
        L = len(self.model.model.layers)
        if index > 0:
            self._dense_out(index - 1)
        if index < L:
            self._dense_in(index, first=index == 0)

    def _projection_launch(self, name, x, weight, out, bias=None):
        """A bound launch of ``_project`` into ``out`` (the kernel's, or PyTorch's GEMM, which
        runs on torch's current stream: the stream the step's launches take)."""
        if self.projection_kernel[name]:
            return prepare_linear_tiled(x, self._tiles[weight.data_ptr()], weight.shape[0], bias, out, self._gemm_ws)
        return lambda stream: out.copy_(F.linear(x, weight, bias))

    def _prepare_boundaries(self):
        """Per layer boundary, the dense launches of ``_boundary`` for the whole batch with
        every argument bound: the same launches, without re-validating and re-packing
        their arguments on every step (the host's time per launch is what paces a step of a
        small model)."""
        cfg = self.model.config
        layers = self.model.model.layers
        L = len(layers)
        eps = cfg.rms_norm_eps
        boundaries = []
        for index in range(L + 1):
            calls = []
            if index > 0:
                layer = layers[index - 1]
                _, _, gate_up_w = self._packed[index - 1]
                attn = self._attn_out.view(self._attn_out.shape[0], -1)
                calls.append(self._projection_launch("o_proj", attn, layer.self_attn.o_proj.weight, self._o))
                calls.append(prepare_add_rms_norm(self._x, self._o, layer.post_attention_layernorm.weight, eps, self._h))
                if self.projection_kernel["gate_up"]:
                    calls.append(prepare_linear_swiglu_tiled(self._h, self._tiles[gate_up_w.data_ptr()],
                                                             cfg.intermediate_size, self._act))
                else:
                    calls.append(self._projection_launch("gate_up", self._h, gate_up_w, self._gate_up))
                    calls.append(prepare_silu_mul(self._gate_up, self._act))
                calls.append(self._projection_launch("down", self._act, layer.mlp.down_proj.weight, self._delta))
            if index < L:
                layer = layers[index]
                qkv_w, qkv_b, _ = self._packed[index]
                calls.append(prepare_add_rms_norm(self._x, None if index == 0 else self._delta,
                                                  layer.input_layernorm.weight, eps, self._h))
                calls.append(self._projection_launch("qkv", self._h, qkv_w, self._qkv, qkv_b))
                calls.append(prepare_rotary_split(self._qkv, self.positions, cfg.num_attention_heads,
                                                  cfg.num_key_value_heads, cfg.head_dim, cfg.rope_theta,
                                                  (self._q, self._k, self._v)))
            boundaries.append(calls)
        return boundaries

    @torch.no_grad()
    def _capture(self):
        """One HIP graph per layer boundary, captured on a side stream (after an eager pass
        of the same launches there, so that every kernel and workspace exists)."""
        L = len(self.model.model.layers)
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        saved = [t.clone() for t in (self._x, self._delta)]
        with torch.cuda.stream(stream):
            for index in range(L + 1):
                self._boundary(index)
        stream.synchronize()
        pool = torch.cuda.graph_pool_handle()
        graphs = []
        for index in range(L + 1):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool, stream=stream):
                self._boundary(index)
            graphs.append(graph)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        self._x.copy_(saved[0])
        self._delta.copy_(saved[1])
        self._graphs = graphs
    @torch.no_grad()
    def _pack_projections(self):
        """One weight (and bias) per layer for q|k|v and for gate|up, so each is one GEMM;
        the model's own parameters become views of the packed tensors (no copy kept)."""
        self._packed = []
        for layer in self.model.model.layers:
            attn, mlp = layer.self_attn, layer.mlp
            parts = (attn.q_proj, attn.k_proj, attn.v_proj)
            qkv_w = torch.cat([m.weight for m in parts], 0)
            qkv_b = torch.cat([m.bias for m in parts], 0)
            start = 0
            for m in parts:
                rows = m.weight.shape[0]
                m.weight.data = qkv_w[start : start + rows]
                m.bias.data = qkv_b[start : start + rows]
                start += rows
            ffn = mlp.gate_proj.weight.shape[0]
            gate_up = torch.cat((mlp.gate_proj.weight, mlp.up_proj.weight), 0)
            mlp.gate_proj.weight.data = gate_up[:ffn]
            mlp.up_proj.weight.data = gate_up[ffn:]
            self._packed.append((qkv_w, qkv_b, gate_up))

    @torch.no_grad()
    def _choose_projections(self, mode="auto"):
        """Per projection, the faster of the skinny-GEMM kernel on tile-major weights
        (hs_skinny_gemm_tiled) and PyTorch's GEMM at this batch, timed over the layers'
        own weights (each call reads another layer's weight from HBM, as in a step).
        Each side runs as the step runs it, into a buffer of the step's shape (PyTorch's
        GEMM followed by the copy into it), and is timed as a replayed HIP graph of its
        calls: device time, which eager calls through Python would hide behind the
        host's time per launch (~10 us, above the kernels' 3-8 us at these shapes).
        For gate|up the kernel is the fused launch with the SiLU gate
        (hs_skinny_gemm_swiglu_tiled) and PyTorch's side is its GEMM followed by
        hs_silu_mul: the two ways the step can run.  Each projection the kernel serves
        keeps a tile-major copy of its weights (the model's row-major parameters stay as
        they are).  The split-K partials of every kernel call go to one workspace owned
        by the engine, sized for the largest plan, so captured graphs keep a buffer
        that lives as long as they do."""
        B, dev, dt = self.state.batch, self.device, self.model.dtype
        layers = self.model.model.layers
        groups = {
            "qkv": [(w, b) for w, b, _ in self._packed],
            "o_proj": [(layer.self_attn.o_proj.weight, None) for layer in layers],
            "gate_up": [(gate_up, None) for _, _, gate_up in self._packed],
            "down": [(layer.mlp.down_proj.weight, None) for layer in layers],
            "lm_head": [(self.model.lm_head.weight, self.model.lm_head.bias)] * 4,
        }
        self.projection_kernel = {}
        self.projection_times = {}  # per projection, the timed choice's device ms of each side
        capture = None
        self._tiles = {}  # data_ptr of a row-major weight -> its tile-major copy
        ffn = self.model.config.intermediate_size
        row_counts = {B} | ({len(rows) for rows, _ in self.groups} if self.groups else set())
        vocab, hidden = self.model.lm_head.weight.shape
        ws_bytes = max(max(gemm_workspace_bytes(r, w.shape[0], w.shape[1]), argmax_workspace_bytes(r, vocab, hidden))
                       for r in row_counts for weights in groups.values() for w, _ in weights[:1])
        self._gemm_ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        for name, weights in groups.items():
            x = torch.full((B, weights[0][0].shape[1]), 0.01, dtype=dt, device=dev)
            if not linear_supported(x, weights[0][0]):
                self.projection_kernel[name] = False
                continue
            for w, _ in weights:
                if w.data_ptr() not in self._tiles:
                    self._tiles[w.data_ptr()] = tile_gate_up(w, ffn) if name == "gate_up" else tile_weight(w)
            if mode != "auto":
                chosen = mode == "kernel"
            else:
                n_out = ffn if name == "gate_up" else weights[0][0].shape[0]
                y = torch.empty(B, n_out, dtype=dt, device=dev)
                if name == "gate_up":
                    kernel = lambda x, w, b: linear_swiglu_tiled(x, self._tiles[w.data_ptr()], ffn, out=y)  # noqa: E731
                    reference = lambda x, w, b: silu_mul(F.linear(x, w, b), out=y)  # noqa: E731
                elif name == "lm_head":  # the step's greedy tokens: the head and its argmax
                    tokens = torch.empty(B, dtype=torch.int64, device=dev)
                    kernel = lambda x, w, b: linear_argmax_tiled(  # noqa: E731
                        x, self._tiles[w.data_ptr()], w.shape[0], b, out=tokens, workspace=self._gemm_ws)
                    reference = lambda x, w, b: tokens.copy_(F.linear(x, w, b).argmax(-1))  # noqa: E731
                else:
                    kernel = lambda x, w, b: linear_tiled(  # noqa: E731
                        x, self._tiles[w.data_ptr()], w.shape[0], b, out=y, workspace=self._gemm_ws)
                    reference = lambda x, w, b: y.copy_(F.linear(x, w, b))  # noqa: E731
                if capture is None:
                    capture = torch.cuda.Stream(dev)  # one capture stream for every timed choice
                elapsed = {label: _graph_time([lambda w=w, b=b, fn=fn: fn(x, w, b) for w, b in weights], capture)
                           for label, fn in (("kernel", kernel), ("torch", reference))}
                chosen = elapsed["kernel"] <= elapsed["torch"]
            self.projection_times[name] = elapsed if mode == "auto" else None
            self.projection_kernel[name] = chosen
            if not chosen:
                for w, _ in weights:
                    self._tiles.pop(w.data_ptr(), None)

    def _next_tokens(self, h):
        """Greedy tokens (int64 [rows]) of the final-normed rows ``h``: the LM head and
        its argmax in the kernel's two launches (hs_skinny_gemm_argmax_tiled, no logits
        written) where the LM head runs on the kernel, else PyTorch's GEMM and argmax."""
        head = self.model.lm_head
        if self.projection_kernel["lm_head"]:
            return linear_argmax_tiled(h, self._tiles[head.weight.data_ptr()], head.weight.shape[0], head.bias,
                                       workspace=self._gemm_ws)
        return F.linear(h, head.weight, head.bias).argmax(-1)

    def _project(self, name, x, weight, bias=None, out=None):
        if self.projection_kernel[name]:
            return linear_tiled(x, self._tiles[weight.data_ptr()], weight.shape[0], bias, out=out,
                                workspace=self._gemm_ws)
        y = F.linear(x, weight, bias)
        if out is None:
            return y
        out.copy_(y)
        return out

    def _append(self, layer, k, v, positions, rows=None, handle=None):
        """Each request's new K/V row (``rows``: a range of requests, default all, whose rows
        are those of ``k``/``v``; or a list of slots whose rows are ``k``/``v`` in that
        order), on the stream ``handle`` (default: the current stream)."""
        st, cfg = self.state, self.state.config
        rows = range(st.batch) if rows is None else rows
        first = rows.start if isinstance(rows, range) else 0
        dev_rows, host_rows, lo, hi = st.append_args(layer, positions, rows)
        _lib.check(
            _lib.load().hs_append_rows(
                k[first].data_ptr(), v[first].data_ptr(), k.stride(0), st.pool.data_ptr(),
                st.blocks * cfg.page_size, _lib.dtype_code(cfg.dtype), cfg.page_size, cfg.kv_heads, cfg.head_dim,
                dev_rows, self._host_alias[layer], host_rows, st.host[layer].shape[0] * cfg.page_size, lo, hi,
                len(rows), handle if handle is not None else _lib.stream_handle(self.device),
            ),
            "hs_append_rows",
        )

    def _rotary_append(self, layer, positions, handle):
        """Layer ``layer``'s rotary embedding of the q|k|v projection and the append of every
        request's new K/V row, in one launch (hs_rotary_split_append)."""
        st, cfg, mc = self.state, self.state.config, self.model.config
        dev_rows, host_rows, lo, hi = st.append_args(layer, positions)
        _lib.check(
            _lib.load().hs_rotary_split_append(
                self._qkv.data_ptr(), self._qkv.stride(0), self._q.data_ptr(), self._k.data_ptr(),
                self._v.data_ptr(), self.positions.data_ptr(), st.batch, mc.num_attention_heads,
                mc.num_key_value_heads, mc.head_dim, mc.rope_theta, _lib.dtype_code(cfg.dtype), st.pool.data_ptr(),
                st.blocks * cfg.page_size, cfg.page_size, dev_rows, self._host_alias[layer], host_rows,
                st.host[layer].shape[0] * cfg.page_size, lo, hi, handle,
            ),
            "hs_rotary_split_append",
        )

    def decoders(self):
        """Every decoder the engine has built (whole batch, per layer, request groups,
        partial batches)."""
        found = [self.dec] + (self.decs or []) + [group for _, group in (self.groups or [])] + [
            sub[0] for sub in self._subsets.values()]
        return list({id(d): d for d in found}.values())

    def set_entry_stats(self, stats):
        """Total the attention's entry counts of every later step into ``stats`` (int64
        [1] on the device; None stops), from the union launches themselves."""
        self._entry_stats = stats
        for dec in self.decoders():
            dec.entry_stats = stats

    def check_status(self):
        """Raise if any layer's union overflowed its buffers in a step so far (reads the
        decoders' status flags back to the host: for tests and debugging, not timed runs)."""
        for dec in self.decoders():
            dec.check_status()

    @torch.inference_mode()
    def step(self, tokens, observer=None, timer=None, probe=None, active=None):
        """One decode step for all B requests: `tokens` [B] int64 (device) -> next tokens.

        ``active`` (optional): the slots that decode this step, in the order their writes
        go through the residency policy (the engine's turn order); the other slots are
        idle (no append, selection, resolve, gather or attention; their rows of the dense
        layers and of the returned tokens are not meaningful).  Default: every slot, in
        slot order.
        ``timer`` (optional list) receives, per layer, the stage events
        ``(layer, {stage: (start, end)}, entries)`` with ``entries`` the layer's
        attention entry total (device tensor) -- for profiling, not for timed runs.
        ``probe`` (optional) is called as ``probe.before_attend(layer, stream, decoder)``
        and ``probe.after_attend(layer, stream, decoder)`` around each layer's attention
        launch on the stream it runs on (light enough for timed runs: events and a copy of
        the decoder's entry counts).
        """
        order = None
        if active is not None:
            order = [int(b) for b in active]
            if sorted(order) != list(range(self.state.batch)):
                return self._step_subset(tokens, order, observer, timer, probe)
        if self.groups is not None:
            return self._step_groups(tokens, observer, timer, probe, order)
        model, st, dec = self.model, self.state, self.dec
        cfg = model.config
        positions = list(st.lengths)
        st.open_tail_pages(positions, order)
        for d in self.decs or (dec,):
            d.set_lengths([p + 1 for p in positions])
        sampled = None
        if self.selector == "uniform":
            sampled = self._draw_pages([p + 1 for p in positions])
        compute = torch.cuda.current_stream(self.device)
        L = st.layers

        def mark(stream):
            if timer is None:
                return None
            event = torch.cuda.Event(enable_timing=True)
            event.record(stream)
            return event

        prefetched = None
        if self.prefetch:
            self._step_start.record(compute)
            self.transfer.wait_event(self._step_start)
            sampled.record_stream(self.transfer)
            # issued PREFETCH_AHEAD layers ahead of the compute stream, so that neither
            # stream waits for the host to issue the other's launches
            prefetched = [self._prefetch(i, sampled, self.transfer, mark) for i in range(min(L, self.PREFETCH_AHEAD))]
        self._x.copy_(model.model.embed_tokens(tokens))
        graphs = self._graphs
        handle = _lib.stream_handle(self.device)  # the compute stream, looked up once per step
        prepared = None
        if graphs is None:
            if self._prepared is None:
                self._prepared = self._prepare_boundaries()
            prepared = self._prepared

        # the rotary launch (the last of a boundary before a layer) fused with the append
        fuse = self.fuse_rotary_append and graphs is None and prepared is not None

        def boundary(index):
            if graphs is not None:
                graphs[index].replay()
            elif prepared is not None:
                for launch in prepared[index][:-1] if fuse and index < L else prepared[index]:
                    launch(handle)
            else:
                self._boundary(index)

        q, k, v = self._q, self._k, self._v
        for index in range(L):
            if prefetched is not None and index + self.PREFETCH_AHEAD < L:
                prefetched.append(self._prefetch(index + self.PREFETCH_AHEAD, sampled, self.transfer, mark))
            marks = {"dense": [mark(compute)]}
            boundary(index)
            marks["dense"].append(mark(compute))
            marks["append"] = [marks["dense"][1]]
            if fuse:  # with the layer's rotary: the append stage holds it
                self._rotary_append(index, positions, handle)
            else:
                self._append(index, k, v, positions, handle=handle)
            lo, hi = st.bounds[index]
            marks["append"].append(mark(compute))
            if prefetched is not None:
                dec = self.decs[index]
                marks.update(prefetched[index])
                compute.wait_event(self._handoff[index][1])
            else:
                marks["select"] = [marks["append"][1]]
                if sampled is None:
                    dec.select(q, lo, hi, stream=handle)
                else:
                    dec.select_pages(sampled[index], stream=handle, validate=False)  # uniform_pages: ascending, tail last
                marks["select"].append(mark(compute))
                marks["resolve"] = [marks["select"][1]]
                dec.resolve(st.tables[index], row_stats=st.row_stats, stream=handle)
                marks["resolve"].append(mark(compute))
                transfer = self.transfer if self.transfer is not None else compute
                if transfer is not compute:
                    resolved, ready = self._handoff[index]
                    resolved.record(compute)
                    transfer.wait_event(resolved)
                marks["gather"] = [mark(transfer)]
                dec.gather(st.alias[index], st.pool, transfer if transfer is not compute else handle)
                marks["gather"].append(mark(transfer))
                if transfer is not compute:
                    ready.record(transfer)
                    compute.wait_event(ready)
            marks["attend"] = [mark(compute)]
            if probe is not None:
                probe.before_attend(index, compute, dec)
            out = dec.attend(q, st.pool, out=self._attn_out, stream=handle)
            if probe is not None:
                probe.after_attend(index, compute, dec)
            marks["attend"].append(mark(compute))
            if observer is not None:
                self.current_group = (range(st.batch), dec)
                observer(index, q, k, v, out)
            if index == L - 1:  # the last layer's o_proj and MLP
                marks["dense_last"] = [marks["attend"][1]]
                boundary(L)
                marks["dense_last"].append(mark(compute))
            if timer is not None:
                timer.append((index, marks, dec.entry_counts.sum(), dec.row_counts[:, 2].sum()))
        tokens = self._next_tokens(add_rms_norm(self._x, self._delta, model.model.norm.weight, cfg.rms_norm_eps))
        st.lengths = [p + 1 for p in positions]
        self.positions += 1
        if self.use_graphs and self._graphs is None:
            self._capture()
        return tokens

    def _subset(self, slots):
        """Decoder and compact buffers of the partial batch ``slots`` (sorted), built on
        first use (a few per run: admissions and finishes change the running set)."""
        key = tuple(slots)
        sub = self._subsets.get(key)
        if sub is None:
            st, cfg = self.state, self.model.config
            if len(self._subsets) >= 8:  # keep the latest few
                self._subsets.pop(next(iter(self._subsets)))
            dec = BatchedSparseDecode(
                st.config, cfg.num_attention_heads, self._top_pages, [max(1, st.lengths[b]) for b in slots],
                keep_sink=self._keep_sink, device=self.device, capacity_lengths=[self._caps[b] for b in slots],
                shared_selection=self.selector == "uniform", workspaces_from=self.dec,
                split_front=self._resolver_split,
            )
            index = torch.tensor(slots, dtype=torch.int64, device=self.device)
            n, dt, dev = len(slots), self.model.dtype, self.device
            Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
            buffers = tuple(torch.empty(shape, dtype=dt, device=dev)
                            for shape in ((n, Hq, D), (n, Hkv, D), (n, Hkv, D), (n, Hq, D)))
            dec.entry_stats = getattr(self, "_entry_stats", None)
            sub = self._subsets[key] = (dec, index, buffers)
        return sub

    def _step_subset(self, tokens, order, observer=None, timer=None, probe=None):
        """A decode step of the slots in ``order`` only (the others idle): the dense
        layers run for the whole batch (their cost is the weights, read once either way),
        the sparse stages for the decoding slots, gathered into compact buffers, in layer
        order on the compute stream."""
        model, st = self.model, self.state
        cfg = model.config
        slots = sorted(order)
        dec, index, (q, k, v, out) = self._subset(slots)
        positions = list(st.lengths)
        st.open_tail_pages(positions, order)
        dec.set_lengths([positions[b] + 1 for b in slots])
        sampled = None
        if self.selector == "uniform":
            sampled = self._draw_pages([positions[b] + 1 for b in slots])
        compute = torch.cuda.current_stream(self.device)
        handle = _lib.stream_handle(self.device)
        if self._prepared is None:
            self._prepared = self._prepare_boundaries()
        L = st.layers

        def mark(stream):
            if timer is None:
                return None
            event = torch.cuda.Event(enable_timing=True)
            event.record(stream)
            return event

        self._x.copy_(model.model.embed_tokens(tokens))
        for layer in range(L):
            marks = {"dense": [mark(compute)]}
            for launch in self._prepared[layer]:
                launch(handle)
            torch.index_select(self._q, 0, index, out=q)
            torch.index_select(self._k, 0, index, out=k)
            torch.index_select(self._v, 0, index, out=v)
            marks["dense"].append(mark(compute))
            marks["append"] = [marks["dense"][1]]
            self._append(layer, k, v, positions, slots, handle=handle)
            marks["append"].append(mark(compute))
            marks["select"] = [marks["append"][1]]
            if sampled is None:
                lo, hi = st.bounds[layer]
                dec.select(q, [lo[b] for b in slots], [hi[b] for b in slots], stream=handle)
            else:
                dec.select_pages(sampled[layer], stream=handle, validate=False)
            marks["select"].append(mark(compute))
            marks["resolve"] = [marks["select"][1]]
            dec.resolve([st.tables[layer][b] for b in slots], row_stats=st.row_stats, stream=handle)
            marks["resolve"].append(mark(compute))
            marks["gather"] = [marks["resolve"][1]]
            dec.gather(st.alias[layer], st.pool, handle)
            marks["gather"].append(mark(compute))
            marks["attend"] = [marks["gather"][1]]
            if probe is not None:
                probe.before_attend(layer, compute, dec)
            dec.attend(q, st.pool, out=out, stream=handle)
            if probe is not None:
                probe.after_attend(layer, compute, dec)
            marks["attend"].append(mark(compute))
            self._attn_out.index_copy_(0, index, out)
            if observer is not None:
                self.current_group = (slots, dec)
                observer(layer, q, k, v, out)
            if layer == L - 1:
                marks["dense_last"] = [marks["attend"][1]]
                for launch in self._prepared[L]:
                    launch(handle)
                marks["dense_last"].append(mark(compute))
            if timer is not None:
                timer.append((layer, marks, dec.entry_counts.sum(), dec.row_counts[:, 2].sum()))
        tokens = self._next_tokens(add_rms_norm(self._x, self._delta, model.model.norm.weight, cfg.rms_norm_eps))
        for b in slots:
            st.lengths[b] = positions[b] + 1
        self.positions.index_add_(0, index, torch.ones_like(index))
        return tokens

    def reset_slot(self, b, length):
        """Slot ``b`` holds a new request with a ``length``-token history (its prefill)."""
        self.positions[b] = length

    def _step_groups(self, tokens, observer=None, timer=None, probe=None, order=None):
        """A decode step with the batch split into request groups pipelined over layers.

        Compute-stream order: for each layer and group, the group's pending attention of
        the previous layer (after its gather's event) and its dense output, then the
        layer's dense input, append, Quest selection and resolve; the group's gather is
        queued on the transfer stream behind its resolve.  While group A's gather reads
        host memory, the compute stream serves group B, and the other way round.  Hot rows
        are rewritten by a gather only after the same group's attention of the previous
        step (the gather waits for a resolve queued after that attention)."""
        model, st = self.model, self.state
        cfg = model.config
        positions = list(st.lengths)
        st.open_tail_pages(positions, order)
        for rows, dec in self.groups:
            dec.set_lengths([positions[b] + 1 for b in rows])
        compute, transfer = torch.cuda.current_stream(self.device), self.transfer
        L = st.layers

        def mark(stream):
            if timer is None:
                return None
            event = torch.cuda.Event(enable_timing=True)
            event.record(stream)
            return event

        marks = [[{} for _ in self.groups] for _ in range(L)]

        def attend(index, g):
            rows, dec = self.groups[g]
            sl = slice(rows.start, rows.stop)
            compute.wait_event(self._group_events[index][g][1])
            m = marks[index][g]
            m["attend"] = [mark(compute)]
            if probe is not None:
                probe.before_attend(index, compute, dec)
            out = dec.attend(self._q[sl], st.pool, out=self._attn_out[sl])
            if probe is not None:
                probe.after_attend(index, compute, dec)
            m["attend"].append(mark(compute))
            if observer is not None:
                self.current_group = (rows, dec)
                observer(index, self._q[sl], self._k[sl], self._v[sl], out)
            m["dense_out"] = [mark(compute)]
            self._dense_out(index, sl)
            m["dense_out"].append(mark(compute))
            if timer is not None:
                timer.append((index, m, dec.entry_counts.sum(), dec.row_counts[:, 2].sum()))

        self._x.copy_(model.model.embed_tokens(tokens))
        for index in range(L):
            lo, hi = st.bounds[index]
            for g, (rows, dec) in enumerate(self.groups):
                sl = slice(rows.start, rows.stop)
                if index > 0:
                    attend(index - 1, g)
                m = marks[index][g]
                m["dense"] = [mark(compute)]
                self._dense_in(index, index == 0, sl)
                m["dense"].append(mark(compute))
                m["append"] = [m["dense"][1]]
                self._append(index, self._k, self._v, positions, rows)
                m["append"].append(mark(compute))
                m["select"] = [m["append"][1]]
                dec.select(self._q[sl], lo[sl], hi[sl])
                m["select"].append(mark(compute))
                m["resolve"] = [m["select"][1]]
                dec.resolve(st.tables[index][sl], row_stats=st.row_stats)
                m["resolve"].append(mark(compute))
                resolved, gathered = self._group_events[index][g]
                resolved.record(compute)
                transfer.wait_event(resolved)
                m["gather"] = [mark(transfer)]
                dec.gather(st.alias[index], st.pool, transfer, grid_x=self.group_gather_workgroups)
                m["gather"].append(mark(transfer))
                gathered.record(transfer)
        for g in range(len(self.groups)):
            attend(L - 1, g)
        tokens = self._next_tokens(add_rms_norm(self._x, self._delta, model.model.norm.weight, cfg.rms_norm_eps))
        st.lengths = [p + 1 for p in positions]
        self.positions += 1
        return tokens


def random_model(workload: DecodeWorkload, device, seed=0):
    """Random-init model of the workload's shape, built directly on the device in its dtype."""
    torch.manual_seed(seed)
    with torch.device(device):
        previous = torch.get_default_dtype()
        torch.set_default_dtype(workload.dtype)
        try:
            model = MiniModel(workload.model_config())
        finally:
            torch.set_default_dtype(previous)
    return model.eval()


def host_bytes_per_request(workload: DecodeWorkload, context=None, steps=None):
    """Pinned host bytes of one request's history (every layer, room for the decode)."""
    context = workload.context if context is None else context
    steps = workload.steps if steps is None else steps
    pages = ceil((context + steps) / workload.page_size)
    element = torch.empty((), dtype=workload.dtype).element_size()
    return workload.layers * pages * 2 * workload.page_size * workload.kv_heads * workload.head_dim * element


def policy_blocks(workload: DecodeWorkload, context=None):
    """Slab of the policy residency: ``resident_fraction`` of every history page, plus the
    blocks the policy's admission promises each (request, layer): its hot region and the
    two active tail pages (hybrid.py:36-37)."""
    context = workload.context if context is None else context
    used = ceil(context / workload.page_size)
    groups = workload.layers * workload.batch
    return round(workload.resident_fraction * groups * used) + groups * (ceil(workload.hot_rows / workload.page_size) + 2)


def empty_state(workload: DecodeWorkload, device, context=None, steps=None, residency="fraction", window=64,
                watermark=None):
    """A state sized for `context` history tokens plus `steps` decoded ones, no history yet.
    ``residency``: "fraction" (a seeded fraction of each layer's pages resident, chosen
    at prefill) or "policy" (the hybrid policy places every page and hot region in a slab
    of :func:`policy_blocks`, with the given resident window and watermark)."""
    context = workload.context if context is None else context
    steps = workload.steps if steps is None else steps
    P = workload.page_size
    cfg = CacheConfig(
        gpu_pages=1, host_pages=1, page_size=P, kv_heads=workload.kv_heads, head_dim=workload.head_dim,
        device=str(device), dtype=workload.dtype,
    )
    if residency == "policy":
        return SparseKVState(workload.layers, workload.batch, context + steps, cfg, workload.hot_rows, 0, 0,
                             policy_blocks=policy_blocks(workload, context), policy_window=window,
                             policy_watermark=watermark)
    if residency != "fraction":
        raise ValueError(f"unknown residency {residency!r}")
    used = ceil(context / P)
    resident = workload.layers * workload.batch * (round(workload.resident_fraction * used) + 1)
    spare = workload.layers * workload.batch * (ceil(steps / P) + 1)
    return SparseKVState(workload.layers, workload.batch, context + steps, cfg, workload.hot_rows, resident, spare)


def random_prompts(workload: DecodeWorkload, device, seed=0, context=None):
    """Uniformly random token ids: [batch, context] (the configs' random prompts)."""
    context = workload.context if context is None else context
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(0, workload.vocab, (workload.batch, context), generator=gen, device=device)


def build_state(workload: DecodeWorkload, device, seed=0, context=None, steps=None):
    """State sized for `context` history tokens plus `steps` decoded ones, history built."""
    context = workload.context if context is None else context
    steps = workload.steps if steps is None else steps
    P = workload.page_size
    cfg = CacheConfig(
        gpu_pages=1, host_pages=1, page_size=P, kv_heads=workload.kv_heads, head_dim=workload.head_dim,
        device=str(device), dtype=workload.dtype,
    )
    used = ceil(context / P)
    resident = workload.layers * workload.batch * (round(workload.resident_fraction * used) + 1)
    spare = workload.layers * workload.batch * (ceil(steps / P) + 1)
    state = SparseKVState(workload.layers, workload.batch, context + steps, cfg, workload.hot_rows, resident, spare)
    state.build_history(context, workload.resident_fraction, seed=seed)
    return state
