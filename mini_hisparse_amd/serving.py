"""The reference's ``Engine`` API over the layer-major batched decode.

``Engine`` (engine.py, the reference's ``engine.py:24-146``) decodes one request at a
time through ``HybridKVCache``.  :class:`LayerMajorEngine` keeps the same interface
-- ``add_request`` / ``step() -> [(request_id, token)]`` / ``run`` / ``cancel``, the
same validation and errors, the same schedule -- and runs every step's decode turns
as one layer-major batched step (:class:`BatchedDecodeEngine`) over the running
requests:

* a step first admits at most one waiting prompt (``engine.py:85-113``): the
  policy's credit check (``HybridKVCache.reserve``), then the prefill through the
  model with every layer's K/V written by ``hs_append_tokens`` and the pages placed
  by the hybrid policy (:class:`PlacementPlan`); the prefill's token is emitted;
* then every running request takes its decode turn (``engine.py:115-128``), in
  turn order: one batched step whose policy writes go request by request in that
  order, then one read of the step's tokens;
* a request finishes on the end-of-sequence token or its last token
  (``engine.py:71-77``) and is released at once: its hot regions and resident
  pages return to the slab (``hybrid.py:487-506``, ``PlacementPlan.release``) and
  its slot (host pool rows, tables, bounds) takes the next admission.

:class:`LayerMajorCache` is the cache side: a slab of ``CacheConfig.gpu_pages``
blocks placed by the reference's hybrid policy (``HotConfig``: hot rows, resident
window, watermark), and ``max_requests`` request slots of ``max_tokens`` tokens each
in pinned host memory.
"""

from __future__ import annotations

from math import ceil

import torch

from .batched_engine import BatchedDecodeEngine, SparseKVState
from .config import CacheConfig, CapacityError
from .engine import Engine, Request
from .hybrid import HotConfig


class LayerMajorCache:
    """Request slots of the layer-major state, with the admission surface of
    ``HybridKVCache`` (``reserve``, ``release_request``, ``collect``,
    ``admission_blocks``, ``index_reservation_bytes``, ``budget``, ``row_stats``).

    ``config.gpu_pages`` is the slab, ``config.host_pages`` bounds the pinned host
    pages of all slots together (``max_requests * layers * ceil(max_tokens / P)``),
    ``hot`` the policy's hot regions, window and watermark."""

    def __init__(self, config: CacheConfig, hot: HotConfig, layers: int, max_requests: int, max_tokens: int):
        if layers < 1 or max_requests < 1 or max_tokens < 1:
            raise ValueError("layers, max_requests and max_tokens must be positive")
        P = config.page_size
        host = max_requests * layers * ceil(max_tokens / P)
        if host > config.host_pages:
            raise CapacityError(f"{max_requests} request slots of {max_tokens} tokens need {host} host pages, "
                                f"above host_pages {config.host_pages}")
        if hot.admission_blocks(P, layers) > config.gpu_pages:
            raise CapacityError("one request's hot regions and tail pages do not fit the slab")
        self.config, self.hot_config, self.layers = config, hot, layers
        self.max_tokens = max_tokens
        self.state = SparseKVState(layers, max_requests, max_tokens, config, hot.hot_rows, 0, 0,
                                   policy_blocks=config.gpu_pages, policy_window=hot.resident_window_pages,
                                   policy_watermark=hot.transition_watermark)
        self.plan = self.state.plan
        self.slot_of: dict[str, int] = {}
        self.free_slots = list(range(max_requests))
        self.stats = {"retired_requests": 0}

    @property
    def pool(self):
        return self.state.pool

    @property
    def budget(self):
        return self.config.gpu_pages

    @property
    def row_stats(self):
        return self.state.row_stats

    def admission_blocks(self, layers):
        return self.hot_config.admission_blocks(self.config.page_size, layers)

    def index_reservation_bytes(self, max_tokens, layers):
        """The index a request reserves (``HybridKVCache.index_reservation_bytes``): page
        tables, Quest bounds and page means per page, the hot tables per layer."""
        cfg = self.config
        pages = ceil(max_tokens / cfg.page_size)
        element = torch.empty((), dtype=cfg.dtype).element_size()
        per_page = cfg.kv_heads * cfg.head_dim * (4 + 2 * element)
        hot_blocks = ceil(self.hot_config.hot_rows / cfg.page_size)
        per_layer = pages * 8 + hot_blocks * 4 + self.hot_config.hot_rows * 12
        return pages * layers * per_page + layers * per_layer

    def reserve(self, request_id, max_tokens, layers):
        """A free slot and the policy's credits (``HybridKVCache.reserve``)."""
        if layers != self.layers:
            raise ValueError("the cache was built for another layer count")
        if max_tokens > self.max_tokens:
            raise CapacityError("request exceeds the slot capacity")
        if not self.free_slots:
            raise CapacityError("every request slot is in use; defer admission")
        slot = self.free_slots[0]
        self.plan.reserve(slot, max_tokens, layers)  # raises CapacityError on the credits
        self.free_slots.pop(0)
        self.slot_of[request_id] = slot
        self.state.reset_slot(slot)
        return slot

    def release_request(self, request_id, wait=True):
        """The request's hot regions and resident pages return to the slab (the policy's
        release), its slot to the free slots."""
        slot = self.slot_of.pop(request_id)
        self.plan.release(slot)
        rows = [(l, b, page) for (b, l), page in self.plan.detached if b != slot]
        self.plan.detached.clear()
        if rows:  # pages of other requests the release tick detached (none: a release frees blocks)
            index = torch.tensor(rows, dtype=torch.int64).T.to(self.state.device)
            self.state.resident[index[0], index[1], index[2]] = -1
        self.state.resident[:, slot] = -1
        self.free_slots.append(slot)
        self.free_slots.sort()
        self.stats["retired_requests"] += 1

    def collect(self, wait=False):
        """Nothing is retired asynchronously: a release returns its blocks and slot at once."""

    def snapshot(self):
        rows = self.state.row_stats.tolist()
        P, Hkv, D = self.config.page_size, self.config.kv_heads, self.config.head_dim
        element = torch.empty((), dtype=self.config.dtype).element_size()
        return {
            "row_stats": {"resident_hits": int(rows[0]), "hot_hits": int(rows[1]), "misses": int(rows[2]),
                          "h2d_bytes": int(rows[2]) * 2 * Hkv * D * element},
            "stats": {**{k: int(v) for k, v in self.plan.stats.items()}, **self.stats},
            "slots": dict(self.slot_of),
        }


class LayerMajorEngine(Engine):
    """``Engine`` (same constructor arguments, methods, errors and schedule) whose decode
    turns run as one layer-major batched step over the running requests.

    ``top_k`` is the Quest page budget per query head (``None``: every page); the
    selector is ``"quest"`` (the reference's ``"mean"`` page-mean selector is not
    provided) or ``"uniform"`` (pages resampled every step, the miss-heavy stress shape).
    ``backend`` is ``"auto"`` or ``"hip"``.  Keyword options go to
    :class:`BatchedDecodeEngine` (request groups, projections, graphs)."""

    def __init__(self, model, cache: LayerMajorCache, top_k=None, backend="auto", eos_token_id=None,
                 selector="quest", **options):
        if backend not in ("auto", "hip"):
            raise ValueError("invalid attention backend")
        if selector not in ("quest", "uniform"):
            raise ValueError(f"selector {selector!r} is not provided by the layer-major engine")
        super().__init__(model, cache, top_k, backend, eos_token_id, selector)
        pages = ceil(cache.max_tokens / cache.config.page_size)
        self.batched = BatchedDecodeEngine(model, cache.state, top_k or pages, selector=selector, **options)
        self._tokens = torch.zeros(cache.state.batch, dtype=torch.int64, device=cache.state.device)

    def _reserve(self, request):
        self.cache.reserve(request.request_id, len(request.prompt) + request.max_new_tokens, self._layers)

    def _admit_one(self):
        if not self.waiting:
            return None
        request = self.waiting[0]
        try:
            self._reserve(request)
        except CapacityError:
            if not self.running:  # nothing decodes, so nothing will free capacity
                raise
            return None
        self.waiting.popleft()
        slot = self.cache.slot_of[request.request_id]
        first = self.cache.state.prefill_slot(self.model, slot, request.prompt)
        self.batched.reset_slot(slot, len(request.prompt))
        with torch.inference_mode():  # the token buffer is a step's output (an inference tensor)
            self._tokens[slot] = first  # the slot's next input token, on the device
        request.prefill_count += 1
        token = int(first.item())
        self._record(request, token)
        if not request.finished:
            self.running.append(request)
        return request.request_id, token

    def _record(self, request, token):
        """Emit a token; a finished request releases its cache at once (engine.py:71-77)."""
        request.generated.append(token)
        request.finished = token == self.eos_token_id or len(request.generated) >= request.max_new_tokens
        if request.finished:
            self.cache.release_request(request.request_id, wait=False)

    def _decode_turns(self, observer=None, timer=None, probe=None):
        if not self.running:
            return []
        turns = list(self.running)
        slots = [self.cache.slot_of[r.request_id] for r in turns]
        # every running request's last token is already on the device: its prefill's in
        # its slot (admission), or its slot of the previous step's output; the step's
        # output is the next step's input, so no token crosses to the device per step
        out = self.batched.step(self._tokens, observer=observer, timer=timer, probe=probe, active=slots)
        self._tokens = out
        host = out.cpu().tolist()
        tokens = [host[slot] for slot in slots]
        emitted = []
        for request, token in zip(turns, tokens):
            request.decode_count += 1
            self._record(request, int(token))
            emitted.append((request.request_id, int(token)))
            if request.finished:
                self.running.remove(request)
        return emitted

    def step(self, observer=None, timer=None, probe=None):
        """Admit at most one prompt, then give every running request a decode turn (one
        batched step); returns the (request id, token) pairs emitted this step.
        ``observer`` (tests), ``timer`` and ``probe`` (measurement) go to the batched
        step (:meth:`BatchedDecodeEngine.step`)."""
        admitted = self._admit_one()
        return ([admitted] if admitted else []) + self._decode_turns(observer, timer, probe)

    def run(self):
        while self.waiting or self.running:
            self.step()
        return {name: request.generated for name, request in self.requests.items()}

    def cancel(self, request_id):
        request = self.requests[request_id]
        if request.finished:
            return
        if request in self.waiting:
            self.waiting.remove(request)
        else:
            self.running.remove(request)
            self.cache.release_request(request_id, wait=False)
        request.finished = request.cancelled = True


__all__ = ["LayerMajorCache", "LayerMajorEngine", "Request"]
