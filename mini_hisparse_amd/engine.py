"""Request scheduler for the sparse-decode cache (the reference's ``Engine``,
``mini_hisparse/engine.py:12-146``, as an interface: ``Request``,
``Engine(model, cache, top_k, backend, eos_token_id, selector)``,
``add_request`` / ``step`` / ``run`` / ``cancel`` and their errors).

Policy: admission is bounded by host backing, hot-region credits and the index
budget, never by whole-request device memory.  Each step first polls retired
requests, then *admits* at most one waiting prompt (a prefill; when admission
fails with nothing running it drains retirements and retries once), then gives
every running request one *decode turn* in arrival order -- a long queue never
starves requests already decoding.  A request leaves the running set on its
last token or the end-of-sequence token, and its cache is released then.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from .config import CapacityError
from .model import MiniModel


@dataclass
class Request:
    request_id: str
    prompt: list[int]
    max_new_tokens: int
    generated: list[int] = field(default_factory=list)
    prefill_count: int = 0
    decode_count: int = 0
    finished: bool = False
    cancelled: bool = False


class Engine:
    def __init__(self, model: MiniModel, cache, top_k=None, backend="auto", eos_token_id: int | None = None,
                 selector: str = "quest"):
        mcfg, ccfg = model.config, cache.config
        if (mcfg.num_key_value_heads, mcfg.head_dim) != (ccfg.kv_heads, ccfg.head_dim):
            raise ValueError("model/cache head dimensions differ")
        if (model.device, model.dtype) != (cache.pool.device, cache.pool.dtype):
            raise ValueError("model/cache dtype or device differ")
        if top_k is not None and top_k < 1:
            raise ValueError("top_k must be positive or None")
        self.model, self.cache = model, cache
        self.top_k, self.backend, self.selector = top_k, backend, selector
        self.eos_token_id = eos_token_id
        self.requests: dict[str, Request] = {}
        self.waiting: deque[Request] = deque()
        self.running: deque[Request] = deque()

    @property
    def _layers(self):
        return self.model.config.num_hidden_layers

    def add_request(self, request_id, prompt, max_new_tokens=16):
        """Queue a prompt; reject what could never be admitted, even into empty pools."""
        if request_id in self.requests or not prompt or max_new_tokens < 1:
            raise ValueError("need a unique ID, nonempty prompt, and positive output length")
        vocab = self.model.config.vocab_size
        if min(prompt) < 0 or max(prompt) >= vocab:
            raise ValueError("token outside model vocabulary")
        tokens, cfg = len(prompt) + max_new_tokens, self.cache.config
        if -(-tokens // cfg.page_size) * self._layers > cfg.host_pages:
            raise CapacityError("request cannot fit even in an empty host pool")
        credits = getattr(self.cache, "admission_blocks", None)
        if credits is not None and credits(self._layers) > self.cache.budget:
            raise CapacityError("request hot-region + tail footprint cannot fit the device pool")
        if self.cache.index_reservation_bytes(tokens, self._layers) > cfg.index_budget_bytes:
            raise CapacityError("request index cannot fit even in an empty index budget")
        request = Request(request_id, list(prompt), max_new_tokens)
        self.requests[request_id] = request
        self.waiting.append(request)
        return request

    def _finish_token(self, request, logits):
        """Greedy token; a request that is done releases its cache right away."""
        token = int(logits.argmax().item())
        request.generated.append(token)
        request.finished = token == self.eos_token_id or len(request.generated) >= request.max_new_tokens
        if request.finished:
            self.cache.release_request(request.request_id, wait=False)
        return token

    def _reserve(self, request):
        self.cache.reserve(request.request_id, len(request.prompt) + request.max_new_tokens, self._layers)

    def _admit_one(self):
        """Admit and prefill the oldest waiting prompt if the cache takes it; returns
        the emitted (request, token) or None."""
        if not self.waiting:
            return None
        request = self.waiting[0]
        try:
            self._reserve(request)
        except CapacityError:
            # with nothing decoding, only retirements can free capacity: drain them
            if self.running or not self.cache.storage.retired:
                if not self.running:
                    raise
                return None
            self.cache.collect(wait=True)
            self._reserve(request)
        self.waiting.popleft()
        logits = self.model.prefill(request.prompt, self.cache, request.request_id)
        request.prefill_count += 1
        token = self._finish_token(request, logits)
        if not request.finished:
            self.running.append(request)
        return request.request_id, token

    def _decode_turns(self):
        emitted = []
        for request in list(self.running):
            logits = self.model.decode(request.generated[-1], request.request_id, self.cache, self.top_k,
                                       self.backend, selector=self.selector)
            request.decode_count += 1
            emitted.append((request.request_id, self._finish_token(request, logits)))
            if request.finished:
                self.running.remove(request)
        return emitted

    def step(self):
        """Admit at most one prompt, then give every running request a decode turn;
        returns the (request id, token) pairs emitted this step."""
        self.cache.collect()
        admitted = self._admit_one()
        return ([admitted] if admitted else []) + self._decode_turns()

    def run(self):
        while self.waiting or self.running:
            self.step()
        self.cache.collect(wait=True)
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
