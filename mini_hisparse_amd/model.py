"""A Qwen2-shaped decoder that drives the sparse decode path.

The reference's ``MiniModel`` (``mini_hisparse/model.py:19-226``) is kept as an
interface: ``ModelConfig`` fields, Hugging Face Qwen2 parameter names and the
order parameters are created in (a seeded random init reproduces the reference's
weights; Qwen2/Qwen2.5 checkpoints load unchanged), ``prefill`` / ``decode`` /
``from_pretrained`` signatures and errors.

Organisation (this module's own): a layer's parameters are declared as linear
specs; one routine, :meth:`MiniModel._layers`, runs the decoder stack for any
number of tokens at given positions and hands each layer's rotated q/k/v to an
attention callback -- causal SDPA for a prefill (PyTorch-ROCm's, not on the
timed path), for a decode the cache append, page selection (Quest through the
cache's kernel backend by default) and sparse row attention.  The arithmetic of
each step (RMSNorm in float32, rotary tables rounded to the model dtype, SiLU
MLP) is Qwen2's, op for op, so logits match the reference bit for bit on the
same device.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch
from torch import nn
from torch.nn import functional as F

from .selection import Selection, select_pages


@dataclass
class ModelConfig:
    vocab_size: int = 256
    hidden_size: int = 128
    intermediate_size: int = 256
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden_size // self.num_attention_heads

    def __post_init__(self):
        if (
            self.hidden_size % self.num_attention_heads
            or self.num_attention_heads % self.num_key_value_heads
            or self.head_dim % 2
        ):
            raise ValueError("model dimensions must support grouped-query attention and RoPE")


class RMSNorm(nn.Module):
    """Root-mean-square norm computed in float32, scaled in the input dtype."""

    def __init__(self, width, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps

    def forward(self, x):
        wide = x.float()
        return (wide * torch.rsqrt(wide.square().mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


def _linears(**specs):
    """A module holding ``nn.Linear`` children created in the keyword order given:
    ``name=(in_features, out_features, bias)``."""
    module = nn.Module()
    for name, (width_in, width_out, bias) in specs.items():
        setattr(module, name, nn.Linear(width_in, width_out, bias=bias))
    return module


def _layer(cfg: ModelConfig):
    """One decoder layer in Qwen2 naming; creation order: the two norms, then q, k, v,
    o, then gate, up, down (the order the random init draws in)."""
    hidden, kv = cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim
    layer = nn.Module()
    layer.input_layernorm = RMSNorm(hidden, cfg.rms_norm_eps)
    layer.post_attention_layernorm = RMSNorm(hidden, cfg.rms_norm_eps)
    layer.self_attn = _linears(q_proj=(hidden, hidden, True), k_proj=(hidden, kv, True), v_proj=(hidden, kv, True),
                               o_proj=(hidden, hidden, False))
    ffn = cfg.intermediate_size
    layer.mlp = _linears(gate_proj=(hidden, ffn, False), up_proj=(hidden, ffn, False), down_proj=(ffn, hidden, False))
    return layer


def rope_tables(start, count, dim, theta, dtype, device):
    """Rotary cos/sin ``[count, 1, dim]`` for positions ``start .. start+count-1``:
    angles in float32, the tables rounded to ``dtype`` (Qwen2's order of operations)."""
    inverse = theta ** (-torch.arange(0, dim, 2, device=device).float() / dim)
    angles = torch.arange(start, start + count, device=device).float()[:, None] * inverse[None, :]
    angles = torch.cat((angles, angles), -1)[:, None, :]
    return angles.cos().to(dtype), angles.sin().to(dtype)


def apply_rope(tensor, cos, sin):
    """``[tokens, heads, dim]`` rotated by half-dimension pairs."""
    first, second = tensor.chunk(2, -1)
    return tensor * cos + torch.cat((-second, first), -1) * sin


def rotary(tensor, start, theta):
    """Rotary embedding of ``[tokens, heads, head_dim]`` at positions start, start+1, ..."""
    cos, sin = rope_tables(start, tensor.shape[0], tensor.shape[-1], theta, tensor.dtype, tensor.device)
    return apply_rope(tensor, cos, sin)


class MiniModel(nn.Module):
    def __init__(self, config: ModelConfig | None = None):
        super().__init__()
        self.config = cfg = config or ModelConfig()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.model.layers = nn.ModuleList(_layer(cfg) for _ in range(cfg.num_hidden_layers))
        self.model.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    @classmethod
    def from_pretrained(cls, name: str, device="cuda", dtype=torch.bfloat16):
        """Adopt the modules of a Qwen2/Qwen2.5 checkpoint (standard RoPE, SiLU, no
        sliding window), given as a local directory or a hub name."""
        from transformers import AutoConfig, AutoModelForCausalLM

        hf_config = AutoConfig.from_pretrained(name)
        # transformers 4 keeps rope_theta on the config; 5 moves it into rope_parameters
        rope = getattr(hf_config, "rope_parameters", None) or getattr(hf_config, "rope_scaling", None) or {}
        kind = rope.get("rope_type", rope.get("type", "default"))
        if hf_config.model_type != "qwen2" or kind != "default":
            raise ValueError("only Qwen2/Qwen2.5 with standard RoPE are supported")
        if getattr(hf_config, "use_sliding_window", False) or hf_config.hidden_act != "silu":
            raise ValueError("sliding window / non-SiLU models are unsupported")
        values = {f.name: getattr(hf_config, f.name) for f in fields(ModelConfig) if f.name != "rope_theta"}
        values["rope_theta"] = rope.get("rope_theta", getattr(hf_config, "rope_theta", 10000.0))
        hf = AutoModelForCausalLM.from_pretrained(name, torch_dtype=dtype).eval().to(device)
        model = cls.__new__(cls)
        nn.Module.__init__(model)
        model.config = ModelConfig(**values)
        model.model, model.lm_head = hf.model, hf.lm_head
        return model.eval()

    @property
    def device(self):
        return self.model.embed_tokens.weight.device

    @property
    def dtype(self):
        return self.model.embed_tokens.weight.dtype

    # -- the decoder stack -----------------------------------------------------------
    def _layers(self, tokens, start, attend):
        """Run every layer over ``tokens`` (1-D device ids) at positions ``start...``;
        ``attend(index, q, k, v)`` returns the layer's attention output ``[tokens,
        heads, head_dim]`` from its rotated q ``[tokens, heads, D]``, k and v
        ``[tokens, kv_heads, D]``.  Returns the final hidden states."""
        cfg = self.config
        x = self.model.embed_tokens(tokens)
        cos, sin = rope_tables(start, len(tokens), cfg.head_dim, cfg.rope_theta, x.dtype, x.device)
        for index, layer in enumerate(self.model.layers):
            h = layer.input_layernorm(x)
            proj = layer.self_attn
            q = proj.q_proj(h).view(len(tokens), cfg.num_attention_heads, cfg.head_dim)
            k = proj.k_proj(h).view(len(tokens), cfg.num_key_value_heads, cfg.head_dim)
            v = proj.v_proj(h).view(len(tokens), cfg.num_key_value_heads, cfg.head_dim)
            attention = attend(index, apply_rope(q, cos, sin), apply_rope(k, cos, sin), v)
            x = x + proj.o_proj(attention.reshape(len(tokens), -1))
            mlp = layer.mlp
            h = layer.post_attention_layernorm(x)
            x = x + mlp.down_proj(F.silu(mlp.gate_proj(h)) * mlp.up_proj(h))
        return x

    def _logits(self, hidden):
        return self.lm_head(self.model.norm(hidden)).float()

    # -- entry points ---------------------------------------------------------------------
    @torch.inference_mode()
    def prefill(self, tokens: list[int], cache=None, request_id=None, observer=None):
        if not tokens:
            raise ValueError("prompt cannot be empty")
        if cache is not None and any(cache.storage.requests[request_id].lengths):
            raise ValueError("prefill is allowed exactly once per request")
        groups = self.config.num_attention_heads // self.config.num_key_value_heads

        def causal(index, q, k, v):
            if cache is not None:
                cache.write(request_id, index, k, v)
            if observer is not None:
                observer.prefill(request_id, index, k, v)
            heads_first = lambda t: t.repeat_interleave(groups, 1).transpose(0, 1)  # noqa: E731
            out = F.scaled_dot_product_attention(q.transpose(0, 1), heads_first(k), heads_first(v), is_causal=True)
            return out.transpose(0, 1)

        hidden = self._layers(torch.tensor(tokens, device=self.device), 0, causal)
        return self._logits(hidden[-1])

    def _select(self, cache, request_id, layer, query, top_k, selector):
        request = cache.storage.requests[request_id]
        length = request.lengths[layer]
        if selector == "quest" and top_k is not None:
            return cache.ops.quest_selection(query, request.minimum[layer], request.maximum[layer], length,
                                             cache.config.page_size, top_k)
        if selector in ("quest", "mean"):
            pages = select_pages(cache, request_id, layer, query, top_k)
            return Selection.from_pages(pages, length, cache.config.page_size, query.shape[0])
        raise ValueError("selector must be quest or mean")

    @torch.inference_mode()
    def decode(self, token: int, request_id, cache, top_k=None, backend="auto", selector="quest", observer=None):
        lengths = cache.storage.requests[request_id].lengths
        if len(set(lengths)) != 1 or lengths[0] == 0:
            raise ValueError("all layers must have the same nonempty history")

        def sparse(index, q, k, v):
            cache.write(request_id, index, k, v)
            if observer is not None:
                observer.decode(request_id, index, q[0], k, v)
            selection = self._select(cache, request_id, index, q[0], top_k, selector)
            return cache.attention(q[0], request_id, index, selection, backend).unsqueeze(0)

        hidden = self._layers(torch.tensor([token], device=self.device), lengths[0], sparse)
        return self._logits(hidden[0])
