"""Read selected physical rows after resolving residency and loading misses.

``row_attention`` keeps the reference's checks and messages (attention.py:7-35).
The backend argument accepts ``"auto"`` and ``"hip"``; the reference's
``"torch"`` and ``"triton"`` paths do not exist here (the gfx950 kernels are
the only implementation) and are rejected as invalid backends.
"""

import torch

BACKENDS = ("auto", "hip")


@torch.inference_mode()
def row_attention(query, cache, request_id, layer, topk, backend="auto"):
    if backend not in BACKENDS:
        raise ValueError("invalid attention backend")
    if query.ndim != 2 or query.shape[1] != cache.config.head_dim:
        raise ValueError("invalid query shape")
    if query.shape[0] % cache.config.kv_heads or query.device != cache.pool.device:
        raise ValueError("query GQA/device mismatch")
    if topk.head_columns is not None and topk.head_columns.shape[0] != query.shape[0]:
        raise ValueError("selection must have one row per query head")
    with cache.resolve(request_id, layer, topk) as lease:
        return cache.ops.attend(query, cache.pool, lease.plan, topk, cache.config)
