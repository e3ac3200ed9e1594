"""mini_hisparse_amd: mini-hisparse's per-step sparse decode path on MI355X (gfx950).

Same Python API as the reference package (``CacheConfig``, ``HotConfig``,
``HybridKVCache``, ``LogicalTopK``, engine and model); the resolver, Quest
selector, host-row gather and row attention run as hand-written HIP kernels
from ``libhisparse_hip.so`` (C ABI: include/hisparse.h).
"""

from .config import CacheConfig, CapacityError
from .hybrid import HotConfig, HybridKVCache
from .row_index import LogicalTopK

__all__ = ["CacheConfig", "CapacityError", "HotConfig", "HybridKVCache", "LogicalTopK"]
