"""Storage dimensions and capacity errors (same fields and checks as config.py:8-30 of
the reference)."""

from dataclasses import dataclass

import torch


class CapacityError(RuntimeError):
    """Admission or allocation cannot be satisfied now (callers defer or retry)."""


_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


@dataclass(frozen=True)
class CacheConfig:
    gpu_pages: int = 16
    host_pages: int = 1024
    page_size: int = 16
    kv_heads: int = 2
    head_dim: int = 32
    device: str = "cuda"
    dtype: torch.dtype = torch.float32
    index_budget_bytes: int = 64 * 1024 * 1024

    def __post_init__(self):
        for name in ("gpu_pages", "host_pages", "page_size", "kv_heads", "head_dim"):
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be positive")
        if self.dtype not in _DTYPES:
            raise ValueError("KV dtype must be float32, float16 or bfloat16")
        if self.index_budget_bytes < 1:
            raise ValueError("index budget must be positive")

    @property
    def row_bytes(self):
        """Bytes of one token row: K and V of every KV head (hybrid.py:569)."""
        return 2 * self.kv_heads * self.head_dim * torch.empty((), dtype=self.dtype).element_size()
