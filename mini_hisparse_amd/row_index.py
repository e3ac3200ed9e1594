"""Logical selection -> physical rows (the resolver boundary).

Same names, arguments and errors as mini_hisparse's ``row_index``
(``row_index.py:15-137``); the resolve itself runs in the gfx950 kernel
``hs_resolve_rows`` (bit-exact with the reference, including the in-place
``tags``/``lru`` update).  It needs ROCm device tensors and never reads
anything back to the host, so it can be captured in a HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class GroupEntries:
    """Per (KV head) deduplicated union columns and query-head masks (hs_build_union)."""

    columns: torch.Tensor  # [Hkv, capacity] int32
    masks: torch.Tensor  # [Hkv, capacity] int32 bit masks (bit i = head kv*g + i)
    counts: torch.Tensor  # [Hkv] int32
    capacity: int


@dataclass(frozen=True)
class LogicalTopK:
    """Selected logical tokens: a shared vector, or a union plus per-head columns.

    ``positions`` may carry trailing -1 padding (device-built unions); padding
    is masked by the resolver exactly like any other invalid position.
    ``entries`` (optional) lets attention read each KV head's rows once.
    """

    positions: torch.Tensor  # shared [K] token positions, or the union for GQA
    head_columns: torch.Tensor | None = None  # [heads, K_head], -1 padding
    entries: GroupEntries | None = None
    union_count: torch.Tensor | None = None  # [1] int32 union size, device-built unions

    @classmethod
    def from_selection(cls, selection, device):
        """Host adapter (row_index.py:20-31); device selections build on the GPU."""
        build = getattr(selection, "logical_topk", None)
        if build is not None:
            return build(device)
        union = sorted({p for row in selection.positions for p in row})
        columns = {token: i for i, token in enumerate(union)}
        width = max(map(len, selection.positions))
        rows = [
            [columns[p] for p in row] + [-1] * (width - len(row)) for row in selection.positions
        ]
        return cls(
            torch.tensor(union, dtype=torch.int32, device=device),
            torch.tensor(rows, dtype=torch.int64, device=device),
        )

    def validate(self, device, maximum):
        positions = self.positions
        if (
            positions.ndim != 1
            or positions.numel() < 1
            or positions.dtype not in (torch.int32, torch.int64)
            or positions.device != torch.device(device)
        ):
            raise ValueError("logical top-k must be a nonempty device integer vector")
        if positions.numel() > maximum:
            raise ValueError("top-k width/union exceeds the admitted max_union_rows")
        if self.head_columns is not None and (
            self.head_columns.ndim != 2
            or self.head_columns.device != torch.device(device)
            or self.head_columns.dtype != torch.int64
        ):
            raise ValueError("head columns must be a device int64 matrix")


@dataclass
class RowPlan:
    physical_rows: torch.Tensor  # shared [K] or per-head [H, K], -1 padding
    miss_host_rows: torch.Tensor  # fixed-width compact prefix; -1 after misses
    miss_device_rows: torch.Tensor
    counts: torch.Tensor  # unique resident hits, hot hits, misses
    union_physical: torch.Tensor | None = None  # [K] physical rows in input order


def _require_device(*tensors):
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                "the HIP resolver needs ROCm device tensors; CPU tables are not supported"
            )


def _as_i32(t):
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def resolve_rows(
    topk, source_table, resident_table, hot_table, tags, lru, length, page_size, *, row_stats=None
):
    """Resident lookup first; protect every selected hot hit before any eviction.

    Mirrors row_index.py:59-137.  ``tags`` (int32) and ``lru`` (int64) are
    updated in place.  ``row_stats`` (optional int64[3]) receives ``counts``
    added on the device, fusing hybrid.py:454.
    """
    positions = topk.positions
    _require_device(positions, source_table, resident_table, hot_table, tags, lru)
    if tags.dtype != torch.int32 or lru.dtype != torch.int64 or not (
        tags.is_contiguous() and lru.is_contiguous()
    ):
        # tables of other integer dtypes: resolve on canonical copies, write back
        tags32 = tags.to(torch.int32).contiguous()
        lru64 = lru.to(torch.int64).contiguous()
        plan = resolve_rows(
            topk, source_table, resident_table, hot_table, tags32, lru64, length, page_size,
            row_stats=row_stats,
        )
        tags.copy_(tags32)
        lru.copy_(lru64)
        return plan
    if positions.dtype not in (torch.int32, torch.int64):
        raise ValueError("logical top-k must be a nonempty device integer vector")
    positions = positions.contiguous()
    n = positions.numel()
    device = positions.device
    source = _as_i32(source_table)
    resident = _as_i32(resident_table)
    hot = _as_i32(hot_table)
    if length > source.numel() * page_size:
        raise ValueError("length exceeds the page tables")
    columns = topk.head_columns
    if columns is not None:
        physical = torch.empty(columns.shape, dtype=torch.int64, device=device)
    else:
        physical = torch.empty(n, dtype=torch.int64, device=device)
    union_physical = torch.empty(n, dtype=torch.int64, device=device)
    miss_host = torch.empty(n, dtype=torch.int64, device=device)
    miss_device = torch.empty(n, dtype=torch.int64, device=device)
    counts = torch.empty(3, dtype=torch.int64, device=device)
    lib = _lib.load()
    ws_bytes = lib.hs_resolve_workspace_bytes(n, length, source.numel(), tags.numel())
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    desc = _lib.ResolveDesc()
    desc.positions = positions.data_ptr()
    desc.n = n
    desc.positions_i64 = int(positions.dtype == torch.int64)
    if columns is not None:
        desc.head_columns = columns.data_ptr()
        desc.heads, desc.width = columns.shape
        desc.hc_stride_h, desc.hc_stride_w = columns.stride()
    desc.source = source.data_ptr()
    desc.resident = resident.data_ptr()
    desc.n_pages = source.numel()
    desc.hot = hot.data_ptr()
    desc.hot_blocks = hot.numel()
    desc.tags = tags.data_ptr()
    desc.lru = lru.data_ptr()
    desc.hot_rows = tags.numel()
    desc.length = int(length)
    desc.page_size = int(page_size)
    desc.physical = physical.data_ptr()
    desc.union_physical = union_physical.data_ptr()
    desc.miss_host_rows = miss_host.data_ptr()
    desc.miss_device_rows = miss_device.data_ptr()
    desc.counts = counts.data_ptr()
    desc.row_stats = _lib.ptr(row_stats)
    status = lib.hs_resolve_rows(
        desc, workspace.data_ptr(), ws_bytes, _lib.stream_handle(device)
    )
    _lib.check(status, "hs_resolve_rows")
    return RowPlan(physical, miss_host, miss_device, counts, union_physical)
