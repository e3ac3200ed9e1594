"""ctypes binding of libhisparse_hip.so (declared in include/hisparse.h).

The library is built in-tree by ``python -m mini_hisparse_amd.build``.  There is
no fallback: when the library is missing every kernel call raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_uint64, POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libhisparse_hip.so"

HS_DTYPE_F32, HS_DTYPE_F16, HS_DTYPE_BF16 = 0, 1, 2


class HipLibraryError(RuntimeError):
    """A libhisparse_hip call failed (the message comes from hs_last_error)."""


class ResolveDesc(ctypes.Structure):
    """``hs_resolve_desc`` of include/hisparse.h."""

    _fields_ = [
        ("positions", c_void_p),
        ("n", c_int64),
        ("positions_i64", c_int32),
        ("lru_i16", c_int32),
        ("page_bits", c_void_p),
        ("head_columns", c_void_p),
        ("heads", c_int64),
        ("width", c_int64),
        ("hc_stride_h", c_int64),
        ("hc_stride_w", c_int64),
        ("source", c_void_p),
        ("resident", c_void_p),
        ("n_pages", c_int64),
        ("hot", c_void_p),
        ("hot_blocks", c_int64),
        ("tags", c_void_p),
        ("lru", c_void_p),
        ("hot_rows", c_int64),
        ("length", c_int64),
        ("page_size", c_int64),
        ("physical", c_void_p),
        ("union_physical", c_void_p),
        ("miss_host_rows", c_void_p),
        ("miss_device_rows", c_void_p),
        ("counts", c_void_p),
        ("row_stats", c_void_p),
        ("workspace", c_void_p),
        ("miss_prefix_only", c_int32),
        ("split_front", c_int32),
    ]


# name -> (restype, argtypes); every symbol of include/hisparse.h
SIGNATURES = {
    "hs_last_error": (c_char_p, []),
    "hs_version": (c_int, []),
    "hs_device_lds_bytes": (c_int, [c_int, POINTER(c_int64)]),
    "hs_host_alias": (c_int, [c_void_p, POINTER(c_void_p)]),
    "hs_host_alloc": (c_int, [c_int64, POINTER(c_void_p)]),
    "hs_host_free": (c_int, [c_void_p]),
    "hs_quest_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "hs_quest_topk": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int32, POINTER(c_void_p), POINTER(c_void_p), c_int32,
         POINTER(c_int64), c_int64, c_int64, c_int64, c_int64, c_int64, c_int32,
         c_void_p, c_int64, c_void_p, c_int64, c_void_p],
    ),
    "hs_build_union": (
        c_int,
        [c_void_p, c_int64, c_int64, POINTER(c_int64), c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
         c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "hs_resolve_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "hs_resolve_rows": (c_int, [POINTER(ResolveDesc), c_void_p, c_int64, c_void_p]),
    "hs_resolve_rows_batched": (c_int, [POINTER(ResolveDesc), c_int32, c_void_p, c_int64, c_void_p]),
    "hs_resolve_noalloc_max_bytes": (c_int64, []),
    "hs_resolve_rows_noalloc": (c_int, [POINTER(ResolveDesc), c_int32, c_void_p]),
    "hs_gather_rows": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
         c_void_p],
    ),
    "hs_gather_rows_batched": (
        c_int,
        [POINTER(c_void_p), c_void_p, POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p),
         POINTER(c_int64), POINTER(c_int64), c_int64, c_int32, c_int64, c_int64, c_int32, c_void_p],
    ),
    "hs_append_rows": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int64, c_int64, c_int64,
         POINTER(c_int64), POINTER(c_void_p), POINTER(c_int64), c_int64, POINTER(c_void_p),
         POINTER(c_void_p), c_int32, c_void_p],
    ),
    "hs_rotary_split_append": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_float,
         c_int32, c_void_p, c_int64, c_int64, POINTER(c_int64), POINTER(c_void_p), POINTER(c_int64), c_int64,
         POINTER(c_void_p), POINTER(c_void_p), c_void_p],
    ),
    "hs_append_tokens": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int32,
         c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, POINTER(c_int64), POINTER(c_int64),
         c_void_p, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "hs_attend_workspace_bytes": (c_int64, [c_int32, c_int64, c_int64, c_int64, c_int64, c_int64]),
    "hs_attend_rows": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p],
    ),
    "hs_probe_row_reads": (
        c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "hs_attend_time_next": (c_int, [c_void_p, c_void_p]),
    "hs_add_rms_norm": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_float,
         c_int32, c_void_p],
    ),
    "hs_rotary_split": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
         c_float, c_int32, c_void_p],
    ),
    "hs_silu_mul": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int32, c_void_p]),
    "hs_uniform_pages": (
        c_int, [c_uint64, c_uint64, POINTER(c_int64), c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "hs_skinny_gemm_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "hs_skinny_gemm": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p,
         c_int64, c_void_p],
    ),
    "hs_skinny_gemm_swiglu_tiled": (
        c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p],
    ),
    "hs_skinny_gemm_tiled": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p,
         c_int64, c_void_p],
    ),
    "hs_skinny_gemm_argmax_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "hs_skinny_gemm_argmax_tiled": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int64,
         c_void_p],
    ),
    "hs_attend_groups": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64,
         c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p],
    ),
    "hs_attend_window": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int64, c_void_p],
    ),
}

_LIB = None
_LIB_PATH = None
_LIB_DEFAULT = False  # the loaded copy is the package's own build


def load(path: Path | str | None = None):
    """Load (once per process) and return the library; raises if it is absent.

    ``path`` names another build of the library; the process holds one copy at most,
    so a path other than the one already loaded is refused (two copies would register
    the same kernels twice with the HIP runtime)."""
    global _LIB, _LIB_PATH, _LIB_DEFAULT
    if path is None and _LIB_DEFAULT:  # every wrapper call: no filesystem lookup
        return _LIB
    target = (Path(path) if path is not None else LIBRARY_PATH).resolve()
    if _LIB is not None and target == _LIB_PATH:
        return _LIB
    if not target.exists():
        raise HipLibraryError(
            f"{target} is missing: build it with `python -m mini_hisparse_amd.build` "
            "(the HIP kernels have no fallback)"
        )
    if _LIB is not None:
        raise HipLibraryError(f"{_LIB_PATH} is already loaded; a second copy ({target}) is refused")
    lib = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB, _LIB_PATH = lib, target
    _LIB_DEFAULT = target == LIBRARY_PATH.resolve()
    return lib


def check(status: int, what: str):
    if status != 0:
        message = load().hs_last_error().decode(errors="replace")
        raise HipLibraryError(f"{what} failed ({status}): {message}")


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: HS_DTYPE_F32, torch.float16: HS_DTYPE_F16, torch.bfloat16: HS_DTYPE_BF16}
    if dtype not in codes:
        raise ValueError("KV dtype must be float32, float16 or bfloat16")
    return codes[dtype]


def ptr(tensor) -> int:
    return 0 if tensor is None else tensor.data_ptr()


def stream_handle(device=None) -> int:
    """Handle of the current stream of ``device`` (default: the current device): the stream
    torch's own work on that device is queued on.  Read without building a Stream object
    (which costs more than a kernel launch)."""
    import torch

    if isinstance(device, torch.device):
        index = device.index
    elif device is None or isinstance(device, int):
        index = device
    else:
        index = torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)
