"""Dense stages of a decoder layer's decode step (HIP kernels).

``linear`` wraps ``hs_skinny_gemm``, the projection of up to 16 token rows
(an HBM stream of the weight on MFMA tiles).  ``add_rms_norm``,
``rotary_split`` and ``silu_mul`` wrap ``hs_add_rms_norm``,
``hs_rotary_split`` and ``hs_silu_mul``: the
RMSNorm (with the residual add before it), the rotary embedding of q and k
(with the split of a packed q|k|v projection) and the SiLU gate of the MLP
(over a packed gate|up projection) of the Qwen2 layer that ``MiniModel``
implements (model.py:53-57 RMSNorm, the rotary and MLP of this package's
``model.py``; the reference's model.py:183-226).  One launch each for B rows.
"""

from __future__ import annotations

import torch

from . import _lib


def _stream(tensor):
    return _lib.stream_handle(tensor.device)


class Launch:
    """One library call with every argument bound but the stream (a ``prepare_*`` result):
    ``launch(stream_handle)`` issues it.  The tensors it names must outlive it."""

    __slots__ = ("fn", "args", "what")

    def __init__(self, fn, args, what):
        self.fn, self.args, self.what = fn, args, what

    def __call__(self, stream):
        status = self.fn(*self.args, stream)
        if status:
            _lib.check(status, self.what)


_WORKSPACE = {}
_GEMM_WS_BYTES = {}


def gemm_workspace_bytes(rows, n, k):
    """Bytes of split-K partials ``linear``/``linear_tiled`` need for [rows, k] x [n, k]."""
    nbytes = _GEMM_WS_BYTES.get((rows, n, k))
    if nbytes is None:
        nbytes = _GEMM_WS_BYTES[(rows, n, k)] = _lib.load().hs_skinny_gemm_workspace_bytes(rows, n, k)
    return nbytes


def _workspace(device, stream, nbytes, given):
    """``given`` when the caller owns the workspace (it must hold ``nbytes``); else a
    module buffer per (device, stream), for eager calls only: a captured graph keeps
    the address of the buffer it saw, which a later, larger call would replace."""
    if given is not None:
        if given.dtype != torch.uint8 or given.device != torch.device(device) or given.numel() < nbytes:
            raise ValueError(f"GEMM workspace must be uint8 on {device} with at least {nbytes} bytes")
        return given
    key = (device, stream)
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def _check_out(out, shape, like, what):
    """An ``out`` buffer the kernels may write: the expected shape and dtype, on the
    device of ``like``, rows of unit inner stride."""
    if out is None:
        return
    if tuple(out.shape) != tuple(shape) or out.dtype != like.dtype or out.device != like.device:
        raise ValueError(f"{what}: out must be {tuple(shape)} {like.dtype} on {like.device}")
    if out.stride(-1) != 1 or (out.dim() == 2 and out.stride(0) < out.shape[1]):
        raise ValueError(f"{what}: out rows must have unit inner stride")
    if out.dim() == 3 and not out.is_contiguous():
        raise ValueError(f"{what}: out must be contiguous")


def linear_supported(x, weight):
    """Shapes ``linear`` takes: 1-16 rows, K a multiple of 32, bf16/f16, 16-byte aligned rows."""
    return (
        x.dim() == 2 and weight.dim() == 2 and 1 <= x.shape[0] <= 16 and x.shape[1] == weight.shape[1]
        and x.shape[1] % 32 == 0 and x.dtype == weight.dtype and x.dtype in (torch.bfloat16, torch.float16)
        and x.stride(1) == 1 and x.stride(0) % 8 == 0 and weight.is_contiguous()
        and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0
    )


def linear(x, weight, bias=None, out=None, workspace=None):
    """``x @ weight.T + bias`` for ``x`` [rows <= 16, K] (F.linear's arguments).
    ``workspace`` (uint8, :func:`gemm_workspace_bytes`) holds the split-K partials; a
    caller that captures the call in a graph passes its own."""
    if not linear_supported(x, weight):
        raise ValueError("linear takes 1-16 rows of a bf16/f16 x with K a multiple of 32 and a contiguous weight")
    if bias is not None and (bias.shape != (weight.shape[0],) or bias.dtype != x.dtype or not bias.is_contiguous()):
        raise ValueError("bias must be [N] contiguous in the dtype of x")
    rows, k = x.shape
    n = weight.shape[0]
    _check_out(out, (rows, n), x, "linear")
    y = torch.empty((rows, n), dtype=x.dtype, device=x.device) if out is None else out
    lib = _lib.load()
    stream = _stream(x)
    ws = _workspace(x.device, stream, gemm_workspace_bytes(rows, n, k), workspace)
    _lib.check(
        lib.hs_skinny_gemm(
            x.data_ptr(), x.stride(0), weight.data_ptr(), n, k, _lib.ptr(bias), y.data_ptr(), y.stride(0), rows,
            _lib.dtype_code(x.dtype), ws.data_ptr(), ws.numel(), stream,
        ),
        "hs_skinny_gemm",
    )
    return y


def tile_weight(weight):
    """``weight`` [N, K] packed tile-major for :func:`linear_tiled`: ceil(N/16) x K/32 blocks
    of 16 rows x 32 k-values (block (t, s) = weight[16t:16t+16, 32s:32s+32]), rows past N zero."""
    if weight.dim() != 2 or weight.shape[1] % 32 != 0 or weight.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("tile_weight takes a bf16/f16 [N, K] weight with K a multiple of 32")
    n, k = weight.shape
    rows = -(-n // 16) * 16
    padded = weight if rows == n else torch.cat((weight, weight.new_zeros(rows - n, k)), 0)
    return padded.reshape(rows // 16, 16, k // 32, 32).transpose(1, 2).contiguous()


def _linear_tiled_launch(x, tiles, n, bias, y, ws):
    k = x.shape[1]
    return Launch(_lib.load().hs_skinny_gemm_tiled,
                  (x.data_ptr(), x.stride(0), tiles.data_ptr(), n, k, _lib.ptr(bias), y.data_ptr(), y.stride(0),
                   x.shape[0], _lib.dtype_code(x.dtype), ws.data_ptr(), ws.numel()),
                  "hs_skinny_gemm_tiled")


def _linear_tiled_check(x, tiles, n, bias, out):
    k = x.shape[1] if x.dim() == 2 else -1
    if not (
        x.dim() == 2 and 1 <= x.shape[0] <= 16 and k % 32 == 0 and k > 0 and n >= 1
        and x.dtype in (torch.bfloat16, torch.float16) and x.stride(1) == 1 and x.stride(0) % 8 == 0
        and x.data_ptr() % 16 == 0 and tiles.dim() == 4 and tiles.shape == (-(-n // 16), k // 32, 16, 32)
        and tiles.is_contiguous() and tiles.dtype == x.dtype and tiles.data_ptr() % 16 == 0
    ):
        raise ValueError("linear_tiled takes 1-16 rows of a bf16/f16 x (K a multiple of 32) and tile_weight's packing")
    if bias is not None and (bias.shape != (n,) or bias.dtype != x.dtype or not bias.is_contiguous()):
        raise ValueError("bias must be [N] contiguous in the dtype of x")
    _check_out(out, (x.shape[0], n), x, "linear_tiled")


def linear_tiled(x, tiles, n, bias=None, out=None, workspace=None):
    """:func:`linear` with the weight as :func:`tile_weight` packed it (``n`` its rows):
    the same arithmetic in the same order, so the same bits."""
    _linear_tiled_check(x, tiles, n, bias, out)
    rows, k = x.shape
    y = torch.empty((rows, n), dtype=x.dtype, device=x.device) if out is None else out
    stream = _stream(x)
    ws = _workspace(x.device, stream, gemm_workspace_bytes(rows, n, k), workspace)
    _linear_tiled_launch(x, tiles, n, bias, y, ws)(stream)
    return y


def prepare_linear_tiled(x, tiles, n, bias, out, workspace):
    """:func:`linear_tiled` into ``out`` with the caller's ``workspace``, bound once."""
    _linear_tiled_check(x, tiles, n, bias, out)
    if out is None:
        raise ValueError("prepare_linear_tiled writes into a given out")
    ws = _workspace(x.device, None, gemm_workspace_bytes(x.shape[0], n, x.shape[1]), workspace)
    return _linear_tiled_launch(x, tiles, n, bias, out, ws)


def argmax_workspace_bytes(rows, n, k):
    """Bytes of per-workgroup keys :func:`linear_argmax_tiled` needs for [rows, k] x [n, k]."""
    return _lib.load().hs_skinny_gemm_argmax_workspace_bytes(rows, n, k)


def linear_argmax_tiled(x, tiles, n, bias=None, out=None, workspace=None):
    """Greedy tokens of the LM head: ``argmax(x @ weight.T + bias, -1)`` as int64 [rows]
    (``hs_skinny_gemm_argmax_tiled``: the logits of :func:`linear_tiled` with one K
    slice, never written; the first maximal index on ties, as torch.argmax)."""
    _linear_tiled_check(x, tiles, n, bias, None)
    rows, k = x.shape
    if out is not None and (out.dtype != torch.int64 or out.shape != (rows,) or out.device != x.device
                            or not out.is_contiguous()):
        raise ValueError(f"linear_argmax_tiled: out must be int64 [{rows}] contiguous on {x.device}")
    tokens = torch.empty(rows, dtype=torch.int64, device=x.device) if out is None else out
    stream = _stream(x)
    ws = _workspace(x.device, stream, argmax_workspace_bytes(rows, n, k), workspace)
    _lib.check(
        _lib.load().hs_skinny_gemm_argmax_tiled(
            x.data_ptr(), x.stride(0), tiles.data_ptr(), n, k, _lib.ptr(bias), tokens.data_ptr(), rows,
            _lib.dtype_code(x.dtype), ws.data_ptr(), ws.numel(), stream,
        ),
        "hs_skinny_gemm_argmax_tiled",
    )
    return tokens


def tile_gate_up(gate_up, ffn):
    """The packed gate|up weight [2 * ffn, K] for :func:`linear_swiglu_tiled`: the gate's
    and the up projection's :func:`tile_weight` tiles interleaved (gate tile i at 2i)."""
    if gate_up.dim() != 2 or gate_up.shape[0] != 2 * ffn:
        raise ValueError("gate_up must be [2 * ffn, K]")
    gate, up = tile_weight(gate_up[:ffn]), tile_weight(gate_up[ffn:])
    return torch.stack((gate, up), 1).reshape(2 * gate.shape[0], *gate.shape[1:]).contiguous()


def _swiglu_check(x, tiles, ffn, out):
    k = x.shape[1] if x.dim() == 2 else -1
    if not (
        x.dim() == 2 and 1 <= x.shape[0] <= 16 and k % 32 == 0 and k > 0 and ffn >= 1
        and x.dtype in (torch.bfloat16, torch.float16) and x.stride(1) == 1 and x.stride(0) % 8 == 0
        and x.data_ptr() % 16 == 0 and tiles.dim() == 4 and tiles.shape == (2 * -(-ffn // 16), k // 32, 16, 32)
        and tiles.is_contiguous() and tiles.dtype == x.dtype and tiles.data_ptr() % 16 == 0
    ):
        raise ValueError("linear_swiglu_tiled takes 1-16 rows of a bf16/f16 x (K a multiple of 32) and "
                         "tile_gate_up's packing")
    _check_out(out, (x.shape[0], ffn), x, "linear_swiglu_tiled")


def _swiglu_launch(x, tiles, ffn, y):
    return Launch(_lib.load().hs_skinny_gemm_swiglu_tiled,
                  (x.data_ptr(), x.stride(0), tiles.data_ptr(), ffn, x.shape[1], y.data_ptr(), y.stride(0),
                   x.shape[0], _lib.dtype_code(x.dtype)),
                  "hs_skinny_gemm_swiglu_tiled")


def linear_swiglu_tiled(x, tiles, ffn, out=None):
    """``silu(x @ gate.T) * (x @ up.T)`` from :func:`tile_gate_up`'s packing, in one launch
    with one K slice.  It has the bits of :func:`linear_tiled` on the packed weight
    followed by :func:`silu_mul` whenever that GEMM also runs in one K slice
    (``gemm_workspace_bytes(rows, 2 * ffn, K)`` at its minimum of 256, with the default
    rounds of 8 k-steps); where the GEMM plans split-K (few output rows, long K) the
    sums are the same up to fp32 summation order."""
    _swiglu_check(x, tiles, ffn, out)
    y = torch.empty((x.shape[0], ffn), dtype=x.dtype, device=x.device) if out is None else out
    _swiglu_launch(x, tiles, ffn, y)(_stream(x))
    return y


def prepare_linear_swiglu_tiled(x, tiles, ffn, out):
    """:func:`linear_swiglu_tiled` into ``out``, bound once."""
    _swiglu_check(x, tiles, ffn, out)
    if out is None:
        raise ValueError("prepare_linear_swiglu_tiled writes into a given out")
    return _swiglu_launch(x, tiles, ffn, out)


def _rms_check(x, delta, weight, out):
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [rows, width] with unit inner stride")
    if delta is not None and (delta.shape != x.shape or delta.stride() != x.stride() or delta.dtype != x.dtype):
        raise ValueError("delta must match x in shape, strides and dtype")
    if weight.shape != (x.shape[1],) or weight.dtype != x.dtype:
        raise ValueError("weight must be [width] in the dtype of x")
    _check_out(out, x.shape, x, "add_rms_norm")


def _rms_launch(x, delta, weight, eps, y):
    return Launch(_lib.load().hs_add_rms_norm,
                  (x.data_ptr(), _lib.ptr(delta), x.data_ptr() if delta is not None else None, y.data_ptr(),
                   weight.data_ptr(), x.shape[0], x.shape[1], x.stride(0), y.stride(0), float(eps),
                   _lib.dtype_code(x.dtype)),
                  "hs_add_rms_norm")


def add_rms_norm(x, delta, weight, eps, out=None):
    """RMSNorm of ``x`` [rows, width] (of ``x + delta`` when ``delta`` is given, and then
    ``x`` is updated in place to the sum).  Returns the normalised rows."""
    _rms_check(x, delta, weight, out)
    y = torch.empty_like(x) if out is None else out
    _rms_launch(x, delta, weight, eps, y)(_stream(x))
    return y


def prepare_add_rms_norm(x, delta, weight, eps, out):
    """:func:`add_rms_norm` into ``out``, bound once."""
    _rms_check(x, delta, weight, out)
    if out is None:
        raise ValueError("prepare_add_rms_norm writes into a given out")
    return _rms_launch(x, delta, weight, eps, out)


def _rotary_check(qkv, positions, heads, kv_heads, head_dim, out):
    rows = qkv.shape[0]
    if qkv.dim() != 2 or qkv.stride(1) != 1 or qkv.shape[1] != (heads + 2 * kv_heads) * head_dim:
        raise ValueError("qkv must be [rows, (heads + 2 kv_heads) head_dim] with unit inner stride")
    if positions.dtype != torch.int64 or positions.shape != (rows,) or positions.device != qkv.device:
        raise ValueError("positions must be int64 [rows] on the device of qkv")
    if out is not None:
        q, k, v = out
        _check_out(q, (rows, heads, head_dim), qkv, "rotary_split q")
        _check_out(k, (rows, kv_heads, head_dim), qkv, "rotary_split k")
        _check_out(v, (rows, kv_heads, head_dim), qkv, "rotary_split v")


def _rotary_launch(qkv, positions, heads, kv_heads, head_dim, theta, q, k, v):
    return Launch(_lib.load().hs_rotary_split,
                  (qkv.data_ptr(), qkv.stride(0), q.data_ptr(), k.data_ptr(), v.data_ptr(), positions.data_ptr(),
                   qkv.shape[0], heads, kv_heads, head_dim, float(theta), _lib.dtype_code(qkv.dtype)),
                  "hs_rotary_split")


def rotary_split(qkv, positions, heads, kv_heads, head_dim, theta, out=None):
    """Split a packed projection ``qkv`` [rows, (heads + 2 kv_heads) head_dim] into q
    [rows, heads, head_dim], k and v [rows, kv_heads, head_dim], with q and k rotated
    at ``positions`` [rows] (int64, device)."""
    _rotary_check(qkv, positions, heads, kv_heads, head_dim, out)
    rows = qkv.shape[0]
    if out is None:
        q = torch.empty((rows, heads, head_dim), dtype=qkv.dtype, device=qkv.device)
        k = torch.empty((rows, kv_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
        v = torch.empty_like(k)
    else:
        q, k, v = out
    _rotary_launch(qkv, positions, heads, kv_heads, head_dim, theta, q, k, v)(_stream(qkv))
    return q, k, v


def prepare_rotary_split(qkv, positions, heads, kv_heads, head_dim, theta, out):
    """:func:`rotary_split` into ``out`` = (q, k, v), bound once (``positions`` is read
    when the launch runs)."""
    _rotary_check(qkv, positions, heads, kv_heads, head_dim, out)
    if out is None:
        raise ValueError("prepare_rotary_split writes into a given out")
    return _rotary_launch(qkv, positions, heads, kv_heads, head_dim, theta, *out)


def _silu_check(gate_up, out):
    if gate_up.dim() != 2 or gate_up.stride(1) != 1 or gate_up.shape[1] % 2:
        raise ValueError("gate_up must be [rows, 2 width] with unit inner stride")
    _check_out(out, (gate_up.shape[0], gate_up.shape[1] // 2), gate_up, "silu_mul")


def _silu_launch(gate_up, y):
    return Launch(_lib.load().hs_silu_mul,
                  (gate_up.data_ptr(), gate_up.stride(0), y.data_ptr(), y.stride(0), gate_up.shape[0],
                   gate_up.shape[1] // 2, _lib.dtype_code(gate_up.dtype)),
                  "hs_silu_mul")


def silu_mul(gate_up, out=None):
    """silu(gate) * up of a packed ``gate_up`` [rows, 2 width] -> [rows, width]."""
    _silu_check(gate_up, out)
    rows, width = gate_up.shape[0], gate_up.shape[1] // 2
    y = torch.empty((rows, width), dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    _silu_launch(gate_up, y)(_stream(gate_up))
    return y


def prepare_silu_mul(gate_up, out):
    """:func:`silu_mul` into ``out``, bound once."""
    _silu_check(gate_up, out)
    if out is None:
        raise ValueError("prepare_silu_mul writes into a given out")
    return _silu_launch(gate_up, out)
