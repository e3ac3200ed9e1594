"""Fused dense-layer kernels of the batched engine against the PyTorch ops they replace
(the model's RMSNorm, the engine's PyTorch rotary, F.silu) and fp32 references."""

import pytest
import torch
from torch.nn import functional as F

from mini_hisparse_amd.batched_engine import rotary_at
from mini_hisparse_amd.dense import add_rms_norm, rotary_split, silu_mul
from mini_hisparse_amd.model import RMSNorm

BF16_ULP = 2.0**-7  # relative spacing of bfloat16 values in [1, 2)


def test_wrappers_check_shapes_without_a_gpu():
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="weight"):
        add_rms_norm(x, None, torch.ones(7, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="delta"):
        add_rms_norm(x, torch.zeros(4, 7, dtype=torch.bfloat16), torch.ones(8, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="qkv"):
        rotary_split(torch.zeros(2, 10, dtype=torch.bfloat16), torch.zeros(2, dtype=torch.int64), 1, 1, 4, 1e4)
    with pytest.raises(ValueError, match="gate_up"):
        silu_mul(torch.zeros(2, 5, dtype=torch.bfloat16))
    # an out buffer of the wrong shape, dtype or layout is refused before any launch
    with pytest.raises(ValueError, match="out"):
        add_rms_norm(x, None, torch.ones(8, dtype=torch.bfloat16), 1e-6, out=torch.empty(4, 7, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="out"):
        silu_mul(torch.zeros(2, 8, dtype=torch.bfloat16), out=torch.empty(2, 4, dtype=torch.float32))
    with pytest.raises(ValueError, match="out"):
        rotary_split(torch.zeros(2, 16, dtype=torch.bfloat16), torch.zeros(2, dtype=torch.int64), 2, 1, 4, 1e4,
                     out=(torch.empty(2, 2, 4, dtype=torch.bfloat16), torch.empty(2, 1, 4, dtype=torch.bfloat16),
                          torch.empty(2, 2, 4, dtype=torch.bfloat16)))
    from mini_hisparse_amd.dense import linear
    with pytest.raises(ValueError, match="out"):
        linear(torch.zeros(2, 32, dtype=torch.bfloat16), torch.zeros(8, 32, dtype=torch.bfloat16),
               out=torch.empty(2, 9, dtype=torch.bfloat16))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,width", [(1, 896), (8, 3584), (3, 5120), (5, 100), (2, 7000)])
def test_add_rms_norm_matches_the_model_norm(gpu, dtype, rows, width):
    gen = torch.Generator(device=gpu).manual_seed(rows * 7 + width)
    x = (torch.randn(rows, width, generator=gen, device=gpu) * 3).to(dtype)
    delta = torch.randn(rows, width, generator=gen, device=gpu).to(dtype)
    norm = RMSNorm(width, 1e-6).to(device=gpu, dtype=dtype)
    with torch.no_grad():
        norm.weight.copy_((torch.rand(width, generator=gen, device=gpu) + 0.5).to(dtype))
        summed = x + delta  # PyTorch's residual add in the model dtype
        expected = norm(summed)
        exact = (summed.double() * torch.rsqrt(summed.double().square().mean(-1, keepdim=True) + 1e-6)) * norm.weight.double()
    got_plain = add_rms_norm(summed.clone(), None, norm.weight, 1e-6)
    inplace = x.clone()
    got = add_rms_norm(inplace, delta, norm.weight, 1e-6)
    torch.testing.assert_close(inplace, summed, rtol=0, atol=0)  # the residual add is exact
    tol = dict(rtol=2 * BF16_ULP if dtype != torch.float32 else 1e-5, atol=1e-5)
    torch.testing.assert_close(got, expected, **tol)
    torch.testing.assert_close(got_plain, got, rtol=0, atol=0)
    torch.testing.assert_close(got.double(), exact, rtol=2 * BF16_ULP if dtype != torch.float32 else 1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(28, 4, 128), (14, 2, 64), (40, 8, 128), (4, 2, 32)])
def test_rotary_split_matches_the_pytorch_rotary(gpu, heads, kv_heads, head_dim):
    rows = 5
    gen = torch.Generator(device=gpu).manual_seed(heads)
    qkv = torch.randn(rows, (heads + 2 * kv_heads) * head_dim, generator=gen, device=gpu).to(torch.bfloat16)
    positions = torch.tensor([0, 1, 639, 65536, 131071], dtype=torch.int64, device=gpu)
    q, k, v = rotary_split(qkv, positions, heads, kv_heads, head_dim, 1e6)
    parts = qkv.view(rows, heads + 2 * kv_heads, head_dim)
    ref_q = rotary_at(parts[:, :heads], positions, 1e6)
    ref_k = rotary_at(parts[:, heads : heads + kv_heads], positions, 1e6)
    torch.testing.assert_close(v, parts[:, heads + kv_heads :], rtol=0, atol=0)
    # same rounding sequence; cos/sin/pow of the device may differ from PyTorch's by an ulp
    torch.testing.assert_close(q, ref_q, rtol=2 * BF16_ULP, atol=2 * BF16_ULP)
    torch.testing.assert_close(k, ref_k, rtol=2 * BF16_ULP, atol=2 * BF16_ULP)
    # fp32 rotation: the bf16 result is within a few roundings of it
    half = head_dim // 2
    inv = 1e6 ** (-torch.arange(0, head_dim, 2, device=gpu, dtype=torch.float64) / head_dim)
    ang = positions.double()[:, None] * inv[None, :]
    t = parts[:, :heads].double()
    a, b = t[..., :half], t[..., half:]
    c, s = ang.cos()[:, None, :], ang.sin()[:, None, :]
    exact = torch.cat((a * c - b * s, b * c + a * s), -1)
    assert (q.double() - exact).abs().max().item() < 0.05


@pytest.mark.gpu
@pytest.mark.parametrize("rows,width", [(1, 4864), (8, 18944), (3, 27648), (2, 33)])
def test_silu_mul_matches_pytorch(gpu, rows, width):
    gen = torch.Generator(device=gpu).manual_seed(width)
    gate_up = (torch.randn(rows, 2 * width, generator=gen, device=gpu) * 4).to(torch.bfloat16)
    got = silu_mul(gate_up)
    gate, up = gate_up[:, :width], gate_up[:, width:]
    torch.testing.assert_close(got, F.silu(gate) * up, rtol=2 * BF16_ULP, atol=1e-6)
    exact = gate.double() * torch.sigmoid(gate.double()) * up.double()
    torch.testing.assert_close(got.double(), exact, rtol=2 * BF16_ULP, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 3, 8, 16])
@pytest.mark.parametrize("n,k,bias", [(4608, 3584, True), (3584, 18944, False), (300, 256, True), (64, 32, False),
                                      (1000, 27648, False)])
def test_linear_matches_an_fp32_reference(gpu, dtype, rows, n, k, bias):
    from mini_hisparse_amd.dense import linear

    gen = torch.Generator(device=gpu).manual_seed(rows + n + k)
    x = torch.randn(rows, k, generator=gen, device=gpu).to(dtype)
    w = (torch.randn(n, k, generator=gen, device=gpu) / k**0.5).to(dtype)
    b = torch.randn(n, generator=gen, device=gpu).to(dtype) if bias else None
    got = linear(x, w, b)
    ref = x.float() @ w.float().T + (b.float() if bias else 0)
    scale = ref.abs().max().item()
    err = (got.float() - ref).abs()
    assert (err <= 2 * BF16_ULP * ref.abs() + 2e-3 * scale).all(), err.max().item()
    assert torch.equal(linear(x, w, b), got)  # split-K partials are summed in a fixed order
    from mini_hisparse_amd.dense import linear_tiled, tile_weight

    # the tile-major weight (rows padded to 16) gives the same bits
    assert torch.equal(linear_tiled(x, tile_weight(w), n, b), got)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 3, 16])
@pytest.mark.parametrize("ffn,k", [(4864, 896), (18944, 3584), (37, 64), (1000, 256), (1000, 4096)])
def test_swiglu_gemm_equals_gemm_then_silu_mul(gpu, dtype, rows, ffn, k):
    """One launch of gate|up with the SiLU gate gives the bits of the tiled GEMM on the packed
    weight followed by hs_silu_mul (ffn not a multiple of 16 included) whenever that GEMM
    runs in one K slice; (1000, 4096) makes it plan split-K, and there both stay within the
    fp32 reference's tolerance."""
    from mini_hisparse_amd.dense import (
        gemm_workspace_bytes, linear_swiglu_tiled, linear_tiled, silu_mul, tile_gate_up, tile_weight,
    )

    gen = torch.Generator(device=gpu).manual_seed(rows + ffn + k)
    x = torch.randn(rows, k, generator=gen, device=gpu).to(dtype)
    w = (torch.randn(2 * ffn, k, generator=gen, device=gpu) / k**0.5).to(dtype)
    want = silu_mul(linear_tiled(x, tile_weight(w), 2 * ffn))
    got = linear_swiglu_tiled(x, tile_gate_up(w, ffn), ffn)
    split_k = gemm_workspace_bytes(rows, 2 * ffn, k) > 256
    assert split_k == (k == 4096)
    if not split_k:
        assert torch.equal(got, want)
    ref = torch.nn.functional.silu(x.float() @ w[:ffn].float().T) * (x.float() @ w[ffn:].float().T)
    assert ((got.float() - ref).abs() <= 0.02 + 0.02 * ref.abs()).all()
    assert ((want.float() - ref).abs() <= 0.02 + 0.02 * ref.abs()).all()


def test_tile_gate_up_interleaves_the_two_projections():
    from mini_hisparse_amd.dense import tile_gate_up, tile_weight

    w = torch.randn(2 * 20, 32).to(torch.bfloat16)
    t = tile_gate_up(w, 20)
    gate, up = tile_weight(w[:20]), tile_weight(w[20:])
    assert t.shape == (4, 1, 16, 32)
    assert torch.equal(t[0], gate[0]) and torch.equal(t[1], up[0]) and torch.equal(t[2], gate[1]) and torch.equal(t[3], up[1])


def test_tile_weight_packs_16_by_32_blocks():
    from mini_hisparse_amd.dense import linear_tiled, tile_weight

    w = torch.randn(37, 64).to(torch.bfloat16)
    t = tile_weight(w)
    assert t.shape == (3, 2, 16, 32) and t.is_contiguous()
    for tile in range(3):
        for step in range(2):
            block = t[tile, step]
            rows = w[16 * tile : 16 * tile + 16, 32 * step : 32 * step + 32]
            assert torch.equal(block[: rows.shape[0]], rows)
            assert not block[rows.shape[0] :].any()  # rows past N are zero
    with pytest.raises(ValueError):
        tile_weight(torch.zeros(8, 40, dtype=torch.bfloat16))
    with pytest.raises(ValueError):  # a row-major weight is not a tile packing
        linear_tiled(torch.zeros(2, 64, dtype=torch.bfloat16), w, 37)


@pytest.mark.gpu
def test_linear_reads_strided_rows_and_rejects_unsupported_shapes(gpu):
    from mini_hisparse_amd.dense import linear

    gen = torch.Generator(device=gpu).manual_seed(9)
    wide = torch.randn(4, 512, generator=gen, device=gpu).to(torch.bfloat16)
    x = wide[:, :256]  # row stride 512
    w = torch.randn(96, 256, generator=gen, device=gpu).to(torch.bfloat16)
    torch.testing.assert_close(linear(x, w).float(), x.float() @ w.float().T, rtol=2 * BF16_ULP, atol=0.05)
    with pytest.raises(ValueError):
        linear(torch.zeros(17, 256, dtype=torch.bfloat16, device=gpu), w)
    with pytest.raises(ValueError):
        linear(torch.zeros(2, 100, dtype=torch.bfloat16, device=gpu), torch.zeros(8, 100, dtype=torch.bfloat16, device=gpu))


@pytest.mark.gpu
def test_split_k_partials_in_a_caller_workspace(gpu):
    """A split-K plan (1000 outputs, K 4096) writes its partials to the caller's workspace
    when given one: the same bits as the module buffer, and a short workspace is refused
    before anything is launched."""
    from mini_hisparse_amd.dense import gemm_workspace_bytes, linear_tiled, tile_weight

    gen = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(2, 4096, generator=gen, device=gpu).to(torch.bfloat16)
    w = (torch.randn(1000, 4096, generator=gen, device=gpu) / 64).to(torch.bfloat16)
    tiles = tile_weight(w)
    need = gemm_workspace_bytes(2, 1000, 4096)
    assert need > 256  # split-K
    own = torch.empty(need, dtype=torch.uint8, device=gpu)
    assert torch.equal(linear_tiled(x, tiles, 1000, workspace=own), linear_tiled(x, tiles, 1000))
    with pytest.raises(ValueError, match="workspace"):
        linear_tiled(x, tiles, 1000, workspace=own[: need - 1])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 4, 16])
@pytest.mark.parametrize("n,k,bias", [(151936, 896, False), (1000, 256, True), (37, 64, False), (50001, 2048, True)])
def test_argmax_gemm_equals_torch_argmax_of_the_logits(gpu, dtype, rows, n, k, bias):
    """hs_skinny_gemm_argmax_tiled against torch.argmax over the logits of
    hs_skinny_gemm_tiled (one K slice at these shapes: the same rounded logits), on
    random rows, then with exact ties planted (the best row copied to index 0 and to
    the last index: the first index wins), all-zero inputs (logits +0 and -0: index 0)
    and NaN rows (the first NaN wins, as torch takes it)."""
    from mini_hisparse_amd.dense import gemm_workspace_bytes, linear_argmax_tiled, linear_tiled, tile_weight

    assert gemm_workspace_bytes(rows, n, k) == 256  # one K slice
    gen = torch.Generator(device=gpu).manual_seed(rows + n + k)
    x = torch.randn(rows, k, generator=gen, device=gpu).to(dtype)
    w = (torch.randn(n, k, generator=gen, device=gpu) / k**0.5).to(dtype)
    b = torch.randn(n, generator=gen, device=gpu).to(dtype) if bias else None

    def check(x, w, what):
        tiles = tile_weight(w)
        expected = linear_tiled(x, tiles, n, b).argmax(-1)
        got = linear_argmax_tiled(x, tiles, n, b)
        assert got.dtype == torch.int64 and torch.equal(got, expected), (what, got.tolist(), expected.tolist())
        return expected

    best = check(x, w, "random")
    if n > 2:
        tied = w.clone()
        r = int(best[0])
        tied[0], tied[n - 1] = w[r], w[r]
        assert int(check(x, tied, "ties")[0]) == 0 or (b is not None and b[0] != b[r])
    zeros = check(torch.zeros_like(x), w, "zeros")
    if b is None:
        assert (zeros == 0).all()
    if n > 8:
        nan = w.clone()
        nan[n // 2, 0] = float("nan")
        nan[n // 3 + 5, 1] = float("nan")
        assert (check(x, nan, "nan") == min(n // 2, n // 3 + 5)).all()


@pytest.mark.gpu
def test_argmax_gemm_rejects_a_short_workspace(gpu):
    from mini_hisparse_amd.dense import argmax_workspace_bytes, linear_argmax_tiled, tile_weight

    x = torch.ones(2, 64, dtype=torch.bfloat16, device=gpu)
    tiles = tile_weight(torch.ones(100, 64, dtype=torch.bfloat16, device=gpu))
    need = argmax_workspace_bytes(2, 100, 64)
    with pytest.raises(ValueError, match="workspace"):
        linear_argmax_tiled(x, tiles, 100, workspace=torch.empty(need - 300, dtype=torch.uint8, device=gpu))


SPLIT_SHAPES = [(4, 1000, 4096), (4, 896, 4864), (8, 3584, 18944), (3, 64, 16384), (1, 5120, 27648), (16, 300, 8192)]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,n,k", SPLIT_SHAPES)
def test_in_kernel_split_merge_equals_the_finalize_launch(gpu, monkeypatch, rows, n, k):
    """Split-K projections merged by each row tile's last workgroup (the default) have
    the bits of the fp32 partials summed by gemm_finalize_kernel (HS_GEMM_FUSED_MERGE=0),
    with and without a bias, from a workspace full of arbitrary bytes."""
    from mini_hisparse_amd.dense import gemm_workspace_bytes, linear_tiled, tile_weight

    gen = torch.Generator(device=gpu).manual_seed(rows + n + k)
    x = torch.randn(rows, k, generator=gen, device=gpu).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=gen, device=gpu) / k**0.5).to(torch.bfloat16)
    bias = torch.randn(n, generator=gen, device=gpu).to(torch.bfloat16)
    tiles = tile_weight(w)
    need = gemm_workspace_bytes(rows, n, k)
    assert need > 256  # split over K
    ws = torch.randint(0, 256, (need,), generator=gen, device=gpu, dtype=torch.uint8)
    for b in (None, bias):
        monkeypatch.setenv("HS_GEMM_FUSED_MERGE", "0")
        expected = linear_tiled(x, tiles, n, b, workspace=torch.empty_like(ws))
        monkeypatch.delenv("HS_GEMM_FUSED_MERGE")
        got = linear_tiled(x, tiles, n, b, workspace=ws)
        again = linear_tiled(x, tiles, n, b, workspace=ws)  # the counters as the first call left them
        torch.cuda.synchronize()
        assert torch.equal(got, expected) and torch.equal(again, expected)


@pytest.mark.gpu
def test_in_kernel_split_merge_replays_from_a_captured_graph(gpu):
    """A captured split-K projection replayed four times with new rows, with eager
    projections of other shapes sharing the workspace between the replays: every replay
    equals the eager result (the counters count each replay in its own round)."""
    from mini_hisparse_amd.dense import gemm_workspace_bytes, linear_tiled, tile_weight

    gen = torch.Generator(device=gpu).manual_seed(3)
    k, n, rows = 4864, 896, 4
    w = (torch.randn(n, k, generator=gen, device=gpu) / 70).to(torch.bfloat16)
    other = (torch.randn(1000, 4096, generator=gen, device=gpu) / 64).to(torch.bfloat16)
    tiles, other_tiles = tile_weight(w), tile_weight(other)
    ws = torch.zeros(max(gemm_workspace_bytes(rows, n, k), gemm_workspace_bytes(2, 1000, 4096)), dtype=torch.uint8,
                     device=gpu)
    x = torch.randn(rows, k, generator=gen, device=gpu).to(torch.bfloat16)
    y = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.Stream(gpu)
    stream.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(stream):
        linear_tiled(x, tiles, n, out=y, workspace=ws)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        linear_tiled(x, tiles, n, out=y, workspace=ws)
    for replay in range(4):
        print(f"[case] split-K graph replay {replay}", flush=True)
        x.copy_(torch.randn(rows, k, generator=gen, device=gpu).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = y.clone()
        expected = linear_tiled(x, tiles, n, workspace=torch.empty_like(ws))
        linear_tiled(torch.randn(2, 4096, generator=gen, device=gpu).to(torch.bfloat16), other_tiles, 1000,
                     workspace=ws)  # another launch's words and counters in the same bytes
        torch.cuda.synchronize()
        assert torch.equal(got, expected), replay
