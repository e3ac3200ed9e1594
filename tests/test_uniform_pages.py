"""hs_uniform_pages, the miss-heavy stress workload's selector (pages
resampled uniformly every step): a CPU restatement of its rule (splitmix64 draws, Floyd's
sampling without replacement) pinned by its distribution, and the kernel against the
restatement bit for bit."""

from itertools import combinations

import numpy as np
import pytest

M64 = (1 << 64) - 1


def splitmix64(x):
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def draw(seed, step, layer, b, batch, count, top):
    """The pages of one (layer, request): ascending, the tail page count - 1 last, -1 past
    min(top, count) -- the rule of hs_uniform_pages, restated."""
    if count <= top:
        return list(range(count)) + [-1] * (top - count)
    n, k = count - 1, top - 1
    base = splitmix64(splitmix64(splitmix64(seed) ^ step) ^ (layer * batch + b))
    taken = set()
    for j in range(n - k, n):
        t = (((splitmix64(base ^ j) >> 32) * (j + 1)) >> 32)
        taken.add(j if t in taken else t)
    return sorted(taken) + [n]


def test_restated_draws_are_uniform_subsets_with_the_tail():
    """Over 12,000 draws of 3 of 6 non-tail pages every one of the 20 subsets appears
    (chi-square over 19 degrees of freedom below 60, p ~ 1e-5), each draw distinct and
    ascending with the tail last; short histories select every page."""
    seen = {c: 0 for c in combinations(range(6), 3)}
    for step in range(12000):
        pages = draw(7, step, step % 5, step % 3, 3, 7, 4)
        assert pages[-1] == 6 and pages == sorted(set(pages)) and len(pages) == 4
        seen[tuple(pages[:3])] += 1
    expected = 12000 / len(seen)
    chi2 = sum((v - expected) ** 2 / expected for v in seen.values())
    assert min(seen.values()) > 0 and chi2 < 60, chi2
    assert draw(1, 2, 0, 0, 1, 3, 8) == [0, 1, 2] + [-1] * 5
    assert draw(1, 2, 0, 0, 1, 9, 9) == list(range(9))
    assert draw(1, 2, 0, 0, 1, 10, 1) == [9]


@pytest.mark.gpu
def test_uniform_pages_kernel_equals_the_restated_rule(gpu):
    """Counts 1 to 65,536 pages (and top 1 / 2 / 64), 17 requests (two launches), three
    heads, four layers and two steps: every row equals the restatement; the heads' rows
    are equal."""
    import torch

    from mini_hisparse_amd.batched_engine import uniform_pages_device

    counts = [1, 5, 64, 65, 66, 129, 4097, 65536, 2, 3, 100, 1000, 17, 18, 4000, 300, 64 * 3]
    P, layers, heads = 16, 4, 3
    lengths = [c * P - 3 if c > 1 else 5 for c in counts]
    for top in (1, 2, 64):
        for step in (0, 12345):
            print(f"[case] uniform pages: top {top}, step {step}", flush=True)
            out = uniform_pages_device(99, step, lengths, P, top, layers, heads, device=gpu)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for layer in range(layers):
                for b, count in enumerate(counts):
                    expected = draw(99, step, layer, b, len(counts), count, top)
                    np.testing.assert_array_equal(got[layer, b], np.tile(expected, (heads, 1)),
                                                  err_msg=f"layer {layer} request {b} count {count} top {top}")


def test_uniform_pages_rejects_bad_shapes_without_a_gpu():
    from mini_hisparse_amd import _lib

    import ctypes

    lib = _lib.load()
    counts = (ctypes.c_int64 * 2)(10, 0)
    assert lib.hs_uniform_pages(1, 2, counts, 2, 3, 4, 1, 0x1000, None) == -1
    assert b"page counts" in lib.hs_last_error()
    counts = (ctypes.c_int64 * 1)(70000)
    assert lib.hs_uniform_pages(1, 2, counts, 1, 3, 4, 1, 0x1000, None) == -1
    assert lib.hs_uniform_pages(1, 2, counts, 1, 0, 4, 1, 0x1000, None) == -1
    assert b"shape" in lib.hs_last_error()
