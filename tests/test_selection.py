"""Selections and the Quest bound, re-expressed from the reference's tests/test_selection.py
(lines 33-55; the paged-cache part at 10-30 is out of scope)."""

from math import ceil

import numpy as np
import pytest
import torch

import oracle
from mini_hisparse_amd.selection import Selection, quest_selection
from tests.conftest import gpu_available


def _bounds(k, page_size):
    count = ceil(len(k) / page_size)
    lo = torch.stack([k[p * page_size : (p + 1) * page_size].amin(0) for p in range(count)])
    hi = torch.stack([k[p * page_size : (p + 1) * page_size].amax(0) for p in range(count)])
    return lo, hi


K_CANCEL = torch.tensor([[[10.0, 0.0]], [[-10.0, 0.0]], [[1.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]])


def test_quest_bound_handles_mean_cancellation_oracle():
    """Page 0 holds +10 and -10: its mean cancels but its bound does not -> pages [0, 2]."""
    lo, hi = _bounds(K_CANCEL, 2)
    pages = oracle.quest_pages(torch.tensor([[1.0, 0.0]]), lo, hi, 5, 2, 2, keep_sink=False)
    assert pages.tolist() == [[0, 2]]  # mean scoring would choose page 1
    torch.testing.assert_close(lo[0], K_CANCEL[:2].amin(0))
    torch.testing.assert_close(hi[0], K_CANCEL[:2].amax(0))


@pytest.mark.gpu
def test_quest_bound_handles_mean_cancellation_gpu():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    lo, hi = _bounds(K_CANCEL, 2)
    q = torch.tensor([[1.0, 0.0]], device="cuda:0")
    selection = quest_selection(q, lo.cuda(), hi.cuda(), 5, 2, 2, keep_sink=False)
    assert selection.pages == [0, 2]
    assert selection.positions == ((0, 1, 4),)


def test_selection_rejects_invalid_and_shared_native_indexer_rows():
    s = Selection.from_tokens([3, 1, 1, -1], 4, 2, 6, source="native_fixture")
    assert all(row == (1, 3) for row in s.positions)
    for rows in [[4], [-2], [-1], [1.2], []]:
        with pytest.raises((ValueError, TypeError)):
            Selection.from_tokens(rows, 4, 2, 2)


def test_selection_from_pages_clips_to_length_and_rejects_bad_pages():
    s = Selection.from_pages([[0, 2], [2]], 10, 4, 2)
    assert s.positions == ((0, 1, 2, 3, 8, 9), (8, 9))
    assert s.pages == [0, 2]
    with pytest.raises(ValueError, match="invalid logical page"):
        Selection.from_pages([[3]], 10, 4, 1)


def test_quest_selection_validates_budget_and_gqa_shape():
    lo = torch.zeros(4, 2, 8)
    with pytest.raises(ValueError, match="GQA"):
        quest_selection(torch.zeros(3, 8), lo, lo, 10, 4, 2)
    with pytest.raises(ValueError, match="budget"):
        quest_selection(torch.zeros(4, 8), lo, lo, 10, 4, 0)
    with pytest.raises(ValueError, match="ROCm"):
        quest_selection(torch.zeros(4, 8), lo, lo, 10, 4, 2)
