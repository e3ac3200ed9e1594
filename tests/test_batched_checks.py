"""Host-side checks of the batched layer decoder that need no GPU: the page list a
caller hands to ``select_pages`` is validated before anything is launched, and an
overflow flag raised by the union builder surfaces as an error.  The decoder's
buffers live on the CPU here; nothing reaches the HIP library but its host-only
size queries."""

import pytest
import torch

from mini_hisparse_amd.batched import BatchedSparseDecode
from mini_hisparse_amd.config import CacheConfig


def decoder(lengths=(40, 100), top=4):
    cfg = CacheConfig(gpu_pages=8, host_pages=64, page_size=16, kv_heads=2, head_dim=64, device="cpu")
    return BatchedSparseDecode(cfg, 4, top, list(lengths), device="cpu", shared_selection=True)


@pytest.mark.parametrize(
    "rows,why",
    [
        ([[0, 2, 1, 0], [0, 3, 5, 6]], "request 0 (3 pages) must give 0, 1, 2 in order"),
        ([[0, 1, 2, 9], [3, 0, 5, 6]], "not ascending"),
        ([[0, 1, 2, 9], [0, 3, 3, 6]], "a repeated page"),
        ([[0, 1, 2, 9], [0, 3, 5, 7]], "page 7 is past the history (7 pages)"),
        ([[0, 1, 2, 9], [0, 2, 3, 5]], "the tail page (6) is not last"),
        ([[-1, 1, 2, 9], [0, 2, 3, 6]], "a negative page"),
    ],
)
def test_select_pages_rejects_malformed_selections_before_launching(rows, why):
    dec = decoder()
    before = dec.pages.clone()
    with pytest.raises(ValueError, match="ascending distinct pages"):
        dec.select_pages(torch.tensor(rows, dtype=torch.int32))
    assert torch.equal(dec.pages, before), "a rejected selection changes nothing"


def test_select_pages_checks_shape_and_dtype():
    dec = decoder()
    with pytest.raises(ValueError, match="int32"):
        dec.select_pages(torch.zeros((2, 4), dtype=torch.int64))
    with pytest.raises(ValueError, match="int32"):
        dec.select_pages(torch.zeros((2, 3), dtype=torch.int32))


@pytest.mark.parametrize("bits,names", [(1, "union positions"), (2, "group entries"), (3, "union positions and group entries")])
def test_status_bits_of_the_union_builder_raise(bits, names):
    dec = decoder()
    dec.check_status()  # a fresh decoder is clean
    dec.status.fill_(bits)
    with pytest.raises(RuntimeError, match=names):
        dec.check_status()
