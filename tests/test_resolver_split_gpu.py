"""The resolver's split front (``hs_resolve_desc.split_front``: the front's work over
several workgroups per request, in three launches; forced on here with
``HS_RESOLVE_SPLIT=1``) against the oracle, bit for bit:
the batched decode's descriptors (union page bitmaps, affine source tables of a
request's contiguous host slots, int16 or int64 LRU), batches of 1 to 17 requests up
to the 7B shape (131,072 tokens, 32,768 hot rows), tags of other requests' host rows,
host-less pages, the miss plan's prefix-only form, and a multi-step trajectory whose
tags and LRU carry from step to step.  A source table that is not affine with base
``source[0]`` is refused on the device: no row, counts 0, tags and LRU unchanged."""

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions
from tests.kernel_cases import resolver_tables

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def split_everywhere(monkeypatch):
    """The library takes the split front for hot regions above 16384 rows only; these
    tests force it for every descriptor that allows it."""
    monkeypatch.setenv("HS_RESOLVE_SPLIT", "1")


TABLES = ("source", "resident", "hot", "tags", "lru")


def page_set_case(rng, length, P, S, sel, affine_base, foreign=40, resident_frac=0.3):
    """Tables and the union of `sel` random pages (the last page always), as positions
    padded with -1 and as the union builder's page bitmap."""
    count = -(-length // P)
    tables = resolver_tables(int(rng.integers(1 << 30)), length, P, S, resident_frac=resident_frac,
                             affine_base=affine_base, foreign_tags=foreign)
    pages = np.unique(np.append(rng.choice(count, size=min(sel, count), replace=False), count - 1))
    union = np.asarray(pages_to_positions(pages[None, :], length, P)[0], np.int32)
    positions = np.full(len(union) + 37, -1, np.int32)
    positions[: len(union)] = union
    marked = np.zeros(-(-count // 32) * 32, bool)
    marked[pages] = True
    bits = np.packbits(marked.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").reshape(-1).astype(np.uint32)
    return tables, positions, bits


class Batch:
    """Device tables and outputs of a list of cases, as resolver descriptors."""

    def __init__(self, gpu, cases, lru_dtype, split, prefix_only=lambda i: 0):
        from mini_hisparse_amd import _lib

        self.lib, self.gpu = _lib.load(), gpu
        self.descs = (_lib.ResolveDesc * len(cases))()
        self.keep, total = [], 0
        for i, (d, (length, P, tables, positions, bits)) in enumerate(zip(self.descs, cases)):
            t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in tables.items()}
            t["lru"] = t["lru"].to(lru_dtype)
            pos = torch.from_numpy(positions).to(gpu)
            pb = torch.from_numpy(bits.view(np.int32)).to(gpu)
            n = pos.numel()
            out = {name: torch.full((n,), -7, dtype=torch.int64, device=gpu) for name in ("phys", "mh", "md")}
            out["counts"] = torch.full((3,), -7, dtype=torch.int64, device=gpu)
            d.positions, d.n, d.positions_i64 = pos.data_ptr(), n, 0
            d.page_bits = pb.data_ptr()
            d.source, d.resident, d.n_pages = t["source"].data_ptr(), t["resident"].data_ptr(), t["source"].numel()
            d.hot, d.hot_blocks = t["hot"].data_ptr(), t["hot"].numel()
            d.tags, d.lru, d.hot_rows = t["tags"].data_ptr(), t["lru"].data_ptr(), t["tags"].numel()
            d.lru_i16 = int(lru_dtype == torch.int16)
            d.length, d.page_size = length, P
            d.physical = d.union_physical = out["phys"].data_ptr()
            d.miss_host_rows, d.miss_device_rows = out["mh"].data_ptr(), out["md"].data_ptr()
            d.counts = out["counts"].data_ptr()
            d.miss_prefix_only = prefix_only(i)
            d.split_front = int(split)
            total += self.lib.hs_resolve_workspace_bytes(n, length, d.n_pages, d.hot_rows)
            self.keep.append((t, pos, pb, out))
        self.ws = torch.empty(total, dtype=torch.uint8, device=gpu)

    def run(self):
        from mini_hisparse_amd import _lib

        _lib.check(self.lib.hs_resolve_rows_batched(self.descs, len(self.keep), self.ws.data_ptr(), self.ws.numel(),
                                                    _lib.stream_handle(torch.device(self.gpu))),
                   "hs_resolve_rows_batched")
        torch.cuda.synchronize()


def check(case_name, out, t, expected, prefix_only):
    phys, mh, md, counts, tags_after, lru_after = expected
    np.testing.assert_array_equal(out["phys"].cpu().numpy(), phys, err_msg=case_name)
    m = int(counts[2])
    if prefix_only:
        np.testing.assert_array_equal(out["mh"][:m].cpu().numpy(), mh[:m], err_msg=case_name)
        np.testing.assert_array_equal(out["md"][:m].cpu().numpy(), md[:m], err_msg=case_name)
        assert (out["mh"][m:] == -7).all() and (out["md"][m:] == -7).all(), case_name
    else:
        np.testing.assert_array_equal(out["mh"].cpu().numpy(), mh, err_msg=case_name)
        np.testing.assert_array_equal(out["md"].cpu().numpy(), md, err_msg=case_name)
    np.testing.assert_array_equal(out["counts"].cpu().numpy(), counts, err_msg=case_name)
    np.testing.assert_array_equal(t["tags"].cpu().numpy(), tags_after, err_msg=case_name)
    np.testing.assert_array_equal(t["lru"].cpu().numpy().astype(np.int64), lru_after, err_msg=case_name)


@pytest.mark.parametrize("lru_dtype", [torch.int16, torch.int64])
@pytest.mark.parametrize("count", [1, 4, 17])
def test_split_front_batches_match_oracle(gpu, lru_dtype, count):
    """Batches of 1, 4 and 17 requests (16 per launch, then 1: 16 to 64 workgroups per
    request) of mixed shapes, every other one with the prefix-only miss plan."""
    rng = np.random.default_rng(1000 + count)
    shapes = [(5000, 16, 2048, 60), (131072, 16, 32768, 900), (64, 4, 64, 16), (40000, 32, 13504, 200),
              (2048, 1, 256, 300), (777, 8, 330, 30), (3001, 2, 1000, 400)]
    cases = []
    for i in range(count):
        length, P, S, sel = shapes[(i + count) % len(shapes)]
        tables, positions, bits = page_set_case(rng, length, P, S, sel, affine_base=int(rng.integers(0, 5000)))
        cases.append((length, P, tables, positions, bits))
    print(f"[case] split front: {count} requests, lru {lru_dtype}", flush=True)
    batch = Batch(gpu, cases, lru_dtype, split=True, prefix_only=lambda i: i % 2)
    batch.run()
    for i, ((length, P, tables, positions, _), (t, _, _, out)) in enumerate(zip(cases, batch.keep)):
        expected = oracle.resolve_rows(positions, *[tables[k] for k in TABLES], length, P)
        check(f"request {i}: length {length}, page {P}, hot rows {tables['tags'].size}", out, t, expected, i % 2)


def test_split_front_trajectory_carries_tags_and_lru(gpu):
    """Four steps over the same tables (tags and LRU rewritten in place each step, new
    page sets, the history growing by a token per step) at the 0.5B and 7B shapes, split
    and single-workgroup fronts side by side: every step of both equals the oracle."""
    rng = np.random.default_rng(7)
    for length, P, S, sel in [(32768, 16, 13504, 224), (131072, 16, 32768, 448)]:
        tables, _, _ = page_set_case(rng, length + 8, P, S, sel, affine_base=4096)
        state = {k: v.copy() for k, v in tables.items()}
        split_t = single_t = None
        for step in range(4):
            L = length + step
            count = -(-L // P)
            pages = np.unique(np.append(rng.choice(count, size=sel, replace=False), count - 1))
            union = np.asarray(pages_to_positions(pages[None, :], L, P)[0], np.int32)
            marked = np.zeros(-(-count // 32) * 32, bool)
            marked[pages] = True
            bits = np.packbits(marked.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").reshape(-1).astype(np.uint32)
            expected = oracle.resolve_rows(union, *[state[k] for k in TABLES], L, P)
            print(f"[case] split trajectory: length {L}, hot rows {S}, step {step}", flush=True)
            for split in (True, False):
                batch = Batch(gpu, [(L, P, tables, union, bits)], torch.int16, split=split)
                t = batch.keep[0][0]
                carried = split_t if split else single_t
                if carried is not None:  # the previous step's tags and LRU, as the device left them
                    t["tags"].copy_(carried["tags"])
                    t["lru"].copy_(carried["lru"])
                batch.run()
                check(f"step {step}, split {split}", batch.keep[0][3], t, expected, 0)
                if split:
                    split_t = t
                else:
                    single_t = t
            state["tags"], state["lru"] = expected[4], expected[5]


def test_split_front_refuses_a_table_that_is_not_affine(gpu):
    """A permuted source table: no row, counts 0, the miss plan all -1, tags and LRU
    untouched (the place launch refuses it before rewriting anything)."""
    rng = np.random.default_rng(3)
    length, P, S = 5000, 16, 2048
    tables, positions, bits = page_set_case(rng, length, P, S, 60, affine_base=None)
    batch = Batch(gpu, [(length, P, tables, positions, bits)], torch.int16, split=True)
    batch.run()
    t, _, _, out = batch.keep[0]
    assert (out["phys"] == -1).all() and (out["mh"] == -1).all() and (out["md"] == -1).all()
    assert out["counts"].tolist() == [0, 0, 0]
    np.testing.assert_array_equal(t["tags"].cpu().numpy(), tables["tags"])
    np.testing.assert_array_equal(t["lru"].cpu().numpy().astype(np.int64), tables["lru"])
