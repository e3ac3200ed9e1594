"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against the reference's own vectors (the
index walkthrough, reference test known answers, golden vectors recorded from
the reference in tests/golden/) and against an independent formulation
written differently from the oracle (sequential / exact rational / scalar),
chosen so that a dropped term, a wrong sign or index, or a swapped operand
fails.
"""

from __future__ import annotations

import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from oracle.quest import pages_to_positions, quest_scores
from oracle.union import from_selection, group_entries
from tests.kernel_cases import random_positions, resolver_tables

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)["cases"] if name != "index_walkthrough.json" else json.load(f)


# --------------------------------------------------------------- resolver
def sequential_resolve(positions, source, resident, hot, tags, lru, length, P, head_columns=None):
    """Independent statement of row_index.py:59-137 as a sequential process over
    the distinct valid tokens in ascending order (no sort/search/scatter)."""
    positions, source, resident, hot = (list(map(int, x)) for x in (positions, source, resident, hot))
    tags, lru = list(map(int, tags)), list(map(int, lru))
    S, NP = len(tags), len(source)
    tokens = sorted({t for t in positions if 0 <= t < length})
    slot_of_tag = {tag: s for s, tag in enumerate(tags) if tag >= 0}
    info, hit_slots = {}, set()
    for t in tokens:
        page, off = min(t // P, NP - 1), t % P
        if source[page] < 0:
            continue
        host = source[page] * P + off
        if resident[page] >= 0:
            info[t] = ("resident", resident[page] * P + off)
        elif host in slot_of_tag:
            hit_slots.add(slot_of_tag[host])
            info[t] = ("hit", slot_of_tag[host])
        else:
            info[t] = ("miss", host)
    victims = [s for s in lru if s not in hit_slots] + [s for s in lru if s in hit_slots]
    filled, miss_host, miss_dev, rank = set(), [], [], 0
    new_tags = list(tags)
    for t in tokens:
        kind, value = info.get(t, (None, None))
        if kind == "miss":
            slot = victims[min(rank, S - 1)]
            rank += 1
            new_tags[slot] = value
            filled.add(slot)
            info[t] = ("loaded", slot, value)
    physical_of = {}
    for t, record in info.items():
        if record[0] == "resident":
            physical_of[t] = record[1]
        else:
            slot = record[1]
            physical_of[t] = hot[slot // P] * P + slot % P
            if record[0] == "loaded":
                miss_host.append(record[2])
                miss_dev.append(physical_of[t])
    n = len(positions)
    seen, result = set(), []
    for t in positions:
        if 0 <= t < length and t not in seen and t in physical_of:
            result.append(physical_of[t])
        else:
            result.append(-1)
        if 0 <= t < length:
            seen.add(t)
    if head_columns is not None:
        result = [[result[c] if 0 <= c < n else -1 for c in row] for row in head_columns]
    untouched = [s for s in lru if s not in filled and s not in hit_slots]
    new_lru = untouched + [s for s in lru if s in filled and s not in hit_slots] + [s for s in lru if s in hit_slots]
    counts = [sum(r[0] == "resident" for r in info.values()), len(hit_slots), len(miss_host)]
    pad = [-1] * (n - len(miss_host))
    return result, miss_host + pad, miss_dev + pad, counts, new_tags, new_lru


def test_resolver_reproduces_the_reference_walkthrough():
    w = _load("index_walkthrough.json")
    lru = [0, 1, 2, 3, 4, 6, 7, 5]
    phys, mh, md, counts, tags, lru_after = oracle.resolve_rows(
        w["logical_tokens"], w["source_table"], w["resident_table"], w["hot_block_table"], w["tags_before"], lru, 16, 4
    )
    assert phys.tolist() == w["physical_rows"]
    assert mh.tolist() == w["miss_host_rows"] and md.tolist() == w["miss_device_rows"]
    assert counts.tolist() == [w["counts"]["resident_hits"], w["counts"]["hot_hits"], w["counts"]["misses"]]
    assert tags.tolist() == w["tags_after"]
    # derived from the LRU rule (untouched, then filled, then hits): slot 0 filled, slot 5 hit
    assert lru_after.tolist() == [1, 2, 3, 4, 6, 7, 0, 5]


def test_resolver_matches_reference_trajectories():
    for case in _load("resolver_trajectories.json"):
        tags, lru = np.asarray(case["tags0"]), np.asarray(case["lru0"])
        for step in case["steps"]:
            cols = None if step["head_columns"] is None else np.asarray(step["head_columns"])
            phys, mh, md, counts, tags, lru = oracle.resolve_rows(
                step["positions"], case["source"], case["resident"], case["hot"], tags, lru,
                case["length"], case["page_size"], head_columns=cols,
            )
            assert phys.tolist() == step["physical"]
            assert mh.tolist() == step["miss_host"] and md.tolist() == step["miss_device"]
            assert counts.tolist() == step["counts"]
            assert tags.tolist() == step["tags"] and lru.tolist() == step["lru"]


@pytest.mark.parametrize("seed", range(12))
def test_resolver_matches_independent_sequential_statement(seed):
    rng = np.random.default_rng(seed)
    P = int(rng.choice([1, 3, 4, 16]))
    length = int(rng.integers(5, 400))
    S = int(rng.choice([8, 30, 64, 256]))
    tables = resolver_tables(seed, length, P, S, resident_frac=float(rng.random()), tag_frac=float(rng.random()))
    n = int(rng.integers(1, S + 1))
    positions = random_positions(seed + 50, n, length)
    args = [tables[k] for k in ("source", "resident", "hot", "tags", "lru")]
    got = oracle.resolve_rows(positions, *args, length, P)
    want = sequential_resolve(positions, *args, length, P)
    for g, w in zip(got, want):
        assert np.asarray(g).tolist() == list(w)
    # per-head columns: positions become a sorted union
    heads = int(rng.integers(1, 5))
    rows = [sorted(set(rng.integers(0, length, size=max(1, n // heads)).tolist())) for _ in range(heads)]
    union, columns = from_selection(rows)
    got = oracle.resolve_rows(union, *args, length, P, head_columns=columns)
    want = sequential_resolve(union, *args, length, P, head_columns=columns.tolist())
    assert got[0].tolist() == want[0]


def test_resolver_invariants_on_random_tables():
    for seed in range(20):
        tables = resolver_tables(seed, 500, 4, 128, tag_frac=0.5)
        positions = random_positions(seed, 100, 500)
        phys, mh, md, counts, tags, lru = oracle.resolve_rows(
            positions, *[tables[k] for k in ("source", "resident", "hot", "tags", "lru")], 500, 4
        )
        assert sorted(lru.tolist()) == list(range(128))  # LRU stays a permutation
        live = tags[tags >= 0]
        assert len(set(live.tolist())) == len(live)  # tags stay unique
        distinct = len({t for t in positions.tolist() if 0 <= t < 500})
        assert counts.sum() == distinct  # every unique valid token is counted once
        assert (mh[: counts[2]] >= 0).all() and (mh[counts[2] :] == -1).all()


# ------------------------------------------------------------------ Quest
def test_quest_known_answer_from_the_reference_tests():
    k = torch.tensor([[[10.0, 0.0]], [[-10.0, 0.0]], [[1.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]])
    lo = torch.stack([k[0:2].amin(0), k[2:4].amin(0), k[4:5].amin(0)])
    hi = torch.stack([k[0:2].amax(0), k[2:4].amax(0), k[4:5].amax(0)])
    assert oracle.quest_pages(torch.tensor([[1.0, 0.0]]), lo, hi, 5, 2, 2, keep_sink=False).tolist() == [[0, 2]]


def brute_quest_pages(q, lo, hi, length, P, top, keep_sink):
    """Exact rational scores, forced pages, ties to the lower page."""
    count = math.ceil(length / P)
    heads, kv = q.shape[0], lo.shape[1]
    g = heads // kv
    if top >= count:
        return [list(range(count))] * heads
    forced = {count - 1} | ({0} if keep_sink and top > 1 and count > 1 else set())
    chosen = []
    for h in range(heads):
        scores = []
        for p in range(count):
            if p in forced:
                scores.append((1, Fraction(0), -p))
                continue
            s = sum(
                max(Fraction(float(q[h, d])) * Fraction(float(lo[p, h // g, d])),
                    Fraction(float(q[h, d])) * Fraction(float(hi[p, h // g, d])))
                for d in range(q.shape[1])
            )
            scores.append((0, s, -p))
        order = sorted(range(count), key=lambda p: scores[p], reverse=True)
        chosen.append(sorted(order[:top]))
    return chosen


@pytest.mark.parametrize("seed", range(6))
def test_quest_matches_exact_rational_brute_force(seed):
    rng = np.random.default_rng(seed)
    pages, P, kv, g, D = int(rng.integers(3, 12)), int(rng.choice([2, 4])), int(rng.integers(1, 3)), int(rng.integers(1, 4)), 6
    length = (pages - 1) * P + int(rng.integers(1, P + 1))
    # small integers: every product and sum is exact, so no rounding can hide an error
    k = rng.integers(-9, 10, size=(pages * P, kv, D)).astype(np.float32)[:length]
    lo = np.stack([k[p * P : (p + 1) * P].min(0) for p in range(pages)])
    hi = np.stack([k[p * P : (p + 1) * P].max(0) for p in range(pages)])
    q = rng.integers(-5, 6, size=(kv * g, D)).astype(np.float32)
    for top in (1, 2, 3, pages, pages + 2):
        for sink in (True, False):
            got = oracle.quest_pages(q, lo, hi, length, P, top, keep_sink=sink)
            assert got.tolist() == brute_quest_pages(q, lo, hi, length, P, top, sink)


def test_quest_scores_are_a_sequential_float32_sum():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 5)).astype(np.float32)
    lo = rng.standard_normal((3, 1, 5)).astype(np.float32)
    hi = lo + np.abs(rng.standard_normal((3, 1, 5))).astype(np.float32)
    scores = quest_scores(q, lo, hi, 3)
    for h in range(2):
        for p in range(3):
            s = np.float32(0)
            for d in range(5):
                s = np.float32(s + np.float32(max(q[h, d] * lo[p, 0, d], q[h, d] * hi[p, 0, d])))
            assert scores[h, p] == s


def test_quest_matches_reference_selections_outside_near_ties():
    data = np.load(os.path.join(GOLDEN, "quest_selections.npz"))
    cases = sorted({key.split("/")[0] for key in data.files}, key=int)
    checked = 0
    for i in cases:
        c = {key.split("/")[1]: data[key] for key in data.files if key.startswith(f"{i}/")}
        length, P, top = int(c["length"]), int(c["page_size"]), int(c["top"])
        got = oracle.quest_pages(c["query"], c["minimum"], c["maximum"], length, P, top, keep_sink=bool(c["keep_sink"]))
        count = math.ceil(length / P)
        q = c["query"].astype(np.float64)
        g = q.shape[0] // c["minimum"].shape[1]
        lo = np.repeat(c["minimum"][:count].astype(np.float64), g, axis=1).transpose(1, 0, 2)
        hi = np.repeat(c["maximum"][:count].astype(np.float64), g, axis=1).transpose(1, 0, 2)
        terms = np.maximum(q[:, None] * lo, q[:, None] * hi)  # exact in float64
        exact = terms.sum(-1)
        # two float32 summation orders of D terms differ by at most 2 * D * 2^-24 * sum|terms|
        bound = 2 * q.shape[1] * 2.0**-24 * np.abs(terms).sum(-1).max(-1)
        forced = [count - 1] + ([0] if c["keep_sink"] and top > 1 and count > 1 else [])
        for h in range(got.shape[0]):
            mine, theirs = set(got[h].tolist()), set(c["chosen"][h].tolist())
            if mine == theirs:
                checked += 1
                continue
            scores = exact[h].copy()
            scores[forced] = np.inf
            kth = np.sort(scores)[::-1][top - 1]
            for p in mine ^ theirs:  # only near-ties may differ
                assert abs(scores[p] - kth) <= 2 * bound[h], (i, h, p)
    assert checked >= 0.9 * sum(len(data[f"{i}/chosen"]) for i in cases)


def test_selection_canonical_positions_from_pages():
    assert pages_to_positions([[0, 2], [2]], 10, 4) == ((0, 1, 2, 3, 8, 9), (8, 9))


# ------------------------------------------------------------------- union
def test_union_columns_and_group_entries_independent_formulation():
    rows = ((1, 5, 9), (5, 6), (0, 9, 12, 13))
    union, columns = from_selection(rows)
    assert union.tolist() == [0, 1, 5, 6, 9, 12, 13]
    for h, row in enumerate(rows):
        assert [union[c] for c in columns[h, : len(row)]] == list(row)
        assert (columns[h, len(row) :] == -1).all()
    (c0, m0), (c1, m1) = group_entries(np.array([[1, 2, -1], [2, 3, -1], [0, 4, 5], [4, -1, -1]]), 2)
    assert c0.tolist() == [1, 2, 3] and m0.tolist() == [1, 3, 2]
    assert c1.tolist() == [0, 4, 5] and m1.tolist() == [1, 3, 1]


# --------------------------------------------------------------- attention
def scalar_attention(q, keys, values, valid):
    """Textbook softmax with math.exp, one head at a time."""
    out = []
    for h in range(len(q)):
        scores = [
            sum(a * b for a, b in zip(q[h], keys[h][j])) / math.sqrt(len(q[h])) if valid[h][j] else None
            for j in range(len(keys[h]))
        ]
        live = [s for s in scores if s is not None]
        if not live:
            out.append([0.0] * len(q[h]))
            continue
        top = max(live)
        weights = [0.0 if s is None else math.exp(s - top) for s in scores]
        total = sum(weights)
        out.append([sum(w * v[d] for w, v in zip(weights, values[h])) / total for d in range(len(q[h]))])
    return np.asarray(out)


def test_row_attention_matches_scalar_softmax():
    rng = np.random.default_rng(5)
    P, kv, D, blocks, heads = 4, 2, 6, 5, 4
    pool = rng.standard_normal((blocks, 2, P, kv, D))
    q = rng.standard_normal((heads, D))
    rows = np.array([[0, 3, 7, -1], [19, 2, -1, -1], [5, 5, 6, 1], [-1, -1, -1, -1]])
    got = oracle.row_attention_rows(q, pool, rows, P)
    g = heads // kv
    keys = [[pool[r // P, 0, r % P, h // g] for r in row] for h, row in enumerate(rows)]
    values = [[pool[r // P, 1, r % P, h // g] for r in row] for h, row in enumerate(rows)]
    want = scalar_attention(q, keys, values, rows >= 0)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert (got[3] == 0).all()  # every row masked -> 0 (row_kernels.py:113)


def test_attention_special_cases():
    rng = np.random.default_rng(6)
    pool = rng.standard_normal((3, 2, 4, 1, 8))
    q = rng.standard_normal((2, 8))
    one = oracle.row_attention_rows(q, pool, np.array([[6], [6]]), 4)
    np.testing.assert_allclose(one, np.stack([pool[1, 1, 2, 0]] * 2))  # a single row returns its V
    zero_q = np.zeros((1, 8))
    mean = oracle.row_attention_rows(zero_q, pool, np.array([[0, 5, 9]]), 4)
    np.testing.assert_allclose(mean[0], (pool[0, 1, 0, 0] + pool[1, 1, 1, 0] + pool[2, 1, 1, 0]) / 3)
    k = rng.standard_normal((6, 1, 8))
    v = rng.standard_normal((6, 1, 8))
    dense = oracle.dense_attention(q, k, v)
    sparse = oracle.selection_oracle(q, k, v, [tuple(range(6)), tuple(range(6))])
    np.testing.assert_allclose(dense, sparse)


def _merge_states(a, b):
    """The window merge of reference/attention.py:11-18 (float64)."""
    (m1, l1, a1), (m2, l2, a2) = a, b
    m = np.maximum(m1, m2)
    w1 = np.where(np.isfinite(m1), np.exp(np.where(np.isfinite(m1), m1 - m, 0.0)), 0.0)
    w2 = np.where(np.isfinite(m2), np.exp(np.where(np.isfinite(m2), m2 - m, 0.0)), 0.0)
    return m, w1 * l1 + w2 * l2, w1[:, None] * a1 + w2[:, None] * a2


def test_window_states_merge_to_scalar_softmax_over_their_tokens():
    """Windows of whole pages (partial tail page, per-head token masks, a head that
    reads nothing in one window): merged states give the textbook softmax of each
    head over exactly the tokens it reads; a head that reads nothing has (-inf, 0, 0)."""
    rng = np.random.default_rng(8)
    P, kv, D, blocks, heads = 4, 2, 6, 7, 4
    pool = rng.standard_normal((blocks, 2, P, kv, D))
    q = rng.standard_normal((heads, D))
    windows = [([5, 1], [4, 4]), ([3], [2])]  # (slots, valid lengths): page 3 is a partial tail
    masks = [rng.random((heads, 2, P)) < 0.6, np.zeros((heads, 1, P), bool)]
    masks[1][0] = True  # head 0 reads the tail window; heads 1-3 read nothing there
    masks[0][3] = False  # head 3 reads nothing in the first window either
    states = [oracle.window_state(q, pool, s, n, m, P) for (s, n), m in zip(windows, masks)]
    m, l, acc = _merge_states(*states)
    g = heads // kv
    for h in range(heads):
        rows = [slot * P + t for (slots, lens), mk in zip(windows, masks)
                for i, (slot, n) in enumerate(zip(slots, lens)) for t in range(n) if mk[h, i, t]]
        if not rows:
            assert m[h] == -np.inf and l[h] == 0 and (acc[h] == 0).all()
            continue
        keys = [[pool[r // P, 0, r % P, h // g] for r in rows]]
        values = [[pool[r // P, 1, r % P, h // g] for r in rows]]
        want = scalar_attention(q[h : h + 1], keys, values, np.ones((1, len(rows)), bool))[0]
        np.testing.assert_allclose(acc[h] / l[h], want, rtol=1e-12, atol=1e-12)
        scores = [np.dot(k, q[h]) * D**-0.5 for k in keys[0]]
        assert m[h] == pytest.approx(max(scores), rel=1e-12, abs=1e-12)
    # no mask: every valid token, i.e. dense attention over the window's tokens
    m0, l0, a0 = oracle.window_state(q, pool, [2, 6], [4, 3], None, P)
    k = np.concatenate([pool[2, 0, :4], pool[6, 0, :3]])
    v = np.concatenate([pool[2, 1, :4], pool[6, 1, :3]])
    np.testing.assert_allclose(a0 / l0[:, None], oracle.dense_attention(q, k, v), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ gather
def test_gather_copies_exactly_the_planned_rows():
    rng = np.random.default_rng(7)
    host = rng.standard_normal((6, 2, 4, 2, 3))
    pool = np.zeros((5, 2, 4, 2, 3))
    oracle.gather_rows(host, pool, [5, 17, -1, 2], [0, 19, 3, -1], 4)
    np.testing.assert_array_equal(pool[0, :, 0], host[1, :, 1])
    np.testing.assert_array_equal(pool[4, :, 3], host[4, :, 1])
    assert np.count_nonzero(pool) == 2 * 2 * 2 * 3  # nothing else written


def test_bounded_gather_skips_rows_past_either_pool():
    """The HIP gather's range rule: an entry whose host row is past the host pool
    (6 pages x 4 = 24 rows) or whose device row is past the device pool (5 x 4 = 20)
    is skipped like -1; every in-range entry is copied as the reference copies it."""
    rng = np.random.default_rng(8)
    host = rng.standard_normal((6, 2, 4, 2, 3))
    plan_h = [5, 24, 23, 2, 9, 0]
    plan_d = [0, 1, 20, 19, 2, 3]
    pool = np.zeros((5, 2, 4, 2, 3))
    oracle.gather_rows(host, pool, plan_h, plan_d, 4, bounded=True)
    expected = np.zeros_like(pool)
    for h, d in ((5, 0), (2, 19), (9, 2), (0, 3)):  # (24, 1) and (23, 20) are out of range
        expected[d // 4, :, d % 4] = host[h // 4, :, h % 4]
    np.testing.assert_array_equal(pool, expected)
    # on a plan inside both pools the bounded rule is the reference's rule
    a, b = np.zeros_like(pool), np.zeros_like(pool)
    oracle.gather_rows(host, a, [5, -1, 23, 7], [0, 3, 19, -1], 4)
    oracle.gather_rows(host, b, [5, -1, 23, 7], [0, 3, 19, -1], 4, bounded=True)
    np.testing.assert_array_equal(a, b)


# --------------------------------------------------------------------- append
def test_append_bound_rule_known_answers():
    """torch.minimum/maximum on the device, as measured on MI355X: a NaN wins (the
    existing bound first); 16-bit ties (+0 vs -0 included) return the new element;
    float32 orders -0 below +0."""
    nan, inf = np.nan, np.inf
    old = np.array([1.0, nan, 2.0, 0.0, -0.0, 3.0, inf, -inf], np.float32)
    new = np.array([0.5, 1.0, nan, -0.0, 0.0, 3.0, 1.0, -2.0], np.float32)
    lo16, hi16 = oracle.bound_min(old, new, 16), oracle.bound_max(old, new, 16)
    lo32, hi32 = oracle.bound_min(old, new, 32), oracle.bound_max(old, new, 32)
    for lo, hi in ((lo16, hi16), (lo32, hi32)):
        np.testing.assert_array_equal(lo[[0, 5, 6, 7]], [0.5, 3.0, 1.0, -inf])
        np.testing.assert_array_equal(hi[[0, 5, 6, 7]], [1.0, 3.0, inf, -2.0])
        assert np.isnan(lo[1]) and np.isnan(lo[2]) and np.isnan(hi[1]) and np.isnan(hi[2])
    # equal zeros: 16-bit takes the new element, float32 takes -0 (min) / +0 (max)
    assert list(np.signbit(lo16[3:5])) == [True, False] and list(np.signbit(hi16[3:5])) == [True, False]
    assert list(np.signbit(lo32[3:5])) == [True, True] and list(np.signbit(hi32[3:5])) == [False, False]


def test_append_bound_rule_is_numpy_min_max_without_nan_or_zero_ties():
    rng = np.random.default_rng(3)
    old, new = rng.standard_normal((2, 4096)).astype(np.float32)
    for bits in (16, 32):
        np.testing.assert_array_equal(oracle.bound_min(old, new, bits), np.minimum(old, new))
        np.testing.assert_array_equal(oracle.bound_max(old, new, bits), np.maximum(old, new))


def test_append_fills_a_page_to_its_column_extrema_and_writes_rows():
    rng = np.random.default_rng(4)
    P, Hkv, D = 8, 2, 16
    keys = rng.standard_normal((P, Hkv, D)).astype(np.float32)
    vals = rng.standard_normal((P, Hkv, D)).astype(np.float32)
    pool = np.zeros((3, 2, P, Hkv, D), np.float32)
    host = np.zeros((5, 2, P, Hkv, D), np.float32)
    lo = np.full((Hkv, D), np.inf, np.float32)
    hi = np.full((Hkv, D), -np.inf, np.float32)
    for t in range(P):  # device block 2, host block 4, one row per step
        oracle.append_rows(pool, host, keys[t : t + 1], vals[t : t + 1], [2 * P + t], [4 * P + t], [lo], [hi], P)
    np.testing.assert_array_equal(lo, keys.min(0))
    np.testing.assert_array_equal(hi, keys.max(0))
    np.testing.assert_array_equal(pool[2, 0], keys)
    np.testing.assert_array_equal(pool[2, 1], vals)
    np.testing.assert_array_equal(host[4], pool[2])
    assert not pool[:2].any() and not host[:4].any()


def test_one_write_of_many_tokens_equals_token_by_token_writes():
    """The batched write's bounds fold rows in order, so one write of T tokens and T
    writes of one token give the same pool, host mirror, bounds and summaries; the
    bounds are the exact extrema of each page's rows (no NaN, no signed-zero ties)."""
    import torch

    P, kv, D, tokens, start = 4, 2, 3, 23, 2
    gen = torch.Generator().manual_seed(5)
    k, v = torch.randn(tokens, kv, D, generator=gen), torch.randn(tokens, kv, D, generator=gen)
    pages = (start + tokens + P - 1) // P
    slots, host_slots = list(range(pages)), list(range(10, 10 + pages))

    def fresh():
        pool, host = torch.zeros(pages, 2, P, kv, D), torch.zeros(20, 2, P, kv, D)
        lo, hi = torch.full((pages, kv, D), float("inf")), torch.full((pages, kv, D), float("-inf"))
        return pool, host, lo, hi, torch.zeros(pages, kv, D)

    bulk = fresh()
    oracle.append_tokens(*bulk[:2], k, v, start // P, start % P, slots[start // P:], host_slots[start // P:],
                         *bulk[2:], P, 32)
    steps = fresh()
    for t in range(tokens):
        page, within = divmod(start + t, P)
        oracle.append_tokens(*steps[:2], k[t : t + 1], v[t : t + 1], page, within, [slots[page]],
                             [host_slots[page]], *steps[2:], P, 32)
    for a, b in zip(bulk, steps):
        assert torch.equal(a, b)
    pool, _, lo, hi, summ = bulk
    for page in range(start // P, pages):
        rows = range(max(0, start - page * P), min(P, start + tokens - page * P))
        keys = torch.stack([k[page * P + r - start] for r in rows])
        assert torch.equal(lo[page], keys.amin(0)) and torch.equal(hi[page], keys.amax(0))
        assert torch.allclose(summ[page], pool[page, 0, : max(rows) + 1].mean(0), atol=1e-6)
