"""Segments of the prefix-tree plan (mentat_amd/tree_plan.py: common prefixes
of neighbours in batch order) on the CPU.

Forests of sequences are grown with the oracle cache's own fork / append
bookkeeping (core/paged_kv_cache.py:152-284 restated in oracle/paged_cache.py),
so block ids are shared exactly as the reference's tables share them. Checked:
  * every query's segments cover its tokens, each exactly once, and the owner
    row's block ids on those pages are the query's own;
  * in depth-first order with all siblings growing in step (as in a rollout),
    each distinct page is read once;
  * any batch order stays correct (shuffled batches);
  * the lcp rule on a hand-made batch, and the segments of a known batch.
"""
import random

import numpy as np
import pytest

from mentat_amd.tree_plan import build_plan, common_prefix_pages, segment_arrays
from oracle.paged_cache import OracleCache


def _forest(seed, B, n_roots=3, steps=40, in_step=False):
    """Leaves of random prefix trees in depth-first order with their layer-0 tables.
    in_step: every live leaf appends each step (the rollout's decode)."""
    rng = random.Random(seed)
    c = OracleCache(1, 8192, B)
    trees = []
    for _ in range(n_roots):
        r = c.allocate()
        c.append(r, 0, list(range(rng.randint(1, 5 * B))))
        trees.append([r])
    for _ in range(steps):
        t = rng.choice(trees)
        leaf = rng.choice(t)
        op = rng.random()
        if op < 0.3 and len(t) < 12:
            t.insert(t.index(leaf) + 1, c.fork(leaf))  # children follow their parent: depth-first order
        elif op < 0.4 and len(t) > 1:
            c.free(leaf)
            t.remove(leaf)
        if in_step or op >= 0.4:
            live = [s for tr in trees for s in tr]
            grow = live if in_step else [s for s in live if rng.random() < 0.7]
            c.append_batched(grow, 0, [0] * len(grow))
    return c, [s for t in trees for s in t]


def _arrays(c, order):
    lens = np.array([c.ntok[s][0] for s in order])
    P = max(1, max(len(c.tables[s][0]) for s in order))
    tab = np.full((len(order), P), -1, dtype=np.int32)
    for i, s in enumerate(order):
        t = c.tables[s][0]
        tab[i, :len(t)] = t
    rows = np.arange(len(order)) * 3 + 1  # table rows differ from batch indices
    return tab, lens, rows


def _check_cover(sg, tab, lens, rows, B):
    row_of = {int(r): i for i, r in enumerate(rows)}
    got = [[] for _ in lens]
    for r, a, b, e, m0, cnt in zip(sg.row, sg.first_page, sg.end_page, sg.end_token, sg.m0, sg.count):
        owner = row_of[int(r)]
        for i in range(int(m0), int(m0 + cnt)):
            assert (tab[owner, a:b] == tab[i, a:b]).all()
            assert e <= lens[i] and (b == (lens[i] + B - 1) // B or e == b * B)
            got[i].append((int(a) * B, int(e)))
    for i, spans in enumerate(got):
        pos = 0
        for a, e in sorted(spans):
            assert a == pos and e > a, (i, spans)
            pos = e
        assert pos == lens[i], (i, spans)


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("B", [16, 32])
def test_segments_cover_each_query_once_and_read_each_page_once(seed, B):
    c, order = _forest(seed, B, in_step=True)
    tab, lens, rows = _arrays(c, order)
    sg = segment_arrays(tab, lens, rows, B)
    _check_cover(sg, tab, lens, rows, B)
    distinct = {(int(tab[i, p]), min(B, int(lens[i]) - p * B)) for i in range(len(order))
                for p in range((int(lens[i]) + B - 1) // B)}
    assert int((sg.end_token - sg.first_page * B).sum()) == sum(v for _, v in distinct)


@pytest.mark.parametrize("seed", range(6))
def test_segments_with_uneven_growth_and_shuffled_orders(seed):
    B = 16
    c, order = _forest(100 + seed, B)
    for shuffle in (False, True):
        o = list(order)
        if shuffle:
            random.Random(seed).shuffle(o)
        tab, lens, rows = _arrays(c, o)
        sg = segment_arrays(tab, lens, rows, B)
        _check_cover(sg, tab, lens, rows, B)
        plan = build_plan(tab, lens, rows, block_size=B, Hkv=2, G=4)
        plan.validate(len(o), 2, 4, int(rows.max()) + 1, tab.shape[1], B)
        assert plan.unique_tokens() <= int(lens.sum())


def test_lcp_rule():
    B = 16
    tab = np.array([[5, 6, 7, 0], [5, 6, 8, 0], [5, 6, 8, 9], [1, 6, 8, 9]], dtype=np.int32)
    lens = np.array([40, 48, 64, 64])
    assert common_prefix_pages(tab, lens, B).tolist() == [0, 2, 3, 0]
    # a partial page is shared when its valid count matches, and ends the run
    lens2 = np.array([40, 40, 40, 64])
    tab2 = np.array([[5, 6, 7, 0], [5, 6, 7, 0], [5, 6, 8, 9], [1, 6, 8, 9]], dtype=np.int32)
    assert common_prefix_pages(tab2, lens2, B).tolist() == [0, 3, 2, 0]


def test_known_segments():
    """Queries 0-3 share 2 pages, 2-3 a third; then each private tail."""
    B = 16
    tab = np.array([[1, 2, 3, 0], [1, 2, 4, 0], [1, 2, 5, 6], [1, 2, 5, 7]], dtype=np.int32)
    lens = np.array([40, 33, 60, 64])
    rows = np.array([10, 11, 12, 13])
    sg = segment_arrays(tab, lens, rows, B)
    got = {(int(r), int(a), int(b), int(e), int(m), int(c))
           for r, a, b, e, m, c in zip(sg.row, sg.first_page, sg.end_page, sg.end_token, sg.m0, sg.count)}
    assert got == {(10, 2, 3, 40, 0, 1), (10, 0, 2, 32, 0, 4), (11, 2, 3, 33, 1, 1),
                   (12, 3, 4, 60, 2, 1), (12, 2, 3, 48, 2, 2), (13, 3, 4, 64, 3, 1)}


def test_empty_and_zero_length_queries():
    sg = segment_arrays(np.zeros((0, 1), np.int32), np.zeros(0), np.zeros(0), 16)
    assert len(sg) == 0
    plan = build_plan(np.zeros((0, 1), np.int32), np.zeros(0), np.zeros(0), block_size=16, Hkv=2, G=4)
    assert plan.items.shape == (0, 8) and plan.q_slot_offsets.tolist() == [0]
    tab = np.array([[3], [3], [4]], dtype=np.int32)
    sg = segment_arrays(tab, np.array([0, 16, 0]), np.array([0, 1, 2]), 16)
    assert [(int(m), int(c)) for m, c in zip(sg.m0, sg.count)] == [(1, 1)]
