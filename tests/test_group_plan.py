"""Host plan of the grouped paged decode (mentat_amd/group_plan.py) on the CPU.

Forests of sequences are grown with the oracle cache's own fork / append
bookkeeping (core/paged_kv_cache.py:152-284 restated in oracle/paged_cache.py),
so the block ids share pages exactly as the reference's tables do. Checked:
  * every query's segments cover its own tiles, each exactly once, and the
    owner row's block ids on those pages are the query's own;
  * every query of a segment holds the segment's pages;
  * in depth-first order with no per-tile cap, each physical page is read once
    (tiles read = distinct (block, tile) pairs); with a cap of c queries a
    page shared by n queries is read ceil(n / c) times at most per run;
  * any batch order stays correct (shuffled batches);
  * the plan validates, and the validator rejects planted index errors.
"""
import random

import numpy as np
import pytest

from mentat_amd.group_plan import GroupPlan, build_group_plan, common_prefix_pages, private_plan
from oracle.paged_cache import OracleCache


def _forest(seed, B, n_roots=3, steps=40):
    """Leaves of random prefix trees, depth-first, with their layer-0 tables."""
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
            kid = c.fork(leaf)
            t.insert(t.index(leaf) + 1, kid)  # children follow their parent: depth-first order
        elif op < 0.4 and len(t) > 1:
            c.free(leaf)
            t.remove(leaf)
        else:
            for s in list(t):
                if rng.random() < 0.7:
                    c.append_batched([s], 0, [0])
    order = [s for t in trees for s in t]
    return c, order


def _arrays(c, order):
    lens = np.array([c.ntok[s][0] for s in order])
    P = max(1, max(len(c.tables[s][0]) for s in order))
    tab = np.full((len(order), P), -1, dtype=np.int32)
    for i, s in enumerate(order):
        t = c.tables[s][0]
        tab[i, :len(t)] = t
    rows = np.arange(len(order)) * 3 + 1  # table rows differ from batch indices
    return tab, lens, rows


def _check_cover(plan, tab, lens, rows, B):
    row_of = {int(r): i for i, r in enumerate(rows)}
    N = lens.size
    tpp = B // 16 if B >= 16 else None
    for i in range(N):
        got = []
        for j in range(plan.seg_off[i], plan.seg_off[i + 1]):
            r, t0, t1, mc = plan.segs[plan.seg_list[j]].tolist()
            m0, cnt = mc & 0xFFFF, mc >> 16
            assert m0 <= i < m0 + cnt
            owner = row_of[r]
            for t in range(t0, t1):
                page = t * 16 // B
                assert tab[owner, page] == tab[i, page], (i, t)   # the owner's page is the query's
                got.append(t)
        want = list(range((int(lens[i]) + 15) // 16))
        assert sorted(got) == want, (i, sorted(got), want)
    return tpp


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("B", [16, 32])
def test_plan_covers_each_query_once_and_reads_each_page_once(seed, B):
    c, order = _forest(seed, B)
    tab, lens, rows = _arrays(c, order)
    plan = build_group_plan(tab, lens, rows, B, per_tile=64)
    plan.validate(len(order), int(rows.max()) + 1, tab.shape[1], B, 64)
    _check_cover(plan, tab, lens, rows, B)
    distinct = set()
    for i in range(len(order)):
        for t in range((int(lens[i]) + 15) // 16):
            page = t * 16 // B
            full = (page + 1) * B <= lens[i]
            # a partial page is private to its query (the kernel masks it with the owner's length)
            distinct.add((int(tab[i, page]), t) if full else (i, -1, t))
    assert plan.tiles_read() == len(distinct)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("per_tile", [1, 2, 4, 8])
def test_plan_with_a_per_tile_cap_and_shuffled_orders(seed, per_tile):
    B = 16
    c, order = _forest(100 + seed, B)
    for shuffle in (False, True):
        o = list(order)
        if shuffle:
            random.Random(seed).shuffle(o)
        tab, lens, rows = _arrays(c, o)
        plan = build_group_plan(tab, lens, rows, B, per_tile=per_tile)
        plan.validate(len(o), int(rows.max()) + 1, tab.shape[1], B, per_tile)
        _check_cover(plan, tab, lens, rows, B)
        assert int((plan.segs[:, 3] >> 16).max()) <= per_tile
        base = private_plan(lens, rows, B)
        assert plan.tiles_read() <= base.tiles_read()


def test_lcp_counts_only_full_equal_pages():
    B = 16
    tab = np.array([[5, 6, 7, 0], [5, 6, 8, 0], [5, 6, 8, 9], [1, 6, 8, 9]], dtype=np.int32)
    lens = np.array([40, 48, 64, 64])
    assert common_prefix_pages(tab, lens, B).tolist() == [0, 2, 3, 0]
    lens2 = np.array([40, 40, 64, 64])  # row 1's third page is partial: not shared
    assert common_prefix_pages(tab, lens2, B).tolist() == [0, 2, 2, 0]


def test_known_segments():
    """Four queries: 0-3 share 2 pages, 2-3 share a third; the plan is
    [0,2) x {0..3}, then each private tail, 3 x {2,3}."""
    B = 16
    tab = np.array([[1, 2, 3], [1, 2, 4], [1, 2, 5], [1, 2, 5]], dtype=np.int32)
    tab[3, 2] = 5
    tab = np.concatenate([tab, np.array([[0], [0], [6], [7]], dtype=np.int32)], axis=1)
    lens = np.array([40, 33, 60, 64])
    rows = np.array([10, 11, 12, 13])
    plan = build_group_plan(tab, lens, rows, B, per_tile=4)
    segs = {tuple(s) for s in plan.segs.tolist()}
    assert segs == {(10, 2, 3, 0 | 1 << 16), (10, 0, 2, 0 | 4 << 16), (11, 2, 3, 1 | 1 << 16),
                    (12, 3, 4, 2 | 1 << 16), (12, 2, 3, 2 | 2 << 16), (13, 3, 4, 3 | 1 << 16)}
    plan.validate(4, 14, 4, B, 4)


def test_empty_and_zero_length_queries():
    plan = build_group_plan(np.zeros((0, 1), np.int32), np.zeros(0), np.zeros(0), 16, per_tile=4)
    assert plan.n_segs == 0 and plan.seg_off.tolist() == [0]
    plan.validate(0, 1, 1, 16, 4)
    tab = np.array([[3], [3], [4]], dtype=np.int32)
    plan = build_group_plan(tab, np.array([0, 16, 0]), np.array([0, 1, 2]), 16, per_tile=4)
    assert plan.seg_off.tolist() == [0, 0, 1, 1]
    plan.validate(3, 3, 1, 16, 4)


def test_validator_rejects_planted_errors():
    c, order = _forest(3, 16)
    tab, lens, rows = _arrays(c, order)
    plan = build_group_plan(tab, lens, rows, 16, per_tile=4)
    N, R = len(order), int(rows.max()) + 1
    plan.validate(N, R, tab.shape[1], 16, 4)

    def bad(mut):
        p = GroupPlan(plan.segs.copy(), plan.seg_off.copy(), plan.seg_list.copy())
        mut(p)
        with pytest.raises(ValueError):
            p.validate(N, R, tab.shape[1], 16, 4)

    bad(lambda p: p.segs.__setitem__((0, 0), R))                   # owner row past the tables
    bad(lambda p: p.segs.__setitem__((0, 2), tab.shape[1] + 1))    # tiles past the table row
    bad(lambda p: p.segs.__setitem__((0, 3), 0 | (5 << 16)))       # more queries than a tile holds
    bad(lambda p: p.seg_list.__setitem__(0, plan.n_segs))           # a segment that does not exist
    bad(lambda p: p.seg_off.__setitem__(1, p.seg_off[1] + 1))       # a query given another's segment
