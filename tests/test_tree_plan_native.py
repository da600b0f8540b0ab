"""The native prefix-tree planner (mentat_tree_plan, host code in the library)
against the Python plan (mentat_amd/tree_plan.py:build_plan) on the CPU:
identical counts, items, members, q_slot_offsets and q_slots, array for array,
over prefix-tree workloads grown through the manager's bookkeeping (forks and
copy-on-write as the reference's manager does them, core/paged_kv_cache.py:
152-284), for every query-heads-per-kv-head geometry, page size and chunking;
share = 0 equals the plan of the same batch with no block ids in common; a
capacity too small returns MENTAT_ESPACE."""
import ctypes

import numpy as np
import pytest
import torch

from mentat_amd import _lib
from mentat_amd.core.paged_kv_cache import PagedKVCacheManager
from mentat_amd.tree_plan import build_plan
from mentat_amd.workloads import replay_tree_ops, tree_ops


def _batch(seed, n_trees, prefix, leaves, max_private, B):
    ops = tree_ops(n_trees=n_trees, prefix=prefix, leaves=leaves, max_private=max_private, seed=seed)
    m = PagedKVCacheManager(1, 2, 32, max_blocks=20000, block_size=B, device="cpu", dtype=torch.bfloat16)
    seq, order = replay_tree_ops(m, ops)
    sts = [m._sequences[seq[x]] for x in order]
    tables = [list(s.page_table[0]) for s in sts]
    lens = [s.num_tokens[0] for s in sts]
    rows = [s.row for s in sts]
    R, P = max(rows) + 1, max(len(t) for t in tables)
    mirror = np.full((R, P + 3), -7, dtype=np.int32)          # rows indexed by table row, stale padding
    for t, r in zip(tables, rows):
        mirror[r, :len(t)] = t
    return tables, lens, rows, mirror


def _native(mirror, rows, lens, B, Hkv, G, chunk, schunk, groups, share=1, caps=(100000, 100000, 400000)):
    N = len(rows)
    ms, mo, msl = caps
    counts = np.zeros(3, np.int32)
    items = np.zeros((ms + mo) * 8 + 1, np.int32)
    members = np.zeros(msl + 1, np.int32)
    off = np.zeros(N * Hkv + 1, np.int32)
    qs = np.zeros(msl + 1, np.int32)
    qr = np.array(rows, np.int32)
    ln = np.array(lens, np.int32)
    st = _lib.get_lib().mentat_tree_plan(mirror.ctypes.data, mirror.shape[1], qr.ctypes.data, ln.ctypes.data, N, B,
                                        Hkv, G, chunk, schunk, groups, share, counts.ctypes.data, items.ctypes.data,
                                        ms, mo, members.ctypes.data, off.ctypes.data, qs.ctypes.data, msl)
    return st, counts, items, members, off, qs


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("B,chunk,schunk,groups", [(16, 4, 32, 3), (32, 2, 3, 1), (16, 16, 32, 99)])
def test_native_plan_equals_python_plan(G, B, chunk, schunk, groups):
    Hkv = 8 if G <= 4 else 2
    for seed, shape in ((0, (4, 300, 12, 80)), (1, (16, 256, 9, 120)), (2, (3, 40, 6, 30))):
        tables, lens, rows, mirror = _batch(seed + G, *shape, B)
        want = build_plan(tables, lens, rows, block_size=B, Hkv=Hkv, G=G, chunk_tiles=chunk,
                          shared_chunk_tiles=schunk, shared_min_groups=groups)
        st, counts, items, members, off, qs = _native(mirror, rows, lens, B, Hkv, G, chunk, schunk, groups)
        assert st == 0
        assert counts.tolist() == [want.n_shared, want.n_solo, want.n_slots]
        n_it = want.items.shape[0]
        assert np.array_equal(items[:n_it * 8].reshape(-1, 8), want.items)
        assert np.array_equal(members[:want.n_slots], want.members)
        assert np.array_equal(off, want.q_slot_offsets)
        assert np.array_equal(qs[:want.n_slots], want.q_slots[:want.n_slots])


def test_native_plan_without_sharing_and_capacity():
    B, Hkv, G = 16, 8, 4
    tables, lens, rows, mirror = _batch(5, 4, 100, 12, 60, B)
    uniq = [[10000 * i + b for b in t] for i, t in enumerate(tables)]      # no ids in common
    want = build_plan(uniq, lens, rows, block_size=B, Hkv=Hkv, G=G, chunk_tiles=4, shared_chunk_tiles=32,
                      shared_min_groups=3)
    st, counts, items, members, off, qs = _native(mirror, rows, lens, B, Hkv, G, 4, 32, 3, share=0)
    assert st == 0 and counts.tolist() == [0, want.n_solo, want.n_slots]
    assert np.array_equal(items[:want.items.shape[0] * 8].reshape(-1, 8), want.items)
    assert np.array_equal(off, want.q_slot_offsets)
    full = build_plan(tables, lens, rows, block_size=B, Hkv=Hkv, G=G, chunk_tiles=4, shared_chunk_tiles=32,
                      shared_min_groups=3)
    assert full.n_shared > 0 and full.n_solo > 0
    for caps in ((full.n_shared - 1, 10 ** 6, 10 ** 6), (10 ** 6, full.n_solo - 1, 10 ** 6),
                 (10 ** 6, 10 ** 6, full.n_slots - 1)):
        assert _native(mirror, rows, lens, B, Hkv, G, 4, 32, 3, caps=caps)[0] == _lib.MENTAT_ESPACE
    assert _native(mirror, rows, lens, B, Hkv, G, 4, 32, 3, caps=(full.n_shared, full.n_solo, full.n_slots))[0] == 0
    bad = mirror[:, :2].copy()                                                 # rows shorter than the pages
    assert _native(bad, rows, lens, B, Hkv, G, 4, 32, 3)[0] == _lib.MENTAT_EINVAL
