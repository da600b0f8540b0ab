"""Host side of prefix-tree decode (CPU): tree workload replay and the segment plan.

The plan must cover every query's context exactly once (segments partition
[0, len) of each member, and a segment's pages are the same block ids in every
member's table), its unique-token count must equal a brute-force count of the
distinct (block, valid tokens) pages, and a float64 evaluation that follows the
plan item by item (partial softmax per item, log-sum-exp merge per query)
must equal the oracle's per-sequence attention.
"""
import dataclasses

import numpy as np
import pytest
import torch

from mentat_amd.core.paged_kv_cache import PagedKVCacheManager
from mentat_amd.tree_plan import ITEM_FIELDS, WAVES_PER_WG, build_plan, find_segments
from mentat_amd.workloads import replay_tree_ops, tree_ops
from oracle.attention import paged_decode_f64
from oracle.paged_cache import OracleCache


def _host_trees(seed, n_trees=4, prefix=2048, leaves=32, max_private=512, B=16, nb=8192):
    ops = tree_ops(n_trees=n_trees, prefix=prefix, leaves=leaves, max_private=max_private, seed=seed)
    m = PagedKVCacheManager(1, 2, 32, max_blocks=nb, block_size=B, device="cpu", dtype=torch.bfloat16)
    seq, order = replay_tree_ops(m, ops)
    ids = [seq[x] for x in order]
    sts = [m._sequences[s] for s in ids]
    return m, ops, ids, [list(s.page_table[0]) for s in sts], [s.num_tokens[0] for s in sts], [s.row for s in sts]


def test_tree_ops_shapes():
    ops = tree_ops(seed=0)
    final = [op for op in ops if op[0] == "final"][0][1]
    assert len(final) == 4 * 32
    assert sum(op[0] == "fork" for op in ops) == 4 * 31
    assert sum(op[0] == "prefill" for op in ops) == 4


def test_tree_replay_matches_oracle_cache():
    """The workload's page tables and refcounts follow the reference's rules (oracle cache)."""
    ops = tree_ops(n_trees=2, prefix=100, leaves=8, max_private=40, seed=3)
    m = PagedKVCacheManager(1, 2, 32, max_blocks=1024, block_size=16, device="cpu", dtype=torch.bfloat16)
    seq, order = replay_tree_ops(m, ops)
    c = OracleCache(1, 1024, 16)
    cs = {}
    hist = {}  # expected token tags of each leaf
    tag = 0
    for op in ops:
        if op[0] == "alloc":
            cs[op[1]] = c.allocate()
            hist[op[1]] = []
        elif op[0] == "prefill":
            tags = list(range(tag, tag + op[2]))
            tag += op[2]
            c.append(cs[op[1]], 0, tags)
            hist[op[1]] += tags
        elif op[0] == "fork":
            cs[op[2]] = c.fork(cs[op[1]])
            hist[op[2]] = list(hist[op[1]])
        elif op[0] == "step":
            tags = list(range(tag, tag + len(op[1])))
            tag += len(op[1])
            c.append_batched([cs[x] for x in op[1]], 0, tags)
            for x, t in zip(op[1], tags):
                hist[x].append(t)
    for leaf in order:
        assert c.gather(cs[leaf], 0) == hist[leaf]  # every leaf reads its own history
    assert m.allocator.refcounts == c.alloc.refcounts
    for leaf, sid in seq.items():
        assert m._sequences[sid].page_table == c.tables[cs[leaf]]
    # refcount = number of tables holding the block
    holders = {}
    for st in m._sequences.values():
        for b in st.page_table[0]:
            holders[b] = holders.get(b, 0) + 1
    assert all(m.allocator.refcounts[b] == n for b, n in holders.items())


@pytest.mark.parametrize("seed", [0, 1])
def test_segments_partition_each_context(seed):
    m, _, ids, tables, lens, rows = _host_trees(seed)
    B = 16
    segs = find_segments(tables, lens, rows, B)
    covered = [[] for _ in ids]
    for s in segs:
        rep = rows.index(s.row)
        for i in s.members:
            assert tables[i][s.first_page:s.end_page] == tables[rep][s.first_page:s.end_page]
            assert s.end_token <= lens[i]
            covered[i].append((s.first_page * B, s.end_token))
    for i, spans in enumerate(covered):
        spans.sort()
        pos = 0
        for a, b in spans:
            assert a == pos and b > a
            pos = b
        assert pos == lens[i]
    seen = {}
    for t, n in zip(tables, lens):
        for p in range((n + B - 1) // B):
            seen[(t[p], min(B, n - p * B))] = 1
    uniq = sum(v for (_, v) in seen)
    plan = build_plan(tables, lens, rows, block_size=B, Hkv=8, G=4)
    # Sharing is found between neighbours in batch order: a partial page that
    # siblings share around a neighbour which already copied it (it grew one
    # more token) is read once per run of neighbours, a few tokens in all.
    assert uniq <= plan.unique_tokens() <= uniq + B * len(ids) // 16
    assert uniq < 0.5 * sum(lens)  # the 2048-token prompts dominate


@pytest.mark.parametrize("min_groups", [1, 3, 99])
def test_plan_items_and_slots(min_groups):
    m, _, ids, tables, lens, rows = _host_trees(0)
    Hkv, G = 8, 4
    mg = 16 // G
    plan = build_plan(tables, lens, rows, block_size=16, Hkv=Hkv, G=G, chunk_tiles=16,
                      shared_min_groups=min_groups)
    plan.validate(len(ids), Hkv, G, max(rows) + 1, max(len(t) for t in tables), 16)
    it = plan.items
    assert it.shape[1] == ITEM_FIELDS and it.dtype == np.int32
    sh, so = it[: plan.n_shared], it[plan.n_shared:]
    assert (so[:, 5] <= mg).all() and (sh[:, 5] <= WAVES_PER_WG * mg).all()
    if min_groups == 99:
        assert plan.n_shared == 0
    else:
        assert plan.n_shared > 0 and (sh[:, 5] > (min_groups - 1) * mg).all()
    # each slot written exactly once and listed exactly once
    written = np.concatenate([np.arange(a[6], a[6] + a[5]) for a in it])
    assert sorted(written.tolist()) == list(range(plan.n_slots))
    assert sorted(plan.q_slots[: plan.q_slot_offsets[-1]].tolist()) == list(range(plan.n_slots))
    # every (query, head) is covered by its members' items, once per token
    cover = np.zeros((len(ids), Hkv), dtype=np.int64)
    for a in it:
        toks = min(16 * (a[1] + a[2]), a[3]) - 16 * a[1]
        for q in plan.members[a[7]: a[7] + a[5]]:
            cover[q, a[4]] += toks
    assert (cover == np.array(lens)[:, None]).all()


def test_validate_requires_slot_counts_to_match_the_items():
    """The merge reads the slots q_slot_offsets lists for each (query, head):
    validate rejects plans whose items write a different number of slots for
    a unit, and items with members but no tiles (the kernel skips those, so
    their slots would hold stale partials)."""
    m, _, ids, tables, lens, rows = _host_trees(1)
    Hkv, G = 8, 4
    args = (len(ids), Hkv, G, max(rows) + 1, max(len(t) for t in tables), 16)
    plan = build_plan(tables, lens, rows, block_size=16, Hkv=Hkv, G=G)
    plan.validate(*args)
    # a member moved to another query: two units' counts no longer match
    it = plan.items[plan.n_shared]
    moved = plan.members.copy()
    moved[it[7]] = (moved[it[7]] + 1) % len(ids)
    bad = dataclasses.replace(plan, members=moved)
    with pytest.raises(ValueError, match="count the slots"):
        bad.validate(*args)
    # an item with members but no tiles
    zero = plan.items.copy()
    zero[plan.n_shared, 2] = 0
    with pytest.raises(ValueError, match="has no tiles"):
        dataclasses.replace(plan, items=zero).validate(*args)
    # a padding item (no tiles, no members) while its slots stay listed
    pad = plan.items.copy()
    pad[plan.n_shared, 2] = 0
    pad[plan.n_shared, 5] = 0
    with pytest.raises(ValueError, match="count the slots"):
        dataclasses.replace(plan, items=pad).validate(*args)


def _plan_eval_f64(q, kp, vp, tables, rows, plan, B, scale):
    """Follow the plan item by item in float64 (what the two kernels compute)."""
    N, Hq, D = q.shape
    Hkv = kp.shape[2]
    G = Hq // Hkv
    tab = {r: t for r, t in zip(rows, tables)}
    part = {}
    for a in plan.items:
        if a[2] == 0:
            continue
        row, t0, nt, valid, h, nm, s0, moff = (int(x) for x in a[:8])
        toks = [t for t in range(16 * t0, min(16 * (t0 + nt), valid))]
        K = np.stack([kp[tab[row][t // B], t % B, h] for t in toks]).astype(np.float64)
        V = np.stack([vp[tab[row][t // B], t % B, h] for t in toks]).astype(np.float64)
        for j in range(nm):
            qi = int(plan.members[moff + j])
            for g in range(G):
                s = K @ q[qi, h * G + g].astype(np.float64) * scale
                mx = s.max()
                p = np.exp(s - mx)
                part[(s0 + j, g)] = (mx, p.sum(), p @ V)
    out = np.zeros((N, Hq, D))
    for qi in range(N):
        for h in range(Hkv):
            sl = plan.q_slots[plan.q_slot_offsets[qi * Hkv + h]: plan.q_slot_offsets[qi * Hkv + h + 1]]
            for g in range(G):
                ps = [part[(int(s), g)] for s in sl]
                M = max(p[0] for p in ps)
                L = sum(p[1] * np.exp(p[0] - M) for p in ps)
                O = sum(p[2] * np.exp(p[0] - M) for p in ps)
                out[qi, h * G + g] = O / L
    return out


def test_plan_evaluation_matches_oracle_attention():
    ops = tree_ops(n_trees=2, prefix=70, leaves=6, max_private=50, seed=5)
    B, Hkv, G, D, nb = 16, 2, 4, 8, 512
    m = PagedKVCacheManager(1, Hkv, 32, max_blocks=nb, block_size=B, device="cpu", dtype=torch.bfloat16)
    seq, order = replay_tree_ops(m, ops)
    ids = [seq[x] for x in order]
    sts = [m._sequences[s] for s in ids]
    tables = [list(s.page_table[0]) for s in sts]
    lens = [s.num_tokens[0] for s in sts]
    rows = [s.row for s in sts]
    rng = np.random.default_rng(0)
    kp = rng.standard_normal((nb, B, Hkv, D))
    vp = rng.standard_normal((nb, B, Hkv, D))
    q = rng.standard_normal((len(ids), Hkv * G, D))
    want = paged_decode_f64(q, kp, vp, tables, lens, B)
    for min_groups in (1, 2, 99):
        plan = build_plan(tables, lens, rows, block_size=B, Hkv=Hkv, G=G, chunk_tiles=2, shared_chunk_tiles=3,
                          shared_min_groups=min_groups)
        got = _plan_eval_f64(q, kp, vp, tables, rows, plan, B, D ** -0.5)
        assert np.abs(got - want).max() < 1e-9
