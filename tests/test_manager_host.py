"""Host bookkeeping of the product PagedKVCacheManager vs the oracle (CPU).

Block ids, refcounts, free sets, page tables and counters must be bit-exact
after every operation, and the device plans the manager emits must name the
same destinations and copy-on-write sources as the oracle.
"""
import random

import numpy as np
import pytest
import torch

from mentat_amd.core.paged_kv_cache import BlockAllocator, PagedKVCacheManager
from oracle.paged_cache import OracleCache


def _same_state(m: PagedKVCacheManager, c: OracleCache):
    assert m.allocator.refcounts == c.alloc.refcounts
    assert m.allocator._free == c.alloc.free
    assert m.allocator.peak_used == c.alloc.peak
    assert set(m._sequences) == set(c.tables)
    h0 = m.host_tables0()
    for sid, st in m._sequences.items():
        assert st.page_table == c.tables[sid]
        assert st.num_tokens == c.ntok[sid]
        assert st.tokens_in_last_block == c.tilb[sid]
        # the host copy of layer 0's rows that the tree planner reads
        assert h0[st.row, :len(st.page_table[0])].tolist() == st.page_table[0]


@pytest.mark.parametrize("seed", range(5))
def test_manager_bookkeeping_matches_oracle(seed):
    rng = random.Random(seed)
    L, nb, B = 3, 2048, 8
    m = PagedKVCacheManager(L, 2, 16, max_blocks=nb, block_size=B, device="cpu", dtype=torch.float32)
    c = OracleCache(L, nb, B)
    for _ in range(150):
        live = list(c.tables)
        op = rng.random()
        if not live or op < 0.15:
            sa, sb = m.allocate_sequence(), c.allocate()
            assert sa == sb
            n = rng.randint(0, 20)
            for l in range(L):
                plan = m.plan_append(sa, l, n)
                c.copies.clear()
                c.append(sb, l, list(range(n)))
                assert plan.shape == (7, n)
                if n:
                    cows = [int(x) for x in plan[2] if x >= 0]
                    assert cows == [src for (_, src, _) in c.copies]
                    assert plan[5, -1] == c.ntok[sb][l] and (plan[5, :-1] == -1).all()
                    assert (plan[6] == np.arange(n)).all()
        elif op < 0.35:
            p = rng.choice(live)
            assert m.fork_sequence(p) == c.fork(p)
        elif (op < 0.45 or len(live) > 12) and len(live) > 1:
            s = rng.choice(live)
            m.free_sequence(s)
            c.free(s)
        else:
            batch = rng.sample(live, rng.randint(1, len(live)))
            for l in range(L):
                plan = m.plan_append_batched(batch, l)
                c.copies.clear()
                dests = c.append_batched(batch, l, list(range(len(batch))))
                assert [(int(b), int(s)) for b, s in zip(plan[0], plan[1])] == dests
                cows = [int(x) for x in plan[2] if x >= 0]
                assert cows == [src for (_, src, _) in c.copies]
                rows = [m._sequences[s].row for s in batch]
                assert plan[3].tolist() == rows
                assert plan[4].tolist() == [len(m._sequences[s].page_table[l]) - 1 for s in batch]
                assert plan[5].tolist() == [m._sequences[s].num_tokens[l] for s in batch]
        _same_state(m, c)
        # live rows are distinct
        rows = [st.row for st in m._sequences.values()]
        assert len(rows) == len(set(rows))


def test_errors_match_reference_types():
    a = BlockAllocator(1)
    a.alloc()
    with pytest.raises(RuntimeError):
        a.alloc()
    with pytest.raises(AssertionError):
        BlockAllocator(2).release(0)
    m = PagedKVCacheManager(1, 1, 32, max_blocks=4, block_size=16, device="cpu", dtype=torch.float32)
    with pytest.raises(KeyError):
        m.free_sequence(123)
    with pytest.raises(KeyError):
        m.fork_sequence(5)


def test_stats_keys_and_formula():
    m = PagedKVCacheManager(28, 8, 128, max_blocks=64, block_size=16, device="cpu", dtype=torch.bfloat16)
    s = m.allocate_sequence()
    m.plan_append(s, 0, 40)
    st = m.get_stats()
    for k in ("num_sequences", "total_cached_tokens", "blocks_used", "blocks_free", "blocks_total",
              "blocks_peak", "utilization", "peak_utilization", "pool_memory_bytes", "peak_kv_cache_bytes"):
        assert k in st
    assert st["blocks_peak"] == 3
    assert st["peak_kv_cache_bytes"] == 3 * 1_835_008
    assert st["peak_kv_cache_bytes_true"] == 3 * 1_835_008 // 28


def test_pool_views_have_reference_shape():
    for dt, layout_native in ((torch.bfloat16, True), (torch.float32, False)):
        m = PagedKVCacheManager(2, 4, 64, max_blocks=8, block_size=16, device="cpu", dtype=dt)
        assert tuple(m.k_pools[1].shape) == (8, 16, 4, 64)
        assert tuple(m.v_pools[0].shape) == (8, 16, 4, 64)
        assert (m.layout == 1) == layout_native
        # one store for all layers: a block id is owned by one layer at a time,
        # so every layer's view of a page is the same memory
        m.k_pools[1][3, 5, 2] = 7.0
        assert float(m.k_pools[1][3, 5, 2, 0]) == 7.0 and float(m.k_pools[0][3, 5, 2, 0]) == 7.0
        assert float(m.k_pools[0].abs().sum()) == 7.0 * 64
        st = m.get_stats()
        assert st["pool_memory_bytes_true"] * 2 == st["pool_memory_bytes"]


def test_block_ids_are_owned_by_one_layer():
    """The invariant that lets all layers share one store: at every point of a
    random trace of allocate / fork / append / free, no block id is in the
    tables of two different layers."""
    rng = random.Random(5)
    L, nb, B = 4, 4096, 8
    m = PagedKVCacheManager(L, 2, 16, max_blocks=nb, block_size=B, device="cpu", dtype=torch.float32)
    for _ in range(300):
        live = list(m._sequences)
        op = rng.random()
        if not live or op < 0.15:
            sid = m.allocate_sequence()
            for layer in range(L):
                m.plan_append(sid, layer, rng.randint(0, 20))
        elif op < 0.35:
            m.fork_sequence(rng.choice(live))
        elif op < 0.5 and len(live) > 1:
            m.free_sequence(rng.choice(live))
        else:
            ids = rng.sample(live, rng.randint(1, len(live)))
            for layer in range(L):
                m.plan_append_batched(ids, layer)
        owner = {}
        for st in m._sequences.values():
            for layer, table in enumerate(st.page_table):
                for b in table:
                    assert owner.setdefault(b, layer) == layer


def test_find_blocked_tokens_closed_forms():
    from mentat_amd.core.generator_utils import _find_blocked_tokens

    assert _find_blocked_tokens([], 3) == set()
    assert _find_blocked_tokens([5], 3) == set()
    # bigram: last token 1 occurred at 0 and 2, followed by 2 and 3
    assert _find_blocked_tokens([1, 2, 1, 3, 1], 2) == {2, 3}
    # trigram adds what followed "3 1"? "3 1" occurs only at the end -> nothing more
    assert _find_blocked_tokens([1, 2, 1, 3, 1], 3) == {2, 3}
    # "1 2" repeated: trigram blocks the 7 that followed the first "1 2"
    assert _find_blocked_tokens([1, 2, 7, 1, 2], 3) == {7}
    rng = random.Random(0)
    for _ in range(50):  # brute force over every earlier window
        ids = [rng.randint(0, 3) for _ in range(rng.randint(0, 12))]
        mx = rng.randint(2, 4)
        want = set()
        for n in range(2, mx + 1):
            for i in range(len(ids) - n + 1):
                if len(ids) >= n and ids[i:i + n - 1] == ids[len(ids) - n + 1:]:
                    want.add(ids[i + n - 1])
        assert _find_blocked_tokens(ids, mx) == want


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("first_layers", [0, 2, 5])
def test_plan_append_step_equals_layer_by_layer_plans(seed, first_layers):
    """One decode step planned for all layers at once (plan_append_step, or its
    two halves with the first `first_layers` layers planned before the rest;
    0: the one-call form) gives the plans, block ids, refcounts, free set and
    counters of plan_append_batched called layer by layer, on random traces
    with forks (shared tails, so copy-on-write), frees and page boundaries; the
    oracle checks the same."""
    rng = random.Random(100 + seed)
    L, nb, B = 5, 4096, 4
    step = PagedKVCacheManager(L, 2, 16, max_blocks=nb, block_size=B, device="cpu", dtype=torch.float32)
    ref = PagedKVCacheManager(L, 2, 16, max_blocks=nb, block_size=B, device="cpu", dtype=torch.float32)
    c = OracleCache(L, nb, B)
    n_steps = 0
    for _ in range(200):
        live = list(c.tables)
        op = rng.random()
        if not live or op < 0.12:
            n = rng.randint(0, 9)
            sa, sb, sc = step.allocate_sequence(), ref.allocate_sequence(), c.allocate()
            for l in range(L):
                step.plan_append(sa, l, n)
                ref.plan_append(sb, l, n)
                c.append(sc, l, list(range(n)))
        elif op < 0.35:
            p = rng.choice(live)
            for _k in range(rng.randint(1, 3)):
                assert step.fork_sequence(p) == ref.fork_sequence(p) == c.fork(p)
            if rng.random() < 0.5 and len(live) > 1:  # the branch parent is freed after its forks
                step.free_sequence(p)
                ref.free_sequence(p)
                c.free(p)
        elif op < 0.45 and len(live) > 1:
            s = rng.choice(live)
            step.free_sequence(s)
            ref.free_sequence(s)
            c.free(s)
        else:
            batch = rng.sample(live, rng.randint(1, len(live)))
            if first_layers:
                st = step.plan_append_step_begin(batch, first_layers)
                head = st["plan"][:first_layers].copy()
                got = step.plan_append_step_finish(st)
                assert (got[:first_layers] == head).all()   # the first layers were final
            else:
                got = step.plan_append_step(batch)
            want = np.stack([ref.plan_append_batched(batch, l) for l in range(L)])
            for l in range(L):
                c.append_batched(batch, l, list(range(len(batch))))
            assert got.dtype == np.int32 and got.shape == (L, 7, len(batch))
            assert (got == want).all()
            n_steps += 1
        assert step.allocator.refcounts == ref.allocator.refcounts
        assert step.allocator._free == ref.allocator._free
        for sid, st in step._sequences.items():
            rt = ref._sequences[sid]
            assert (st.page_table, st.num_tokens, st.tokens_in_last_block) == \
                (rt.page_table, rt.num_tokens, rt.tokens_in_last_block)
        _same_state(step, c)
    assert n_steps > 40


def test_plan_append_step_non_uniform_layers_fall_back():
    """Layers appended unevenly (not what decode, prefill or fork do) take the
    layer-by-layer path and still match it exactly."""
    L, B = 3, 4
    step = PagedKVCacheManager(L, 2, 16, max_blocks=256, block_size=B, device="cpu", dtype=torch.float32)
    ref = PagedKVCacheManager(L, 2, 16, max_blocks=256, block_size=B, device="cpu", dtype=torch.float32)
    for m in (step, ref):
        a = m.allocate_sequence()
        for l in range(L):
            m.plan_append(a, l, 5 + l)  # different lengths per layer
        m.fork_sequence(a)
    got = step.plan_append_step([0, 1])
    want = np.stack([ref.plan_append_batched([0, 1], l) for l in range(L)])
    assert (got == want).all()
    assert step.allocator.refcounts == ref.allocator.refcounts


@pytest.mark.parametrize("first_layers", [1, 2, 4])
def test_plan_append_step_mixes_replay_and_layer_plans(first_layers):
    """Equal counters in every layer but one layer whose tail is no longer
    shared (its tail re-pointed at a private copy by hand): that layer is
    planned on its own, the others replay layer 0, and the result is still the
    layer-by-layer plans, ids and refcounts."""
    L, B = 4, 4
    mgrs = [PagedKVCacheManager(L, 2, 16, max_blocks=256, block_size=B, device="cpu", dtype=torch.float32)
            for _ in range(2)]
    for m in mgrs:
        a = m.allocate_sequence()
        for l in range(L):
            m.plan_append(a, l, 6)
        b = m.fork_sequence(a)
        sb = m._sequences[b]
        old = sb.page_table[2][-1]
        new = m.allocator.alloc()
        m.allocator.release(old)
        sb.page_table[2][-1] = new
    step, ref = mgrs
    st = step.plan_append_step_begin([0, 1], first_layers)
    got = step.plan_append_step_finish(st)
    want = np.stack([ref.plan_append_batched([0, 1], l) for l in range(L)])
    assert (got == want).all()
    assert step.allocator.refcounts == ref.allocator.refcounts
    assert step.allocator._free == ref.allocator._free
    for sid in (0, 1):
        s, r = step._sequences[sid], ref._sequences[sid]
        assert (s.page_table, s.num_tokens, s.tokens_in_last_block) == (r.page_table, r.num_tokens,
                                                                         r.tokens_in_last_block)
