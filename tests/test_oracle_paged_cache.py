"""Pins the paged-cache oracle (CPU): closed-form id order, invariants, known answers."""
import random

import pytest

from oracle.paged_cache import OracleAllocator, OracleCache, next_fit_order, peak_kv_cache_bytes


def _random_alloc_free_events(n, steps, rng):
    """Alloc/free events driven by a set allocator (ids needed for the frees)."""
    a = OracleAllocator(n)
    used, events, got = [], [], []
    for _ in range(steps):
        if used and (rng.random() < 0.45 or not a.free):
            b = used.pop(rng.randrange(len(used)))
            a.release(b)
            events.append(("f", b))
        else:
            b = a.alloc()
            used.append(b)
            events.append(("a",))
            got.append(b)
    return events, got


@pytest.mark.parametrize("n", [64, 256, 8192])
def test_set_pop_is_next_fit_before_wrap(n):
    rng = random.Random(n)
    for _ in range(5):
        events, got = _random_alloc_free_events(n, 3 * n, rng)
        first = []
        k = 0
        for ev in events:
            if ev[0] == "a":
                k += 1
                if k > n:
                    break
            first.append(ev)
        model = next_fit_order(n, first)
        assert got[: len(model)] == model
        assert model == list(range(len(model)))


def test_allocator_errors():
    a = OracleAllocator(2)
    a.alloc(), a.alloc()
    with pytest.raises(RuntimeError):
        a.alloc()
    with pytest.raises(AssertionError):
        OracleAllocator(3).release(1)
    with pytest.raises(AssertionError):
        OracleAllocator(3).ref(2)


def _check_invariants(c: OracleCache, hist):
    assert sum(c.alloc.refcounts) == c.table_entries()
    assert c.alloc.free == {b for b, r in enumerate(c.alloc.refcounts) if r == 0}
    for sid, layers in hist.items():
        for l in range(c.L):
            assert c.gather(sid, l) == layers[l], (sid, l)


def _random_trace(seed, L=2, nb=4096, B=4, steps=200):
    rng = random.Random(seed)
    c = OracleCache(L, nb, B)
    hist = {}  # sid -> per-layer list of tags
    tag = [0]

    def new_tags(k):
        out = list(range(tag[0], tag[0] + k))
        tag[0] += k
        return out

    for _ in range(steps):
        op = rng.random()
        live = list(hist)
        if not live or op < 0.15:
            sid = c.allocate()
            hist[sid] = [[] for _ in range(L)]
            n = rng.randint(0, 9)
            for l in range(L):
                t = new_tags(n)
                c.append(sid, l, t)
                hist[sid][l] += t
        elif op < 0.35:
            p = rng.choice(live)
            cid = c.fork(p)
            hist[cid] = [list(x) for x in hist[p]]
        elif (op < 0.45 or len(live) > 10) and len(live) > 1:
            sid = rng.choice(live)
            c.free(sid)
            del hist[sid]
        else:
            batch = rng.sample(live, rng.randint(1, len(live)))
            for l in range(L):
                t = new_tags(len(batch))
                c.append_batched(batch, l, t)
                for s, x in zip(batch, t):
                    hist[s][l].append(x)
        _check_invariants(c, hist)
    return c, hist


@pytest.mark.parametrize("seed", range(6))
def test_random_traces_keep_invariants(seed):
    _random_trace(seed)


def test_k_way_branch_copy_pattern():
    # A parent with a partially filled tail branches into K=3 children and is
    # freed; in the next decode append the first K-1 children copy the shared
    # tail, the last one writes in place.
    B = 16
    c = OracleCache(1, 64, B)
    p = c.allocate()
    c.append(p, 0, list(range(21)))  # tail block holds 5 tokens
    tail = c.tables[p][0][-1]
    kids = [c.fork(p) for _ in range(3)]
    c.free(p)
    assert c.alloc.refcounts[tail] == 3
    c.copies.clear()
    dests = c.append_batched(kids, 0, [100, 101, 102])
    assert [src for (_, src, _) in c.copies] == [tail, tail]
    assert dests[2] == (tail, 5)
    assert dests[0][0] != tail and dests[1][0] != tail
    assert c.alloc.refcounts[tail] == 1
    # An EOS child freed before the append removes one sharer.
    c2 = OracleCache(1, 64, B)
    p = c2.allocate()
    c2.append(p, 0, list(range(21)))
    kids = [c2.fork(p) for _ in range(3)]
    c2.free(p)
    c2.free(kids[1])
    c2.copies.clear()
    c2.append_batched([kids[0], kids[2]], 0, [7, 8])
    assert len(c2.copies) == 1
    # A full tail never copies: the first append opens a fresh block.
    c3 = OracleCache(1, 64, B)
    p = c3.allocate()
    c3.append(p, 0, list(range(32)))
    kids = [c3.fork(p) for _ in range(2)]
    c3.free(p)
    c3.copies.clear()
    c3.append_batched(kids, 0, [1, 2])
    assert c3.copies == []


def test_peak_kv_bytes_matches_published_run():
    # The reference's sample run (Qwen3-1.7B: 28 layers, 8 kv heads, head_dim 128,
    # block 16, bf16) reports 1316 peak blocks and 2,414,870,528 peak KV bytes.
    assert peak_kv_cache_bytes(1316, 28, 16, 8, 128, 2) == 2_414_870_528
