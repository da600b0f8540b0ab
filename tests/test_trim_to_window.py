"""trim_to_window (core/paged_kv_cache.py:370-417) on the CPU: the oracle and
the product manager's host bookkeeping against what the reference's own
manager recorded on scripted scenarios (tests/golden/trim_to_window.json,
written by tests/golden/make_trim_vectors.py), and the oracle against the
closed form of page-aligned eviction.

The reference moves only the kept slots of a partially evicted front page to
its front and leaves the later pages where they are, so after such a trim the
gather reads some slots twice and misses others; the vectors record that, and
both the oracle and the product reproduce it."""
import json
import os
import random

import numpy as np
import pytest
import torch

from mentat_amd.core.paged_kv_cache import PagedKVCacheManager
from oracle.paged_cache import OracleCache

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "trim_to_window.json")))
L, NB, OFF = GOLD["num_layers"], GOLD["max_blocks"], GOLD["tag_layer_offset"]
CASES = sorted(GOLD["cases"])


def _replay_oracle(case):
    B = case["block_size"]
    c = OracleCache(L, NB, B)
    tag = 0
    for rec in case["steps"]:
        op = rec["step"]
        if op[0] == "alloc":
            c.allocate()
        elif op[0] == "fork":
            c.fork(op[1])
        elif op[0] == "free":
            c.free(op[1])
        elif op[0] == "prefill":
            ts = list(range(tag + 1, tag + 1 + op[2]))
            tag += op[2]
            for layer in range(L):
                c.append(op[1], layer, [t + OFF * layer for t in ts])
        elif op[0] == "decode":
            ts = list(range(tag + 1, tag + 1 + len(op[1])))
            tag += len(op[1])
            for layer in range(L):
                c.append_batched(list(op[1]), layer, [t + OFF * layer for t in ts])
        elif op[0] == "trim":
            c.trim_to_window(op[1], op[2])
        yield rec, c


@pytest.mark.parametrize("name", CASES)
def test_oracle_trim_matches_reference_vectors(name):
    case = GOLD["cases"][name]
    c = None
    for rec, c in _replay_oracle(case):
        st = rec["state"]
        assert c.alloc.refcounts == st["refcounts"], rec["step"]
        assert sorted(c.alloc.free) == st["free"], rec["step"]
        assert sorted(c.tables) == sorted(int(s) for s in st["seqs"])
        for sid, want in st["seqs"].items():
            sid = int(sid)
            assert c.tables[sid] == want["page_table"], (rec["step"], sid)
            assert c.ntok[sid] == want["num_tokens"], (rec["step"], sid)
            assert c.tilb[sid] == want["tokens_in_last_block"], (rec["step"], sid)
            for layer in range(L):
                got = [max(t, 0) for t in c.gather(sid, layer)]  # never-written slots hold 0 in the reference
                assert got == want["gather"][layer], (rec["step"], sid, layer)
    assert np.array_equal(np.maximum(c.pool, 0).reshape(L, NB, -1), np.array(case["k_pools"]))


def test_vectors_cover_every_trim_branch():
    """Between them the scenarios evict whole pages, shift a private front
    page, copy a shared front page, trim to zero and leave a short sequence
    alone."""
    seen = set()
    for name in CASES:
        case = GOLD["cases"][name]
        prev = None
        for rec in case["steps"]:
            op = rec["step"]
            if op[0] == "trim" and prev is not None:
                sid, w = str(op[1]), op[2]
                before, after = prev["seqs"][sid], rec["state"]["seqs"][sid]
                B = case["block_size"]
                evict = before["num_tokens"][0] - w
                if evict <= 0:
                    seen.add("noop")
                    assert after == before
                    continue
                if w == 0:
                    seen.add("zero")
                if evict % B == 0:
                    seen.add("aligned")
                else:
                    front = before["page_table"][0][evict // B]
                    shared = prev["refcounts"][front] > 1
                    seen.add("shared_partial" if shared else "private_partial")
                    assert (after["page_table"][0][0] != front) == shared
            prev = rec["state"]
    assert seen == {"noop", "zero", "aligned", "shared_partial", "private_partial"}


@pytest.mark.parametrize("seed", range(6))
def test_oracle_page_aligned_trim_keeps_the_last_window_tokens(seed):
    """Evicting a whole number of pages leaves exactly the last `window`
    tokens of the history, in order, and releases exactly the evicted pages."""
    rng = random.Random(seed)
    B = rng.choice([4, 8, 16])
    c = OracleCache(2, 256, B)
    sid = c.allocate()
    n = rng.randint(2 * B, 6 * B)
    hist = list(range(1, n + 1))
    for layer in range(2):
        c.append(sid, layer, [t + 1000 * layer for t in hist])
    pages = (n - 1) // B  # pages that can go while keeping at least one token
    k = rng.randint(1, pages)
    w = n - k * B
    before = [list(t) for t in c.tables[sid]]
    c.trim_to_window(sid, w)
    for layer in range(2):
        assert c.gather(sid, layer) == [t + 1000 * layer for t in hist[-w:]]
        assert c.tables[sid][layer] == before[layer][k:]
        for b in before[layer][:k]:
            assert c.alloc.refcounts[b] == 0 and b in c.alloc.free
    assert c.ntok[sid] == [w, w]


@pytest.mark.parametrize("name", CASES)
def test_product_trim_bookkeeping_matches_reference_vectors(name):
    """The product manager's host half (block ids, refcounts, free set, page
    tables, counters) on the CPU, its appends planned but not written."""
    case = GOLD["cases"][name]
    B = case["block_size"]
    m = PagedKVCacheManager(L, 1, 16, max_blocks=NB, block_size=B, device="cpu", dtype=torch.float32)
    for rec in case["steps"]:
        op = rec["step"]
        if op[0] == "alloc":
            m.allocate_sequence()
        elif op[0] == "fork":
            m.fork_sequence(op[1])
        elif op[0] == "free":
            m.free_sequence(op[1])
        elif op[0] == "prefill":
            for layer in range(L):
                m.plan_append(op[1], layer, op[2])
        elif op[0] == "decode":
            for layer in range(L):
                m.plan_append_batched(list(op[1]), layer)
        elif op[0] == "trim":
            m.trim_to_window(op[1], op[2])
        st = rec["state"]
        assert m.allocator.refcounts == st["refcounts"], op
        assert sorted(m.allocator._free) == st["free"], op
        assert sorted(m._sequences) == sorted(int(s) for s in st["seqs"])
        for sid, want in st["seqs"].items():
            seq = m._sequences[int(sid)]
            assert seq.page_table == want["page_table"], (op, sid)
            assert seq.num_tokens == want["num_tokens"], (op, sid)
            assert seq.tokens_in_last_block == want["tokens_in_last_block"], (op, sid)
