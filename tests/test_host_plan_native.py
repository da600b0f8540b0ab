"""The C host planner (mentat_amd/csrc/host_plan.c) against the Python planner (CPU).

Two managers run the same random traces, one through the C planner and one
with it switched off: every plan, page table, counter, refcount, the free
set's iteration order (its pop order), the peak and the host copy of layer 0
must be identical after every operation, including steps whose layers are
not uniform (some layers prefilled separately), copy-on-write of shared tails,
and running out of blocks part-way through a step.
"""
import contextlib
import random

import numpy as np
import pytest
import torch

from mentat_amd.core import paged_kv_cache as pkv
from mentat_amd.core.paged_kv_cache import PagedKVCacheManager

pytestmark = pytest.mark.skipif(pkv._host_plan is None, reason="host planner extension not built")


@contextlib.contextmanager
def _python_planner():
    saved = pkv._host_plan
    pkv._host_plan = None
    try:
        yield
    finally:
        pkv._host_plan = saved


def _same(a: PagedKVCacheManager, b: PagedKVCacheManager):
    assert a.allocator.refcounts == b.allocator.refcounts
    assert list(a.allocator._free) == list(b.allocator._free)   # same set, same table order
    assert a.allocator.peak_used == b.allocator.peak_used
    assert a._sequences.keys() == b._sequences.keys()
    for sid, sa in a._sequences.items():
        sb = b._sequences[sid]
        assert sa.page_table == sb.page_table
        assert sa.num_tokens == sb.num_tokens
        assert sa.tokens_in_last_block == sb.tokens_in_last_block
        assert sa.row == sb.row
    ha, hb = a.host_tables0(), b.host_tables0()
    for sa in a._sequences.values():
        n = len(sa.page_table[0])
        assert ha[sa.row, :n].tolist() == hb[sa.row, :n].tolist() == sa.page_table[0]


def _both(a, b, f):
    """f(manager) on both; results (or the raised error's type and text) must agree."""
    try:
        ra, ea = f(a), None
    except Exception as e:  # noqa: BLE001
        ra, ea = None, e
    with _python_planner():
        try:
            rb, eb = f(b), None
        except Exception as e:  # noqa: BLE001
            rb, eb = None, e
    assert (ea is None) == (eb is None), (ea, eb)
    if ea is not None:
        assert type(ea) is type(eb) and str(ea) == str(eb)
        return None
    if isinstance(ra, np.ndarray):
        assert ra.dtype == rb.dtype and np.array_equal(ra, rb)
    else:
        assert ra == rb
    return ra


@pytest.mark.parametrize("seed", range(8))
def test_native_planner_equals_python_planner(seed):
    rng = random.Random(seed)
    L = rng.choice([1, 2, 5])
    B = rng.choice([4, 16])
    nb = rng.choice([64, 400, 4096])   # small pools run out part-way through steps
    mk = lambda: PagedKVCacheManager(L, 2, 8, max_blocks=nb, block_size=B, device="cpu", dtype=torch.float32)  # noqa: E731
    a, b = mk(), mk()
    exhausted = 0
    for _ in range(120):
        live = list(a._sequences)
        op = rng.random()
        if not live or op < 0.12:
            sid = _both(a, b, lambda m: m.allocate_sequence())
            n = rng.randint(0, 3 * B)
            layers = range(L) if rng.random() < 0.8 else rng.sample(range(L), rng.randint(1, L))  # non-uniform
            for l in layers:
                if _both(a, b, lambda m: m.plan_append(sid, l, n)) is None:
                    exhausted += 1
                    break
        elif op < 0.30:
            p = rng.choice(live)
            if _both(a, b, lambda m: m.fork_sequence(p)) is None:
                exhausted += 1
        elif op < 0.40 and len(live) > 1:
            s = rng.choice(live)
            _both(a, b, lambda m: m.free_sequence(s))
        elif op < 0.55:
            ids = rng.sample(live, rng.randint(1, len(live)))
            l = rng.randrange(L)
            if _both(a, b, lambda m: m.plan_append_batched(ids, l)) is None:
                exhausted += 1
        else:
            ids = rng.sample(live, rng.randint(1, len(live)))
            first = rng.randint(1, L)

            def step(m):
                st = m.plan_append_step_begin(ids, first)
                head = st["plan"][:first].copy()
                return np.concatenate([head, m.plan_append_step_finish(st)])

            if _both(a, b, step) is None:
                exhausted += 1
        _same(a, b)
        if len(a._sequences) > 24:
            for s in rng.sample(list(a._sequences), 8):
                _both(a, b, lambda m: m.free_sequence(s))
    if nb == 64:
        assert exhausted > 0


def test_native_step_reports_uniform_like_python():
    L, B = 4, 4
    mk = lambda: PagedKVCacheManager(L, 2, 8, max_blocks=256, block_size=B, device="cpu", dtype=torch.float32)  # noqa: E731
    a, b = mk(), mk()
    for m in (a, b):
        ctx = _python_planner() if m is b else contextlib.nullcontext()
        with ctx:
            s0 = m.allocate_sequence()
            for l in range(L):
                m.plan_append(s0, l, 6)
            m.fork_sequence(s0)
            s2 = m.allocate_sequence()
            m.plan_append(s2, 0, 3)   # only layer 0: not uniform
    for ids in ([0, 1], [0, 1, 2]):
        sa = a.plan_append_step_begin(ids, 2)
        with _python_planner():
            sb = b.plan_append_step_begin(ids, 2)
        assert sa["uniform"] == sb["uniform"] == (2 not in ids)
        assert "native" in sa and "native" not in sb
        pa = a.plan_append_step_finish(sa)
        with _python_planner():
            pb = b.plan_append_step_finish(sb)
        assert np.array_equal(pa, pb)
        _same(a, b)


def test_native_planner_declines_foreign_objects():
    """Lists replaced by other sequences types: the C planner returns None
    before touching anything, and the Python planner runs."""
    m = PagedKVCacheManager(2, 2, 8, max_blocks=64, block_size=4, device="cpu", dtype=torch.float32)
    s = m.allocate_sequence()
    for l in range(2):
        m.plan_append(s, l, 3)
    seq = m._sequences[s]
    seq.num_tokens = tuple(seq.num_tokens)   # not a list
    free_before = list(m.allocator._free)
    plan = np.empty((7, 1), dtype=np.int32)
    assert pkv._host_plan.append_batched([seq], 0, 4, m.allocator, plan) is None
    assert list(m.allocator._free) == free_before
    seq.num_tokens = list(seq.num_tokens)
    got = m.plan_append_batched([s], 0)
    assert got[5, 0] == 4 and seq.num_tokens == [4, 3]
