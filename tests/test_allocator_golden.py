"""Block ids after set.pop()'s cursor wraps, against the reference's own
allocator: tests/golden/allocator_traces.json holds seeded alloc / ref /
release traces and the ids, free set and refcounts that the reference's
BlockAllocator (core/paged_kv_cache.py:21-72) produced on them
(tests/golden/make_allocator_traces.py). The product allocator and the
oracle's must reproduce every id, past the wrap that the closed-form next-fit
model of oracle.paged_cache.next_fit_order does not cover."""
import json
import os

import pytest

from mentat_amd.core.paged_kv_cache import BlockAllocator
from oracle.paged_cache import OracleAllocator

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "allocator_traces.json")
TRACES = json.load(open(FIXTURE))["traces"]


def _replay(alloc, events):
    out = []
    for ev in events:
        if ev[0] == "a":
            out.append(alloc.alloc())
        elif ev[0] == "r":
            alloc.ref(ev[1])
        else:
            alloc.release(ev[1])
    return out


@pytest.mark.parametrize("i", range(len(TRACES)))
def test_allocators_reproduce_reference_ids_past_the_wrap(i):
    tr = TRACES[i]
    ids = tr["allocs"]
    # the trace wraps: consecutive ids decrease only when the cursor wraps
    assert sum(b < a for a, b in zip(ids, ids[1:])) >= 5
    prod = BlockAllocator(tr["n"])
    assert _replay(prod, tr["events"]) == ids
    assert sorted(prod._free) == tr["free"] and prod.refcounts == tr["refcounts"]
    orc = OracleAllocator(tr["n"])
    assert _replay(orc, tr["events"]) == ids
    assert sorted(orc.free) == tr["free"] and orc.refcounts == tr["refcounts"]
