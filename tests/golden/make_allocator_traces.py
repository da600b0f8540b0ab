"""Writes allocator_traces.json: the block ids that the reference's
BlockAllocator (core/paged_kv_cache.py:21-72, a Python ``set`` popped for
every allocation) hands out on seeded alloc / ref / release traces that run
long enough for ``set.pop()``'s cursor to wrap round the table many times.

Run only where the reference sources are readable (the build container):
    python tests/golden/make_allocator_traces.py /root/reference
The fixture holds inputs (the event sequence) and outputs (allocated ids,
final free set and refcounts); no reference code is copied into it.
"""
import json
import os
import random
import sys


def trace(BlockAllocator, n: int, ops: int, seed: int) -> dict:
    rng = random.Random(seed)
    a = BlockAllocator(n)
    held: list[int] = []  # one entry per outstanding reference
    events, allocs = [], []
    for _ in range(ops):
        r = rng.random()
        if held and (r < 0.45 or a.num_free == 0):
            b = held.pop(rng.randrange(len(held)))
            a.release(b)
            events.append(["f", b])
        elif held and r < 0.55:
            b = rng.choice(held)
            a.ref(b)
            held.append(b)
            events.append(["r", b])
        else:
            b = a.alloc()
            held.append(b)
            events.append(["a"])
            allocs.append(b)
    return {"n": n, "seed": seed, "events": events, "allocs": allocs, "free": sorted(a._free),
            "refcounts": list(a.refcounts)}


def main() -> None:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from core.paged_kv_cache import BlockAllocator  # the reference's allocator

    traces = [trace(BlockAllocator, n, ops, seed)
              for n, ops, seed in ((16, 2000, 1), (100, 3000, 2), (1000, 4000, 3))]
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "allocator_traces.json")
    with open(out, "w") as f:
        json.dump({"source": "core/paged_kv_cache.py:21-72 BlockAllocator", "traces": traces}, f,
                  separators=(",", ":"))
    print(f"wrote {out}: {[len(t['allocs']) for t in traces]} allocations")


if __name__ == "__main__":
    main()
