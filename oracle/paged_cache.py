"""Oracle: paged KV-cache bookkeeping (test infrastructure only).

Restates core/paged_kv_cache.py of the reference on plain Python/numpy:
  * ``OracleAllocator``        BlockAllocator (:21-72): list refcounts, a ``set``
                               free list popped with ``set.pop()``, peak tracking,
                               RuntimeError when empty, AssertionError on ref/release
                               of a free block.
  * ``OracleCache.allocate`` / ``fork`` / ``free``   (:143-176)
  * ``OracleCache.append``      append_tokens, prefill (:178-225)
  * ``OracleCache.append_batched``  append_tokens_batched, decode (:227-284)
  * ``OracleCache.gather``      build_packed_kv's gather order (:289-368)
  * ``OracleCache.trim_to_window``  sliding-window eviction (:370-417)
  * ``peak_kv_cache_bytes``     get_stats' formula (:419-439)

Instead of K/V tensors the pools hold integer *tags* (one per written token,
per layer), so a test can check exactly which token each slot holds after
copy-on-write, fork and free.

Pinned by (tests/test_oracle_paged_cache.py): the closed-form next-fit order
of ``set.pop()`` before the first wrap-around of the id range; refcount
conservation (sum of refcounts == number of table entries over all
(sequence, layer)); free set == ids with refcount 0; every sequence's gathered
tags equal its own token history (a fork inherits the history at fork time);
the K-way branch consequence (first K-1 children in batch order copy, the
last writes in place); the peak_kv_cache_bytes figure of the reference's
published run (1316 blocks -> 2,414,870,528 bytes for Qwen3-1.7B).
trim_to_window (tests/test_trim_to_window.py): the states and tags the
reference's own manager recorded on scripted scenarios
(tests/golden/trim_to_window.json), and, where eviction is page-aligned, the
closed form gather == the last `window` tokens of the history.
"""
from __future__ import annotations

import numpy as np


class OracleAllocator:
    """core/paged_kv_cache.py:21-72."""

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self.refcounts = [0] * num_blocks
        self.free = set(range(num_blocks))
        self.peak = 0

    def alloc(self) -> int:
        if not self.free:  # :46-50
            raise RuntimeError("out of blocks")
        b = self.free.pop()  # :51
        self.refcounts[b] = 1
        self.peak = max(self.peak, self.num_blocks - len(self.free))
        return b

    def ref(self, b: int) -> None:  # :58-60
        assert self.refcounts[b] > 0
        self.refcounts[b] += 1

    def release(self, b: int) -> None:  # :62-66
        assert self.refcounts[b] > 0
        self.refcounts[b] -= 1
        if self.refcounts[b] == 0:
            self.free.add(b)

    def is_shared(self, b: int) -> bool:  # :68-69
        return self.refcounts[b] > 1


class OracleCache:
    """Bookkeeping + tag pools of the reference manager (no tensors)."""

    def __init__(self, num_layers: int, max_blocks: int, block_size: int):
        self.L = num_layers
        self.B = block_size
        self.alloc = OracleAllocator(max_blocks)
        # pool[l][blk][slot] = tag of the token stored there (-1: never written)
        self.pool = np.full((num_layers, max_blocks, block_size), -1, dtype=np.int64)
        self.tables: dict[int, list[list[int]]] = {}
        self.ntok: dict[int, list[int]] = {}
        self.tilb: dict[int, list[int]] = {}
        self.next_id = 0
        self.copies: list[tuple] = []  # (layer, src, dst) of every copy-on-write

    # :143-150
    def allocate(self) -> int:
        sid = self.next_id
        self.next_id += 1
        self.tables[sid] = [[] for _ in range(self.L)]
        self.ntok[sid] = [0] * self.L
        self.tilb[sid] = [0] * self.L
        return sid

    # :152-170
    def fork(self, pid: int) -> int:
        cid = self.next_id
        self.next_id += 1
        self.tables[cid] = []
        for layer_blocks in self.tables[pid]:
            self.tables[cid].append(list(layer_blocks))
            for b in layer_blocks:
                self.alloc.ref(b)
        self.ntok[cid] = list(self.ntok[pid])
        self.tilb[cid] = list(self.tilb[pid])
        return cid

    # :172-176
    def free(self, sid: int) -> None:
        tables = self.tables.pop(sid)
        self.ntok.pop(sid)
        self.tilb.pop(sid)
        for layer_blocks in tables:
            for b in layer_blocks:
                self.alloc.release(b)

    def _new_tail_if_needed(self, sid: int, layer: int) -> int:
        table = self.tables[sid][layer]
        if not table or self.tilb[sid][layer] == self.B:  # :190 / :251
            table.append(self.alloc.alloc())
            self.tilb[sid][layer] = 0
        tail = table[-1]
        if self.alloc.is_shared(tail):  # :199-209 / :258-265
            new = self.alloc.alloc()
            self.pool[layer, new] = self.pool[layer, tail]  # whole-block copy_
            self.copies.append((layer, tail, new))
            self.alloc.release(tail)
            table[-1] = new
            tail = new
        return tail

    # :178-225
    def append(self, sid: int, layer: int, tags: list[int]) -> None:
        written = 0
        n = len(tags)
        while written < n:
            tail = self._new_tail_if_needed(sid, layer)
            start = self.tilb[sid][layer]
            k = min(self.B - start, n - written)
            self.pool[layer, tail, start:start + k] = tags[written:written + k]
            written += k
            self.tilb[sid][layer] += k
        self.ntok[sid][layer] += n

    # :227-284
    def append_batched(self, sids: list[int], layer: int, tags: list[int]) -> list[tuple]:
        dests = []
        for sid in sids:
            tail = self._new_tail_if_needed(sid, layer)
            slot = self.tilb[sid][layer]
            dests.append((tail, slot))
            self.tilb[sid][layer] += 1
            self.ntok[sid][layer] += 1
        for (blk, slot), tag in zip(dests, tags):  # the vectorised scatter (:283-284)
            self.pool[layer, blk, slot] = tag
        return dests

    # :289-368 (gather order only)
    def gather(self, sid: int, layer: int) -> list[int]:
        out = []
        rem = self.ntok[sid][layer]
        for b in self.tables[sid][layer]:
            if rem == 0:
                break
            k = min(self.B, rem)
            out.extend(self.pool[layer, b, :k].tolist())
            rem -= k
        return out

    # :370-417
    def trim_to_window(self, sid: int, window: int) -> None:
        """Evict all but the last `window` tokens. Whole pages at the front are
        released; a partially evicted front page has its kept slots moved to
        the front (in place when private, into a newly allocated page when
        shared), and later pages are left where they are, exactly as the
        reference does. The counters become `window`."""
        if self.ntok[sid][0] <= window:  # :373-374 (layer 0 decides)
            return
        for layer in range(self.L):
            remaining = self.ntok[sid][layer] - window
            table = self.tables[sid][layer]
            while remaining > 0 and table:
                blk = table[0]
                n_in = min(self.B, remaining)
                if n_in >= self.B:
                    table.pop(0)
                    self.alloc.release(blk)
                    remaining -= self.B
                    continue
                keep = self.B - n_in
                if self.alloc.is_shared(blk):
                    new = self.alloc.alloc()
                    self.pool[layer, new, :keep] = self.pool[layer, blk, n_in:n_in + keep]
                    self.alloc.release(blk)
                    table[0] = new
                else:
                    self.pool[layer, blk, :keep] = self.pool[layer, blk, n_in:n_in + keep].copy()
                remaining = 0
            self.ntok[sid][layer] = window
            self.tilb[sid][layer] = 0 if window == 0 else (window % self.B or self.B)

    def table_entries(self) -> int:
        return sum(len(t) for tables in self.tables.values() for t in tables)


def peak_kv_cache_bytes(blocks_peak: int, num_layers: int, block_size: int, kv_heads: int, head_dim: int,
                        elem_bytes: int) -> int:
    """get_stats' figure (core/paged_kv_cache.py:425-427, 438): counts every layer per block id."""
    return 2 * num_layers * block_size * kv_heads * head_dim * elem_bytes * blocks_peak


def next_fit_order(n: int, events: list) -> list[int]:
    """Closed-form model of ``set(range(n)).pop()`` before the first wrap:
    the lowest free id at or above a cursor that only moves forward.

    ``events``: sequence of ('a',) / ('f', id). Returns the allocated ids;
    valid while the cursor has not passed n - 1.
    """
    free = [True] * n
    cur = 0
    out = []
    for ev in events:
        if ev[0] == "a":
            while cur < n and not free[cur]:
                cur += 1
            if cur >= n:
                raise ValueError("wrap-around: the closed form no longer applies")
            free[cur] = False
            out.append(cur)
            cur += 1
        else:
            free[ev[1]] = True
    return out
