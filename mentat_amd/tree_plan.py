"""Host plan for the prefix-tree decode kernel (mentat_tree_decode).

The decode batch's contexts are split into segments: maximal runs of pages
that a set of sequences reaches through the same block ids (with the same
number of valid tokens), i.e. the edges of the prefix tree the batch forms —
a shared prompt, internal branches, each leaf's private tail. The sharing
structure is the same in every layer (forks, frees and copy-on-write treat all
layers alike; only the block ids differ), so a plan is built once per decode
step from layer 0's tables and reused by every layer: a segment names a
representative table row and the kernel reads that layer's ids from it.

Work: each segment is cut into chunks of 16-token tiles and each (chunk, kv
head) gets its members' queries in groups of 16 / G (one MFMA query tile;
G = query heads per kv head). A chunk with at least ``shared_min_groups``
groups becomes a shared task (one workgroup stages the chunk's pages in LDS
once, up to WAVES_PER_WG groups on its wavefronts); other chunks become solo
items, one wavefront per group, reading the pages directly. Every (member,
chunk, head) gets a partial slot; ``q_slot_offsets`` / ``q_slots`` list each
(query, head)'s slots for the merge.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

ITEM_FIELDS = 8
WAVES_PER_WG = 8
SHARED_MAX_TILES = 32  # tiles per shared task (the kernel's unrolled tile loop)


@dataclass
class Segment:
    first_page: int
    end_page: int          # exclusive
    end_token: int         # exclusive absolute token index
    members: list          # batch indices
    row: int               # representative table row
    block_size: int

    @property
    def tokens(self) -> int:
        return self.end_token - self.first_page * self.block_size


@dataclass
class TreePlan:
    items: np.ndarray          # int32 [n_shared + n_solo, ITEM_FIELDS]
    n_shared: int
    members: np.ndarray        # int32 member query indices (items point into it)
    q_slot_offsets: np.ndarray  # int32 [N * Hkv + 1]
    q_slots: np.ndarray        # int32 [n_slots]
    n_slots: int
    segments: list

    @property
    def n_solo(self) -> int:
        return self.items.shape[0] - self.n_shared

    def unique_tokens(self) -> int:
        """Distinct cached token positions the batch reads (the same count in every layer)."""
        return sum(s.tokens for s in self.segments)

    def validate(self, Nq: int, Hkv: int, G: int, rows: int, table_stride: int, block_size: int) -> None:
        """Host check that every index the kernels take from the plan is in bounds."""
        it = self.items
        if it.ndim != 2 or it.shape[1] != ITEM_FIELDS or it.dtype != np.int32:
            raise ValueError("items must be int32 [n, %d]" % ITEM_FIELDS)
        if not 0 <= self.n_shared <= it.shape[0]:
            raise ValueError("n_shared out of range")
        off, qs = self.q_slot_offsets, self.q_slots
        if off.shape != (Nq * Hkv + 1,) or off[0] != 0 or np.any(np.diff(off) < 0) or off[-1] > qs.size:
            raise ValueError("q_slot_offsets is not a CSR offset array over Nq * Hkv (query, head) pairs")
        if off[-1] and (qs[: off[-1]].min() < 0 or qs[: off[-1]].max() >= self.n_slots):
            raise ValueError("q_slots names a slot outside [0, n_slots)")
        mem = self.members
        if mem.dtype != np.int32 or mem.ndim != 1:
            raise ValueError("members must be int32 [n]")
        live = it[:, 2] > 0
        if not live.any():
            return
        a = it[live]
        mg = 16 // G
        cap = np.where(np.arange(it.shape[0])[live] < self.n_shared, WAVES_PER_WG * mg, mg)
        if np.any((a[:, 0] < 0) | (a[:, 0] >= rows)):
            raise ValueError("item table row out of range")
        if np.any((a[:, 1] < 0) | ((a[:, 1].astype(np.int64) + a[:, 2]) * 16 > table_stride * block_size)):
            raise ValueError("item tiles run past the table rows")
        if np.any((a[:, 4] < 0) | (a[:, 4] >= Hkv)):
            raise ValueError("item kv head out of range")
        if np.any((a[:, 5] < 1) | (a[:, 5] > cap)):
            raise ValueError("item member count out of range")
        if np.any(it[: self.n_shared, 2] > SHARED_MAX_TILES):
            raise ValueError("shared task longer than %d tiles" % SHARED_MAX_TILES)
        if np.any((a[:, 6] < 0) | (a[:, 6].astype(np.int64) + a[:, 5] > self.n_slots)):
            raise ValueError("item partial slots out of range")
        if np.any((a[:, 7] < 0) | (a[:, 7].astype(np.int64) + a[:, 5] > mem.size)):
            raise ValueError("item member list out of range")
        idx = np.concatenate([np.arange(o, o + n) for o, n in zip(a[:, 7], a[:, 5])])
        if np.any((mem[idx] < 0) | (mem[idx] >= Nq)):
            raise ValueError("member query index out of range")

    def device_arrays(self, device) -> tuple:
        """(items, members, q_slot_offsets, q_slots) as int32 device tensors (uploaded once)."""
        import torch

        key = str(device)
        cached = getattr(self, "_dev", None)
        if cached is None or cached[0] != key:
            host = (self.items.reshape(-1), self.members if self.members.size else np.zeros(1, np.int32),
                    self.q_slot_offsets, self.q_slots)
            cached = (key, tuple(torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in host))
            self._dev = cached
        return cached[1]


def find_segments(tables: list, lens: list, rows: list, block_size: int) -> list:
    """Recursive partition of the batch's page paths (see module docstring)."""
    B = block_size
    npages = [(int(n) + B - 1) // B for n in lens]

    def key(i, p):
        return (int(tables[i][p]), min(B, int(lens[i]) - p * B))

    segs: list[Segment] = []
    stack = [(list(range(len(tables))), 0)]
    while stack:
        members, p = stack.pop()
        members = [i for i in members if npages[i] > p]
        if not members:
            continue
        start = p
        while True:
            if any(npages[i] <= p for i in members):
                break
            k0 = key(members[0], p)
            if any(key(i, p) != k0 for i in members[1:]):
                break
            p += 1
            if k0[1] < B:
                break
        if p > start:
            last_valid = key(members[0], p - 1)[1]
            segs.append(Segment(start, p, (p - 1) * B + last_valid, list(members), int(rows[members[0]]), B))
        rest = [i for i in members if npages[i] > p]
        groups: dict = {}
        for i in rest:
            groups.setdefault(key(i, p), []).append(i)
        for g in reversed(list(groups.values())):
            stack.append((g, p))
    return segs


def build_plan(tables: list, lens: list, rows: list, *, block_size: int, Hkv: int, G: int,
               chunk_tiles: int = 4, shared_chunk_tiles: int = 32, shared_min_groups: int = 3) -> TreePlan:
    """Segments -> shared tasks, solo items and per-(query, head) partial slots."""
    if G < 1 or 16 % G:
        raise ValueError("query heads per kv head must divide 16")
    if not 1 <= shared_chunk_tiles <= SHARED_MAX_TILES or chunk_tiles < 1:
        raise ValueError("chunk sizes must be >= 1 (shared: <= %d tiles)" % SHARED_MAX_TILES)
    N = len(tables)
    segs = find_segments(tables, lens, rows, block_size)
    mg = 16 // G
    shared: list = []
    solo: list = []
    members: list = []
    slots_of: list[list[int]] = [[] for _ in range(N * Hkv)]
    n_slots = 0

    def add(dst, seg, c0, nt, h, mem):
        nonlocal n_slots
        dst.append([seg.row, c0, nt, seg.end_token, h, len(mem), n_slots, len(members)])
        members.extend(mem)
        for m in mem:
            slots_of[m * Hkv + h].append(n_slots)
            n_slots += 1

    for seg in segs:
        t0 = seg.first_page * block_size // 16
        t1 = (seg.end_token + 15) // 16
        groups = (len(seg.members) + mg - 1) // mg
        if groups >= shared_min_groups:
            cap = WAVES_PER_WG * mg
            sets = [seg.members[j:j + cap] for j in range(0, len(seg.members), cap)]
            for c0 in range(t0, t1, shared_chunk_tiles):
                nt = min(shared_chunk_tiles, t1 - c0)
                for h in range(Hkv):
                    for mem in sets:
                        add(shared, seg, c0, nt, h, mem)
        else:
            sets = [seg.members[j:j + mg] for j in range(0, len(seg.members), mg)]
            for c0 in range(t0, t1, chunk_tiles):
                nt = min(chunk_tiles, t1 - c0)
                for h in range(Hkv):
                    for mem in sets:
                        add(solo, seg, c0, nt, h, mem)
    off = np.zeros(N * Hkv + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(s) for s in slots_of])
    q_slots = np.array([s for lst in slots_of for s in lst] or [0], dtype=np.int32)
    items = shared + solo
    arr = np.array(items, dtype=np.int32).reshape(-1, ITEM_FIELDS) if items else np.zeros((0, ITEM_FIELDS), np.int32)
    return TreePlan(items=arr, n_shared=len(shared), members=np.array(members, dtype=np.int32),
                    q_slot_offsets=off, q_slots=q_slots, n_slots=n_slots, segments=segs)
