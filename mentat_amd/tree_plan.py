"""Host plan for the prefix-tree decode kernel (mentat_tree_decode).

The decode batch's contexts are split into segments: maximal runs of pages
that a set of sequences reaches through the same block ids (with the same
number of valid tokens), i.e. the edges of the prefix tree the batch forms —
a shared prompt, internal branches, each leaf's private tail. The sharing
structure is the same in every layer (forks, frees and copy-on-write treat all
layers alike; only the block ids differ), so a plan is built once per decode
step from layer 0's tables and reused by every layer: a segment names a
representative table row and the kernel reads that layer's ids from it.

Work items: each segment is cut into chunks of at most `chunk_tiles` 16-token
tiles, and each (chunk, kv head) into member groups of 16 / G queries (one
MFMA query tile; G = query heads per kv head). The groups of one (chunk, head)
are consecutive and start on a workgroup boundary, so a shared chunk is read
by one CU. Every (member, chunk, head) gets a partial slot; `q_slot_offsets`
/ `q_slots` list each (query, head)'s slots for the merge.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

ITEM_FIELDS = 24
ITEM_MEMBERS = ITEM_FIELDS - 7
WAVES_PER_WG = 8


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
    items: np.ndarray          # int32 [n_items, ITEM_FIELDS]
    q_slot_offsets: np.ndarray  # int32 [N * Hkv + 1]
    q_slots: np.ndarray        # int32 [n_slots]
    n_slots: int
    segments: list

    def unique_tokens(self) -> int:
        """Distinct cached token positions the batch reads (the same count in every layer)."""
        return sum(s.tokens for s in self.segments)

    def validate(self, Nq: int, Hkv: int, G: int, rows: int, table_stride: int, block_size: int) -> None:
        """Host check that every index the kernels take from the plan is in bounds."""
        it = self.items
        if it.ndim != 2 or it.shape[1] != ITEM_FIELDS or it.dtype != np.int32:
            raise ValueError("items must be int32 [n, %d]" % ITEM_FIELDS)
        off, qs = self.q_slot_offsets, self.q_slots
        if off.shape != (Nq * Hkv + 1,) or off[0] != 0 or np.any(np.diff(off) < 0) or off[-1] > qs.size:
            raise ValueError("q_slot_offsets is not a CSR offset array over Nq * Hkv (query, head) pairs")
        if off[-1] and (qs[: off[-1]].min() < 0 or qs[: off[-1]].max() >= self.n_slots):
            raise ValueError("q_slots names a slot outside [0, n_slots)")
        live = it[:, 2] > 0
        if not live.any():
            return
        a = it[live]
        mg = 16 // G
        if np.any((a[:, 0] < 0) | (a[:, 0] >= rows)):
            raise ValueError("item table row out of range")
        if np.any((a[:, 1] < 0) | ((a[:, 1] + a[:, 2]) * 16 > table_stride * block_size)):
            raise ValueError("item tiles run past the table rows")
        if np.any((a[:, 4] < 0) | (a[:, 4] >= Hkv)):
            raise ValueError("item kv head out of range")
        if np.any((a[:, 5] < 1) | (a[:, 5] > min(mg, ITEM_MEMBERS))):
            raise ValueError("item member count out of range")
        if np.any((a[:, 6] < 0) | (a[:, 6] + a[:, 5] > self.n_slots)):
            raise ValueError("item partial slots out of range")
        cols = np.arange(ITEM_MEMBERS)[None, :] < a[:, 5:6]
        mem = a[:, 7:]
        if np.any(cols & ((mem < 0) | (mem >= Nq))):
            raise ValueError("item member query index out of range")

    def device_arrays(self, device) -> tuple:
        """(items, q_slot_offsets, q_slots) as int32 device tensors (uploaded once)."""
        import torch

        key = str(device)
        cached = getattr(self, "_dev", None)
        if cached is None or cached[0] != key:
            up = tuple(torch.from_numpy(np.ascontiguousarray(a)).to(device)
                       for a in (self.items.reshape(-1), self.q_slot_offsets, self.q_slots))
            cached = (key, up)
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
               chunk_tiles: int = 32) -> TreePlan:
    """Segments -> work items and per-(query, head) partial slots."""
    if 16 % G:
        raise ValueError("query heads per kv head must divide 16")
    N = len(tables)
    segs = find_segments(tables, lens, rows, block_size)
    mg = min(16 // G, ITEM_MEMBERS)
    items: list[list[int]] = []
    slots_of: list[list[int]] = [[] for _ in range(N * Hkv)]
    n_slots = 0
    for seg in segs:
        t0 = seg.first_page * block_size // 16
        t1 = (seg.end_token + 15) // 16
        groups = [seg.members[j:j + mg] for j in range(0, len(seg.members), mg)]
        for c0 in range(t0, t1, chunk_tiles):
            nt = min(chunk_tiles, t1 - c0)
            for h in range(Hkv):
                if len(groups) > 1 and len(items) % WAVES_PER_WG:
                    # start a shared chunk on a workgroup boundary (padding items are empty)
                    pad = WAVES_PER_WG - len(items) % WAVES_PER_WG
                    if pad < len(groups):
                        items.extend([[0] * ITEM_FIELDS for _ in range(pad)])
                for grp in groups:
                    it = [seg.row, c0, nt, seg.end_token, h, len(grp), n_slots] + list(grp)
                    it += [0] * (ITEM_FIELDS - len(it))
                    items.append(it)
                    for m in grp:
                        slots_of[m * Hkv + h].append(n_slots)
                        n_slots += 1
    off = np.zeros(N * Hkv + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(s) for s in slots_of])
    q_slots = np.array([s for lst in slots_of for s in lst] or [0], dtype=np.int32)
    arr = np.array(items, dtype=np.int32).reshape(-1, ITEM_FIELDS) if items else np.zeros((0, ITEM_FIELDS), np.int32)
    return TreePlan(items=arr, q_slot_offsets=off, q_slots=q_slots, n_slots=n_slots, segments=segs)
