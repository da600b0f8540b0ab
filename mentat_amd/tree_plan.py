"""Host plan for the prefix-tree decode kernel (mentat_tree_decode).

The decode batch's contexts are split into segments: runs of pages that a set
of sequences reaches through the same block ids (with the same number of valid
tokens), i.e. the edges of the prefix tree the batch forms — a shared prompt,
internal branches, each leaf's private tail. The sharing structure is the same
in every layer (forks, frees and copy-on-write treat all layers alike; only
the block ids differ), so a plan is built once per decode step from layer 0's
tables and reused by every layer: a segment names a representative table row
and the kernel reads that layer's ids from it.

Segments come from the common prefixes of neighbours in batch order. A fork
copies its parent's block ids (core/paged_kv_cache.py:152-170), so two
sequences share exactly the pages on which their tables agree, and in the
reference's depth-first leaf order (core/generator_utils.py:171-189) the
sequences holding a page are consecutive. lcp[i] = the leading pages whose
ids (and valid token counts) sequence i has in common with sequence i - 1; a
page p of sequence i is then shared by i .. j exactly when lcp[k] > p for
i < k <= j, and each sequence's pages past lcp[i] are cut where that run of
neighbours gets shorter. Any batch order gives a correct plan (pages shared by
sequences that are not neighbours are read once per run of neighbours).

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
# Default plan: solo items of 4 tiles, shared tasks of up to 32 tiles for chunks of
# at least 2 member groups (measured best at the prefix-tree and rollout shapes)
CHUNK_TILES = 4
SHARED_CHUNK_TILES = 32
SHARED_MIN_GROUPS = 2


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
class SegmentArrays:
    """Segments as int64 arrays: owner table row, first page, end page
    (exclusive), end token (exclusive, absolute), first query, query count
    (queries m0 .. m0 + count - 1)."""
    row: np.ndarray
    first_page: np.ndarray
    end_page: np.ndarray
    end_token: np.ndarray
    m0: np.ndarray
    count: np.ndarray

    def __len__(self) -> int:
        return int(self.row.size)

    def segments(self, block_size: int) -> list:
        return [Segment(int(a), int(b), int(e), list(range(int(m), int(m) + int(c))), int(r), block_size)
                for r, a, b, e, m, c in zip(self.row, self.first_page, self.end_page, self.end_token, self.m0,
                                            self.count)]


@dataclass
class TreePlan:
    items: np.ndarray          # int32 [n_shared + n_solo, ITEM_FIELDS]
    n_shared: int
    members: np.ndarray        # int32 member query indices (items point into it)
    q_slot_offsets: np.ndarray  # int32 [N * Hkv + 1]
    q_slots: np.ndarray        # int32 [n_slots]
    n_slots: int
    seg: SegmentArrays
    block_size: int

    @property
    def n_solo(self) -> int:
        return self.items.shape[0] - self.n_shared

    @property
    def segments(self) -> list:
        return self.seg.segments(self.block_size)

    def unique_tokens(self) -> int:
        """Distinct cached token positions the batch reads (the same count in every layer)."""
        if not len(self.seg):
            return 0
        return int((self.seg.end_token - self.seg.first_page * self.block_size).sum())

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
        # Items with tiles write their members' slots; padding items (no tiles)
        # are skipped by the kernel and must have no members.
        if np.any((it[:, 2] <= 0) & (it[:, 5] != 0)):
            raise ValueError("an item with members has no tiles: its slots would never be written")
        live = it[:, 2] > 0
        if not live.any():
            if off[-1]:
                raise ValueError("q_slot_offsets lists slots that no item writes")
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
        tot = int(a[:, 5].sum())
        idx = np.repeat(a[:, 7].astype(np.int64) - np.cumsum(a[:, 5]) + a[:, 5], a[:, 5]) + np.arange(tot)
        if np.any((mem[idx] < 0) | (mem[idx] >= Nq)):
            raise ValueError("member query index out of range")
        # The merge reads the slots q_slot_offsets lists per (query, head): as
        # many as the items write for it (with slots in range and each written
        # once, the merge then reads exactly the written ones).
        keys = mem[idx].astype(np.int64) * Hkv + np.repeat(a[:, 4], a[:, 5])
        if not np.array_equal(np.bincount(keys, minlength=Nq * Hkv), np.diff(off.astype(np.int64))):
            raise ValueError("q_slot_offsets does not count the slots the items write per (query, head)")

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


def table_array(tables) -> np.ndarray:
    """Page tables (lists of block ids) as one int32 [N, P] array padded with -1."""
    if isinstance(tables, np.ndarray):
        return tables
    P = max([len(t) for t in tables] + [1])
    arr = np.full((len(tables), P), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        arr[i, :len(t)] = t
    return arr


def common_prefix_pages(tab: np.ndarray, lens, block_size: int) -> np.ndarray:
    """lcp[i]: leading pages on which rows i - 1 and i hold the same block id
    with the same number of valid tokens (lcp[0] = 0). A shared partial page
    ends the run."""
    N, P = tab.shape
    lcp = np.zeros(N, dtype=np.int64)
    if N < 2:
        return lcp
    lens = np.asarray(lens, dtype=np.int64)
    valid = np.clip(lens[:, None] - np.arange(P)[None, :] * block_size, 0, block_size)
    ok = (tab[1:] == tab[:-1]) & (valid[1:] == valid[:-1]) & (valid[1:] > 0)
    ok = np.concatenate([ok, np.zeros((N - 1, 1), dtype=bool)], axis=1)
    lcp[1:] = np.argmin(ok, axis=1)
    return lcp


def segment_arrays(tables, lens, rows, block_size: int) -> SegmentArrays:
    """Segments of the batch (see the module docstring)."""
    tab = table_array(tables)
    lens = np.asarray(lens, dtype=np.int64)
    B = block_size
    N = int(lens.size)
    npg = ((lens + B - 1) // B).tolist()
    lcp = common_prefix_pages(tab, lens, B).tolist()
    out: list = []
    for i in range(N):
        lo, hi = lcp[i], npg[i]
        if hi <= lo:
            continue
        j, r = i + 1, hi
        while j < N and lcp[j] > lo:
            if lcp[j] < r:
                out.append((i, lcp[j], hi, j - i))  # pages [lcp[j], hi) of queries i .. j - 1
                hi = r = lcp[j]
            j += 1
        out.append((i, lo, hi, j - i))
    if not out:
        z = np.zeros(0, dtype=np.int64)
        return SegmentArrays(z, z, z, z, z, z)
    a = np.array(out, dtype=np.int64)
    owner = a[:, 0]
    end_token = np.minimum(a[:, 2] * B, lens[owner])
    return SegmentArrays(row=np.asarray(rows, dtype=np.int64)[owner], first_page=a[:, 1], end_page=a[:, 2],
                         end_token=end_token, m0=owner, count=a[:, 3])


def find_segments(tables, lens, rows, block_size: int) -> list:
    """The batch's segments as Segment objects."""
    return segment_arrays(tables, lens, rows, block_size).segments(block_size)


def _items_of(sg: SegmentArrays, sel: np.ndarray, B: int, Hkv: int, chunk: int, cap: int):
    """Items of the segments `sel`, chunk-major, then kv head, then member set."""
    t0 = sg.first_page[sel] * B // 16
    t1 = (sg.end_token[sel] + 15) // 16
    cnt = sg.count[sel]
    nch = (t1 - t0 + chunk - 1) // chunk
    nset = (cnt + cap - 1) // cap
    per = nch * Hkv * nset
    tot = int(per.sum())
    sid = np.repeat(np.arange(sel.size), per)
    loc = np.arange(tot) - np.repeat(np.cumsum(per) - per, per)
    ns = nset[sid]
    iset = loc % ns
    rest = loc // ns
    h = rest % Hkv
    ch = rest // Hkv
    c0 = t0[sid] + ch * chunk
    nt = np.minimum(chunk, t1[sid] - c0)
    m_start = sg.m0[sel][sid] + iset * cap
    m_cnt = np.minimum(cap, cnt[sid] - iset * cap)
    return np.stack([sg.row[sel][sid], c0, nt, sg.end_token[sel][sid], h, m_cnt], axis=1), m_start


def build_plan(tables, lens, rows, *, block_size: int, Hkv: int, G: int,
               chunk_tiles: int = CHUNK_TILES, shared_chunk_tiles: int = SHARED_CHUNK_TILES,
               shared_min_groups: int = SHARED_MIN_GROUPS) -> TreePlan:
    """Segments -> shared tasks, solo items and per-(query, head) partial slots.

    ``tables``: the queries' page tables (lists, or an int32 [N, P] array whose
    rows past a query's pages are ignored); ``rows``: each query's table row."""
    if G < 1 or 16 % G:
        raise ValueError("query heads per kv head must divide 16")
    if not 1 <= shared_chunk_tiles <= SHARED_MAX_TILES or chunk_tiles < 1:
        raise ValueError("chunk sizes must be >= 1 (shared: <= %d tiles)" % SHARED_MAX_TILES)
    N = int(np.asarray(lens).size)
    sg = segment_arrays(tables, lens, rows, block_size)
    mg = 16 // G
    groups = (sg.count + mg - 1) // mg
    shared = groups >= shared_min_groups
    a_sh, m_sh = _items_of(sg, np.nonzero(shared)[0], block_size, Hkv, shared_chunk_tiles, WAVES_PER_WG * mg)
    order = np.argsort(-a_sh[:, 2], kind="stable")   # shared tasks longest first (the kernel's queue order)
    a_sh, m_sh = a_sh[order], m_sh[order]
    a_so, m_so = _items_of(sg, np.nonzero(~shared)[0], block_size, Hkv, chunk_tiles, mg)
    body = np.concatenate([a_sh, a_so])
    m_start = np.concatenate([m_sh, m_so])
    m_cnt = body[:, 5]
    first = np.cumsum(m_cnt) - m_cnt          # member offset = first slot of the item
    items = np.concatenate([body, first[:, None], first[:, None]], axis=1).astype(np.int32)
    n_slots = int(m_cnt.sum())
    members = (np.repeat(m_start - first, m_cnt) + np.arange(n_slots)).astype(np.int32)
    keys = members.astype(np.int64) * Hkv + np.repeat(body[:, 4], m_cnt)
    off = np.zeros(N * Hkv + 1, dtype=np.int32)
    off[1:] = np.cumsum(np.bincount(keys, minlength=N * Hkv))
    q_slots = np.argsort(keys, kind="stable").astype(np.int32) if n_slots else np.zeros(1, np.int32)
    return TreePlan(items=items.reshape(-1, ITEM_FIELDS), n_shared=int(a_sh.shape[0]), members=members,
                    q_slot_offsets=off, q_slots=q_slots, n_slots=n_slots, seg=sg, block_size=block_size)
