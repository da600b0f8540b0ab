"""Host plan of the grouped paged decode (mentat_paged_decode_grouped).

Sequences of a branching rollout share the pages they inherited at a fork
(core/paged_kv_cache.py:152-170: fork_sequence copies the block ids, so a
shared page has one id in every table that holds it). In the depth-first
batch order of the reference's leaves (core/generator_utils.py:171-189) the
sequences that share a page are consecutive, so comparing each sequence's
block ids with its predecessor's finds all the sharing: lcp[i] is the number
of leading full pages sequence i has in common with sequence i - 1, and a page
p of sequence i is shared by i .. j exactly when lcp[k] > p for i < k <= j.

From those common prefixes every sequence's pages are cut into segments: a
page run held by one set of consecutive queries, read from the table row of
the first (the owner). The decode kernel reads each segment once for all of
its queries, up to 16 / G of them in one MFMA query tile (G = query heads per
kv head); a larger set is split into several such groups. Any batch order is
correct: pages shared by sequences that are not neighbours are read once per
neighbourhood.

The sharing pattern is the same in every layer (forks, frees, appends and
copy-on-write act on all layers alike; only the ids differ), so one plan built
from layer 0's ids serves every layer: a segment names tiles and an owner row,
and the kernel reads that layer's ids from the row.

Arrays (int32):
  segs      [S, 4]  owner table row, first 16-token tile, end tile (exclusive),
                    m0 | count << 16 (queries m0 .. m0 + count - 1)
  seg_off   [N + 1] query i's segments are seg_list[seg_off[i] .. seg_off[i + 1]],
                    in page order
  seg_list  [sum over queries of their segments]
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class GroupPlan:
    segs: np.ndarray
    seg_off: np.ndarray
    seg_list: np.ndarray

    @property
    def n_segs(self) -> int:
        return int(self.segs.shape[0])

    def tiles_read(self) -> int:
        """16-token tiles the kernel reads per kv head (each segment once)."""
        return int((self.segs[:, 2] - self.segs[:, 1]).sum()) if self.n_segs else 0

    def validate(self, N: int, rows: int, table_stride: int, block_size: int, per_tile: int) -> None:
        """Host check of every index the kernel takes from the plan."""
        s, off, lst = self.segs, self.seg_off, self.seg_list
        for a, name in ((s, "segs"), (off, "seg_off"), (lst, "seg_list")):
            if a.dtype != np.int32:
                raise ValueError(f"{name} must be int32")
        if s.ndim != 2 or s.shape[1] != 4:
            raise ValueError("segs must be [S, 4]")
        if off.shape != (N + 1,) or off[0] != 0 or np.any(np.diff(off) < 0) or off[-1] != lst.size:
            raise ValueError("seg_off is not a CSR offset array over the N queries")
        S = s.shape[0]
        if S == 0:
            if lst.size:
                raise ValueError("seg_list names segments of an empty plan")
            return
        m0, cnt = s[:, 3] & 0xFFFF, s[:, 3] >> 16
        if np.any((s[:, 0] < 0) | (s[:, 0] >= rows)):
            raise ValueError("segment owner row out of range")
        if np.any((s[:, 1] < 0) | (s[:, 2] <= s[:, 1]) | (s[:, 2].astype(np.int64) * 16 > table_stride * block_size)):
            raise ValueError("segment tiles out of range")
        if np.any((cnt < 1) | (cnt > per_tile) | (m0.astype(np.int64) + cnt > N)):
            raise ValueError("segment queries out of range")
        if lst.size and (lst.min() < 0 or lst.max() >= S):
            raise ValueError("seg_list names a segment outside [0, S)")
        q = np.repeat(np.arange(N), np.diff(off))
        sm = m0[lst]
        if np.any((q < sm) | (q >= sm + cnt[lst])):
            raise ValueError("a query's segment does not hold it")
        if np.unique(q.astype(np.int64) * S + lst).size != lst.size:
            raise ValueError("a query lists one segment twice")


def common_prefix_pages(tables: np.ndarray, lens: np.ndarray, block_size: int) -> np.ndarray:
    """lcp[i]: leading full pages with the same block ids in rows i - 1 and i (lcp[0] = 0)."""
    N = tables.shape[0]
    lcp = np.zeros(N, dtype=np.int64)
    if N < 2:
        return lcp
    full = np.asarray(lens, dtype=np.int64) // block_size
    lim = np.minimum(full[1:], full[:-1])
    P = tables.shape[1]
    ok = (tables[1:] == tables[:-1]) & (np.arange(P)[None, :] < lim[:, None])
    ok = np.concatenate([ok, np.zeros((N - 1, 1), dtype=bool)], axis=1)
    lcp[1:] = np.argmin(ok, axis=1)
    return lcp


def build_group_plan(tables: np.ndarray, lens, rows, block_size: int, per_tile: int) -> GroupPlan:
    """Segments of the N queries (see the module docstring).

    tables: [N, P] int32, row i = query i's layer-0 block ids (entries past its
    pages are ignored); lens: tokens per query; rows: the table row of each
    query; per_tile: queries per MFMA tile (16 // G)."""
    tables = np.asarray(tables)
    lens = np.asarray(lens, dtype=np.int64)
    rows = np.asarray(rows, dtype=np.int64)
    N = int(lens.size)
    B = block_size
    tiles_per_page = B // 16
    npg = (lens + B - 1) // B
    lcp = common_prefix_pages(tables, lens, B).tolist()
    npg_l, lens_l, rows_l = npg.tolist(), lens.tolist(), rows.tolist()
    segs: list = []
    per_q: list = [[] for _ in range(N)]

    def emit(owner, a, b, m0, c):
        t0 = a * tiles_per_page
        t1 = b * tiles_per_page if b < npg_l[owner] else (lens_l[owner] + 15) // 16
        for k in range(0, c, per_tile):
            cc = min(per_tile, c - k)
            idx = len(segs)
            segs.append((rows_l[owner], t0, t1, (m0 + k) | (cc << 16)))
            for q in range(m0 + k, m0 + k + cc):
                per_q[q].append((a, idx))

    for i in range(N):
        lo, hi = lcp[i], npg_l[i]
        if hi <= lo:
            continue
        j, r = i + 1, hi
        while j < N and lcp[j] > lo:
            if lcp[j] < r:
                emit(i, lcp[j], hi, i, j - i)  # pages [lcp[j], hi) held by queries i .. j - 1
                hi = r = lcp[j]
            j += 1
        emit(i, lo, hi, i, j - i)
    off = np.zeros(N + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(p) for p in per_q])
    lst = np.array([idx for p in per_q for _, idx in sorted(p)], dtype=np.int32)
    seg_arr = np.array(segs, dtype=np.int32).reshape(-1, 4)
    return GroupPlan(segs=seg_arr, seg_off=off, seg_list=lst)


def private_plan(lens, rows, block_size: int) -> GroupPlan:
    """The plan without sharing: one segment per query holding all its pages."""
    lens = np.asarray(lens, dtype=np.int64)
    rows = np.asarray(rows, dtype=np.int64)
    N = int(lens.size)
    nz = np.nonzero(lens > 0)[0]
    segs = np.zeros((nz.size, 4), dtype=np.int32)
    segs[:, 0] = rows[nz]
    segs[:, 2] = (lens[nz] + 15) // 16
    segs[:, 3] = nz | (1 << 16)
    off = np.zeros(N + 1, dtype=np.int32)
    off[1:] = np.cumsum(lens > 0)
    return GroupPlan(segs=segs, seg_off=off, seg_list=np.arange(nz.size, dtype=np.int32))
