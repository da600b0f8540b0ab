"""Paged KV-cache manager for MI355X — drop-in for the reference's core/paged_kv_cache.py.

Host side (bit-exact with the reference): a refcounted block allocator whose
free list is a Python ``set`` popped with ``set.pop()`` (so block ids follow
exactly the reference's order, core/paged_kv_cache.py:21-72), per-layer page
tables and counters per sequence (:79-96), fork/free (:152-176) and the lazy
copy-on-write rules of append (:178-284).

Device side (new):
  * one K store and one V store of ``max_blocks`` pages serve every layer. The
    reference gives each layer its own ``max_blocks`` pool (:124-138), but its
    single allocator hands every block id to exactly one (sequence, layer) —
    fork shares an id within its layer, copy-on-write takes a fresh one — so a
    page id is never live in two layers and one store holds them all, with
    1/num_layers of the memory. 16-bit pools with block_size % 16 == 0 use the
    native layout read by the MFMA decode kernel (K [blk][Hkv][B][D],
    V [blk][Hkv][D][B]); other pools keep the reference layout. ``k_pools[l]`` /
    ``v_pools[l]`` are ``[max_blocks, block_size, Hkv, D]``-shaped views of the
    shared stores (permuted views for the native layout), so
    ``k_pools[l][blk, slot]`` means what it means in the reference for every
    block id that layer ``l`` owns.
  * every live sequence owns a row of int32 device block tables
    ``[num_layers, rows, pages]`` and lengths ``[num_layers, rows]``. The append
    kernel writes the table entry and length of each token it stores and
    performs the copy-on-write of a shared tail page in the same launch; a fork
    copies the parent's rows with one launch. No table is re-uploaded per step.
  * ``build_packed_kv`` gathers nothing: it returns zero-copy ``PagedKVView``s
    that ``adapters.attention_backend.attn_decode`` hands to the paged decode
    kernel.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from .. import ops
from .._lib import LAYOUT_NATIVE, LAYOUT_REFERENCE

try:  # the host planner in C (mentat_amd/csrc/host_plan.c): the same steps on the same objects
    from .. import _host_plan
except ImportError:  # not built: the Python planner below
    _host_plan = None

__all__ = ["BlockAllocator", "SequenceState", "PagedKVCacheManager", "PagedKVView"]


# ============================================================================
# Block allocator (reference: core/paged_kv_cache.py:21-72)
# ============================================================================

class BlockAllocator:
    """Refcounted pool of block ids.

    ``alloc`` takes ``set.pop()`` of the free set, like the reference; in
    CPython that hands out ids in ascending next-fit order until the first
    wrap-around of the id range, and in a hash-table-defined order after it.
    """

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self.refcounts = [0] * num_blocks
        self._free: set[int] = set(range(num_blocks))
        self._peak_used = 0

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._free)

    @property
    def peak_used(self) -> int:
        return self._peak_used

    def alloc(self) -> int:
        if not self._free:
            raise RuntimeError(
                f"PagedKVCache: out of blocks (pool size={self.num_blocks}).  "
                "Increase max_blocks or prune more aggressively."
            )
        blk = self._free.pop()
        self.refcounts[blk] = 1
        used = self.num_blocks - len(self._free)
        if used > self._peak_used:
            self._peak_used = used
        return blk

    def ref(self, block_idx: int) -> None:
        assert self.refcounts[block_idx] > 0, f"ref() on free block {block_idx}"
        self.refcounts[block_idx] += 1

    def release(self, block_idx: int) -> None:
        assert self.refcounts[block_idx] > 0, f"release() on free block {block_idx}"
        self.refcounts[block_idx] -= 1
        if self.refcounts[block_idx] == 0:
            self._free.add(block_idx)

    def is_shared(self, block_idx: int) -> bool:
        return self.refcounts[block_idx] > 1

    def can_alloc(self, n: int = 1) -> bool:
        return len(self._free) >= n


# ============================================================================
# Sequence metadata (reference: core/paged_kv_cache.py:79-96)
# ============================================================================

@dataclass
class SequenceState:
    """Per-sequence, per-layer page tables and counters; ``row`` is the sequence's
    row in the device block tables."""

    seq_id: int
    num_layers: int
    num_tokens: list[int] = field(default_factory=list)
    tokens_in_last_block: list[int] = field(default_factory=list)
    page_table: list[list[int]] = field(default_factory=list)
    row: int = -1

    def __post_init__(self):
        if not self.page_table:
            self.page_table = [[] for _ in range(self.num_layers)]
        if not self.num_tokens:
            self.num_tokens = [0] * self.num_layers
        if not self.tokens_in_last_block:
            self.tokens_in_last_block = [0] * self.num_layers


@dataclass
class PagedKVView:
    """Zero-copy stand-in for one packed K (or V) tensor of ``build_packed_kv``.

    Carries what the paged decode kernel needs to read the pages in place.
    """

    store: torch.Tensor          # this layer's K (or V) store
    tables: torch.Tensor         # this layer's [rows, pages] int32 block tables
    lens: torch.Tensor           # this layer's [rows] int32 lengths
    rows: torch.Tensor           # [N] int32 table row of each batch sequence
    block_size: int
    layout: int
    max_seqlen: int

    @property
    def shape(self):  # informational: the logical packed shape the reference would return
        return (int(self.lens.numel()), ) + tuple(self.store.shape[-2:])


# ============================================================================
# Manager (reference: core/paged_kv_cache.py:104-455)
# ============================================================================

class PagedKVCacheManager:
    def __init__(
        self,
        num_layers: int,
        num_key_value_heads: int,
        head_dim: int,
        max_blocks: int = 4096,
        block_size: int = 16,
        device: str | torch.device = "cuda",
        dtype: torch.dtype = torch.bfloat16,
    ):
        self.num_layers = num_layers
        self.num_key_value_heads = num_key_value_heads
        self.head_dim = head_dim
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dtype = dtype

        self.allocator = BlockAllocator(max_blocks)

        L, nb, B, H, D = num_layers, max_blocks, block_size, num_key_value_heads, head_dim
        native = dtype in (torch.bfloat16, torch.float16) and B % 16 == 0 and D % 32 == 0
        self.layout = LAYOUT_NATIVE if native else LAYOUT_REFERENCE
        # Pools are zero-initialised, as in the reference (:124-138); one store per
        # K/V for all layers (see the module docstring).
        if native:
            self._k_store = torch.zeros(nb, H, B, D, device=self.device, dtype=dtype)
            self._v_store = torch.zeros(nb, H, D, B, device=self.device, dtype=dtype)
            self.k_pools = [self._k_store.permute(0, 2, 1, 3)] * L
            self.v_pools = [self._v_store.permute(0, 3, 1, 2)] * L
        else:
            self._k_store = torch.zeros(nb, B, H, D, device=self.device, dtype=dtype)
            self._v_store = torch.zeros(nb, B, H, D, device=self.device, dtype=dtype)
            self.k_pools = [self._k_store] * L
            self.v_pools = [self._v_store] * L

        # Device block tables / lengths, one row per live sequence (grown on demand).
        self._rows_cap = 64
        self._pages_cap = 64
        self._tables = torch.zeros(L, self._rows_cap, self._pages_cap, dtype=torch.int32, device=self.device)
        self._lens = torch.zeros(L, self._rows_cap, dtype=torch.int32, device=self.device)
        self._free_rows: list[int] = list(range(self._rows_cap - 1, -1, -1))
        # Host copy of layer 0's table rows (indexed like the device rows): the
        # prefix-tree planner compares block ids on it each decode step. Every
        # layer shares layer 0's sharing pattern, so one layer is enough.
        self._host_t0 = np.zeros((self._rows_cap, self._pages_cap), dtype=np.int32)
        self._rows_cache: dict[tuple, torch.Tensor] = {}
        self._cu_cache: dict[tuple, torch.Tensor] = {}
        # Bumped whenever _tables / _lens are reallocated: captured launches that
        # hold their addresses must be captured again.
        self.tables_version = 0
        self._empty_row = -1

        self._sequences: dict[int, SequenceState] = {}
        self._next_seq_id = 0

    # ------------------------------------------------------------------
    #  Device table capacity
    # ------------------------------------------------------------------
    def _grow_rows(self) -> None:
        old = self._rows_cap
        new = old * 2
        t = torch.zeros(self.num_layers, new, self._pages_cap, dtype=torch.int32, device=self.device)
        t[:, :old] = self._tables
        n = torch.zeros(self.num_layers, new, dtype=torch.int32, device=self.device)
        n[:, :old] = self._lens
        self._tables, self._lens, self._rows_cap = t, n, new
        h = np.zeros((new, self._host_t0.shape[1]), dtype=np.int32)
        h[:old] = self._host_t0
        self._host_t0 = h
        self._free_rows = list(range(new - 1, old - 1, -1)) + self._free_rows
        self.tables_version += 1

    def _ensure_pages(self, npages: int) -> None:
        if npages <= self._pages_cap:
            return
        new = self._pages_cap
        while new < npages:
            new *= 2
        t = torch.zeros(self.num_layers, self._rows_cap, new, dtype=torch.int32, device=self.device)
        t[:, :, : self._pages_cap] = self._tables
        self._tables, self._pages_cap = t, new
        self._widen_host_t0(new)
        self._rows_cache.clear()
        self.tables_version += 1

    def _widen_host_t0(self, pages: int) -> None:
        w = self._host_t0.shape[1]
        if pages <= w:
            return
        while w < pages:
            w *= 2
        h = np.zeros((self._host_t0.shape[0], w), dtype=np.int32)
        h[:, : self._host_t0.shape[1]] = self._host_t0
        self._host_t0 = h

    def _host_t0_row(self, seq: SequenceState) -> None:
        t = seq.page_table[0]
        self._widen_host_t0(len(t))
        self._host_t0[seq.row, : len(t)] = t

    def host_tables0(self) -> np.ndarray:
        """Layer 0's block ids on the host, [rows, stride] int32 indexed by table
        row (entries past a row's pages are stale)."""
        return self._host_t0

    def reserve(self, rows: int, pages: int) -> None:
        """Grow the device tables to at least ``rows`` free rows and ``pages``
        pages per row now, so that later steps do not reallocate them."""
        while len(self._free_rows) < rows:
            self._grow_rows()
        self._ensure_pages(pages)

    def empty_row(self) -> int:
        """A table row that no sequence owns and whose length is 0 in every
        layer (decode of a padding entry reads nothing and writes zeros)."""
        if self._empty_row < 0:
            self._empty_row = self._take_row()
            self._lens[:, self._empty_row] = 0
        return self._empty_row

    def _take_row(self) -> int:
        if not self._free_rows:
            self._grow_rows()
        return self._free_rows.pop()

    # ------------------------------------------------------------------
    #  Sequences (reference :143-176)
    # ------------------------------------------------------------------
    def allocate_sequence(self) -> int:
        seq_id = self._next_seq_id
        self._next_seq_id += 1
        row = self._take_row()
        self._sequences[seq_id] = SequenceState(seq_id=seq_id, num_layers=self.num_layers, row=row)
        if self.device.type == "cuda":
            # a reused row still holds its previous sequence's lengths: the new
            # sequence has no tokens until its first append
            self._lens[:, row] = 0
        return seq_id

    def fork_sequence(self, parent_id: int) -> int:
        parent = self._sequences[parent_id]
        child_id = self._next_seq_id
        self._next_seq_id += 1
        tables: list[list[int]] = []
        for layer_blocks in parent.page_table:
            tables.append(list(layer_blocks))
            for blk in layer_blocks:
                self.allocator.ref(blk)
        child = SequenceState(
            seq_id=child_id,
            num_layers=self.num_layers,
            num_tokens=list(parent.num_tokens),
            tokens_in_last_block=list(parent.tokens_in_last_block),
            page_table=tables,
            row=self._take_row(),
        )
        self._sequences[child_id] = child
        n0 = len(tables[0]) if tables else 0
        self._host_t0[child.row, :n0] = self._host_t0[parent.row, :n0]
        if self.device.type == "cuda":
            n_entries = max((len(t) for t in tables), default=0)
            idx = torch.tensor([parent.row, child.row], dtype=torch.int32).to(self.device, non_blocking=True)
            ops.table_copy_rows(self._tables, self._lens, idx[:1], idx[1:], n_entries)
        return child_id

    def free_sequence(self, seq_id: int) -> None:
        seq = self._sequences.pop(seq_id)
        for layer_blocks in seq.page_table:
            for blk in layer_blocks:
                self.allocator.release(blk)
        if seq.row >= 0:
            self._free_rows.append(seq.row)

    # ------------------------------------------------------------------
    #  Append (reference :178-284): host plan + one fused device launch
    # ------------------------------------------------------------------
    def plan_append(self, seq_id: int, layer_idx: int, num_new: int) -> np.ndarray:
        """Host half of ``append_tokens``: update the allocator and page tables
        exactly as the reference does and return the int32 [7, num_new] plan."""
        seq = self._sequences[seq_id]
        table = seq.page_table[layer_idx]
        B = self.block_size
        plan = np.empty((7, num_new), dtype=np.int32)
        written = 0
        while written < num_new:
            if not table or seq.tokens_in_last_block[layer_idx] == B:
                table.append(self.allocator.alloc())
                seq.tokens_in_last_block[layer_idx] = 0
            tail = table[-1]
            cow = -1
            if self.allocator.is_shared(tail):
                new_blk = self.allocator.alloc()
                self.allocator.release(tail)
                table[-1] = new_blk
                cow, tail = tail, new_blk
            start = seq.tokens_in_last_block[layer_idx]
            n = min(B - start, num_new - written)
            cols = slice(written, written + n)
            plan[0, cols] = tail
            plan[1, cols] = np.arange(start, start + n)
            plan[2, cols] = -1
            plan[2, written] = cow
            plan[3, cols] = seq.row
            plan[4, cols] = len(table) - 1
            plan[5, cols] = -1
            plan[6, cols] = np.arange(written, written + n)
            written += n
            seq.tokens_in_last_block[layer_idx] += n
        seq.num_tokens[layer_idx] += num_new
        if num_new:
            plan[5, num_new - 1] = seq.num_tokens[layer_idx]
        if layer_idx == 0:
            self._host_t0_row(seq)
        return plan

    def _native_plan(self) -> bool:
        return _host_plan is not None and type(self.allocator) is BlockAllocator

    def _mirror_t0(self, plan0: np.ndarray) -> None:
        """Layer 0's planned table entries into the host copy of its tables."""
        self._widen_host_t0(int(plan0[4].max()) + 1)
        self._host_t0[plan0[3], plan0[4]] = plan0[0]

    def plan_append_batched(self, seq_ids: list[int], layer_idx: int) -> np.ndarray:
        """Host half of ``append_tokens_batched`` (one token per sequence, in
        batch order): returns the int32 [7, N] plan. Rows: destination block,
        slot, copy-on-write source (-1: none), table row, page index, new
        length, batch index."""
        if layer_idx != 0 or not seq_ids:
            return self._plan_batched(seq_ids, layer_idx)
        try:
            return self._plan_batched(seq_ids, 0)
        except Exception:
            self._resync_t0(seq_ids)
            raise

    def _resync_t0(self, seq_ids) -> None:
        """Layer 0's rows of the host copy from the page tables (after a plan
        that failed part-way, e.g. out of blocks, left some tables grown)."""
        for sid in seq_ids:
            seq = self._sequences.get(sid)
            if seq is not None and seq.row >= 0:
                self._host_t0_row(seq)

    def _plan_batched(self, seq_ids: list[int], layer_idx: int) -> np.ndarray:
        if seq_ids and self._native_plan():
            plan = np.empty((7, len(seq_ids)), dtype=np.int32)
            seqs = self._sequences
            if _host_plan.append_batched([seqs[s] for s in seq_ids], layer_idx, self.block_size, self.allocator,
                                         plan) is not None:
                if layer_idx == 0:
                    self._mirror_t0(plan)
                return plan
        B = self.block_size
        alloc = self.allocator
        rc = alloc.refcounts
        seqs = self._sequences
        L = layer_idx
        dst, slots, cows, rows, pages, lens = [], [], [], [], [], []
        for sid in seq_ids:
            seq = seqs[sid]
            table = seq.page_table[L]
            tilb = seq.tokens_in_last_block
            if not table or tilb[L] == B:
                table.append(alloc.alloc())
                tilb[L] = 0
            tail = table[-1]
            cow = -1
            if rc[tail] > 1:  # shared tail: copy-on-write (reference :258-265)
                new_blk = alloc.alloc()
                alloc.release(tail)
                table[-1] = new_blk
                cow, tail = tail, new_blk
            slot = tilb[L]
            tilb[L] = slot + 1
            nt = seq.num_tokens
            nt[L] += 1
            dst.append(tail)
            slots.append(slot)
            cows.append(cow)
            rows.append(seq.row)
            pages.append(len(table) - 1)
            lens.append(nt[L])
        plan = np.array([dst, slots, cows, rows, pages, lens, list(range(len(seq_ids)))],
                        dtype=np.int32).reshape(7, len(seq_ids))
        if L == 0 and seq_ids:
            self._mirror_t0(plan)
        return plan

    def plan_append_step(self, seq_ids: list[int]) -> np.ndarray:
        """Host half of one decode step's appends for every layer: the int32
        [num_layers, 7, N] plans that ``plan_append_batched(seq_ids, l)`` for
        l = 0, 1, ... would return, with the same allocator calls in the same
        order (layer-major, sequence-minor), so block ids and refcounts match.

        Decode, prefill, fork and free act on every layer alike, so every layer
        of a sequence has the same counters, the same refcount on its tail and
        the same tail-sharing partition across the batch. Then layer l makes
        the allocations layer 0 makes, at the same sequences: layer 0 is planned
        exactly, and the other layers replay its new-page and copy-on-write
        events on their own tables. The precondition is checked per step
        (counters, tail refcounts, sharing partition); if it does not hold the
        layers are planned one by one.
        """
        return self.plan_append_step_finish(self.plan_append_step_begin(seq_ids))

    def plan_append_step_begin(self, seq_ids: list[int], first_layers: int = 1) -> dict:
        """First half of plan_append_step: layers 0 .. first_layers - 1 are
        planned (``state["plan"][:first_layers]`` is final); plan_append_step_finish
        plans the rest. Nothing else may touch the manager in between. A caller
        can start the first layers' device work while the rest is planned."""
        L = self.num_layers
        N = len(seq_ids)
        plan = np.empty((L, 7, N), dtype=np.int32)
        st = {"seq_ids": seq_ids, "plan": plan, "next": L}
        if N == 0:
            return st
        seqs = [self._sequences[s] for s in seq_ids]
        upto = min(max(first_layers, 1), L)
        if self._native_plan():
            try:
                r = _host_plan.step_begin(seqs, L, self.block_size, self.allocator, plan)
            except Exception:
                self._resync_t0(seq_ids)
                raise
            if r is not None:  # the C planner: layer 0, then layers 1 .. upto - 1
                self._mirror_t0(plan[0])
                st.update(seqs=seqs, native=r[0], uniform=r[1], next=1)
                self._plan_layers(st, upto)
                return st
        rc = self.allocator.refcounts
        # Every layer's counters equal layer 0's (else every layer is planned on its own).
        uniform = all(s.num_tokens.count(s.num_tokens[0]) == L
                      and s.tokens_in_last_block.count(s.tokens_in_last_block[0]) == L for s in seqs)
        pts = [s.page_table for s in seqs]
        tails0 = [pt[0][-1] if pt[0] else -1 for pt in pts]
        paged = -1 not in tails0   # every sequence has a page in layer 0 (decode)
        rc0 = list(map(rc.__getitem__, tails0)) if paged else [rc[t] if t >= 0 else 0 for t in tails0]
        pages_before = [len(pt[0]) for pt in pts]
        p0 = self.plan_append_batched(seq_ids, 0)
        plan[0] = p0
        # Layer 0's events, in batch order: a new tail page, and/or a copy-on-write.
        new_at = [i for i, pt in enumerate(pts) if len(pt[0]) > pages_before[i]]
        cow_at = [i for i in range(N) if p0[2, i] >= 0]
        st.update(seqs=seqs, pts=pts, uniform=uniform, paged=paged, tails0=tails0, rc0=rc0,
                  shared0=any(r > 1 for r in rc0), ngroups0=len(set(tails0)), p0=p0,
                  events=sorted([(i, 0) for i in new_at] + [(i, 1) for i in cow_at]), next=1)
        self._plan_layers(st, upto)
        return st

    def plan_append_step_finish(self, st: dict) -> np.ndarray:
        """Second half of plan_append_step: the remaining layers; returns the
        int32 [num_layers, 7, N] plans."""
        self._plan_layers(st, self.num_layers)
        return st["plan"]

    def _plan_layers(self, st: dict, upto: int) -> None:
        """Layers st["next"] .. upto - 1, in order. A layer whose structure is
        layer 0's before the step (counters, tail refcounts, tail-sharing
        partition) replays layer 0's new-page and copy-on-write events on its
        own tables: the allocator calls plan_append_batched would make for it,
        in the same order. Any other layer runs plan_append_batched itself.
        Refcounts of a layer's blocks change only when that layer is planned,
        so each check sees the layer as it was before the step."""
        l0 = st["next"]
        if l0 >= upto:
            return
        st["next"] = upto
        if "native" in st:
            _host_plan.step_layers(st["native"], l0, upto, self.num_layers, self.block_size, self.allocator,
                                   st["plan"])
            return
        plan, seqs, pts, rc = st["plan"], st["seqs"], st["pts"], self.allocator.refcounts
        tails0, rc0, p0, events = st["tails0"], st["rc0"], st["p0"], st["events"]
        alloc, release = self.allocator.alloc, self.allocator.release
        replayed = []
        for l in range(l0, upto):
            ok = st["uniform"]
            tl = None
            if ok:
                if st["paged"]:
                    try:
                        tl = [pt[l][-1] for pt in pts]
                    except IndexError:  # an empty table where layer 0 has pages
                        ok = False
                    if ok:
                        ok = list(map(rc.__getitem__, tl)) == rc0
                else:
                    tl = [pt[l][-1] if pt[l] else -1 for pt in pts]
                    ok = [rc[t] if t >= 0 else 0 for t in tl] == rc0
                if ok and st["shared0"]:
                    ok = len(set(tl)) == st["ngroups0"] == len(set(zip(tails0, tl)))
            if not ok:
                plan[l] = self.plan_append_batched(st["seq_ids"], l)
                continue
            pl = plan[l]
            pl[1:] = p0[1:]
            pl[2] = -1
            for i, kind in events:
                table = pts[i][l]
                if kind == 0:
                    tl[i] = alloc()
                    table.append(tl[i])
                else:
                    old = table[-1]
                    tl[i] = alloc()
                    release(old)
                    table[-1] = tl[i]
                    pl[2, i] = old
            pl[0] = tl
            replayed.append(l)
        if replayed:
            # Layer 0's counters are the step's counters for every replayed layer.
            lo, hi = replayed[0], replayed[-1] + 1
            if len(replayed) == hi - lo:
                for s in seqs:
                    s.tokens_in_last_block[lo:hi] = [s.tokens_in_last_block[0]] * (hi - lo)
                    s.num_tokens[lo:hi] = [s.num_tokens[0]] * (hi - lo)
            else:
                for s in seqs:
                    for l in replayed:
                        s.tokens_in_last_block[l] = s.tokens_in_last_block[0]
                        s.num_tokens[l] = s.num_tokens[0]

    def _launch_append(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, plan: np.ndarray) -> None:
        if plan.shape[1] == 0:
            return
        if self.device.type != "cuda":
            raise RuntimeError("PagedKVCacheManager: K/V writes run on the HIP device only")
        self._ensure_pages(int(plan[4].max()) + 1)
        plan_t = torch.from_numpy(plan).to(self.device, non_blocking=False)
        k = k.to(self.dtype).contiguous()
        v = v.to(self.dtype).contiguous()
        ops.kv_append(
            k, v, self._k_store, self._v_store, plan_t,
            block_size=self.block_size, layout=self.layout,
            block_tables=self._tables[layer_idx], seq_lens=self._lens[layer_idx],
        )

    def append_tokens(self, seq_id: int, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> None:
        plan = self.plan_append(seq_id, layer_idx, int(k.shape[0]))
        self._launch_append(layer_idx, k, v, plan)

    def append_tokens_batched(self, seq_ids: list[int], layer_idx: int, k: torch.Tensor,
                              v: torch.Tensor) -> None:
        """Append 1 token for N sequences; k, v: (N, num_key_value_heads, head_dim)."""
        if len(seq_ids) == 0:
            return
        plan = self.plan_append_batched(seq_ids, layer_idx)
        self._launch_append(layer_idx, k, v, plan)

    def get_kv_length(self, seq_id: int) -> int:
        return self._sequences[seq_id].num_tokens[0]

    # ------------------------------------------------------------------
    #  Zero-copy "packed" KV (reference :289-368)
    # ------------------------------------------------------------------
    def _rows_tensor(self, seq_ids: tuple) -> torch.Tensor:
        t = self._rows_cache.get(seq_ids)
        if t is None:
            rows = [self._sequences[s].row for s in seq_ids]
            t = torch.tensor(rows, dtype=torch.int32).to(self.device)
            if len(self._rows_cache) > 64:
                self._rows_cache.clear()
            self._rows_cache[seq_ids] = t
        return t

    def build_packed_kv(self, seq_ids: list[int], layer_idx: int, cached_metadata=None):
        """Returns (k_view, v_view, cu_seqlens_k, max_seqlen_k) like the reference,
        with zero-copy views in place of the packed tensors (nothing is gathered)."""
        key = tuple(seq_ids)
        lens = [self._sequences[s].num_tokens[layer_idx] for s in seq_ids]
        max_len = max(lens) if lens else 0
        ck = (key, tuple(lens))
        cu = self._cu_cache.get(ck)
        if cu is None:
            cu_host = np.zeros(len(lens) + 1, dtype=np.int32)
            if lens:
                cu_host[1:] = np.cumsum(lens)
            cu = torch.from_numpy(cu_host).to(self.device)
            if len(self._cu_cache) > 64:
                self._cu_cache.clear()
            self._cu_cache[ck] = cu
        rows = self._rows_tensor(key) if seq_ids else torch.zeros(0, dtype=torch.int32, device=self.device)
        common = dict(tables=self._tables[layer_idx], lens=self._lens[layer_idx], rows=rows,
                      block_size=self.block_size, layout=self.layout, max_seqlen=max_len)
        kv = PagedKVView(store=self._k_store, **common)
        vv = PagedKVView(store=self._v_store, **common)
        return kv, vv, cu, max_len

    def gather_packed_kv(self, seq_ids: list[int], layer_idx: int):
        """The reference's materialised packed copy (for callers that need real
        tensors): (packed_k, packed_v, cu_seqlens_k, max_seqlen_k)."""
        blk, slot, lens = [], [], []
        for sid in seq_ids:
            seq = self._sequences[sid]
            n = seq.num_tokens[layer_idx]
            lens.append(n)
            rem = n
            for b in seq.page_table[layer_idx]:
                if rem == 0:
                    break
                c = min(self.block_size, rem)
                blk.extend([b] * c)
                slot.extend(range(c))
                rem -= c
        b_t = torch.tensor(blk, dtype=torch.long, device=self.device)
        s_t = torch.tensor(slot, dtype=torch.long, device=self.device)
        cu = torch.tensor([0] + lens, dtype=torch.int32).cumsum(0, dtype=torch.int32).to(self.device)
        pk = self.k_pools[layer_idx][b_t, s_t]
        pv = self.v_pools[layer_idx][b_t, s_t]
        return pk, pv, cu, (max(lens) if lens else 0)

    # ------------------------------------------------------------------
    #  Sliding-window trim (reference :370-417; no caller in the reference)
    # ------------------------------------------------------------------
    def trim_to_window(self, seq_id: int, window_size: int) -> None:
        seq = self._sequences[seq_id]
        if seq.num_tokens[0] <= window_size:
            return
        B = self.block_size
        for layer_idx in range(self.num_layers):
            evict = seq.num_tokens[layer_idx] - window_size
            table = seq.page_table[layer_idx]
            kp, vp = self.k_pools[layer_idx], self.v_pools[layer_idx]
            remaining = evict
            while remaining > 0 and table:
                blk = table[0]
                n_in = min(B, remaining)
                if n_in >= B:
                    table.pop(0)
                    self.allocator.release(blk)
                    remaining -= B
                else:
                    keep = B - n_in
                    if self.allocator.is_shared(blk):
                        new_blk = self.allocator.alloc()
                        kp[new_blk, :keep] = kp[blk, n_in:n_in + keep]
                        vp[new_blk, :keep] = vp[blk, n_in:n_in + keep]
                        self.allocator.release(blk)
                        table[0] = new_blk
                    else:
                        kp[blk, :keep] = kp[blk, n_in:n_in + keep].clone()
                        vp[blk, :keep] = vp[blk, n_in:n_in + keep].clone()
                    remaining = 0
            seq.num_tokens[layer_idx] = window_size
            if window_size == 0:
                seq.tokens_in_last_block[layer_idx] = 0
            else:
                r = window_size % B
                seq.tokens_in_last_block[layer_idx] = r if r else B
        self._upload_row(seq)

    def _upload_row(self, seq: SequenceState) -> None:
        """Re-write a sequence's device table row and lengths from the host lists."""
        self._host_t0_row(seq)
        if self.device.type != "cuda":
            return
        npg = max((len(t) for t in seq.page_table), default=0)
        self._ensure_pages(max(npg, 1))
        host = np.zeros((self.num_layers, self._pages_cap), dtype=np.int32)
        for l, t in enumerate(seq.page_table):
            host[l, :len(t)] = t
        self._tables[:, seq.row] = torch.from_numpy(host).to(self.device)
        self._lens[:, seq.row] = torch.tensor(seq.num_tokens, dtype=torch.int32).to(self.device)

    # ------------------------------------------------------------------
    #  Stats (reference :419-455)
    # ------------------------------------------------------------------
    def get_stats(self) -> dict:
        total_tokens = sum(s.num_tokens[0] if s.num_tokens else 0 for s in self._sequences.values())
        # Reference formula: counts every layer for each block id (overstates by L x).
        bytes_per_block = 2 * self.num_layers * self.block_size * self.num_key_value_heads * self.head_dim * self.dtype_size
        true_bytes_per_block = bytes_per_block // max(self.num_layers, 1)
        return {
            "num_sequences": len(self._sequences),
            "total_cached_tokens": total_tokens,
            "blocks_used": self.allocator.num_used,
            "blocks_free": self.allocator.num_free,
            "blocks_total": self.max_blocks,
            "blocks_peak": self.allocator.peak_used,
            "utilization": self.allocator.num_used / self.max_blocks,
            "peak_utilization": self.allocator.peak_used / self.max_blocks,
            "pool_memory_bytes": bytes_per_block * self.max_blocks,  # reference formula (L pools)
            "pool_memory_bytes_true": true_bytes_per_block * self.max_blocks,  # the shared stores
            "peak_kv_cache_bytes": bytes_per_block * self.allocator.peak_used,
            # Each block id holds one layer's K and V page: the bytes actually in use.
            "peak_kv_cache_bytes_true": true_bytes_per_block * self.allocator.peak_used,
        }

    @property
    def dtype_size(self) -> int:
        return torch.tensor([], dtype=self.dtype).element_size()

    def __repr__(self) -> str:
        st = self.get_stats()
        return (
            f"PagedKVCacheManager(layers={self.num_layers}, heads={self.num_key_value_heads}, "
            f"head_dim={self.head_dim}, block_size={self.block_size}, "
            f"blocks={st['blocks_used']}/{self.max_blocks}, seqs={st['num_sequences']}, "
            f"tokens={st['total_cached_tokens']})"
        )
