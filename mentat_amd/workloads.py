"""Seeded synthetic inputs for the branching-decode kernels.

These are the measured workloads (sizes, distributions and seeds fixed here):

* ``paged_decode_batch``: paged decode at Llama-3-8B attention shapes (pools
  in either layout) —
  bf16, 32 query / 8 kv heads, head_dim 128, page size 16, 64 sequences with
  context lengths uniform in [512, 4096], block tables = consecutive slices of
  a seeded random permutation of a 65,536-page pool, Q/K/V ~ N(0, 1),
  scale 1/sqrt(128).
* ``prefix_tree_batch``: prefix-tree decode at Qwen3-8B attention shapes —
  bf16, 32 query / 8 kv heads, head_dim 128, page size 16, q and k through
  RMSNorm (weight 1, eps 1e-6), 4 trees of 32 leaves over 2048-token shared
  prompts (``tree_ops`` fixes the shapes), written through the paged cache
  manager so sharing, refcounts and copy-on-write are the manager's own.
* ``sampling_logits``: [256, 151936] bf16 logits, row r ~ sigma_r * N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


from ._lib import LAYOUT_NATIVE, LAYOUT_REFERENCE


def logical_views(k_store: torch.Tensor, v_store: torch.Tensor, layout: int):
    """[num_blocks, B, Hkv, D]-shaped views of K/V stores of either layout."""
    if layout == LAYOUT_NATIVE:
        return k_store.permute(0, 2, 1, 3), v_store.permute(0, 3, 1, 2)
    return k_store, v_store


@dataclass
class PagedBatch:
    q: torch.Tensor            # [N, Hq, D]
    k_store: torch.Tensor      # pool storage in `layout`
    v_store: torch.Tensor
    block_tables: torch.Tensor  # [N, max_pages] int32 (unused entries = 0)
    seq_lens: torch.Tensor     # [N] int32
    lens: list                 # host copy of seq_lens
    tables: list               # host page tables (list of lists)
    block_size: int
    scale: float
    layout: int = LAYOUT_REFERENCE

    @property
    def k_pool(self) -> torch.Tensor:
        """K as [num_blocks, B, Hkv, D] (a view; non-contiguous for the native layout)."""
        return logical_views(self.k_store, self.v_store, self.layout)[0]

    @property
    def v_pool(self) -> torch.Tensor:
        return logical_views(self.k_store, self.v_store, self.layout)[1]

    @property
    def max_seqlen(self) -> int:
        return max(self.lens) if self.lens else 0

    def algorithmic_bytes(self) -> int:
        """HBM bytes one decode over this batch must move at minimum.

        K and V of every cached token (Hkv*D elements each), Q read once, O
        written once, one int32 table entry per page and one length per sequence.
        """
        N, Hq, D = self.q.shape
        Hkv = self.k_pool.shape[2]  # logical [num_blocks, B, Hkv, D]
        esz = self.q.element_size()
        ctx = sum(self.lens)
        pages = sum((n + self.block_size - 1) // self.block_size for n in self.lens)
        return ctx * Hkv * D * esz * 2 + 2 * N * Hq * D * esz + 4 * pages + 4 * N


def paged_decode_batch(
    *,
    N: int = 64,
    Hq: int = 32,
    Hkv: int = 8,
    D: int = 128,
    block_size: int = 16,
    ctx_lo: int = 512,
    ctx_hi: int = 4096,
    num_blocks: int = 65536,
    dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cuda",
    seed: int = 0,
    lens: list | None = None,
    layout: int = LAYOUT_REFERENCE,
) -> PagedBatch:
    rng = np.random.default_rng(seed)
    if lens is None:
        lens = rng.integers(ctx_lo, ctx_hi + 1, size=N).tolist()
    else:
        lens = [int(x) for x in lens]
        N = len(lens)
    perm = rng.permutation(num_blocks)
    pages = [(n + block_size - 1) // block_size for n in lens]
    if sum(pages) > num_blocks:
        raise ValueError("pool too small for the requested contexts")
    max_pages = max(1, max(pages) if pages else 1)
    tables = []
    tab = np.zeros((N, max_pages), dtype=np.int32)
    off = 0
    for i, npg in enumerate(pages):
        row = perm[off:off + npg]
        off += npg
        tables.append(row.tolist())
        tab[i, :npg] = row
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q = torch.randn(N, Hq, D, generator=g, device=device, dtype=torch.float32).to(dtype)
    if layout == LAYOUT_NATIVE:
        k_store = torch.empty(num_blocks, Hkv, block_size, D, device=device, dtype=dtype)
        v_store = torch.empty(num_blocks, Hkv, D, block_size, device=device, dtype=dtype)
    else:
        k_store = torch.empty(num_blocks, block_size, Hkv, D, device=device, dtype=dtype)
        v_store = torch.empty_like(k_store)
    # Fill in slices to bound the fp32 temporaries (i.i.d. entries: the layout
    # does not change the distribution).
    step = max(1, (1 << 26) // (block_size * Hkv * D))
    for s in range(0, num_blocks, step):
        e = min(num_blocks, s + step)
        k_store[s:e] = torch.randn(k_store[s:e].shape, generator=g, device=device).to(dtype)
        v_store[s:e] = torch.randn(v_store[s:e].shape, generator=g, device=device).to(dtype)
    return PagedBatch(
        q=q,
        k_store=k_store,
        v_store=v_store,
        layout=layout,
        block_tables=torch.from_numpy(tab).to(device),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        lens=lens,
        tables=tables,
        block_size=block_size,
        scale=1.0 / float(np.sqrt(D)),
    )


def sampling_logits(*, R: int = 256, V: int = 151936, sigma_lo: float = 0.5, sigma_hi: float = 4.0,
                    dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cuda",
                    seed: int = 0):
    """Logits for the fused entropy-gate + sampling step: row r is sigma_r * N(0, 1)
    with sigma_r uniform in [sigma_lo, sigma_hi] (seeded), so entropies at
    T = 0.7 span a 3-nat gate. Returns (logits [R, V], sigmas)."""
    rng = np.random.default_rng(seed)
    sig = rng.uniform(sigma_lo, sigma_hi, size=R).astype(np.float32)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.empty(R, V, device=device, dtype=dtype)
    for r0 in range(0, R, 16):
        r1 = min(R, r0 + 16)
        z = torch.randn(r1 - r0, V, generator=g, device=device)
        x[r0:r1] = (z * torch.from_numpy(sig[r0:r1]).to(device)[:, None]).to(dtype)
    return x, sig


# ----------------------------------------------------------------------------
# Prefix-tree decode workload
# ----------------------------------------------------------------------------

def tree_ops(*, n_trees: int = 4, prefix: int = 2048, leaves: int = 32, max_private: int = 512,
             seed: int = 0) -> list:
    """Seeded event list that grows ``n_trees`` branching trees in a paged cache.

    Shapes: each tree starts as one leaf with U{0..max_private} private tokens
    after its ``prefix``-token prompt. A split picks a leaf uniformly and a
    depth d uniformly along its private span [f, P] (f = depth of the leaf's
    last fork, P = its length past the prompt); the leaf keeps P, a new leaf
    starts at d with length U{d..max_private}; both leaves' private spans now
    start at d. Splits repeat until the tree has ``leaves`` leaves.

    The events replay that as decode would: one step appends one token to every
    leaf still growing, forks happen at the step of their depth (in split
    order), and a new leaf sits right after its parent in batch order, so the
    parent (first in batch order) copies a shared partial tail on its next
    append and the new leaf writes it in place.

    Events: ("alloc", leaf), ("prefill", leaf, n), ("fork", parent, child),
    ("step", [leaf, ...] in batch order). Leaves are numbered globally.
    """
    rng = np.random.default_rng(seed)
    ops: list = []
    forks_at: dict = {}
    target: dict = {}
    order: list = []
    nid = 0
    for _ in range(n_trees):
        root = nid
        nid += 1
        f = {root: 0}
        target[root] = int(rng.integers(0, max_private + 1))
        live = [root]
        while len(live) < leaves:
            j = live[int(rng.integers(len(live)))]
            d = int(rng.integers(f[j], target[j] + 1))
            i = nid
            nid += 1
            target[i] = int(rng.integers(d, max_private + 1))
            f[j] = f[i] = d
            forks_at.setdefault(d, []).append((j, i))
            live.append(i)
        ops.append(("alloc", root))
        ops.append(("prefill", root, prefix))
        order.append(root)
    for t in range(max_private + 1):
        for j, i in forks_at.get(t, []):
            ops.append(("fork", j, i))
            order.insert(order.index(j) + 1, i)
        grow = [x for x in order if target[x] > t]
        if grow:
            ops.append(("step", grow))
    ops.append(("final", list(order)))
    return ops


def replay_tree_ops(mgr, ops: list, layer: int = 0, kv=None) -> tuple:
    """Apply ``tree_ops`` events to a PagedKVCacheManager.

    ``kv(n)`` returns the (k, v) rows [n, Hkv, D] to write; with ``kv=None``
    only the host bookkeeping runs (page tables, refcounts, copy-on-write
    decisions). Returns (sequence id of each leaf, leaves in batch order).
    """
    seq = {}
    order = []
    for op in ops:
        if op[0] == "alloc":
            seq[op[1]] = mgr.allocate_sequence()
        elif op[0] == "prefill":
            sid = seq[op[1]]
            if kv is None:
                mgr.plan_append(sid, layer, op[2])
            else:
                mgr.append_tokens(sid, layer, *kv(op[2]))
        elif op[0] == "fork":
            seq[op[2]] = mgr.fork_sequence(seq[op[1]])
        elif op[0] == "step":
            ids = [seq[x] for x in op[1]]
            if kv is None:
                mgr.plan_append_batched(ids, layer)
            else:
                mgr.append_tokens_batched(ids, layer, *kv(len(ids)))
        elif op[0] == "final":
            order = list(op[1])
    return seq, order


def _rms_normed(shape, g, device, eps=1e-6):
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


@dataclass
class TreeBatch:
    q: torch.Tensor            # [Nq, Hq, D], one query per leaf in batch order
    mgr: object                # the PagedKVCacheManager holding the trees (one layer)
    seq_ids: list              # sequence id of each query
    lens: list                 # cached tokens of each query
    tables: list               # host page table of each query
    rows: list                 # device table row of each query
    block_tables: torch.Tensor  # the layer's [rows, pages] int32 tables
    seq_lens: torch.Tensor     # the layer's [rows] int32 lengths
    k_store: torch.Tensor      # native stores of the layer
    v_store: torch.Tensor
    block_size: int
    scale: float

    def unique_tokens(self) -> int:
        seen = set()
        B = self.block_size
        for t, n in zip(self.tables, self.lens):
            for p in range((n + B - 1) // B):
                seen.add((t[p], min(B, n - p * B)))
        return sum(v for _, v in seen)

    def logical_tokens(self) -> int:
        return sum(self.lens)

    def _bytes(self, tokens: int) -> int:
        N, Hq, D = self.q.shape
        Hkv = self.k_store.shape[1]
        esz = self.q.element_size()
        pages = sum((n + self.block_size - 1) // self.block_size for n in self.lens)
        return tokens * Hkv * D * esz * 2 + 2 * N * Hq * D * esz + 4 * pages + 4 * N

    def unique_bytes(self) -> int:
        """K/V of every distinct cached token once, Q and O once, the table entries."""
        return self._bytes(self.unique_tokens())

    def logical_bytes(self) -> int:
        """The same with every leaf's full context counted (no sharing)."""
        return self._bytes(self.logical_tokens())


def prefix_tree_batch(*, n_trees: int = 4, prefix: int = 2048, leaves: int = 32, max_private: int = 512,
                      Hq: int = 32, Hkv: int = 8, D: int = 128, block_size: int = 16,
                      max_blocks: int = 8192, dtype: torch.dtype = torch.bfloat16,
                      device: str | torch.device = "cuda", seed: int = 0) -> TreeBatch:
    from .core.paged_kv_cache import PagedKVCacheManager

    ops = tree_ops(n_trees=n_trees, prefix=prefix, leaves=leaves, max_private=max_private, seed=seed)
    mgr = PagedKVCacheManager(1, Hkv, D, max_blocks=max_blocks, block_size=block_size, device=device,
                              dtype=dtype)
    if mgr.layout != LAYOUT_NATIVE:
        raise ValueError("the prefix-tree workload needs the native pool layout")
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def kv(n):
        k = _rms_normed((n, Hkv, D), g, device).to(dtype)
        v = torch.randn(n, Hkv, D, generator=g, device=device).to(dtype)
        return k, v

    seq, order = replay_tree_ops(mgr, ops, 0, kv)
    ids = [seq[x] for x in order]
    q = _rms_normed((len(ids), Hq, D), g, device).to(dtype)
    states = [mgr._sequences[s] for s in ids]
    return TreeBatch(
        q=q, mgr=mgr, seq_ids=ids,
        lens=[st.num_tokens[0] for st in states],
        tables=[list(st.page_table[0]) for st in states],
        rows=[st.row for st in states],
        block_tables=mgr._tables[0], seq_lens=mgr._lens[0],
        k_store=mgr._k_store, v_store=mgr._v_store,
        block_size=block_size, scale=1.0 / float(np.sqrt(D)),
    )
