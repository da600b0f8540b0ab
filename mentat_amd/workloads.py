"""Seeded synthetic inputs for the branching-decode kernels.

These are the measured workloads (sizes, distributions and seeds fixed here):

* ``paged_decode_batch``: paged decode at Llama-3-8B attention shapes (pools
  in either layout) —
  bf16, 32 query / 8 kv heads, head_dim 128, page size 16, 64 sequences with
  context lengths uniform in [512, 4096], block tables = consecutive slices of
  a seeded random permutation of a 65,536-page pool, Q/K/V ~ N(0, 1),
  scale 1/sqrt(128).
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
