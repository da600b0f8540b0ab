"""Seeded synthetic inputs for the branching-decode kernels.

These are the measured workloads (sizes, distributions and seeds fixed here):

* ``paged_decode_batch``: paged decode at Llama-3-8B attention shapes —
  bf16, 32 query / 8 kv heads, head_dim 128, page size 16, 64 sequences with
  context lengths uniform in [512, 4096], block tables = consecutive slices of
  a seeded random permutation of a 65,536-page pool, Q/K/V ~ N(0, 1),
  scale 1/sqrt(128).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class PagedBatch:
    q: torch.Tensor            # [N, Hq, D]
    k_pool: torch.Tensor       # [num_blocks, B, Hkv, D]
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # [N, max_pages] int32 (unused entries = 0)
    seq_lens: torch.Tensor     # [N] int32
    lens: list                 # host copy of seq_lens
    tables: list               # host page tables (list of lists)
    block_size: int
    scale: float

    @property
    def max_seqlen(self) -> int:
        return max(self.lens) if self.lens else 0

    def algorithmic_bytes(self) -> int:
        """HBM bytes one decode over this batch must move at minimum.

        K and V of every cached token (Hkv*D elements each), Q read once, O
        written once, one int32 table entry per page and one length per sequence.
        """
        N, Hq, D = self.q.shape
        Hkv = self.k_pool.shape[2]
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
    k_pool = torch.empty(num_blocks, block_size, Hkv, D, device=device, dtype=dtype)
    v_pool = torch.empty_like(k_pool)
    # Fill in slices to bound the fp32 temporaries.
    step = max(1, (1 << 26) // (block_size * Hkv * D))
    for s in range(0, num_blocks, step):
        e = min(num_blocks, s + step)
        k_pool[s:e] = torch.randn(e - s, block_size, Hkv, D, generator=g, device=device).to(dtype)
        v_pool[s:e] = torch.randn(e - s, block_size, Hkv, D, generator=g, device=device).to(dtype)
    return PagedBatch(
        q=q,
        k_pool=k_pool,
        v_pool=v_pool,
        block_tables=torch.from_numpy(tab).to(device),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        lens=lens,
        tables=tables,
        block_size=block_size,
        scale=1.0 / float(np.sqrt(D)),
    )
