"""Attention backend for MI355X — drop-in for the reference's adapters/attention_backend.py.

Same names and signatures (adapters/attention_backend.py:32-36, :175-229):

    BACKEND                         "hip"
    attn_prefill(q, k, v, window_size=None)                         (B, S, H, D) -> (B, S, Hq, D)
    attn_decode(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_k, N, window_size=None) -> (N, Hq, D)

``attn_decode`` runs the HIP paged-decode kernel (libmentat_hip.so). When
``k``/``v`` are the zero-copy ``PagedKVView``s that
``PagedKVCacheManager.build_packed_kv`` returns, the kernel reads the pages
in place; given packed tensors (the reference's varlen layout) it reads those.
There is no fallback: without the library or a HIP device it raises.

``attn_prefill`` (causal attention over a batch of prompts) runs the HIP
prefill kernels (``mentat_prefill_attention``: GQA, sliding window; MFMA for
bf16/f16, the VALU decode kernel with one query per position for fp32); only
shapes no kernel takes (head_dim other than 64/128) use torch's device
matmuls in fp32.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import ops
from ..core.paged_kv_cache import PagedKVView

BACKEND = "hip"

__all__ = ["BACKEND", "attn_prefill", "attn_decode"]


def attn_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    window_size: Optional[int] = None,
) -> torch.Tensor:
    """Causal (optionally sliding-window) attention, (batch, seq, heads, head_dim).

    Position i attends to positions max(0, i - window_size + 1) .. i, as the
    reference's SDPA path does (adapters/attention_backend.py:43-96). K/V may
    have fewer heads than Q (GQA: query head h reads kv head h // (Hq/Hkv)).
    head_dim 64/128: the HIP kernels (MFMA for bf16/f16, VALU for fp32); other
    shapes (no kernel) run torch's device matmuls in fp32.
    """
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    if q.dtype in ops.PREFILL_GROUPS and D in (64, 128) and Hq % Hkv == 0 and G in ops.PREFILL_GROUPS[q.dtype]:
        return ops.prefill_attention(q, k, v, window_size=window_size)
    out_dtype = q.dtype
    qf = q.float().permute(0, 2, 1, 3).contiguous()                     # B, Hq, S, D
    kf = k.float().permute(0, 2, 1, 3)                                  # B, Hkv, S, D
    vf = v.float().permute(0, 2, 1, 3)
    if G > 1:
        kf = kf.repeat_interleave(G, dim=1)
        vf = vf.repeat_interleave(G, dim=1)
    kt = kf.transpose(-1, -2).contiguous()                              # B, Hq, D, S
    vf = vf.contiguous()
    scores = torch.matmul(qf, kt) * (1.0 / math.sqrt(D))                # B, Hq, S, S
    pos = torch.arange(S, device=q.device)
    mask = pos[None, :] <= pos[:, None]
    if window_size is not None and window_size < S:
        mask = mask & (pos[None, :] >= (pos[:, None] - window_size + 1))
    scores = scores.masked_fill(~mask, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    o = torch.matmul(probs, vf)                                         # B, Hq, S, D
    return o.permute(0, 2, 1, 3).to(out_dtype)


def attn_decode(
    q: torch.Tensor,
    k,
    v,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_k: int,
    N: int,
    window_size: Optional[int] = None,
) -> torch.Tensor:
    """One query per sequence over its cached context (reference semantics: the
    token appended this step included, default scale head_dim**-0.5). With
    window_size w, sequence i of length len attends to its last w tokens,
    [max(0, len - w), len): the reference's flash path
    (adapters/attention_backend.py:219-228, window_size=(w - 1, 0) with the
    query aligned to the end of the keys). The reference's SDPA fallback
    (:99-168) ignores the window; the two agree whenever len <= w, which
    trim_to_window keeps true."""
    q = q.contiguous()
    if isinstance(k, PagedKVView):
        if not isinstance(v, PagedKVView):
            raise TypeError("attn_decode: k and v must both be PagedKVView or both tensors")
        return ops.paged_decode(
            q, k.store, v.store, layout=k.layout, block_tables=k.tables, seq_lens=k.lens, seq_rows=k.rows,
            max_seqlen=max(int(max_seqlen_k), 1), window_size=window_size,
        )
    cu = cu_seqlens_k.to(device=q.device, dtype=torch.int32)
    return ops.paged_decode(q, k.contiguous(), v.contiguous(), cu_seqlens_k=cu,
                            max_seqlen=max(int(max_seqlen_k), 1), window_size=window_size)
