"""Oracle: paged decode attention (test infrastructure only).

Restates
  * ``PagedKVCacheManager.build_packed_kv`` (core/paged_kv_cache.py:289-368):
    for each sequence in batch order, its first ``num_tokens`` cached tokens
    are gathered page by page (``min(block_size, remaining)`` slots of each
    page in table order) into a packed ``[sum_ctx, Hkv, D]`` copy, with
    ``cu_seqlens_k`` = exclusive prefix sum of the lengths (int32) and
    ``max_seqlen_k`` = the longest length (0 for an empty batch).
  * ``_sdpa_decode`` (adapters/attention_backend.py:99-168): one query per
    sequence attends to every packed token of that sequence with
    ``is_causal=False`` and the default scale ``D**-0.5``; GQA query head h
    reads kv head ``h // (Hq // Hkv)`` (the expand/reshape at :152-155).
  * the decode window of the flash path (adapters/attention_backend.py:219-228):
    ``window_size=(w - 1, 0)`` with ``causal=True`` and one query aligned to the
    end of its keys keeps a sequence's last ``w`` tokens.

Pinned by (tests/test_oracle_attention.py): one cached token gives o = v;
identical keys give o = mean(V); a GQA head-mapping probe; agreement with
torch's own scaled_dot_product_attention in float64 (an independent library
routine) on random ragged batches. The window: the last row of the
reference's sliding-window prefill mask (adapters/attention_backend.py:81-86)
through torch's SDPA in float64, and w >= len reduces to no window.
"""
from __future__ import annotations

import numpy as np


def gather_packed_kv(k_pool, v_pool, page_tables, num_tokens, block_size):
    """Restates core/paged_kv_cache.py:289-368 on numpy arrays.

    k_pool, v_pool: [num_blocks, block_size, Hkv, D]; page_tables: list of
    lists of block ids (one per sequence); num_tokens: list of lengths.
    Returns (packed_k, packed_v, cu_seqlens int32 [N+1], max_seqlen).
    """
    blk_idx: list[int] = []
    slot_idx: list[int] = []
    for table, n_tok in zip(page_tables, num_tokens):  # :316-328
        remaining = int(n_tok)
        for blk in table:
            if remaining == 0:
                break
            n = min(block_size, remaining)
            blk_idx.extend([int(blk)] * n)
            slot_idx.extend(range(n))
            remaining -= n
    lens = [int(n) for n in num_tokens]
    cu = np.zeros(len(lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(lens, dtype=np.int64).astype(np.int32)
    max_len = max(lens) if lens else 0
    b = np.asarray(blk_idx, dtype=np.int64)
    s = np.asarray(slot_idx, dtype=np.int64)
    return k_pool[b, s], v_pool[b, s], cu, max_len


def sdpa_decode_f64(q, packed_k, packed_v, cu_seqlens_k, scale=None, window_size=None):
    """Restates adapters/attention_backend.py:99-168 in float64.

    q: [N, Hq, D]; packed_k/v: [total, Hkv, D]. Returns [N, Hq, D] float64.
    A sequence with no cached tokens yields zeros. window_size w keeps each
    sequence's last w tokens (the flash path, :219-228).
    """
    q = np.asarray(q, dtype=np.float64)
    N, Hq, D = q.shape
    Hkv = packed_k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    out = np.zeros((N, Hq, D), dtype=np.float64)
    cu = np.asarray(cu_seqlens_k, dtype=np.int64)
    for i in range(N):
        lo = cu[i]
        if window_size is not None and cu[i + 1] - cu[i] > window_size:
            lo = cu[i + 1] - window_size
        k = np.asarray(packed_k[lo:cu[i + 1]], dtype=np.float64)  # [L, Hkv, D]
        v = np.asarray(packed_v[lo:cu[i + 1]], dtype=np.float64)
        if k.shape[0] == 0:
            continue
        kh = np.repeat(k, G, axis=1)  # GQA expand: q head h -> kv head h // G
        vh = np.repeat(v, G, axis=1)
        s = np.einsum("hd,lhd->hl", q[i], kh) * scale
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[i] = np.einsum("hl,lhd->hd", p, vh)
    return out


def paged_decode_f64(q, k_pool, v_pool, page_tables, num_tokens, block_size, scale=None, window_size=None):
    """build_packed_kv followed by the SDPA decode, in float64."""
    pk, pv, cu, _ = gather_packed_kv(k_pool, v_pool, page_tables, num_tokens, block_size)
    return sdpa_decode_f64(q, pk, pv, cu, scale, window_size)


def reference_cpu_decode(q, k_pool, v_pool, page_tables, num_tokens, block_size):
    """The reference's CPU decode path in torch, in the model dtype.

    Gathers with one advanced-indexing copy per pool (core/paged_kv_cache.py:
    347-359) and runs one SDPA call per sequence with the GQA expand
    (adapters/attention_backend.py:141-168). Used as the timed CPU baseline.
    """
    import torch
    import torch.nn.functional as F

    blk_idx: list[int] = []
    slot_idx: list[int] = []
    lens: list[int] = []
    for table, n_tok in zip(page_tables, num_tokens):
        remaining = int(n_tok)
        lens.append(remaining)
        for blk in table:
            if remaining == 0:
                break
            n = min(block_size, remaining)
            blk_idx.extend([int(blk)] * n)
            slot_idx.extend(range(n))
            remaining -= n
    b = torch.tensor(blk_idx, dtype=torch.long)
    s = torch.tensor(slot_idx, dtype=torch.long)
    pk = k_pool[b, s]
    pv = v_pool[b, s]
    N, Hq, D = q.shape
    Hkv = pk.shape[1]
    G = Hq // Hkv
    outs = []
    start = 0
    for i in range(N):
        L = lens[i]
        ki = pk[start:start + L]
        vi = pv[start:start + L]
        start += L
        if G > 1:
            ki = ki.unsqueeze(2).expand(-1, -1, G, -1).reshape(L, Hq, D)
            vi = vi.unsqueeze(2).expand(-1, -1, G, -1).reshape(L, Hq, D)
        qi = q[i].unsqueeze(0).unsqueeze(2)
        ki = ki.permute(1, 0, 2).unsqueeze(0)
        vi = vi.permute(1, 0, 2).unsqueeze(0)
        oi = F.scaled_dot_product_attention(qi, ki, vi, is_causal=False)
        outs.append(oi.squeeze(0).squeeze(1))
    return torch.stack(outs, dim=0)


def reference_cpu_prefill(q, k, v, window_size=None):
    """The reference's SDPA prefill path in torch on the CPU, in the model dtype
    (adapters/attention_backend.py:43-96): transpose to (B, H, S, D), expand the
    kv heads to the query heads (GQA), causal SDPA, or an explicit
    sliding-window mask when window_size < S. Used as the timed CPU baseline of
    the prefill kernel; the kernel's parity tests use a float64 restatement."""
    import torch
    import torch.nn.functional as F

    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    Hq, Hkv, S = q.size(1), k.size(1), q.size(2)
    if Hkv != Hq:
        g = Hq // Hkv
        k = k.unsqueeze(2).expand(-1, -1, g, -1, -1).reshape(k.size(0), Hq, S, k.size(-1))
        v = v.unsqueeze(2).expand(-1, -1, g, -1, -1).reshape(v.size(0), Hq, S, v.size(-1))
    if window_size is not None and window_size < S:
        i = torch.arange(S)
        mask = (i[None, :] <= i[:, None]) & (i[None, :] >= (i[:, None] - window_size + 1))
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    else:
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    return o.transpose(1, 2)
