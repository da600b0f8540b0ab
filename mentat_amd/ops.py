"""Tensor-level wrappers over the C ABI (include/mentat_capi.h).

Each wrapper validates shapes, dtypes and devices on the host (a kernel is
never launched on operands that do not match what its grid assumes), then
calls the library on torch's current stream.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from ._lib import DTYPE_CODES, MentatError, check, get_lib, ptr, stream_handle

__all__ = ["paged_decode", "MentatError", "workspace"]

# One workspace per (device, stream): calls on one stream are ordered, so they
# may share it; calls on different streams get different buffers.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A zero-initialised uint8 device buffer of at least nbytes (cached, grows)."""
    if nbytes <= 0:
        nbytes = 1
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream_handle(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = 1 << max(20, (nbytes - 1).bit_length())
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_i32(t: Optional[torch.Tensor], name: str, device) -> None:
    if t is None:
        return
    _require(t.dtype == torch.int32, f"{name} must be int32, got {t.dtype}")
    _require(t.device == device, f"{name} must be on {device}, got {t.device}")
    _require(t.is_contiguous(), f"{name} must be contiguous")


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    *,
    max_seqlen: int,
    block_tables: Optional[torch.Tensor] = None,
    seq_lens: Optional[torch.Tensor] = None,
    seq_rows: Optional[torch.Tensor] = None,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    chunk_tokens: int = 0,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """One-query-per-sequence attention over a paged (or packed varlen) KV cache.

    Paged mode (``block_tables`` given): k_cache/v_cache are pools
    ``[num_blocks, block_size, Hkv, D]``; sequence i uses table row
    ``seq_rows[i]`` (or i) and has ``seq_lens[row]`` tokens.
    Packed mode: k_cache/v_cache are ``[total, Hkv, D]`` and ``cu_seqlens_k``
    (int32, N+1) delimits the sequences, as in the reference's
    ``build_packed_kv`` output (core/paged_kv_cache.py:289-368).

    ``max_seqlen`` must be >= every sequence length (it sizes the split-K grid).
    Returns ``out`` [N, Hq, D] in q's dtype.
    """
    _require(q.dim() == 3, f"q must be [N, Hq, D], got {tuple(q.shape)}")
    N, Hq, D = q.shape
    dev = q.device
    _require(dev.type == "cuda", "paged_decode runs on the GPU only (q is on the CPU)")
    _require(q.dtype in DTYPE_CODES, f"unsupported dtype {q.dtype}")
    _require(k_cache.dtype == q.dtype and v_cache.dtype == q.dtype, "q/k/v dtypes differ")
    _require(k_cache.device == dev and v_cache.device == dev, "q/k/v devices differ")
    _require(q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous(),
             "q, k_cache and v_cache must be contiguous")
    _require(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if block_tables is not None:
        _require(k_cache.dim() == 4, "paged k_cache must be [num_blocks, block_size, Hkv, D]")
        num_blocks, block_size, Hkv, Dk = k_cache.shape
        _require(seq_lens is not None, "paged mode needs seq_lens")
        _require(block_tables.dim() == 2, "block_tables must be [rows, stride]")
        _check_i32(block_tables, "block_tables", dev)
        _check_i32(seq_lens, "seq_lens", dev)
        _check_i32(seq_rows, "seq_rows", dev)
        rows = block_tables.shape[0]
        if seq_rows is None:
            _require(rows >= N and seq_lens.numel() >= N, "block_tables/seq_lens have fewer rows than N")
        else:
            _require(seq_rows.numel() == N, "seq_rows must have N entries")
            _require(seq_lens.numel() >= rows, "seq_lens must have one entry per table row")
        _require(block_tables.shape[1] * block_size >= max_seqlen,
                 "block_tables rows are too short for max_seqlen")
        stride = block_tables.stride(0)
    else:
        _require(cu_seqlens_k is not None, "packed mode needs cu_seqlens_k")
        _require(k_cache.dim() == 3, "packed k_cache must be [total, Hkv, D]")
        _check_i32(cu_seqlens_k, "cu_seqlens_k", dev)
        _require(cu_seqlens_k.numel() == N + 1, "cu_seqlens_k must have N+1 entries")
        _, Hkv, Dk = k_cache.shape
        num_blocks, block_size, stride = 0, 0, 0
    _require(Dk == D, f"head_dim mismatch q {D} vs cache {Dk}")
    _require(Hq % Hkv == 0, f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if out is None:
        out = torch.empty_like(q)
    else:
        _require(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    if N == 0:
        return out
    lib = get_lib()
    max_seqlen = max(int(max_seqlen), 1)
    nbytes = lib.mentat_paged_decode_workspace_bytes(N, Hq, Hkv, D, block_size, max_seqlen, chunk_tokens)
    ws = workspace(dev, nbytes) if nbytes else None
    st = lib.mentat_paged_decode(
        ptr(q), ptr(k_cache), ptr(v_cache),
        ptr(block_tables), stride,
        ptr(seq_rows), ptr(seq_lens),
        ptr(cu_seqlens_k), num_blocks,
        ptr(out), N, Hq, Hkv, D, block_size,
        max_seqlen, float(scale), DTYPE_CODES[q.dtype], int(chunk_tokens),
        ptr(ws), nbytes, stream_handle(dev),
    )
    check(st, "mentat_paged_decode")
    return out
