"""Tensor-level wrappers over the C ABI (include/mentat_capi.h).

Each wrapper validates shapes, dtypes and devices on the host (a kernel is
never launched on operands that do not match what its grid assumes), then
calls the library on torch's current stream.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from ._lib import (
    DTYPE_CODES,
    LAYOUT_NATIVE,
    LAYOUT_REFERENCE,
    MENTAT_ESPACE,
    MentatError,
    check,
    get_lib,
    ptr,
    stream_handle,
)
from . import tree_plan

__all__ = [
    "paged_decode",
    "prefill_attention",
    "semantic_ema",
    "semantic_similar_mask",
    "tree_decode",
    "kv_append",
    "page_copy",
    "table_copy_rows",
    "row_stats",
    "RowStats",
    "philox4x32_10",
    "MentatError",
    "workspace",
    "LAYOUT_NATIVE",
    "LAYOUT_REFERENCE",
    "PLAN_FIELDS",
]

# Rows of the int32 [7, n] append plan (see mentat_kv_append in include/mentat_capi.h).
PLAN_FIELDS = ("dst_block", "dst_slot", "cow_src", "row", "page", "new_len", "src_tok")

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
    layout: int = LAYOUT_REFERENCE,
    window_size: Optional[int] = None,
) -> torch.Tensor:
    """One-query-per-sequence attention over a paged (or packed varlen) KV cache.

    Paged mode (``block_tables`` given): k_cache/v_cache are pools
    ``[num_blocks, block_size, Hkv, D]`` (``layout=LAYOUT_REFERENCE``), or the
    native stores K ``[num_blocks, Hkv, block_size, D]`` and V
    ``[num_blocks, Hkv, D, block_size]`` (``layout=LAYOUT_NATIVE``, 16-bit
    dtypes, block_size a multiple of 16); sequence i uses table row
    ``seq_rows[i]`` (or i) and has ``seq_lens[row]`` tokens.
    Packed mode: k_cache/v_cache are ``[total, Hkv, D]`` and ``cu_seqlens_k``
    (int32, N+1) delimits the sequences, as in the reference's
    ``build_packed_kv`` output (core/paged_kv_cache.py:289-368).

    ``max_seqlen`` must be >= every sequence length (it sizes the split-K grid).
    ``window_size`` (positive, or None for the whole context): sequence i of
    length len attends to its last window_size tokens, [max(0, len - w), len),
    as flash_attn_varlen_func(causal=True, window_size=(w - 1, 0)) does in the
    reference's decode (adapters/attention_backend.py:219-228).
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
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    window = 0 if window_size is None else int(window_size)
    _require(window_size is None or window > 0, "window_size must be positive")
    if layout == LAYOUT_NATIVE:
        _require(block_tables is not None, "the native layout needs block_tables")
        _require(q.dtype in (torch.bfloat16, torch.float16), "the native layout needs a 16-bit dtype")
        _require(k_cache.dim() == 4 and v_cache.dim() == 4, "native stores are 4-d")
        num_blocks, Hkv, block_size, Dk = k_cache.shape
        _require(tuple(v_cache.shape) == (num_blocks, Hkv, Dk, block_size),
                 "native V store must be [num_blocks, Hkv, D, block_size]")
        _require(block_size % 16 == 0, "the native layout needs block_size % 16 == 0")
    else:
        _require(layout == LAYOUT_REFERENCE, f"unknown layout {layout}")
        _require(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
    if block_tables is not None:
        if layout == LAYOUT_REFERENCE:
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
    nbytes = lib.mentat_paged_decode_workspace_bytes(layout, N, Hq, Hkv, D, block_size, max_seqlen, window,
                                                     chunk_tokens)
    ws = workspace(dev, nbytes) if nbytes else None
    st = lib.mentat_paged_decode(
        layout, ptr(q), ptr(k_cache), ptr(v_cache),
        ptr(block_tables), stride,
        ptr(seq_rows), ptr(seq_lens),
        ptr(cu_seqlens_k), num_blocks,
        ptr(out), N, Hq, Hkv, D, block_size,
        max_seqlen, window, float(scale), DTYPE_CODES[q.dtype], int(chunk_tokens),
        ptr(ws), nbytes, stream_handle(dev),
    )
    check(st, "mentat_paged_decode")
    return out


# query heads per kv head that the prefill kernels take, per dtype
PREFILL_GROUPS = {torch.bfloat16: (1, 2, 4, 8, 16), torch.float16: (1, 2, 4, 8, 16), torch.float32: (1, 2, 4, 8)}


def prefill_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    window_size: Optional[int] = None,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal (optionally sliding-window) GQA attention over a batch of prompts.

    q [B, S, Hq, D], k/v [B, S, Hkv, D] (D in {64, 128}; bf16 or f16 with
    Hq/Hkv in {1, 2, 4, 8, 16} on the MFMA kernel, fp32 with Hq/Hkv in
    {1, 2, 4, 8} on the VALU kernel); position i attends to keys
    max(0, i - window_size + 1) .. i (all of 0 .. i when window_size is None
    or >= S), softmax scale D^-1/2 by default. Returns [B, S, Hq, D].
    """
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be [B, S, H, D]")
    B, S, Hq, D = q.shape
    _require(k.shape == v.shape and k.shape[0] == B and k.shape[1] == S and k.shape[3] == D,
             f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    Hkv = k.shape[2]
    dev = q.device
    _require(dev.type == "cuda", "prefill_attention runs on the GPU only (q is on the CPU)")
    _require(q.dtype in PREFILL_GROUPS, f"prefill_attention needs bf16/f16/fp32, got {q.dtype}")
    _require(k.dtype == q.dtype and v.dtype == q.dtype, "q/k/v dtypes differ")
    _require(k.device == dev and v.device == dev, "q/k/v devices differ")
    _require(D in (64, 128), f"head_dim {D} not supported (64, 128)")
    _require(Hq % Hkv == 0 and Hq // Hkv in PREFILL_GROUPS[q.dtype], f"Hq/Hkv = {Hq}/{Hkv} not supported")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if out is None:
        out = torch.empty_like(q)
    else:
        _require(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    if B == 0 or S == 0:
        return out
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    window = 0 if window_size is None else int(window_size)
    _require(window_size is None or window > 0, "window_size must be positive")
    st = get_lib().mentat_prefill_attention(ptr(q), ptr(k), ptr(v), ptr(out), B, S, Hq, Hkv, D, window,
                                            float(scale), DTYPE_CODES[q.dtype], stream_handle(dev))
    check(st, "mentat_prefill_attention")
    return out


_GLUE_DTYPES = (torch.bfloat16, torch.float16)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None):
    """HF RMSNorm of the rows of ``x`` (last dim H), or of ``residual + x``
    when ``residual`` is given (the residual add fused in). Returns
    ``(out, h)`` with h = residual + x (None without a residual). 16-bit
    dtypes; torch's rounding per op (mentat_rmsnorm)."""
    _require(x.dtype in _GLUE_DTYPES and weight.dtype == x.dtype, "rmsnorm takes bf16/f16 x and weight")
    _require(x.is_contiguous() and weight.is_contiguous() and weight.dim() == 1, "contiguous x and 1-d weight")
    H = x.shape[-1]
    _require(weight.numel() == H, "weight length must match the last dim")
    rows = x.numel() // H
    out = torch.empty_like(x)
    h = None
    if residual is not None:
        _require(residual.shape == x.shape and residual.dtype == x.dtype and residual.is_contiguous(),
                 "residual must match x")
        h = torch.empty_like(x)
    st = get_lib().mentat_rmsnorm(ptr(x), ptr(residual), ptr(h), ptr(weight), ptr(out), rows, H, float(eps),
                                  DTYPE_CODES[x.dtype], stream_handle(x.device))
    check(st, "mentat_rmsnorm")
    return out, h


def rope_(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """Rotary embedding in place: q [..., Hq, D] and k [..., Hk, D] (same
    leading rows), cos/sin with D trailing elements per row;
    t = t*cos + rotate_half(t)*sin with torch's rounding (mentat_rope)."""
    _require(q.dtype in _GLUE_DTYPES and k.dtype == q.dtype and cos.dtype == q.dtype and sin.dtype == q.dtype,
             "rope takes bf16/f16 tensors of one dtype")
    _require(q.is_contiguous() and k.is_contiguous() and cos.is_contiguous() and sin.is_contiguous(),
             "rope takes contiguous tensors")
    D = q.shape[-1]
    rows = cos.numel() // D
    _require(sin.numel() == rows * D and q.numel() % (rows * D) == 0 and k.numel() % (rows * D) == 0,
             "q, k, cos and sin must share the leading rows")
    Hq, Hk = q.numel() // (rows * D), k.numel() // (rows * D)
    st = get_lib().mentat_rope(ptr(q), ptr(k), ptr(cos), ptr(sin), rows, Hq, Hk, D, DTYPE_CODES[q.dtype],
                               stream_handle(q.device))
    check(st, "mentat_rope")


def rope_qkv(qkv: torch.Tensor, Hq: int, Hk: int, cos: torch.Tensor, sin: torch.Tensor):
    """Split a merged q/k/v projection output (rows of Hq + 2 Hk heads of D,
    last dim dense) into dense q [rows, Hq, D], k and v [rows, Hk, D], with
    RoPE applied to q and k (mentat_rope_qkv)."""
    _require(qkv.dtype in _GLUE_DTYPES and cos.dtype == qkv.dtype and sin.dtype == qkv.dtype,
             "rope_qkv takes bf16/f16 tensors of one dtype")
    _require(qkv.stride(-1) == 1 and cos.is_contiguous() and sin.is_contiguous(), "dense rows required")
    D = cos.shape[-1]
    rows = cos.numel() // D
    W = (Hq + 2 * Hk) * D
    _require(qkv.shape[-1] == W and qkv.numel() == rows * W and qkv.is_contiguous(),
             "qkv must be contiguous [rows, (Hq + 2 Hk) * D]")
    q = torch.empty(rows, Hq, D, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty(rows, Hk, D, dtype=qkv.dtype, device=qkv.device)
    v = torch.empty(rows, Hk, D, dtype=qkv.dtype, device=qkv.device)
    st = get_lib().mentat_rope_qkv(ptr(qkv), W, ptr(q), ptr(k), ptr(v), ptr(cos), ptr(sin), rows, Hq, Hk, D,
                                   DTYPE_CODES[qkv.dtype], stream_handle(qkv.device))
    check(st, "mentat_rope_qkv")
    return q, k, v


def rope_qkv_append(
    qkv: torch.Tensor,
    Hq: int,
    Hk: int,
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_store: torch.Tensor,
    v_store: torch.Tensor,
    plan: torch.Tensor,
    *,
    block_size: int,
    layout: int = LAYOUT_REFERENCE,
    block_tables: Optional[torch.Tensor] = None,
    seq_lens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """:func:`rope_qkv` followed by :func:`kv_append` of its k and v in one
    launch (mentat_rope_qkv_append): returns the rotated q [rows, Hq, D]; the
    rotated k and the v of each plan column's source row go straight into the
    stores (same bits as the two calls)."""
    _require(qkv.dtype in _GLUE_DTYPES and cos.dtype == qkv.dtype and sin.dtype == qkv.dtype,
             "rope_qkv_append takes bf16/f16 tensors of one dtype")
    _require(cos.is_contiguous() and sin.is_contiguous(), "dense cos / sin rows required")
    D = cos.shape[-1]
    rows = cos.numel() // D
    W = (Hq + 2 * Hk) * D
    _require(qkv.shape[-1] == W and qkv.numel() == rows * W and qkv.is_contiguous(),
             "qkv must be contiguous [rows, (Hq + 2 Hk) * D]")
    dev = qkv.device
    _require(k_store.device == dev and v_store.device == dev, "qkv and the stores must share a device")
    _require(k_store.dtype == qkv.dtype and v_store.dtype == qkv.dtype, "store dtype differs from qkv")
    _require(k_store.is_contiguous() and v_store.is_contiguous(), "stores must be contiguous")
    _require(plan.dim() == 2 and plan.shape[0] == len(PLAN_FIELDS), "plan must be int32 [7, n]")
    _check_i32(plan, "plan", dev)
    _check_i32(block_tables, "block_tables", dev)
    _check_i32(seq_lens, "seq_lens", dev)
    num_blocks = k_store.shape[0]
    if layout == LAYOUT_NATIVE:
        _require(tuple(k_store.shape) == (num_blocks, Hk, block_size, D), "bad native K store")
        _require(tuple(v_store.shape) == (num_blocks, Hk, D, block_size), "bad native V store")
    else:
        _require(tuple(k_store.shape) == (num_blocks, block_size, Hk, D), "bad K pool")
        _require(tuple(v_store.shape) == (num_blocks, block_size, Hk, D), "bad V pool")
    trows = stride = 0
    if block_tables is not None:
        _require(block_tables.dim() == 2, "block_tables must be [rows, stride]")
        trows, stride = block_tables.shape
        _require(block_tables.stride(0) == stride, "block_tables rows must be dense")
        if seq_lens is not None:
            _require(seq_lens.numel() >= trows, "seq_lens shorter than block_tables")
    elif seq_lens is not None:
        trows = seq_lens.numel()
    q = torch.empty(rows, Hq, D, dtype=qkv.dtype, device=dev)
    st = get_lib().mentat_rope_qkv_append(
        layout, ptr(qkv), W, ptr(q), ptr(cos), ptr(sin), rows, Hq, Hk, D, ptr(k_store), ptr(v_store), ptr(plan),
        plan.shape[1], block_size, num_blocks, DTYPE_CODES[qkv.dtype], ptr(block_tables), stride, trows,
        ptr(seq_lens), stream_handle(dev),
    )
    check(st, "mentat_rope_qkv_append")
    return q


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with torch's rounding per op (mentat_silu_mul)."""
    _require(gate.dtype in _GLUE_DTYPES and up.dtype == gate.dtype and up.shape == gate.shape,
             "silu_mul takes bf16/f16 tensors of one shape")
    _require(gate.is_contiguous() and up.is_contiguous(), "silu_mul takes contiguous tensors")
    out = torch.empty_like(gate)
    F = gate.shape[-1]
    st = get_lib().mentat_silu_mul(ptr(gate), ptr(up), ptr(out), gate.numel() // F, F, F, DTYPE_CODES[gate.dtype],
                                   stream_handle(gate.device))
    check(st, "mentat_silu_mul")
    return out


def silu_mul_merged(gu: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up from a merged gate/up projection output [..., 2F]
    (gate = first half of each row, up = second half): [..., F]."""
    _require(gu.dtype in _GLUE_DTYPES and gu.is_contiguous() and gu.shape[-1] % 2 == 0,
             "silu_mul_merged takes a contiguous bf16/f16 [..., 2F] tensor")
    F = gu.shape[-1] // 2
    rows = gu.numel() // (2 * F)
    out = torch.empty(*gu.shape[:-1], F, dtype=gu.dtype, device=gu.device)
    st = get_lib().mentat_silu_mul(ptr(gu), gu.data_ptr() + F * gu.element_size(), ptr(out), rows, F, 2 * F,
                                   DTYPE_CODES[gu.dtype], stream_handle(gu.device))
    check(st, "mentat_silu_mul")
    return out


def silu_mul_merged_split(gu: torch.Tensor, split: int) -> torch.Tensor:
    """silu_mul_merged of a [rows, 2F] projection output, returned as the
    column slices [split, rows, F / split] that a split-K down projection
    takes as its batched left operand (mentat_silu_mul_split)."""
    _require(gu.dtype in _GLUE_DTYPES and gu.is_contiguous() and gu.dim() == 2 and gu.shape[-1] % 2 == 0,
             "silu_mul_merged_split takes a contiguous bf16/f16 [rows, 2F] tensor")
    F = gu.shape[-1] // 2
    rows = gu.shape[0]
    _require(split >= 1 and F % (8 * split) == 0, "F must split into slices of a multiple of 8")
    out = torch.empty(split, rows, F // split, dtype=gu.dtype, device=gu.device)
    st = get_lib().mentat_silu_mul_split(ptr(gu), gu.data_ptr() + F * gu.element_size(), ptr(out), rows, F, 2 * F,
                                         split, DTYPE_CODES[gu.dtype], stream_handle(gu.device))
    check(st, "mentat_silu_mul_split")
    return out


def rmsnorm_partials(parts: torch.Tensor, weight: torch.Tensor, eps: float,
                     residual: Optional[torch.Tensor] = None):
    """rmsnorm of x = the sum of the fp32 partial products ``parts``
    [S, rows, H] (S in 2, 4, 8) rounded once to weight's dtype, with the
    residual add fused in as in rmsnorm. Returns ``(out, h)``
    (mentat_rmsnorm_partials)."""
    _require(parts.dtype == torch.float32 and parts.is_contiguous() and parts.dim() == 3,
             "rmsnorm_partials takes contiguous fp32 partials [S, rows, H]")
    _require(weight.dtype in _GLUE_DTYPES and weight.is_contiguous() and weight.dim() == 1
             and weight.numel() == parts.shape[2], "weight must be a bf16/f16 vector of length H")
    S, rows, H = parts.shape
    out = torch.empty(rows, H, dtype=weight.dtype, device=parts.device)
    h = None
    if residual is not None:
        _require(residual.shape == (rows, H) and residual.dtype == weight.dtype and residual.is_contiguous(),
                 "residual must be [rows, H] of weight's dtype")
        h = torch.empty_like(residual)
    st = get_lib().mentat_rmsnorm_partials(ptr(parts), S, ptr(residual), ptr(h), ptr(weight), ptr(out), rows, H,
                                           float(eps), DTYPE_CODES[weight.dtype], stream_handle(parts.device))
    check(st, "mentat_rmsnorm_partials")
    return out, h


def semantic_ema(vectors: list, hidden: torch.Tensor, fresh: list, alpha: float) -> None:
    """Fold row i of ``hidden`` [n, H] into ``vectors[i]`` (an H-element
    contiguous tensor on the same device, updated in place): copied when
    ``fresh[i]``, else ``v.mul_(1 - alpha).add_(h, alpha=alpha)`` with torch's
    rounding. One launch for all rows."""
    n = len(vectors)
    if n == 0:
        return
    _require(hidden.dim() == 2 and hidden.shape[0] == n and hidden.stride(1) == 1, "hidden must be [n, H], rows dense")
    _require(hidden.dtype in DTYPE_CODES, f"unsupported dtype {hidden.dtype}")
    dev, H = hidden.device, hidden.shape[1]
    _require(dev.type == "cuda", "semantic_ema runs on the GPU only")
    for v in vectors:
        _require(v.dtype == hidden.dtype and v.device == dev and v.is_contiguous() and v.numel() == H,
                 "every vector must be a contiguous H-element tensor of hidden's dtype and device")
    # pinned + asynchronous: the host does not wait for queued GPU work here
    meta = torch.tensor([v.data_ptr() for v in vectors] + [int(bool(f)) for f in fresh], dtype=torch.int64)
    meta = meta.pin_memory().to(dev, non_blocking=True)
    init = meta[n:].to(torch.int32)
    st = get_lib().mentat_semantic_ema(ptr(meta), ptr(hidden), ptr(init), n, H, hidden.stride(0),
                                       float(np.float32(1.0 - alpha)), float(np.float32(alpha)),
                                       DTYPE_CODES[hidden.dtype], stream_handle(dev))
    check(st, "mentat_semantic_ema")


def semantic_similar_mask(vectors: list, parent_key: list, group: list, threshold: float,
                          wait: bool = True):
    """Host bool [M, M]: entry (i, j) is set iff i < j, same group, different
    parent key, and the cosine similarity of the two vectors (F.normalize +
    mm in their dtype) exceeds ``threshold``. With ``wait=False`` the mask is
    returned as a pinned uint8 [M, M] tensor whose copy is still in flight on
    the current stream (read it after that stream's next synchronisation)."""
    M = len(vectors)
    if M == 0:
        return np.zeros((0, 0), dtype=bool) if wait else torch.zeros(0, 0, dtype=torch.uint8)
    dev, dt = vectors[0].device, vectors[0].dtype
    H = vectors[0].numel()
    _require(dev.type == "cuda", "semantic_similar_mask runs on the GPU only")
    _require(dt in DTYPE_CODES, f"unsupported dtype {dt}")
    for v in vectors:
        _require(v.dtype == dt and v.device == dev and v.is_contiguous() and v.numel() == H,
                 "vectors must be contiguous, of one dtype, device and length")
    meta = torch.tensor([v.data_ptr() for v in vectors] + [int(k) for k in parent_key] + [int(g) for g in group],
                        dtype=torch.int64).pin_memory().to(dev, non_blocking=True)
    keys = meta[M:].to(torch.int32)
    scratch = torch.empty(M * H, dtype=dt, device=dev)
    mask = torch.empty(M * M, dtype=torch.uint8, device=dev)
    st = get_lib().mentat_semantic_similar(ptr(meta), ptr(keys[:M]), ptr(keys[M:]), M, H, float(threshold),
                                           DTYPE_CODES[dt], ptr(scratch), scratch.numel() * scratch.element_size(),
                                           ptr(mask), stream_handle(dev))
    check(st, "mentat_semantic_similar")
    if not wait:
        host = torch.empty(M * M, dtype=torch.uint8, pin_memory=True)
        host.copy_(mask, non_blocking=True)
        return host.view(M, M)
    return mask.cpu().numpy().reshape(M, M).astype(bool)


def kv_append(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_store: torch.Tensor,
    v_store: torch.Tensor,
    plan: torch.Tensor,
    *,
    block_size: int,
    layout: int = LAYOUT_REFERENCE,
    block_tables: Optional[torch.Tensor] = None,
    seq_lens: Optional[torch.Tensor] = None,
) -> None:
    """Write new token rows into the pools per ``plan`` (int32 [7, n], PLAN_FIELDS).

    Fused with the lazy copy-on-write of shared tail pages and the device
    table/length update of this layer (``block_tables`` [rows, stride],
    ``seq_lens`` [rows]). k_new/v_new: [n_src, Hkv, D].
    """
    dev = k_store.device
    _require(dev.type == "cuda", "kv_append runs on the GPU only")
    _require(plan.dim() == 2 and plan.shape[0] == len(PLAN_FIELDS), "plan must be int32 [7, n]")
    _check_i32(plan, "plan", dev)
    _check_i32(block_tables, "block_tables", dev)
    _check_i32(seq_lens, "seq_lens", dev)
    _require(k_new.dim() == 3 and k_new.shape == v_new.shape, "k_new/v_new must be [n, Hkv, D]")
    _require(k_new.is_contiguous() and v_new.is_contiguous(), "k_new/v_new must be contiguous")
    _require(k_new.dtype == k_store.dtype == v_store.dtype == v_new.dtype, "dtype mismatch")
    _require(k_store.is_contiguous() and v_store.is_contiguous(), "stores must be contiguous")
    n_src, Hkv, D = k_new.shape
    num_blocks = k_store.shape[0]
    if layout == LAYOUT_NATIVE:
        _require(tuple(k_store.shape) == (num_blocks, Hkv, block_size, D), "bad native K store")
        _require(tuple(v_store.shape) == (num_blocks, Hkv, D, block_size), "bad native V store")
    else:
        _require(tuple(k_store.shape) == (num_blocks, block_size, Hkv, D), "bad K pool")
        _require(tuple(v_store.shape) == (num_blocks, block_size, Hkv, D), "bad V pool")
    n = plan.shape[1]
    if n == 0:
        return
    rows = stride = 0
    if block_tables is not None:
        _require(block_tables.dim() == 2, "block_tables must be [rows, stride]")
        rows, stride = block_tables.shape
        _require(block_tables.stride(0) == stride, "block_tables rows must be dense")
        if seq_lens is not None:
            _require(seq_lens.numel() >= rows, "seq_lens shorter than block_tables")
    elif seq_lens is not None:
        rows = seq_lens.numel()
    st = get_lib().mentat_kv_append(
        layout, ptr(k_new), ptr(v_new), ptr(k_store), ptr(v_store), ptr(plan), n, n_src, Hkv, D,
        block_size, num_blocks, DTYPE_CODES[k_store.dtype], ptr(block_tables), stride, rows,
        ptr(seq_lens), stream_handle(dev),
    )
    check(st, "mentat_kv_append")


def page_copy(pools: list, src: torch.Tensor, dst: torch.Tensor) -> None:
    """dst[i] <- src[i] (whole pages) in every pool of ``pools`` with one launch."""
    if not pools or src.numel() == 0:
        return
    dev = pools[0].device
    _check_i32(src, "src", dev)
    _check_i32(dst, "dst", dev)
    _require(src.numel() == dst.numel(), "src/dst lengths differ")
    nb = pools[0].shape[0]
    bb = pools[0][0].numel() * pools[0].element_size()
    for t in pools:
        _require(t.is_contiguous() and t.device == dev, "pools must be contiguous on one device")
        _require(t.shape[0] == nb and t[0].numel() * t.element_size() == bb, "pools differ in geometry")
    ptrs = torch.tensor([t.data_ptr() for t in pools], dtype=torch.int64, device=dev)
    st = get_lib().mentat_page_copy(ptr(ptrs), len(pools), ptr(src), ptr(dst), src.numel(), bb, nb,
                                    stream_handle(dev))
    check(st, "mentat_page_copy")


def table_copy_rows(tables: torch.Tensor, seq_lens: Optional[torch.Tensor], src_rows: torch.Tensor,
                    dst_rows: torch.Tensor, n_entries: int) -> None:
    """tables[:, dst] <- tables[:, src] (first n_entries entries) and lengths, all layers."""
    if src_rows.numel() == 0:
        return
    dev = tables.device
    _check_i32(tables, "tables", dev)
    _check_i32(seq_lens, "seq_lens", dev)
    _check_i32(src_rows, "src_rows", dev)
    _check_i32(dst_rows, "dst_rows", dev)
    _require(tables.dim() == 3, "tables must be [L, rows, stride]")
    L, rows, stride = tables.shape
    if seq_lens is not None:
        _require(tuple(seq_lens.shape) == (L, rows), "seq_lens must be [L, rows]")
    _require(0 <= n_entries <= stride, "n_entries out of range")
    st = get_lib().mentat_table_copy_rows(ptr(tables), ptr(seq_lens), L, rows, stride, ptr(src_rows),
                                          ptr(dst_rows), src_rows.numel(), n_entries, stream_handle(dev))
    check(st, "mentat_table_copy_rows")


@dataclass
class RowStats:
    entropy: torch.Tensor                 # [R] f32, entropy of softmax(x / T), rounded as torch in the dtype
    entropy_f32: Optional[torch.Tensor]   # [R] f32, the same with fp32 arithmetic (no dtype rounding)
    gate: torch.Tensor                    # [R] u8, entropy > gate_threshold
    entropy_pen: Optional[torch.Tensor]   # [R] f32, entropy of softmax(xp)
    lse: Optional[torch.Tensor]           # [R] f32, log-sum-exp of xp
    topk_ids: Optional[torch.Tensor]      # [R, K] i32
    topk_lp: Optional[torch.Tensor]       # [R, K] f32
    sample: Optional[torch.Tensor]        # [R] i32


def row_stats(
    logits: torch.Tensor,
    *,
    temperature: float = 1.0,
    penalty: float = 1.0,
    pen_offsets: Optional[torch.Tensor] = None,
    pen_ids: Optional[torch.Tensor] = None,
    gate_threshold: float = float("inf"),
    topk: int = 0,
    sample: bool = False,
    sample_temperature: float = 1.0,
    top_p: float = 1.0,
    seed: int = 0,
    step: int = 0,
    pen_stats: Optional[bool] = None,
    entropy_f32: bool = False,
) -> RowStats:
    """Fused per-row entropy, gate, repetition penalty, top-K and top-p draw
    (mentat_row_stats in include/mentat_capi.h) over logits [R, V].

    ``pen_stats`` (default: ``topk > 0``) also returns the entropy and
    log-sum-exp of the penalised row (``entropy_pen``, ``lse``; None otherwise).
    ``entropy`` is rounded as the reference's compute_entropy is in the logits
    dtype; ``entropy_f32=True`` also returns it computed in fp32 throughout.
    """
    if pen_stats is None:
        pen_stats = topk > 0
    _require(logits.dim() == 2, "logits must be [R, V]")
    dev = logits.device
    _require(dev.type == "cuda", "row_stats runs on the GPU only")
    _require(logits.dtype in DTYPE_CODES, f"unsupported dtype {logits.dtype}")
    _require(logits.stride(1) == 1, "logits rows must be contiguous")
    R, V = logits.shape
    _require(0 <= topk <= 8, "topk must be in [0, 8]")
    _require(topk <= V, "topk larger than the vocabulary")
    _require(temperature > 0, "temperature must be > 0")
    if pen_offsets is not None:
        _check_i32(pen_offsets, "pen_offsets", dev)
        _check_i32(pen_ids, "pen_ids", dev)
        _require(pen_offsets.numel() == R + 1, "pen_offsets must have R+1 entries")
    if sample:
        _require(sample_temperature > 0 and 0 < top_p <= 1, "bad sampling parameters")
    f32 = dict(dtype=torch.float32, device=dev)
    out = RowStats(
        entropy=torch.empty(R, **f32),
        entropy_f32=torch.empty(R, **f32) if entropy_f32 else None,
        gate=torch.empty(R, dtype=torch.uint8, device=dev),
        entropy_pen=torch.empty(R, **f32) if pen_stats else None,
        lse=torch.empty(R, **f32) if pen_stats else None,
        topk_ids=torch.empty(R, topk, dtype=torch.int32, device=dev) if topk else None,
        topk_lp=torch.empty(R, topk, **f32) if topk else None,
        sample=torch.full((R,), -1, dtype=torch.int32, device=dev) if sample else None,
    )
    if R == 0:
        return out
    st = get_lib().mentat_row_stats(
        ptr(logits), logits.stride(0), R, V, DTYPE_CODES[logits.dtype], float(temperature),
        float(penalty), ptr(pen_offsets), ptr(pen_ids),
        float(gate_threshold), int(topk), int(bool(sample)), float(sample_temperature),
        float(top_p), int(seed) & (2**64 - 1), int(step) & (2**64 - 1),
        ptr(out.entropy), ptr(out.entropy_f32), ptr(out.entropy_pen), ptr(out.lse), ptr(out.gate),
        ptr(out.topk_ids), ptr(out.topk_lp), ptr(out.sample), stream_handle(dev),
    )
    check(st, "mentat_row_stats")
    return out


def philox4x32_10(counters: torch.Tensor, keys: torch.Tensor) -> torch.Tensor:
    """Philox4x32-10 blocks on the device: counters int32/uint32 [n, 4], keys [n, 2]."""
    dev = counters.device
    _require(counters.dim() == 2 and counters.shape[1] == 4, "counters must be [n, 4]")
    _require(keys.shape == (counters.shape[0], 2), "keys must be [n, 2]")
    c = counters.contiguous().to(torch.int32)
    k = keys.contiguous().to(torch.int32)
    out = torch.empty_like(c)
    st = get_lib().mentat_philox4x32_10(ptr(c), ptr(k), ptr(out), c.shape[0], stream_handle(dev))
    check(st, "mentat_philox4x32_10")
    return out


class TreePlanBuffers:
    """Device arrays of prefix-tree plans with fixed capacities, refilled per
    call (for launches captured once and replayed with new plans): one int32
    buffer holding counts [2], q_slot_offsets [Nq * Hkv + 1], items
    [max_items, 8], members [max_slots] and q_slots [max_slots], and a pinned
    host twin the plan is written into; upload copies the parts in use."""

    def __init__(self, device, Nq: int, Hkv: int, max_shared: int, max_solo: int, max_slots: int):
        self.Nq, self.Hkv = Nq, Hkv
        self.max_shared, self.max_solo, self.max_slots = max_shared, max_solo, max_slots
        mi = max_shared + max_solo
        # regions: counts | q_slot_offsets | items | members | q_slots
        self._cuts = np.cumsum([0, 2, Nq * Hkv + 1, 8 * max(mi, 1), max(max_slots, 1), max(max_slots, 1)])
        n = int(self._cuts[-1])
        self.host = torch.zeros(n, dtype=torch.int32, pin_memory=True)
        self.host_np = self.host.numpy()
        self.dev = torch.zeros(n, dtype=torch.int32, device=device)
        c = self._cuts
        self.counts = self.dev[c[0]:c[1]]
        self.q_slot_offsets = self.dev[c[1]:c[2]]
        self.items = self.dev[c[2]:c[3]]
        self.members = self.dev[c[3]:c[4]]
        self.q_slots = self.dev[c[4]:c[5]]
        self._used = (mi, max_slots)  # items and slots the last plan holds

    def fits(self, plan) -> bool:
        return plan.n_shared <= self.max_shared and plan.n_solo <= self.max_solo and plan.n_slots <= self.max_slots

    def write(self, plan, n: int) -> None:
        """Plan of n <= Nq queries into the host twin (queries n .. Nq - 1 get no slots)."""
        _require(self.fits(plan), "the plan exceeds the buffers' capacities")
        c, h = self._cuts, self.host_np
        h[0], h[1] = plan.n_shared, plan.n_solo
        off = h[c[1]:c[2]]
        off[:n * self.Hkv + 1] = plan.q_slot_offsets
        off[n * self.Hkv + 1:] = plan.q_slot_offsets[-1]
        k = plan.items.size
        h[c[2]:c[2] + k] = plan.items.reshape(-1)
        h[c[3]:c[3] + plan.n_slots] = plan.members[:plan.n_slots]
        h[c[4]:c[4] + plan.n_slots] = plan.q_slots[:plan.n_slots]
        self._used = (plan.items.shape[0], plan.n_slots)

    def upload(self) -> None:
        """Queue the copies of the parts the last plan uses (three copies)."""
        c = self._cuts
        items, slots = self._used
        a = int(c[2]) + 8 * items
        self.dev[:a].copy_(self.host[:a], non_blocking=True)
        if slots:
            for lo in (int(c[3]), int(c[4])):
                self.dev[lo:lo + slots].copy_(self.host[lo:lo + slots], non_blocking=True)

    def plan(self, tables: np.ndarray, qrows: np.ndarray, lens: np.ndarray, block_size: int, G: int,
             chunk_tiles: int = tree_plan.CHUNK_TILES, shared_chunk_tiles: int = tree_plan.SHARED_CHUNK_TILES,
             shared_min_groups: int = tree_plan.SHARED_MIN_GROUPS) -> tuple:
        """Plan n queries with the native planner (mentat_tree_plan) straight
        into the host twin. tables: host int32 [rows, stride] block ids indexed
        by table row; qrows, lens: int32 per query. When a capacity is exceeded
        the queries get a plan without sharing (one segment each), which the
        capacities hold by construction. Returns (n_shared, n_solo, n_slots, shared)."""
        n = int(qrows.size)
        _require(n <= self.Nq, "more queries than the buffers hold")
        _require(tables.dtype == np.int32 and tables.flags.c_contiguous, "tables must be C-contiguous int32")
        qrows = np.ascontiguousarray(qrows, dtype=np.int32)
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        c, h = self._cuts, self.host_np
        base = h.ctypes.data
        cnt = np.zeros(3, dtype=np.int32)
        off = h[c[1]:c[2]]
        lib = get_lib()
        for share in (1, 0):
            st = lib.mentat_tree_plan(
                tables.ctypes.data, tables.shape[1], qrows.ctypes.data, lens.ctypes.data, n, block_size,
                self.Hkv, G, chunk_tiles, shared_chunk_tiles, shared_min_groups, share, cnt.ctypes.data,
                base + 4 * int(c[2]), self.max_shared, self.max_solo, base + 4 * int(c[3]),
                base + 4 * int(c[1]), base + 4 * int(c[4]), self.max_slots)
            if st == 0:
                break
            _require(st == MENTAT_ESPACE and share, f"mentat_tree_plan failed ({st})")
        h[0], h[1] = cnt[0], cnt[1]
        off[n * self.Hkv + 1:] = off[n * self.Hkv]
        self._used = (int(cnt[0] + cnt[1]), int(cnt[2]))
        return int(cnt[0]), int(cnt[1]), int(cnt[2]), bool(share)


def tree_decode_counted(
    q: torch.Tensor,
    k_store: torch.Tensor,
    v_store: torch.Tensor,
    *,
    block_tables: torch.Tensor,
    bufs: TreePlanBuffers,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """:func:`tree_decode` with the plan in ``bufs`` (device arrays of fixed
    capacity; mentat_tree_decode_counted reads the item counts on the device).
    The plan written there must have been validated against these tables."""
    _require(q.dim() == 3, f"q must be [N, Hq, D], got {tuple(q.shape)}")
    Nq, Hq, D = q.shape
    dev = q.device
    _require(dev.type == "cuda", "tree_decode runs on the GPU only")
    _require(q.dtype in (torch.bfloat16, torch.float16), "tree_decode needs a 16-bit dtype")
    _require(k_store.dtype == q.dtype and v_store.dtype == q.dtype, "q/k/v dtypes differ")
    _require(q.is_contiguous() and k_store.is_contiguous() and v_store.is_contiguous(),
             "q and the stores must be contiguous")
    _require(k_store.dim() == 4, "native K store must be [num_blocks, Hkv, block_size, D]")
    num_blocks, Hkv, block_size, Dk = k_store.shape
    _require(tuple(v_store.shape) == (num_blocks, Hkv, Dk, block_size),
             "native V store must be [num_blocks, Hkv, D, block_size]")
    _require(Dk == D and Hq % Hkv == 0 and 16 % (Hq // Hkv) == 0, "bad head geometry")
    _require(block_tables.dim() == 2 and block_tables.stride(1) == 1, "block_tables must be [rows, stride]")
    _check_i32(block_tables, "block_tables", dev)
    _require(bufs.Nq == Nq and bufs.Hkv == Hkv, "the plan buffers were sized for another batch")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty_like(q)
    if Nq == 0:
        return out
    lib = get_lib()
    nbytes = lib.mentat_tree_decode_workspace_bytes(bufs.max_slots, Hq, Hkv, D)
    ws = workspace(dev, nbytes) if nbytes else None
    st = lib.mentat_tree_decode_counted(
        ptr(q), ptr(k_store), ptr(v_store), ptr(block_tables), block_tables.stride(0), num_blocks,
        ptr(bufs.items), ptr(bufs.counts), bufs.max_shared, bufs.max_solo, ptr(bufs.members),
        ptr(bufs.q_slot_offsets), ptr(bufs.q_slots), bufs.max_slots, ptr(out), Nq, Hq, Hkv, D, block_size,
        float(scale), DTYPE_CODES[q.dtype], ptr(ws), nbytes, stream_handle(dev),
    )
    check(st, "mentat_tree_decode_counted")
    return out


def tree_decode(
    q: torch.Tensor,
    k_store: torch.Tensor,
    v_store: torch.Tensor,
    *,
    block_tables: torch.Tensor,
    plan,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Prefix-shared decode attention over native stores (mentat_tree_decode).

    ``plan`` is a :class:`mentat_amd.tree_plan.TreePlan` built from the same
    batch's page tables (one layer's ``block_tables`` [rows, stride] give the
    page ids). Same result as :func:`paged_decode` on that batch.
    """
    _require(q.dim() == 3, f"q must be [N, Hq, D], got {tuple(q.shape)}")
    Nq, Hq, D = q.shape
    dev = q.device
    _require(dev.type == "cuda", "tree_decode runs on the GPU only")
    _require(q.dtype in (torch.bfloat16, torch.float16), "tree_decode needs a 16-bit dtype")
    _require(k_store.dtype == q.dtype and v_store.dtype == q.dtype, "q/k/v dtypes differ")
    _require(k_store.device == dev and v_store.device == dev, "q/k/v devices differ")
    _require(q.is_contiguous() and k_store.is_contiguous() and v_store.is_contiguous(),
             "q and the stores must be contiguous")
    _require(k_store.dim() == 4, "native K store must be [num_blocks, Hkv, block_size, D]")
    num_blocks, Hkv, block_size, Dk = k_store.shape
    _require(tuple(v_store.shape) == (num_blocks, Hkv, Dk, block_size),
             "native V store must be [num_blocks, Hkv, D, block_size]")
    _require(Dk == D, f"head_dim mismatch q {D} vs cache {Dk}")
    _require(Hq % Hkv == 0 and 16 % (Hq // Hkv) == 0, "Hq/Hkv must divide 16")
    _require(block_size % 16 == 0, "tree_decode needs block_size % 16 == 0")
    _require(block_tables.dim() == 2, "block_tables must be [rows, stride]")
    _check_i32(block_tables, "block_tables", dev)
    rows, _ = block_tables.shape
    stride = block_tables.stride(0)
    _require(block_tables.stride(1) == 1, "block_tables rows must be contiguous")
    G = Hq // Hkv
    if getattr(plan, "_validated", None) != (Nq, Hkv, G, rows, block_tables.shape[1], block_size):
        plan.validate(Nq, Hkv, G, rows, block_tables.shape[1], block_size)
        plan._validated = (Nq, Hkv, G, rows, block_tables.shape[1], block_size)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty_like(q)
    else:
        _require(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    if Nq == 0:
        return out
    items, members, off, slots = plan.device_arrays(dev)
    lib = get_lib()
    nbytes = lib.mentat_tree_decode_workspace_bytes(plan.n_slots, Hq, Hkv, D)
    ws = workspace(dev, nbytes) if nbytes else None
    st = lib.mentat_tree_decode(
        ptr(q), ptr(k_store), ptr(v_store), ptr(block_tables), stride, num_blocks,
        ptr(items), plan.n_shared, plan.n_solo, ptr(members), ptr(off), ptr(slots), plan.n_slots, ptr(out),
        Nq, Hq, Hkv, D, block_size, float(scale), DTYPE_CODES[q.dtype], ptr(ws), nbytes, stream_handle(dev),
    )
    check(st, "mentat_tree_decode")
    return out
