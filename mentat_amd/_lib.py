"""ctypes binding of libmentat_hip.so (C ABI declared in include/mentat_capi.h).

torch is imported first so the library's HIP runtime dependency resolves to
the runtime torch already loaded: one HIP runtime per process, and the raw
stream handles torch hands out are valid for the library's launches.

There is no fallback: if the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmentat_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "mentat_capi.h")

MENTAT_OK = 0
MENTAT_EINVAL = -1
MENTAT_EUNSUP = -2
MENTAT_ESPACE = -3

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float
_c_u64 = ctypes.c_uint64
_c_u32 = ctypes.c_uint32

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "mentat_abi_version": (_c_int, []),
    "mentat_device_count": (_c_int, []),
    "mentat_paged_decode_workspace_bytes": (_c_size, [_c_int] * 9),
    "mentat_paged_decode_auto_chunk": (_c_int, [_c_int] * 4),
    "mentat_paged_decode": (
        _c_int,
        [
            _c_int,  # layout
            _c_void_p, _c_void_p, _c_void_p,  # q, k_cache, v_cache
            _c_void_p, _c_i64,  # block_tables, table_stride
            _c_void_p, _c_void_p,  # seq_rows, seq_lens
            _c_void_p, _c_i64,  # cu_seqlens_k, num_blocks
            _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,  # out, N, Hq, Hkv, D, block_size
            _c_int, _c_int, _c_float, _c_int, _c_int,  # max_seqlen, window_size, scale, dtype, chunk_tokens
            _c_void_p, _c_size, _c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "mentat_paged_decode_noalloc": (
        _c_int,
        [
            _c_int,  # layout
            _c_void_p, _c_void_p, _c_void_p,  # q, k_cache, v_cache
            _c_void_p, _c_i64,  # block_tables, table_stride
            _c_void_p, _c_void_p,  # seq_rows, seq_lens
            _c_void_p, _c_i64,  # cu_seqlens_k, num_blocks
            _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,  # out, N, Hq, Hkv, D, block_size
            _c_int, _c_int, _c_float, _c_int, _c_int,  # max_seqlen, window_size, scale, dtype, chunk_tokens
            _c_void_p,  # stream
        ],
    ),
    "mentat_tree_decode_workspace_bytes": (_c_size, [_c_int] * 4),
    "mentat_tree_decode": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q, k_store, v_store, block_tables
            _c_i64, _c_i64, _c_void_p, _c_int, _c_int,  # table_stride, num_blocks, items, n_shared, n_solo
            _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p,  # members, q_slot_offsets, q_slots, n_slots, out
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int,  # Nq, Hq, Hkv, D, block_size, scale, dtype
            _c_void_p, _c_size, _c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "mentat_tree_decode_counted": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q, k_store, v_store, block_tables
            _c_i64, _c_i64, _c_void_p, _c_void_p, _c_int, _c_int,  # table_stride, num_blocks, items, counts, caps
            _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p,  # members, q_slot_offsets, q_slots, max_slots, out
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int,  # Nq, Hq, Hkv, D, block_size, scale, dtype
            _c_void_p, _c_size, _c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "mentat_tree_plan": (
        _c_int,
        [
            _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_int,  # tables, table_stride, qrows, lens, N
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,  # block_size, Hkv, G, chunks, min groups, share
            _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p,  # counts, items, max_shared, max_solo, members
            _c_void_p, _c_void_p, _c_int,  # q_slot_offsets, q_slots, max_slots
        ],
    ),
    "mentat_prefill_attention": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q, k, v, out
            _c_int, _c_int, _c_int, _c_int, _c_int,  # batch, seqlen, Hq, Hkv, D
            _c_int, _c_float, _c_int, _c_void_p,  # window, scale, dtype, stream
        ],
    ),
    "mentat_rmsnorm": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # x, residual_in, residual_out, weight, out
            _c_int, _c_int, _c_float, _c_int, _c_void_p,  # rows, H, eps, dtype, stream
        ],
    ),
    "mentat_rope": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q, k, cos, sin
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,  # rows, Hq, Hk, D, dtype, stream
        ],
    ),
    "mentat_rope_qkv": (
        _c_int,
        [
            _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p,  # qkv, row_stride, q, k, v
            _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,  # cos, sin, rows, Hq, Hk, D, dtype, stream
        ],
    ),
    "mentat_silu_mul": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_i64, _c_int, _c_void_p]),
    "mentat_silu_mul_split": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_i64, _c_int, _c_int, _c_void_p],
    ),
    "mentat_rmsnorm_partials": (
        _c_int,
        [
            _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # parts, n_parts, res_in, res_out, w, out
            _c_int, _c_int, _c_float, _c_int, _c_void_p,  # rows, H, eps, dtype, stream
        ],
    ),
    "mentat_semantic_ema": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,  # dst_ptrs, hidden, init, n, H
            _c_i64, _c_float, _c_float, _c_int, _c_void_p,  # hidden_stride, mul_scale, add_scale, dtype, stream
        ],
    ),
    "mentat_semantic_similar": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,  # ptrs, parent_key, group, M, H
            _c_float, _c_int, _c_void_p, _c_size, _c_void_p, _c_void_p,  # thr, dtype, scratch, bytes, mask, stream
        ],
    ),
    "mentat_kv_append": (
        _c_int,
        [
            _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # layout, k_new, v_new, k_pool, v_pool
            _c_void_p, _c_int, _c_i64, _c_int, _c_int, _c_int,  # plan, n, n_src, Hkv, D, block_size
            _c_i64, _c_int, _c_void_p, _c_i64, _c_i64, _c_void_p,  # num_blocks, dtype, tables, stride, rows, lens
            _c_void_p,  # stream
        ],
    ),
    "mentat_rope_qkv_append": (
        _c_int,
        [
            _c_int, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p,  # layout, qkv, row_stride, q, cos, sin
            _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p,  # rows, Hq, Hk, D, k_pool, v_pool
            _c_void_p, _c_int, _c_int, _c_i64, _c_int,  # plan, n, block_size, num_blocks, dtype
            _c_void_p, _c_i64, _c_i64, _c_void_p, _c_void_p,  # tables, stride, table rows, lens, stream
        ],
    ),
    "mentat_page_copy": (
        _c_int,
        [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_void_p],
    ),
    "mentat_table_copy_rows": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_void_p, _c_void_p, _c_int, _c_i64, _c_void_p],
    ),
    "mentat_row_stats": (
        _c_int,
        [
            _c_void_p, _c_i64, _c_int, _c_int, _c_int, _c_float,  # logits, stride, R, V, dtype, temperature
            _c_float, _c_void_p, _c_void_p,  # penalty, pen_offsets, pen_ids
            _c_float, _c_int, _c_int, _c_float,  # gate_threshold, topk, do_sample, sample_temperature
            _c_float, _c_u64, _c_u64,  # top_p, seed, step
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # outputs
            _c_void_p,  # stream
        ],
    ),
    "mentat_philox4x32_10": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p]),
}

LAYOUT_REFERENCE = 0
LAYOUT_NATIVE = 1


class MentatError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


_LIB = None


def declared_symbols(header: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in the C header (for export checks)."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mentat_[a-z0-9_]+)\s*\(", text)))


def get_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise MentatError(
                f"{LIB_PATH} is missing: build it with `python -m mentat_amd.build` "
                "(there is no fallback path)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


_STATUS_TEXT = {
    MENTAT_EINVAL: "invalid argument",
    MENTAT_EUNSUP: "unsupported shape/dtype combination",
    MENTAT_ESPACE: "workspace too small",
}


def check(status: int, what: str) -> None:
    if status != MENTAT_OK:
        txt = _STATUS_TEXT.get(status, f"HIP error {status}")
        raise MentatError(f"{what} failed: {txt} (status {status})")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
