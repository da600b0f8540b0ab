/*
 * mentat_capi.h — C ABI of the MI355X (gfx950) branching-decode library
 * (libmentat_hip.so).
 *
 * Every entry point takes raw device pointers, plain integers and a
 * hipStream_t (passed as void*), launches stream-ordered work and returns an
 * int status:
 *      0                  success
 *      MENTAT_EINVAL (-1) an argument is out of range (null pointer, size <= 0 ...)
 *      MENTAT_EUNSUP (-2) the shape / dtype combination has no compiled kernel
 *      MENTAT_ESPACE (-3) the caller's workspace is smaller than required
 *      > 0                a hipError_t returned by the launch
 * The library never allocates device memory: workspaces are passed in by the
 * caller, sized with the matching *_workspace_bytes() query.
 *
 * Pool layout (identical to the reference's PagedKVCacheManager pools,
 * core/paged_kv_cache.py:124-138): pool[num_blocks][block_size][num_kv_heads][head_dim],
 * row-major, in the model dtype. Block tables are int32, one row per sequence
 * slot, `table_stride` entries per row.
 *
 * dtype codes: MENTAT_F32 = 0, MENTAT_F16 = 1, MENTAT_BF16 = 2.
 */
#ifndef MENTAT_CAPI_H
#define MENTAT_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MENTAT_OK 0
#define MENTAT_EINVAL (-1)
#define MENTAT_EUNSUP (-2)
#define MENTAT_ESPACE (-3)

#define MENTAT_F32 0
#define MENTAT_F16 1
#define MENTAT_BF16 2

/* ABI version of this header; bumped on any signature change. */
int mentat_abi_version(void);

/* Number of HIP devices visible to the library's runtime (negative on error). */
int mentat_device_count(void);

/* ------------------------------------------------------------------------
 * Paged decode attention (one query token per sequence).
 *
 * Replaces the pair build_packed_kv + attn_decode of the reference:
 *   core/paged_kv_cache.py:289-368   (gather of every cached token into a
 *                                      packed [sum_ctx, Hkv, D] copy)
 *   adapters/attention_backend.py:192-229 (flash_attn_varlen_func, or the
 *                                      per-sequence SDPA loop at :99-168)
 * Semantics: for sequence i, query head h attends to ALL of its cached
 * tokens (the token appended this step included) with kv head
 * h / (Hq/Hkv) and softmax scale `scale`:  out[i,h] = softmax(q·Kᵀ·scale)·V.
 *
 * Two addressing modes:
 *   paged  (block_tables != NULL): token t of sequence i lives in
 *          k_cache[block_tables[row*table_stride + t/block_size]][t%block_size],
 *          row = seq_rows ? seq_rows[i] : i, length = seq_lens[row].
 *          Reads the pages in place (no gather copy).
 *   packed (block_tables == NULL): the reference's varlen layout,
 *          k_cache = packed [total, Hkv, D], token t of sequence i at row
 *          cu_seqlens_k[i] + t, length = cu_seqlens_k[i+1] - cu_seqlens_k[i].
 *
 * q, out: [N, Hq, D] contiguous, dtype. Long contexts are split into
 * chunks of `chunk_tokens` (0 = automatic) whose partial softmax states are
 * merged in a second kernel through `workspace`.
 * Page ids outside [0, num_blocks) are skipped (treated as masked) rather
 * than read.
 * ---------------------------------------------------------------------- */
size_t mentat_paged_decode_workspace_bytes(int N, int Hq, int Hkv, int D, int block_size,
                                           int max_seqlen, int chunk_tokens);

int mentat_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, int64_t table_stride,
                        const int32_t* seq_rows, const int32_t* seq_lens,
                        const int32_t* cu_seqlens_k, int64_t num_blocks,
                        void* out, int N, int Hq, int Hkv, int D, int block_size,
                        int max_seqlen, float scale, int dtype, int chunk_tokens,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The chunk length (tokens) mentat_paged_decode uses when chunk_tokens == 0. */
int mentat_paged_decode_auto_chunk(int N, int Hkv, int block_size, int max_seqlen);

#ifdef __cplusplus
}
#endif

#endif /* MENTAT_CAPI_H */
