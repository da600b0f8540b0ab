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
 * caller, sized with the matching *_workspace_bytes() query. Every workspace
 * begins with MENTAT_WORKSPACE_RESERVED bytes of arrival counters (native
 * paged decode) that must be zero before the workspace's first use; every
 * call leaves them zero and keeps its own data after them, so one zero-filled
 * workspace per stream can serve every entry point. Calls that share a
 * workspace must be ordered (the same stream).
 *
 * Pools hold num_blocks pages of block_size tokens x num_kv_heads x head_dim
 * elements in the model dtype, in one of two layouts (MENTAT_LAYOUT_* below);
 * the reference layout is the reference's own PagedKVCacheManager pool
 * (core/paged_kv_cache.py:124-138). Block tables are int32, one row per
 * sequence slot, `table_stride` entries per row.
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

#define MENTAT_WORKSPACE_RESERVED 262144

#define MENTAT_F32 0
#define MENTAT_F16 1
#define MENTAT_BF16 2

/* Pool layouts.
 * MENTAT_LAYOUT_REFERENCE: K and V stored [num_blocks][block_size][Hkv][D]
 *   (the reference's own layout).
 * MENTAT_LAYOUT_NATIVE (16-bit dtypes, block_size a multiple of 16):
 *   K stored [num_blocks][Hkv][block_size][D], V stored [num_blocks][Hkv][D][block_size],
 *   so one (page, kv head) is contiguous and V is transposed inside it; this is
 *   the layout the MFMA decode kernel reads. */
#define MENTAT_LAYOUT_REFERENCE 0
#define MENTAT_LAYOUT_NATIVE 1

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
 * window_size > 0 restricts sequence i of length len to its last window_size
 * tokens, [max(0, len - window_size), len): the reference's window argument
 * (attention_backend.py:192-229), which flash_attn_varlen_func applies as
 * window_size=(window_size - 1, 0) with the query aligned to the end of its
 * keys. 0 attends to all tokens (the reference's window_size=None); negative
 * values return MENTAT_EINVAL.
 *
 * `layout` selects the pool layout (MENTAT_LAYOUT_*). The native layout runs
 * on the MFMA kernel with a persistent, equal-work (stream-K) partition of all
 * (sequence, kv head, 16-token tile) triples; it needs block_tables.
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
size_t mentat_paged_decode_workspace_bytes(int layout, int N, int Hq, int Hkv, int D, int block_size,
                                           int max_seqlen, int window_size, int chunk_tokens);

int mentat_paged_decode(int layout, const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, int64_t table_stride,
                        const int32_t* seq_rows, const int32_t* seq_lens,
                        const int32_t* cu_seqlens_k, int64_t num_blocks,
                        void* out, int N, int Hq, int Hkv, int D, int block_size,
                        int max_seqlen, int window_size, float scale, int dtype, int chunk_tokens,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The chunk length (tokens) the reference-layout path uses when chunk_tokens == 0. */
int mentat_paged_decode_auto_chunk(int N, int Hkv, int block_size, int max_seqlen);

/* mentat_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * The workspace is a static device array of MENTAT_NOALLOC_SCRATCH_BYTES
 * inside the library, one per device, held until the process ends; the call
 * itself allocates nothing. A call whose workspace need
 * (mentat_paged_decode_workspace_bytes) exceeds that size returns
 * MENTAT_ESPACE. Every call on a device shares that device's array, so calls
 * that overlap on one device (other streams or threads) race; calls ordered
 * on one stream are safe. Results equal mentat_paged_decode's. */
#define MENTAT_NOALLOC_SCRATCH_BYTES 8388608

int mentat_paged_decode_noalloc(int layout, const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_tables, int64_t table_stride,
                                const int32_t* seq_rows, const int32_t* seq_lens,
                                const int32_t* cu_seqlens_k, int64_t num_blocks,
                                void* out, int N, int Hq, int Hkv, int D, int block_size,
                                int max_seqlen, int window_size, float scale, int dtype, int chunk_tokens,
                                void* stream);

/* ------------------------------------------------------------------------
 * Prefix-tree decode attention: the same result as mentat_paged_decode for
 * every query (core/paged_kv_cache.py:289-368 + adapters/attention_backend.py:
 * 192-229: query i attends to all of its cached tokens), computed so that a
 * page shared by several sequences of a branching tree (fork_sequence,
 * core/paged_kv_cache.py:152-170) is read from HBM once for all of them.
 * Native pool layout only (K [blk][Hkv][B][D], V [blk][Hkv][D][B]),
 * bf16/f16, block_size 16/32/64, Hq/Hkv in {1,2,4,8,16}, D in {64,128}.
 *
 * The host plan (built once per decode step, shared by all layers):
 *   items[n_shared + n_solo][8] int32, one per (segment chunk, kv head,
 *     member set): [0] table row whose ids the chunk reads; [1] first 16-token
 *     tile; [2] tile count; [3] tokens of the segment (exclusive end,
 *     absolute); [4] kv head; [5] member count m; [6] first partial slot
 *     (member j writes slot [6]+j); [7] offset of the m member query indices
 *     in members[]. Items with [2] == 0 are padding.
 *     The first n_shared items are shared tasks (m <= 8 * 16/(Hq/Hkv)): one
 *     workgroup stages the chunk's pages through LDS once for all members.
 *     The other n_solo items have m <= 16/(Hq/Hkv) and run one per wavefront.
 *   q_slot_offsets[Nq*Hkv+1], q_slots[]: the partial slots of (query, kv head)
 *     q*Hkv+h, merged with the log-sum-exp rule into out.
 * block_tables: [rows, table_stride] int32 (one layer). Workspace:
 * mentat_tree_decode_workspace_bytes(n_slots, ...) bytes. Page ids outside
 * [0, num_blocks) are masked, not read. Every index the plan holds must be in
 * range (rows, tiles, heads, members < Nq, slots < n_slots): the host
 * validates plans before the call.
 * ---------------------------------------------------------------------- */
size_t mentat_tree_decode_workspace_bytes(int n_slots, int Hq, int Hkv, int D);

int mentat_tree_decode(const void* q, const void* k_store, const void* v_store, const int32_t* block_tables,
                       int64_t table_stride, int64_t num_blocks, const int32_t* items, int n_shared, int n_solo,
                       const int32_t* members, const int32_t* q_slot_offsets, const int32_t* q_slots, int n_slots,
                       void* out, int Nq, int Hq, int Hkv, int D, int block_size, float scale, int dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* mentat_tree_decode with the plan's item counts in device memory, so that a
 * captured launch (a rollout's decode step replayed as a HIP graph) takes a new
 * plan each step: counts = device int32 [n_shared, n_solo], at most
 * max_shared / max_solo, the capacities the items, members and q_slots arrays
 * and the workspace (mentat_tree_decode_workspace_bytes(max_slots, ...)) were
 * sized for; q_slot_offsets [Nq * Hkv + 1] is read from device memory too. The
 * kernel runs a fixed grid whose workgroups stride over the items. Same
 * result as mentat_tree_decode with n_shared / n_solo = the counts. */
int mentat_tree_decode_counted(const void* q, const void* k_store, const void* v_store,
                               const int32_t* block_tables, int64_t table_stride, int64_t num_blocks,
                               const int32_t* items, const int32_t* counts, int max_shared, int max_solo,
                               const int32_t* members, const int32_t* q_slot_offsets, const int32_t* q_slots,
                               int max_slots, void* out, int Nq, int Hq, int Hkv, int D, int block_size,
                               float scale, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Host planner of the prefix-tree decode (no device work): the plan of
 * mentat_amd/tree_plan.py:build_plan for N queries, written into the arrays
 * mentat_tree_decode_counted reads. Segments are the pages a run of
 * neighbouring queries holds through the same block ids (forks copy their
 * parent's ids, core/paged_kv_cache.py:152-170); share = 0 gives every query
 * one segment of its own. tables: host block ids, query i's at
 * tables[qrows[i] * table_stride ...]; lens: tokens per query.
 * Outputs: counts [3] = n_shared, n_solo, n_slots; items [(max_shared +
 * max_solo) * 8] with the solo items right after the shared ones; members and
 * q_slots [max_slots]; q_slot_offsets [N * Hkv + 1]. Returns MENTAT_ESPACE
 * when a capacity is exceeded (the outputs are then incomplete). */
int mentat_tree_plan(const int32_t* tables, int64_t table_stride, const int32_t* qrows, const int32_t* lens, int N,
                     int block_size, int Hkv, int G, int chunk_tiles, int shared_chunk_tiles, int shared_min_groups,
                     int share, int32_t* counts, int32_t* items, int max_shared, int max_solo, int32_t* members,
                     int32_t* q_slot_offsets, int32_t* q_slots, int max_slots);

/* ------------------------------------------------------------------------
 * Prefill attention: causal (optionally sliding-window) attention over one
 * batch of prompts, GQA.
 *
 * Replaces adapters/attention_backend.py:175-189 attn_prefill (and its SDPA
 * path :43-96 / flash_attn_func(causal=True, window_size=...)).
 * q [batch, seqlen, Hq, D], k/v [batch, seqlen, Hkv, D], out [batch, seqlen,
 * Hq, D], all contiguous, D in {64, 128}; bf16 or f16 with Hq/Hkv in
 * {1, 2, 4, 8, 16} (MFMA kernel), or fp32 with Hq/Hkv in {1, 2, 4, 8} (VALU
 * kernel, one query per position). Query head h reads kv head h / (Hq/Hkv).
 * Position i attends to keys max(0, i - window + 1) .. i when
 * 0 < window < seqlen, to 0 .. i otherwise. scale: softmax scale (the
 * reference uses D^-1/2). No workspace.
 * ---------------------------------------------------------------------- */
int mentat_prefill_attention(const void* q, const void* k, const void* v, void* out, int batch, int seqlen,
                             int Hq, int Hkv, int D, int window, float scale, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Semantic-diversity prune.
 *
 * mentat_semantic_ema replaces core/generator.py:376-398
 * (_update_semantic_vectors): for each of n leaves, row i of `hidden`
 * ([n, hidden_stride], H used) is written to the H-element vector at
 * dst_ptrs[i] when init[i] != 0 (a new leaf clones its hidden state), and
 * otherwise folded in as v.mul_(mul_scale).add_(h, alpha=add_scale) with the
 * rounding of torch's kernels: rnd(fma(add_scale, h, rnd(v * mul_scale))).
 * dst_ptrs, init: device arrays of n entries. Vectors in `dtype`.
 *
 * mentat_semantic_similar replaces the similarity mask of
 * core/generator.py:400-460 (_prune_similar): for M candidate vectors at
 * ptrs[i], mask[i*M + j] = 1 iff i < j, group[i] == group[j],
 * parent_key[i] != parent_key[j] (siblings are never compared) and
 * rnd(dot(n_i, n_j)) > rnd(threshold), where n_i = F.normalize(v_i, p=2) in
 * the vectors' dtype (float norm rounded, clamp_min(1e-12), float divide
 * rounded) and rnd rounds to that dtype, as torch's comparison with a scalar
 * does. scratch: at least M*H elements of the dtype. mask: M*M bytes.
 * ---------------------------------------------------------------------- */
int mentat_semantic_ema(const int64_t* dst_ptrs, const void* hidden, const int32_t* init, int n, int H,
                        int64_t hidden_stride, float mul_scale, float add_scale, int dtype, void* stream);

int mentat_semantic_similar(const int64_t* ptrs, const int32_t* parent_key, const int32_t* group, int M, int H,
                            float threshold, int dtype, void* scratch, size_t scratch_bytes, uint8_t* mask,
                            void* stream);

/* ------------------------------------------------------------------------
 * Per-layer glue of the captured decode step (16-bit models; dtype
 * MENTAT_BF16 or MENTAT_F16). The reference's decode loop
 * (core/generator_utils.py:340-418) runs each layer with the model's own
 * modules: input_layernorm, RoPE in the adapters' rotate_half form
 * (adapters/llama_adapter.py:70-113), post_attention_layernorm, the MLP and
 * two residual adds. Each entry point is one launch and rounds as the torch
 * kernels it replaces (one rounding to the dtype per torch op).
 *
 * mentat_rmsnorm: for each of `rows` rows of H elements (H % 8 == 0,
 * H <= 8192, 16-byte aligned buffers): h = x, or h = rnd(residual_in + x)
 * written to residual_out when residual_in is given; then
 * out = rnd(weight * rnd(h * rsqrt(mean(h^2) + eps))) (HF LlamaRMSNorm /
 * Qwen3RMSNorm). The fp32 summation order of the mean differs from torch's.
 *
 * mentat_rope: in place on q [rows][Hq][D] and k [rows][Hk][D] with cos/sin
 * [rows][D]: t = rnd(rnd(t * cos) + rnd(rotate_half(t) * sin)).
 *
 * mentat_rope_qkv: the same rotation, reading row r's q, k and v heads from one
 * merged projection output (qkv + r * row_stride: Hq q heads, then Hk k heads,
 * then Hk v heads) and writing rotated q, rotated k and plain v to dense
 * [rows][H][D] buffers (q_proj / k_proj / v_proj computed as one GEMM).
 *
 * mentat_silu_mul: out[r][j] = rnd(rnd(silu(gate[r][j])) * up[r][j]) for
 * j < F (F % 8 == 0), gate and up rows in_row_stride elements apart (F for
 * separate tensors, 2F for the halves of a merged gate/up projection), out
 * dense [rows][F], 16-byte aligned; silu(g) = g / (1 + exp(-g)) in fp32 (the
 * LlamaMLP / Qwen3MLP activation and product).
 *
 * mentat_silu_mul_split: the same product written as `split` column slices
 * [split][rows][F / split] (F % (8 * split) == 0), the operand layout of a
 * split-K down projection computed as one batched product over the slices.
 *
 * mentat_rmsnorm_partials: mentat_rmsnorm with x given as n_parts (2, 4 or 8)
 * fp32 partial products parts[s][rows][H]: x = rnd(sum over s of parts[s]),
 * the value one un-split down projection would have stored (up to the fp32
 * summation order), then the residual add and the norm as above.
 * ------------------------------------------------------------------------ */
int mentat_rmsnorm(const void* x, const void* residual_in, void* residual_out, const void* weight, void* out,
                   int rows, int H, float eps, int dtype, void* stream);

int mentat_rope(void* q, void* k, const void* cos, const void* sin, int rows, int Hq, int Hk, int D, int dtype,
                void* stream);

int mentat_rope_qkv(const void* qkv, int64_t row_stride, void* q, void* k, void* v, const void* cos,
                    const void* sin, int rows, int Hq, int Hk, int D, int dtype, void* stream);

int mentat_silu_mul(const void* gate, const void* up, void* out, int rows, int F, int64_t in_row_stride, int dtype,
                    void* stream);

int mentat_silu_mul_split(const void* gate, const void* up, void* out, int rows, int F, int64_t in_row_stride,
                          int split, int dtype, void* stream);

int mentat_rmsnorm_partials(const float* parts, int n_parts, const void* residual_in, void* residual_out,
                            const void* weight, void* out, int rows, int H, float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * KV append: write n new token rows into the pools, fused with the lazy
 * copy-on-write of a shared tail page and the device block-table update.
 *
 * Replaces the device half of
 *   core/paged_kv_cache.py:178-225  append_tokens (prefill: a while-loop over blocks)
 *   core/paged_kv_cache.py:227-284  append_tokens_batched (decode: one token per sequence)
 * The host keeps the reference's allocator/refcount bookkeeping and produces
 * `plan`, int32 [7][n] (structure of arrays), one column per new token:
 *   [0] dst block   [1] dst slot   [2] copy-on-write source block (-1: none)
 *   [3] table row (-1: no table update)   [4] page index within the row
 *   [5] new sequence length to store in seq_lens[row] (-1: leave)
 *   [6] source token index into k_new / v_new
 * A copy-on-write copies the source block's first `dst slot` tokens (the valid
 * ones; the reference's copy_ also moves the unused tail slots, which no read
 * ever reaches), so it never overlaps another write of the same launch.
 * k_new/v_new: [n_src, Hkv, D] contiguous.
 * block_tables ([table_rows, table_stride]) and seq_lens ([table_rows]) are the
 * tables of this layer and may be NULL. Out-of-range plan entries are skipped.
 * ---------------------------------------------------------------------- */
int mentat_kv_append(int layout, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                     const int32_t* plan, int n, int64_t n_src, int Hkv, int D, int block_size,
                     int64_t num_blocks, int dtype, int32_t* block_tables, int64_t table_stride,
                     int64_t table_rows, int32_t* seq_lens, void* stream);

/* mentat_rope_qkv followed by mentat_kv_append of its k and v, in one launch
 * (bf16/f16): rotated q goes to the dense q [rows][Hq][D]; for each plan column
 * the rotated k and the v of source row plan[6] (< rows) are written straight
 * into the pools (K/V heads Hk) at the column's (block, slot), with that
 * column's copy-on-write and table / length update. Pools, tables, lengths and
 * q hold the same bits as the two calls. Replaces, for one decode step's layer,
 * the adapters' RoPE of q and k (adapters/llama_adapter.py:70-113) and the
 * device half of append_tokens_batched (core/paged_kv_cache.py:227-284). */
int mentat_rope_qkv_append(int layout, const void* qkv, int64_t row_stride, void* q, const void* cos,
                           const void* sin, int rows, int Hq, int Hk, int D, void* k_pool, void* v_pool,
                           const int32_t* plan, int n, int block_size, int64_t num_blocks, int dtype,
                           int32_t* block_tables, int64_t table_stride, int64_t table_rows, int32_t* seq_lens,
                           void* stream);

/* Batched whole-page copy dst[i] <- src[i] in each of n_pools pools (e.g. the
 * K and V pools of every layer in one launch). `pools` is a DEVICE array of
 * n_pools base pointers; block_bytes = bytes of one page. Pairs with an
 * out-of-range id are skipped.
 * Replaces the per-layer block copies of core/paged_kv_cache.py:201-206,
 * :261-262 and :398-405 when many pages move at once. */
int mentat_page_copy(void* const* pools, int n_pools, const int32_t* src, const int32_t* dst, int n,
                     int64_t block_bytes, int64_t num_blocks, void* stream);

/* Copy block-table rows (first n_entries entries) and lengths, for every layer:
 * tables [L][rows][stride], seq_lens [L][rows] (may be NULL).
 * The device half of fork_sequence, core/paged_kv_cache.py:152-170, whose
 * host half copies the page-table lists and bumps the refcounts. */
int mentat_table_copy_rows(int32_t* tables, int32_t* seq_lens, int L, int64_t rows, int64_t stride,
                           const int32_t* src_rows, const int32_t* dst_rows, int n, int64_t n_entries,
                           void* stream);

/* ------------------------------------------------------------------------
 * Fused per-row statistics, gate and sampling over [R, V] logits (row_stride
 * elements apart), one workgroup per row, all outputs device arrays:
 *   out_entropy[R]      entropy (nats) of softmax(x / temperature), raw logits
 *                       (compute_entropy at the gate temperature,
 *                       core/generator_utils.py:196-202, core/generator.py:342),
 *                       rounded as torch's device kernels round it in the logits
 *                       dtype: y = rnd(x * fl(1/T)), p = rnd(e/s), lp = rnd(fl(y-m) - ln s),
 *                       t = rnd(p*lp) (NaN -> 0), H = -rnd(sum t), e = exp2(fl(y-m)*log2 e)
 *   out_entropy_f32[R]  the same entropy with fp32 arithmetic and no dtype rounding
 *                       (the reference's value for fp32 logits; may be NULL)
 *   out_gate[R]         out_entropy > gate_threshold (may be NULL)
 *   xp                  repetition penalty over the row's ids in CSR
 *                       pen_offsets[R+1] / pen_ids (duplicates ignored; NULL or
 *                       penalty == 1: none), core/generator_utils.py:205-230
 *   out_entropy_pen[R]  entropy of softmax(xp) (core/generator.py:293; may be NULL),
 *                       rounded as out_entropy (T = 1)
 *   out_lse[R]          log-sum-exp of xp (may be NULL)
 *   out_topk[R,topk], out_topk_lp[R,topk]
 *                       the topk (0..8) best log_softmax(xp) values in the logits
 *                       dtype and their ids, ties to the lowest id; topk = 1 is the
 *                       argmax of core/generator.py:308-310, topk = K the branch
 *                       children of :283-287
 *   out_sample[R]       if do_sample: temperature + top-p draw from xp with
 *                       Philox4x32-10 (key = seed, counter = (row, step, 0)),
 *                       bit-exact per the oracle's sampling_ref.c; the only
 *                       temperature/top-p sampling of the reference is HF
 *                       generate (baseline_rollout.py:56-66)
 * V <= 524288. dtype: MENTAT_BF16 / MENTAT_F16 / MENTAT_F32.
 * ---------------------------------------------------------------------- */
int mentat_row_stats(const void* logits, int64_t row_stride, int R, int V, int dtype, float temperature,
                     float penalty, const int32_t* pen_offsets, const int32_t* pen_ids,
                     float gate_threshold, int topk, int do_sample, float sample_temperature,
                     float top_p, uint64_t seed, uint64_t step, float* out_entropy,
                     float* out_entropy_f32, float* out_entropy_pen, float* out_lse, uint8_t* out_gate,
                     int32_t* out_topk,
                     float* out_topk_lp, int32_t* out_sample, void* stream);

/* Philox4x32-10 blocks: out[4i..4i+3] = rounds(counters[4i..], keys[2i..]) for
 * i < n (device arrays). The generator mentat_row_stats draws from. */
int mentat_philox4x32_10(const uint32_t* counters, const uint32_t* keys, uint32_t* out, int n,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MENTAT_CAPI_H */
