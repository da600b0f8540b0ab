// Paged KV-cache device operations for gfx950.
//
//  kv_append     K/V write of new tokens fused with the lazy copy-on-write of a
//                shared tail page and the device block-table / length update.
//                Replaces the per-layer scatter and CoW copy_ of
//                core/paged_kv_cache.py:178-225 (append_tokens, prefill) and
//                :227-284 (append_tokens_batched, decode).
//  page_copy     batched whole-page copy src->dst over any number of pools (all
//                layers' K and V in one launch).
//  table_copy    block-table row copy (every layer) for fork_sequence,
//                core/paged_kv_cache.py:152-170.
//
// All copies move 16-byte vectors; one workgroup per token / page / row.
#include "mentat_common.h"

namespace mentat {

// Plan layout: int32 [7][n] (structure of arrays), one column per token.
enum PlanField { kDstBlock = 0, kDstSlot, kCowSrc, kRow, kPage, kNewLen, kSrcTok, kPlanFields };

struct AppendParams {
  const char* k_new;  // [n_src, Hkv*D] elements
  const char* v_new;
  char* k_pool;  // [num_blocks, B, Hkv*D]
  char* v_pool;
  const int32_t* plan;
  int n;
  long row_bytes;  // Hkv*D*esz: bytes of one cached token
  int block_size;
  long num_blocks;
  int32_t* tables;  // this layer's [rows, stride] (may be null)
  long table_stride;
  long table_rows;
  int32_t* lens;  // this layer's [rows] (may be null)
  long n_src;
};

__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  const int i = blockIdx.x;
  if (i >= p.n) return;
  const int32_t dst = p.plan[kDstBlock * p.n + i];
  const int32_t slot = p.plan[kDstSlot * p.n + i];
  const int32_t cow = p.plan[kCowSrc * p.n + i];
  const int32_t row = p.plan[kRow * p.n + i];
  const int32_t page = p.plan[kPage * p.n + i];
  const int32_t new_len = p.plan[kNewLen * p.n + i];
  const int32_t src_tok = p.plan[kSrcTok * p.n + i];
  if (dst < 0 || dst >= p.num_blocks || slot < 0 || slot >= p.block_size) return;
  if (src_tok < 0 || src_tok >= p.n_src) return;
  const long nvec = p.row_bytes / 16;  // 16-byte vectors per token row
  const long blk_bytes = (long)p.block_size * p.row_bytes;

  // Lazy copy-on-write: the first `slot` (valid) tokens of the shared tail page.
  if (cow >= 0 && cow < p.num_blocks && cow != dst) {
    const long nv = (long)slot * nvec;
    const uint4* sk = (const uint4*)(p.k_pool + (long)cow * blk_bytes);
    const uint4* sv = (const uint4*)(p.v_pool + (long)cow * blk_bytes);
    uint4* dk = (uint4*)(p.k_pool + (long)dst * blk_bytes);
    uint4* dv = (uint4*)(p.v_pool + (long)dst * blk_bytes);
    for (long j = threadIdx.x; j < nv; j += blockDim.x) {
      dk[j] = sk[j];
      dv[j] = sv[j];
    }
  }
  // New token row.
  {
    const uint4* sk = (const uint4*)(p.k_new + (long)src_tok * p.row_bytes);
    const uint4* sv = (const uint4*)(p.v_new + (long)src_tok * p.row_bytes);
    uint4* dk = (uint4*)(p.k_pool + (long)dst * blk_bytes + (long)slot * p.row_bytes);
    uint4* dv = (uint4*)(p.v_pool + (long)dst * blk_bytes + (long)slot * p.row_bytes);
    for (long j = threadIdx.x; j < nvec; j += blockDim.x) {
      dk[j] = sk[j];
      dv[j] = sv[j];
    }
  }
  if (threadIdx.x == 0 && row >= 0 && row < p.table_rows) {
    if (p.tables && page >= 0 && page < p.table_stride) p.tables[(long)row * p.table_stride + page] = dst;
    if (p.lens && new_len >= 0) p.lens[row] = new_len;
  }
}

struct PageCopyParams {
  char* const* pools;  // device array of n_pools pool base pointers
  int n_pools;
  const int32_t* src;
  const int32_t* dst;
  int n;
  long block_bytes;
  long num_blocks;
};

// grid: (n pairs, n_pools)
__global__ __launch_bounds__(256) void page_copy_kernel(PageCopyParams p) {
  const int i = blockIdx.x;
  const int pool = blockIdx.y;
  if (i >= p.n || pool >= p.n_pools) return;
  const int32_t s = p.src[i], d = p.dst[i];
  if (s < 0 || s >= p.num_blocks || d < 0 || d >= p.num_blocks || s == d) return;
  char* base = p.pools[pool];
  const uint4* sp = (const uint4*)(base + (long)s * p.block_bytes);
  uint4* dp = (uint4*)(base + (long)d * p.block_bytes);
  const long nv = p.block_bytes / 16;
  for (long j = threadIdx.x; j < nv; j += blockDim.x) dp[j] = sp[j];
}

struct TableCopyParams {
  int32_t* tables;  // [L, rows, stride]
  int32_t* lens;    // [L, rows]
  int L;
  long rows;
  long stride;
  const int32_t* src_rows;
  const int32_t* dst_rows;
  int n;
  long n_entries;  // entries copied per row (<= stride)
};

// grid: (n pairs, L)
__global__ __launch_bounds__(256) void table_copy_kernel(TableCopyParams p) {
  const int i = blockIdx.x;
  const int l = blockIdx.y;
  if (i >= p.n || l >= p.L) return;
  const int32_t s = p.src_rows[i], d = p.dst_rows[i];
  if (s < 0 || s >= p.rows || d < 0 || d >= p.rows || s == d) return;
  const int32_t* sp = p.tables + ((long)l * p.rows + s) * p.stride;
  int32_t* dp = p.tables + ((long)l * p.rows + d) * p.stride;
  for (long j = threadIdx.x; j < p.n_entries; j += blockDim.x) dp[j] = sp[j];
  if (threadIdx.x == 0 && p.lens) p.lens[(long)l * p.rows + d] = p.lens[(long)l * p.rows + s];
}

}  // namespace mentat

using namespace mentat;

static int esize(int dtype) {
  switch (dtype) {
    case MENTAT_F32: return 4;
    case MENTAT_F16: return 2;
    case MENTAT_BF16: return 2;
    default: return 0;
  }
}

extern "C" int mentat_kv_append(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                                const int32_t* plan, int n, int64_t n_src, int Hkv, int D,
                                int block_size, int64_t num_blocks, int dtype, int32_t* block_tables,
                                int64_t table_stride, int64_t table_rows, int32_t* seq_lens,
                                void* stream) {
  if (n == 0) return MENTAT_OK;
  const int es = esize(dtype);
  if (es == 0) return MENTAT_EUNSUP;
  if (!k_new || !v_new || !k_pool || !v_pool || !plan || n < 0 || Hkv <= 0 || D <= 0 ||
      block_size <= 0 || num_blocks <= 0 || n_src <= 0)
    return MENTAT_EINVAL;
  const long row_bytes = (long)Hkv * D * es;
  if (row_bytes % 16 != 0) return MENTAT_EUNSUP;
  AppendParams p;
  p.k_new = (const char*)k_new; p.v_new = (const char*)v_new;
  p.k_pool = (char*)k_pool; p.v_pool = (char*)v_pool;
  p.plan = plan; p.n = n; p.row_bytes = row_bytes; p.block_size = block_size; p.num_blocks = num_blocks;
  p.tables = block_tables; p.table_stride = table_stride; p.table_rows = table_rows; p.lens = seq_lens;
  p.n_src = n_src;
  hipLaunchKernelGGL(kv_append_kernel, dim3(n), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

extern "C" int mentat_page_copy(void* const* pools, int n_pools, const int32_t* src, const int32_t* dst,
                                int n, int64_t block_bytes, int64_t num_blocks, void* stream) {
  if (n == 0 || n_pools == 0) return MENTAT_OK;
  if (!pools || !src || !dst || n < 0 || n_pools < 0 || block_bytes <= 0 || num_blocks <= 0)
    return MENTAT_EINVAL;
  if (block_bytes % 16 != 0 || n_pools > 65535) return MENTAT_EUNSUP;
  PageCopyParams p;
  p.pools = (char* const*)pools; p.n_pools = n_pools; p.src = src; p.dst = dst; p.n = n;
  p.block_bytes = block_bytes; p.num_blocks = num_blocks;
  hipLaunchKernelGGL(page_copy_kernel, dim3(n, n_pools), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

extern "C" int mentat_table_copy_rows(int32_t* tables, int32_t* seq_lens, int L, int64_t rows,
                                      int64_t stride, const int32_t* src_rows, const int32_t* dst_rows,
                                      int n, int64_t n_entries, void* stream) {
  if (n == 0) return MENTAT_OK;
  if (!tables || !src_rows || !dst_rows || n < 0 || L <= 0 || rows <= 0 || stride <= 0 || L > 65535)
    return MENTAT_EINVAL;
  if (n_entries < 0 || n_entries > stride) return MENTAT_EINVAL;
  TableCopyParams p;
  p.tables = tables; p.lens = seq_lens; p.L = L; p.rows = rows; p.stride = stride;
  p.src_rows = src_rows; p.dst_rows = dst_rows; p.n = n; p.n_entries = n_entries;
  hipLaunchKernelGGL(table_copy_kernel, dim3(n, L), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}
