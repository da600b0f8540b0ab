// Paged KV-cache device operations for gfx950.
//
//  kv_append     K/V write of new tokens fused with the lazy copy-on-write of a
//                shared tail page and the device block-table / length update.
//                Replaces the per-layer scatter and CoW copy_ of
//                core/paged_kv_cache.py:178-225 (append_tokens, prefill) and
//                :227-284 (append_tokens_batched, decode).
//  rope_qkv_append  the RoPE split of a merged q/k/v projection fused with
//                kv_append: rotated k and v go straight into the pools.
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
  char* k_pool;
  char* v_pool;
  const int32_t* plan;
  int n;
  int Hkv, D, esz;
  long row_bytes;  // Hkv*D*esz: bytes of one cached token
  int block_size;
  long num_blocks;
  int32_t* tables;  // this layer's [rows, stride] (may be null)
  long table_stride;
  long table_rows;
  int32_t* lens;  // this layer's [rows] (may be null)
  long n_src;
  int layout;
};

// Copy-on-write of a shared tail page: the first `slot` (valid) tokens of K and
// V from block cow to block dst, threads first, first + step, ... taking the
// 16-byte vectors (elements, for the native V). Every other write of an append
// targets slots >= slot of dst or a different block, so the copy needs no
// ordering against them.
__device__ __forceinline__ void cow_tokens(const AppendParams& p, int dst, int cow, int slot, long first, long step) {
  const long blk_bytes = (long)p.block_size * p.row_bytes;
  const char* ks = p.k_pool + (long)cow * blk_bytes;
  const char* vs = p.v_pool + (long)cow * blk_bytes;
  char* kd = p.k_pool + (long)dst * blk_bytes;
  char* vd = p.v_pool + (long)dst * blk_bytes;
  if (p.layout == MENTAT_LAYOUT_REFERENCE) {
    const long nv = (long)slot * p.row_bytes / 16;
    for (long j = first; j < nv; j += step) {
      ((uint4*)kd)[j] = ((const uint4*)ks)[j];
      ((uint4*)vd)[j] = ((const uint4*)vs)[j];
    }
  } else {
    // K [Hkv][B][D]: rows 0..slot-1 of each head are contiguous.
    const long hv = (long)slot * p.D * p.esz / 16;  // vectors per head
    const long hstride = (long)p.block_size * p.D * p.esz;
    for (long j = first; j < (long)p.Hkv * hv; j += step) {
      const long h = j / hv, e = j - h * hv;
      ((uint4*)(kd + h * hstride))[e] = ((const uint4*)(ks + h * hstride))[e];
    }
    // V [Hkv][D][B]: elements 0..slot-1 of every (head, d) row.
    const long nel = (long)p.Hkv * p.D * slot;
    for (long j = first; j < nel; j += step) {
      const long hd = j / slot, t = j - hd * slot;
      const long idx = hd * p.block_size + t;
      if (p.esz == 2) ((uint16_t*)vd)[idx] = ((const uint16_t*)vs)[idx];
      else ((uint32_t*)vd)[idx] = ((const uint32_t*)vs)[idx];
    }
  }
}

__device__ __forceinline__ void table_update(const AppendParams& p, int32_t dst, int32_t row, int32_t page,
                                             int32_t new_len) {
  if (row >= 0 && row < p.table_rows) {
    if (p.tables && page >= 0 && page < p.table_stride) p.tables[(long)row * p.table_stride + page] = dst;
    if (p.lens && new_len >= 0) p.lens[row] = new_len;
  }
}

// One workgroup per new token: optional whole-page copy-on-write, then the
// token row, then the table entry and length.
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
  const long blk_bytes = (long)p.block_size * p.row_bytes;
  if (cow >= 0 && cow < p.num_blocks && cow != dst && slot > 0) cow_tokens(p, dst, cow, slot, threadIdx.x, blockDim.x);
  const char* srck = p.k_new + (long)src_tok * p.row_bytes;
  const char* srcv = p.v_new + (long)src_tok * p.row_bytes;
  char* kblk = p.k_pool + (long)dst * blk_bytes;
  char* vblk = p.v_pool + (long)dst * blk_bytes;
  if (p.layout == MENTAT_LAYOUT_REFERENCE) {
    // [B][Hkv][D]: the token row is contiguous.
    const long nvec = p.row_bytes / 16;
    const uint4* sk = (const uint4*)srck;
    const uint4* sv = (const uint4*)srcv;
    uint4* dk = (uint4*)(kblk + (long)slot * p.row_bytes);
    uint4* dv = (uint4*)(vblk + (long)slot * p.row_bytes);
    for (long j = threadIdx.x; j < nvec; j += blockDim.x) {
      dk[j] = sk[j];
      dv[j] = sv[j];
    }
  } else {
    // K: [Hkv][B][D] -> head h's D elements are contiguous at (h*B + slot)*D.
    const long dvec = (long)p.D * p.esz / 16;
    const long nvec = (long)p.Hkv * dvec;
    for (long j = threadIdx.x; j < nvec; j += blockDim.x) {
      const long h = j / dvec, e = j - h * dvec;
      ((uint4*)(kblk + ((h * p.block_size + slot) * p.D) * p.esz))[e] = ((const uint4*)srck)[j];
    }
    // V: [Hkv][D][B] -> element (h, d) at ((h*D + d)*B + slot).
    const long nel = (long)p.Hkv * p.D;
    if (p.esz == 2) {
      for (long j = threadIdx.x; j < nel; j += blockDim.x)
        ((uint16_t*)vblk)[j * p.block_size + slot] = ((const uint16_t*)srcv)[j];
    } else {
      for (long j = threadIdx.x; j < nel; j += blockDim.x)
        ((uint32_t*)vblk)[j * p.block_size + slot] = ((const uint32_t*)srcv)[j];
    }
  }
  if (threadIdx.x == 0) table_update(p, dst, row, page, new_len);
}

// rope_qkv + kv_append in one launch (16-bit models). Rows of qkv hold Hq q
// heads, then Hk k heads, then Hk v heads, row_stride elements apart; cos and
// sin are [rows][D]. Grid (max(rows, n), ceil((Hq + 2 Hk) * D/2 / 256)); thread
// (j, x = 256 y + t) with h = x / (D/2), i = x % (D/2):
//   h < Hq:           rotates pair (i, i + D/2) of q head h of row j into q [rows][Hq][D];
//   Hq <= h < Hq+Hk:  rotates that pair of k head h - Hq of plan column j's source
//                     row into the K pool at the column's (block, slot);
//   h >= Hq + Hk:     copies elements i and i + D/2 of v head h - Hq - Hk there.
// The rotation rounds as mentat_rope_qkv does, so the pools and q hold the bits
// of mentat_rope_qkv followed by mentat_kv_append. Column j's copy-on-write is
// spread over all of its workgroups' threads; workgroup (j, 0) updates the
// table entry and length.
struct RopeAppendParams {
  AppendParams a;  // k_new / v_new unused; n_src = rows
  const uint16_t* qkv;
  long row_stride;
  uint16_t* q;
  const uint16_t* cs;
  const uint16_t* sn;
  int rows, Hq;
};

template <typename T>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendParams r) {
  using E = G16<T>;
  const AppendParams& p = r.a;
  const int j = blockIdx.x;
  const int D = p.D, half = D / 2, Hk = p.Hkv;
  const int x = blockIdx.y * 256 + threadIdx.x;
  const int h = x / half, i = x - h * half;
  auto ld = [](const uint16_t* b, long e) __attribute__((always_inline)) { return E::lo((uint32_t)b[e]); };
  if (h < r.Hq) {
    if (j < r.rows) {
      const uint16_t* src = r.qkv + (long)j * r.row_stride + (long)h * D;
      const uint16_t* c = r.cs + (long)j * D;
      const uint16_t* s = r.sn + (long)j * D;
      float ya, yb;
      rope_pair<T>(ld(src, i), ld(src, i + half), ld(c, i), ld(s, i), ld(c, i + half), ld(s, i + half), ya, yb);
      uint16_t* dst = r.q + ((long)j * r.Hq + h) * D;
      dst[i] = (uint16_t)E::bits(ya);
      dst[i + half] = (uint16_t)E::bits(yb);
    }
  }
  if (j >= p.n) return;
  const int32_t dst = p.plan[kDstBlock * p.n + j];
  const int32_t slot = p.plan[kDstSlot * p.n + j];
  const int32_t src_tok = p.plan[kSrcTok * p.n + j];
  if (dst < 0 || dst >= p.num_blocks || slot < 0 || slot >= p.block_size) return;
  if (src_tok < 0 || src_tok >= r.rows) return;
  const long blk_bytes = (long)p.block_size * p.row_bytes;
  uint16_t* kblk = (uint16_t*)(p.k_pool + (long)dst * blk_bytes);
  uint16_t* vblk = (uint16_t*)(p.v_pool + (long)dst * blk_bytes);
  const bool native = p.layout != MENTAT_LAYOUT_REFERENCE;
  if (h >= r.Hq && h < r.Hq + 2 * Hk) {
    const uint16_t* src = r.qkv + (long)src_tok * r.row_stride + (long)h * D;
    const int hk = h < r.Hq + Hk ? h - r.Hq : h - r.Hq - Hk;
    float ya, yb;
    if (h < r.Hq + Hk) {
      const uint16_t* c = r.cs + (long)src_tok * D;
      const uint16_t* s = r.sn + (long)src_tok * D;
      rope_pair<T>(ld(src, i), ld(src, i + half), ld(c, i), ld(s, i), ld(c, i + half), ld(s, i + half), ya, yb);
      // K: reference [B][Hkv][D] (token row contiguous), native [Hkv][B][D]
      uint16_t* kr = kblk + (native ? ((long)hk * p.block_size + slot) * D : ((long)slot * Hk + hk) * D);
      kr[i] = (uint16_t)E::bits(ya);
      kr[i + half] = (uint16_t)E::bits(yb);
    } else {
      // V: reference [B][Hkv][D], native [Hkv][D][B] (element (hk, d) at (hk*D + d)*B + slot)
      if (native) {
        vblk[((long)hk * D + i) * p.block_size + slot] = src[i];
        vblk[((long)hk * D + i + half) * p.block_size + slot] = src[i + half];
      } else {
        uint16_t* vr = vblk + ((long)slot * Hk + hk) * D;
        vr[i] = src[i];
        vr[i + half] = src[i + half];
      }
    }
  }
  const int32_t cow = p.plan[kCowSrc * p.n + j];
  if (cow >= 0 && cow < p.num_blocks && cow != dst && slot > 0)
    cow_tokens(p, dst, cow, slot, x, (long)gridDim.y * 256);
  if (blockIdx.y == 0 && threadIdx.x == 0)
    table_update(p, dst, p.plan[kRow * p.n + j], p.plan[kPage * p.n + j], p.plan[kNewLen * p.n + j]);
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

extern "C" int mentat_kv_append(int layout, const void* k_new, const void* v_new, void* k_pool,
                                void* v_pool, const int32_t* plan, int n, int64_t n_src, int Hkv, int D,
                                int block_size, int64_t num_blocks, int dtype, int32_t* block_tables,
                                int64_t table_stride, int64_t table_rows, int32_t* seq_lens,
                                void* stream) {
  if (n == 0) return MENTAT_OK;
  const int es = esize(dtype);
  if (es == 0) return MENTAT_EUNSUP;
  if (!k_new || !v_new || !k_pool || !v_pool || !plan || n < 0 || Hkv <= 0 || D <= 0 ||
      block_size <= 0 || num_blocks <= 0 || n_src <= 0)
    return MENTAT_EINVAL;
  if (layout != MENTAT_LAYOUT_REFERENCE && layout != MENTAT_LAYOUT_NATIVE) return MENTAT_EINVAL;
  const long row_bytes = (long)Hkv * D * es;
  if (((long)D * es) % 16 != 0) return MENTAT_EUNSUP;
  AppendParams p;
  p.k_new = (const char*)k_new; p.v_new = (const char*)v_new;
  p.k_pool = (char*)k_pool; p.v_pool = (char*)v_pool;
  p.plan = plan; p.n = n; p.Hkv = Hkv; p.D = D; p.esz = es;
  p.row_bytes = row_bytes; p.block_size = block_size; p.num_blocks = num_blocks;
  p.tables = block_tables; p.table_stride = table_stride; p.table_rows = table_rows; p.lens = seq_lens;
  p.n_src = n_src; p.layout = layout;
  hipLaunchKernelGGL(kv_append_kernel, dim3(n), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

extern "C" int mentat_rope_qkv_append(int layout, const void* qkv, int64_t row_stride, void* q, const void* cos,
                                      const void* sin, int rows, int Hq, int Hk, int D, void* k_pool, void* v_pool,
                                      const int32_t* plan, int n, int block_size, int64_t num_blocks, int dtype,
                                      int32_t* block_tables, int64_t table_stride, int64_t table_rows,
                                      int32_t* seq_lens, void* stream) {
  if (rows < 0 || n < 0 || Hq <= 0 || Hk <= 0 || D <= 0 || D % 2 != 0 || row_stride < (int64_t)(Hq + 2 * Hk) * D ||
      block_size <= 0 || num_blocks <= 0)
    return MENTAT_EINVAL;
  if (layout != MENTAT_LAYOUT_REFERENCE && layout != MENTAT_LAYOUT_NATIVE) return MENTAT_EINVAL;
  if (rows == 0 && n == 0) return MENTAT_OK;
  if ((rows > 0 && (!qkv || !q || !cos || !sin)) || (n > 0 && (!k_pool || !v_pool || !plan))) return MENTAT_EINVAL;
  if (dtype != MENTAT_BF16 && dtype != MENTAT_F16) return MENTAT_EUNSUP;
  if (((long)D * 2) % 16 != 0) return MENTAT_EUNSUP;  // the copy-on-write moves 16-byte vectors
  RopeAppendParams r;
  AppendParams& p = r.a;
  p.k_new = nullptr; p.v_new = nullptr;
  p.k_pool = (char*)k_pool; p.v_pool = (char*)v_pool;
  p.plan = plan; p.n = n; p.Hkv = Hk; p.D = D; p.esz = 2;
  p.row_bytes = (long)Hk * D * 2; p.block_size = block_size; p.num_blocks = num_blocks;
  p.tables = block_tables; p.table_stride = table_stride; p.table_rows = table_rows; p.lens = seq_lens;
  p.n_src = rows; p.layout = layout;
  r.qkv = (const uint16_t*)qkv; r.row_stride = (long)row_stride; r.q = (uint16_t*)q;
  r.cs = (const uint16_t*)cos; r.sn = (const uint16_t*)sin; r.rows = rows; r.Hq = Hq;
  const dim3 grid((unsigned)(rows > n ? rows : n), (unsigned)(((Hq + 2 * Hk) * (D / 2) + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MENTAT_BF16) hipLaunchKernelGGL(rope_append_kernel<BF16>, grid, dim3(256), 0, s, r);
  else hipLaunchKernelGGL(rope_append_kernel<F16>, grid, dim3(256), 0, s, r);
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
