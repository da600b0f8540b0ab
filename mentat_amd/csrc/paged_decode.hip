// Paged decode attention for gfx950 (CDNA4, wave64).
//
// Replaces the gather in core/paged_kv_cache.py:289-368 (build_packed_kv) plus
// the varlen attention of adapters/attention_backend.py:192-229: pages are read
// in place through the block table, nothing is copied.
//
// Work decomposition
//   unit = (sequence, chunk of `chunk_tokens` cached tokens, kv head); one
//   wavefront per unit, 4 independent wavefronts per workgroup. All Hq/Hkv query
//   heads of the kv head (the GQA group) are packed into that wavefront, so each
//   K/V byte is read from HBM once and used G times.
//
// Lane layout inside the wavefront (bf16, D = 128):
//   LPT = 16 lanes per token, each lane owns 8 consecutive head-dim elements
//   (one 16-byte load), TPI = 4 tokens per load instruction. One wave load of K
//   therefore covers 4 tokens x 256 contiguous bytes: every 128-byte line it
//   touches is used whole.
//   q·k: 4 x v_dot2_f32_bf16 per lane and head, then a 16-lane DPP butterfly.
//   Online softmax (base 2) is kept per token group (lanes with the same tg), so
//   the inner loop needs no cross-group traffic; groups are merged once at the end.
//
// Split-K: when a launch has more than one chunk per sequence, each unit writes
// its (m, l, acc) to the workspace and combine_kernel merges them with the usual
// log-sum-exp rescaling.
//
// Sliding window (window > 0): a sequence of length len attends to its tokens
// [max(0, len - window), len), the last `window` of them, as
// flash_attn_varlen_func(causal=True, window_size=(window - 1, 0)) does for one
// query aligned to the end of its keys (adapters/attention_backend.py:219-228).
// The chunks start at the window's first token.
//
// Causal prefill (causal_S > 0, packed mode, fp32 prompts): query n of the
// [B*S, Hq, D] batch is position i = n % S of prompt b = n / S and attends to
// the keys [b*S, b*S + i] of the [B*S, Hkv, D] K/V (with the window: the last
// `window` of them), which is the reference's causal prefill attention
// (adapters/attention_backend.py:43-96) restated as one decode query per
// position.
#include <mutex>

#include "mentat_common.h"

namespace mentat {

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* rows;
  const int32_t* lens;
  const int32_t* cu;
  int64_t num_blocks;
  void* out;
  float* ws_acc;  // [N, Hq, max_chunks, D]
  float* ws_ml;   // [N, Hq, max_chunks, 2]
  int N, Hq, Hkv, block_size, chunk_tokens, max_chunks;
  int window;        // attend to the last `window` tokens; 0 = all of them
  int causal_S;      // > 0: packed causal prefill of prompts of causal_S tokens (no cu)
  float scale_log2;  // softmax scale * log2(e)
};

// First token a sequence of length len attends to.
__device__ __forceinline__ int window_start(int len, int window) {
  return window > 0 && len > window ? len - window : 0;
}

constexpr int kWavesPerBlock = 4;

template <typename T, int D, int G, bool PAGED>
__global__ __launch_bounds__(kWavesPerBlock * 64) void paged_decode_kernel(DecodeParams p) {
  constexpr int EPL = Elem<T>::per16;  // elements per lane
  constexpr int LPT = D / EPL;         // lanes per token
  constexpr int TPI = 64 / LPT;        // tokens per wave iteration
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "bad lane layout");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tg = lane / LPT;
  const int dl = lane % LPT;

  long unit = (long)blockIdx.x * kWavesPerBlock + wave;
  const int head = (int)(unit % p.Hkv);
  unit /= p.Hkv;
  const int chunk = (int)(unit % p.max_chunks);
  const int seq = (int)(unit / p.max_chunks);
  if (seq >= p.N) return;

  int row = seq, len, base_tok = 0;
  if constexpr (PAGED) {
    row = p.rows ? p.rows[seq] : seq;
    len = p.lens[row];
  } else if (p.causal_S > 0) {
    base_tok = seq - seq % p.causal_S;
    len = seq % p.causal_S + 1;
  } else {
    base_tok = p.cu[seq];
    len = p.cu[seq + 1] - base_tok;
  }
  const int t0 = window_start(len, p.window) + chunk * p.chunk_tokens;
  if (t0 >= len && chunk > 0) return;  // empty chunk (chunk 0 always writes a state)
  const int t1 = min(len, t0 + p.chunk_tokens);

  // Query fragment of the G heads of this kv head, kept packed for v_dot2.
  const long row_elems = (long)p.Hkv * D;  // elements per cached token
  uint4 qv[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const char* qp = (const char*)p.q +
                     (((long)seq * p.Hq + (long)head * G + h) * D + (long)dl * EPL) * sizeof(typename T::storage);
    qv[h] = *(const uint4*)qp;
  }

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegInf;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }

  const char* kbase = (const char*)p.k + ((long)head * D + (long)dl * EPL) * sizeof(typename T::storage);
  const char* vbase = (const char*)p.v + ((long)head * D + (long)dl * EPL) * sizeof(typename T::storage);
  const long tok_bytes = row_elems * sizeof(typename T::storage);

  // Token step: every lane group handles token t + tg.
  for (int t = t0; t < t1; t += TPI) {
    const int tok = t + tg;
    const bool valid = tok < t1;
    long off;
    bool ok = valid;
    if constexpr (PAGED) {
      const int tc = valid ? tok : (t1 - 1);
      int pi = tc / p.block_size;
      const int slot = tc - pi * p.block_size;
      ok = ok && pi < p.table_stride;
      pi = pi < p.table_stride ? pi : (int)p.table_stride - 1;
      const int blk = p.tables[(long)row * p.table_stride + pi];
      ok = ok && blk >= 0 && blk < p.num_blocks;
      const long blk_c = (blk >= 0 && blk < p.num_blocks) ? blk : 0;
      off = (blk_c * p.block_size + slot) * tok_bytes;
    } else {
      const int tc = valid ? tok : (t1 - 1);
      off = (long)(base_tok + tc) * tok_bytes;
    }
    const uint4 kw = *(const uint4*)(kbase + off);
    const uint4 vw = *(const uint4*)(vbase + off);

    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s[h] = group_sum<LPT>(Dot16<T>::dot(qv[h], kw, 0.f)) * p.scale_log2;
      if (!ok) s[h] = kNegInf;
    }
    float vf[EPL];
    Elem<T>::unpack(vw, vf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mn = fmaxf(m[h], s[h]);
      const float ms = (mn == kNegInf) ? 0.f : mn;
      const float alpha = fast_exp2(m[h] - ms);
      const float pr = fast_exp2(s[h] - ms);
      l[h] = l[h] * alpha + pr;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(acc[h][e], alpha, pr * vf[e]);
      m[h] = mn;
    }
  }

  // Merge the TPI token groups of the wavefront (lanes dl + LPT*g).
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mw = m[h];
#pragma unroll
    for (int o = LPT; o < 64; o <<= 1) mw = fmaxf(mw, __shfl_xor(mw, o));
    const float ms = (mw == kNegInf) ? 0.f : mw;
    const float sc = fast_exp2(m[h] - ms);
    float lw = l[h] * sc;
#pragma unroll
    for (int o = LPT; o < 64; o <<= 1) lw += __shfl_xor(lw, o);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float a = acc[h][e] * sc;
#pragma unroll
      for (int o = LPT; o < 64; o <<= 1) a += __shfl_xor(a, o);
      acc[h][e] = a;
    }
    m[h] = mw;
    l[h] = lw;
  }
  if (tg != 0) return;

#pragma unroll
  for (int h = 0; h < G; ++h) {
    const int qh = head * G + h;
    if (p.max_chunks == 1) {
      const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
      const long o = ((long)seq * p.Hq + qh) * D + (long)dl * EPL;
#pragma unroll
      for (int e = 0; e < EPL; ++e) Elem<T>::store1(p.out, o + e, acc[h][e] * inv);
    } else {
      const long slot = ((long)seq * p.Hq + qh) * p.max_chunks + chunk;
      float* wa = p.ws_acc + slot * D + (long)dl * EPL;
#pragma unroll
      for (int e = 0; e < EPL; e += 4)
        *(float4*)(wa + e) = make_float4(acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]);
      if (dl == 0) {
        p.ws_ml[slot * 2] = m[h];
        p.ws_ml[slot * 2 + 1] = l[h];
      }
    }
  }
}

// Merge the per-chunk partial states of one (sequence, query head) per wavefront.
template <typename T, int D, bool PAGED>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
  const int qh = blockIdx.x % p.Hq;
  const int seq = blockIdx.x / p.Hq;
  const int lane = threadIdx.x;
  int len;
  if constexpr (PAGED) {
    const int row = p.rows ? p.rows[seq] : seq;
    len = p.lens[row];
  } else if (p.causal_S > 0) {
    len = seq % p.causal_S + 1;
  } else {
    len = p.cu[seq + 1] - p.cu[seq];
  }
  const int span = len - window_start(len, p.window);
  const int nch = max(1, min(p.max_chunks, (span + p.chunk_tokens - 1) / p.chunk_tokens));
  const long slot0 = ((long)seq * p.Hq + qh) * p.max_chunks;
  float mx = kNegInf;
  for (int c = 0; c < nch; ++c) mx = fmaxf(mx, p.ws_ml[(slot0 + c) * 2]);
  const float ms = (mx == kNegInf) ? 0.f : mx;
  constexpr int PER = (D + 63) / 64;
  float o[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) o[j] = 0.f;
  float lt = 0.f;
  for (int c = 0; c < nch; ++c) {
    const float sc = fast_exp2(p.ws_ml[(slot0 + c) * 2] - ms);
    lt += p.ws_ml[(slot0 + c) * 2 + 1] * sc;
    const float* wa = p.ws_acc + (slot0 + c) * D;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int d = lane + 64 * j;
      if (d < D) o[j] = fmaf(wa[d], sc, o[j]);
    }
  }
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = lane + 64 * j;
    if (d < D) Elem<T>::store1(p.out, ((long)seq * p.Hq + qh) * D + d, o[j] * inv);
  }
}

template <typename T, int D, int G, bool PAGED>
static hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
  const long units = (long)p.N * p.max_chunks * p.Hkv;
  const long blocks = (units + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL((paged_decode_kernel<T, D, G, PAGED>), dim3((unsigned)blocks),
                     dim3(kWavesPerBlock * 64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_chunks == 1) return e;
  hipLaunchKernelGGL((decode_combine_kernel<T, D, PAGED>), dim3((unsigned)(p.N * p.Hq)), dim3(64), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename T, int D, bool PAGED>
static int dispatch_g(int G, const DecodeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return (int)launch_decode<T, D, 1, PAGED>(p, s);
    case 2: return (int)launch_decode<T, D, 2, PAGED>(p, s);
    case 4: return (int)launch_decode<T, D, 4, PAGED>(p, s);
    case 8: return (int)launch_decode<T, D, 8, PAGED>(p, s);
    default: return MENTAT_EUNSUP;
  }
}

template <typename T, bool PAGED>
static int dispatch_d(int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<T, 64, PAGED>(G, p, s);
    case 128: return dispatch_g<T, 128, PAGED>(G, p, s);
    default: return MENTAT_EUNSUP;
  }
}

static int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

static int auto_chunk(int N, int Hkv, int block_size, int max_seqlen) {
  // Aim for roughly 8 wavefronts of work per CU (256 CUs) across the launch,
  // assuming sequences average ~60% of the longest; chunks are whole pages and
  // at least 256 tokens so the per-chunk merge traffic stays small.
  const long target_units = 2048;
  long total = (long)N * Hkv * (long)max_seqlen * 6 / 10;
  long c = total / target_units;
  long bs = block_size > 0 ? block_size : 16;
  long chunk = 256;
  while (chunk < c) chunk <<= 1;
  chunk = ((chunk + bs - 1) / bs) * bs;
  if (chunk >= max_seqlen) chunk = max_seqlen > 0 ? ((max_seqlen + bs - 1) / bs) * bs : bs;
  return (int)chunk;
}

}  // namespace mentat

using namespace mentat;

extern "C" int mentat_paged_decode_auto_chunk(int N, int Hkv, int block_size, int max_seqlen) {
  return auto_chunk(N, Hkv, block_size, max_seqlen);
}

size_t native_workspace_bytes(int N, int Hq, int Hkv, int D);
int native_paged_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                        int64_t table_stride, const int32_t* seq_rows, const int32_t* seq_lens,
                        int64_t num_blocks, void* out, int N, int Hq, int Hkv, int D, int block_size,
                        int window_size, float scale, int dtype, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

// Longest attended span: the window caps it.
static int attended_span(int max_seqlen, int window) {
  return window > 0 && window < max_seqlen ? window : max_seqlen;
}

extern "C" size_t mentat_paged_decode_workspace_bytes(int layout, int N, int Hq, int Hkv, int D,
                                                      int block_size, int max_seqlen, int window_size,
                                                      int chunk_tokens) {
  if (N <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_seqlen <= 0 || window_size < 0) return 0;
  if (layout == MENTAT_LAYOUT_NATIVE) return native_workspace_bytes(N, Hq, Hkv, D);
  const int span = attended_span(max_seqlen, window_size);
  const int chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(N, Hkv, block_size, span);
  const int mc = ceil_div(span, chunk);
  if (mc <= 1) return 0;
  return kWsReserved + (size_t)N * Hq * mc * (D + 2) * sizeof(float);
}

extern "C" int mentat_paged_decode(int layout, const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, int64_t table_stride,
                                   const int32_t* seq_rows, const int32_t* seq_lens,
                                   const int32_t* cu_seqlens_k, int64_t num_blocks, void* out, int N,
                                   int Hq, int Hkv, int D, int block_size, int max_seqlen,
                                   int window_size, float scale, int dtype, int chunk_tokens,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (N == 0) return MENTAT_OK;
  if (!q || !k_cache || !v_cache || !out || N < 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return MENTAT_EINVAL;
  if (Hq % Hkv != 0) return MENTAT_EINVAL;
  const bool paged = block_tables != nullptr;
  if (paged && (!seq_lens || block_size <= 0 || table_stride <= 0 || num_blocks <= 0)) return MENTAT_EINVAL;
  if (!paged && !cu_seqlens_k) return MENTAT_EINVAL;
  if (max_seqlen < 0 || window_size < 0) return MENTAT_EINVAL;
  if (layout == MENTAT_LAYOUT_NATIVE) {
    if (!paged) return MENTAT_EINVAL;
    return native_paged_decode(q, k_cache, v_cache, block_tables, table_stride, seq_rows, seq_lens, num_blocks,
                               out, N, Hq, Hkv, D, block_size, window_size, scale, dtype, workspace,
                               workspace_bytes, (hipStream_t)stream);
  }
  if (layout != MENTAT_LAYOUT_REFERENCE) return MENTAT_EINVAL;
  const int ms = attended_span(max_seqlen > 0 ? max_seqlen : 1, window_size);
  DecodeParams p;
  p.q = q; p.k = k_cache; p.v = v_cache;
  p.tables = block_tables; p.table_stride = table_stride; p.rows = seq_rows; p.lens = seq_lens;
  p.cu = cu_seqlens_k; p.num_blocks = num_blocks; p.out = out;
  p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.block_size = block_size; p.window = window_size; p.causal_S = 0;
  p.chunk_tokens = chunk_tokens > 0 ? chunk_tokens : auto_chunk(N, Hkv, block_size, ms);
  p.max_chunks = ceil_div(ms, p.chunk_tokens);
  p.scale_log2 = scale * kLog2e;
  p.ws_acc = nullptr; p.ws_ml = nullptr;
  if (p.max_chunks > 1) {
    const size_t need = kWsReserved + (size_t)N * Hq * p.max_chunks * (D + 2) * sizeof(float);
    if (!workspace || workspace_bytes < need) return MENTAT_ESPACE;
    p.ws_acc = (float*)((char*)workspace + kWsReserved);
    p.ws_ml = p.ws_acc + (size_t)N * Hq * p.max_chunks * D;
  }
  const int G = Hq / Hkv;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16: return paged ? dispatch_d<BF16, true>(D, G, p, s) : dispatch_d<BF16, false>(D, G, p, s);
    case MENTAT_F16: return paged ? dispatch_d<F16, true>(D, G, p, s) : dispatch_d<F16, false>(D, G, p, s);
    case MENTAT_F32: return paged ? dispatch_d<F32, true>(D, G, p, s) : dispatch_d<F32, false>(D, G, p, s);
    default: return MENTAT_EUNSUP;
  }
}

namespace mentat {

// Causal fp32 prefill over [batch, S] prompts on the decode kernel's packed
// mode: one query per position, one chunk per query (no workspace).
int causal_prefill_f32(const void* q, const void* k, const void* v, void* out, int batch, int S, int Hq, int Hkv,
                       int D, int window, float scale, hipStream_t stream) {
  const long n = (long)batch * S;
  if (n * Hkv > 0x7fffffffL || (long)S * Hkv * D > 0x7fffffffL) return MENTAT_EUNSUP;
  DecodeParams p;
  p.q = q; p.k = k; p.v = v;
  p.tables = nullptr; p.table_stride = 0; p.rows = nullptr; p.lens = nullptr;
  p.cu = nullptr; p.num_blocks = 0; p.out = out;
  p.N = (int)n; p.Hq = Hq; p.Hkv = Hkv; p.block_size = 0; p.window = window; p.causal_S = S;
  p.chunk_tokens = S; p.max_chunks = 1;
  p.scale_log2 = scale * kLog2e;
  p.ws_acc = nullptr; p.ws_ml = nullptr;
  return dispatch_d<F32, false>(D, Hq / Hkv, p, stream);
}

}  // namespace mentat

// ---- the allocation-free variant ----------------------------------------------------------
// mentat_paged_decode_noalloc runs mentat_paged_decode with its workspace in this
// file-scope device array: every device the library runs on holds its own copy
// (MENTAT_NOALLOC_SCRATCH_BYTES) until the process ends. Its first
// MENTAT_WORKSPACE_RESERVED bytes are the native path's arrival counters, zeroed
// once per device by a fill kernel on the first call's stream and left zero by
// every call; the rest holds a call's partials and is overwritten by the next
// call. Calls that overlap on one device (other streams, other threads) race
// on it.
static __device__ __align__(256) unsigned char scratch[MENTAT_NOALLOC_SCRATCH_BYTES];

namespace mentat {

constexpr int kScratchMaxDevices = 64;

__global__ void zero_words_kernel(uint32_t* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0u;
}

static std::mutex g_scratch_mu;
static void* g_scratch_dev[kScratchMaxDevices] = {};

// The device address of the current device's scratch (its host-side name is not
// a device address). Looked up, and its counters zeroed, once per device.
static int scratch_address(void** out, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kScratchMaxDevices) return MENTAT_EUNSUP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return (int)hipErrorInvalidSymbol;
    const long words = (long)(kWsReserved / sizeof(uint32_t));
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                       (uint32_t*)p, words);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return MENTAT_OK;
}

}  // namespace mentat

extern "C" int mentat_paged_decode_noalloc(int layout, const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_tables, int64_t table_stride,
                                           const int32_t* seq_rows, const int32_t* seq_lens,
                                           const int32_t* cu_seqlens_k, int64_t num_blocks, void* out, int N,
                                           int Hq, int Hkv, int D, int block_size, int max_seqlen,
                                           int window_size, float scale, int dtype, int chunk_tokens,
                                           void* stream) {
  if (N == 0) return MENTAT_OK;
  if (N < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_seqlen < 0 || window_size < 0) return MENTAT_EINVAL;
  const size_t need = mentat_paged_decode_workspace_bytes(layout, N, Hq, Hkv, D, block_size,
                                                          max_seqlen > 0 ? max_seqlen : 1, window_size,
                                                          chunk_tokens);
  if (need > (size_t)MENTAT_NOALLOC_SCRATCH_BYTES) return MENTAT_ESPACE;
  void* ws = nullptr;
  const int st = scratch_address(&ws, (hipStream_t)stream);
  if (st != MENTAT_OK) return st;
  return mentat_paged_decode(layout, q, k_cache, v_cache, block_tables, table_stride, seq_rows, seq_lens,
                             cu_seqlens_k, num_blocks, out, N, Hq, Hkv, D, block_size, max_seqlen, window_size,
                             scale, dtype, chunk_tokens, ws, (size_t)MENTAT_NOALLOC_SCRATCH_BYTES, stream);
}
