// Paged decode attention on the MFMA matrix cores (gfx950), native pool layout.
//
// Same semantics as paged_decode.hip (the gather + varlen attention of
// core/paged_kv_cache.py:289-368 and adapters/attention_backend.py:192-229),
// for 16-bit pools stored page-major and head-major:
//     K store [num_blocks][Hkv][B][D]      (a page-head is B*D contiguous elements)
//     V store [num_blocks][Hkv][D][B]      (transposed inside the page-head)
// B must be a multiple of 16; a page is processed as B/16 tiles of 16 tokens.
//
// Per tile and kv head (one wavefront, all G = Hq/Hkv query heads of the group):
//   S^T[16 tok x 16 q] = K[16 tok x D] . Q^T[D x 16 q]      v_mfma_f32_16x16x32_{bf16,f16}, D/32 steps
//   O[16 q x 16 d]   += P[16 q x 16 tok] . V[16 tok x 16 d]  v_mfma_f32_16x16x16_{bf16,f16}, D/16 tiles
// The accumulator layout of S^T (lane l: tokens 4*(l/16)+i, column q = l%16) is
// exactly the A-operand layout of P for the second product, so the softmax
// probabilities never leave their registers. Query rows q >= G are zero.
// K rows load as 16 bytes per lane (16 tokens x 64 contiguous bytes per
// instruction); V loads as 8 bytes per lane from the transposed page-head
// (512 contiguous bytes per instruction).
//
// Online softmax in base 2, one (m, l) per column lane. The rescale of O is
// lazy: the running max only moves when some column's tile max exceeds it by
// more than 8 (probabilities stay <= 2^8 otherwise, exact in fp32/16-bit).
//
// Work partition (stream-K): the (sequence, head unit, tile) triples are laid
// out in one flat index space, split into equal contiguous ranges. With Hkv a
// multiple of 4 a head unit is a team of 4 kv heads and the ranges go to the W/4
// persistent workgroups: the 4 waves of a workgroup take the 4 heads of the same
// tiles, so the workgroup reads each page's K (and V) of those heads as one
// contiguous 16 KiB piece at a time (the native store holds a page's heads next
// to each other), which the memory system serves faster than 4 KiB pieces of
// unrelated pages. Otherwise a head unit is one kv head and each of the W waves
// takes a range. A range that covers a whole (sequence, kv head) unit writes the
// output directly; split units leave (m, l, O) partials in the workspace, merged
// inside the kernel by the last piece to arrive.
//
// Sliding window (window > 0): a sequence of length len attends to its last
// `window` tokens, [max(0, len - window), len), as flash_attn_varlen_func with
// causal=True, window_size=(window - 1, 0) does for one query aligned to the end
// of its keys (adapters/attention_backend.py:219-228). Its tiles run from the
// one holding the window's first token; earlier tokens of that tile are masked.
#include "mentat_common.h"

namespace mentat {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma;
template <> struct Mfma<BF16> {
  __device__ static f32x4_t qk(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(const uint2& a, const uint2& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  __device__ static uint2 pack(f32x4_t v) {
    return __builtin_bit_cast(uint2, __builtin_convertvector(v, bf16x4_t));
  }
};
template <> struct Mfma<F16> {
  __device__ static f32x4_t qk(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(const uint2& a, const uint2& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
  __device__ static uint2 pack(f32x4_t v) {
    return __builtin_bit_cast(uint2, __builtin_convertvector(v, f16x4_t));
  }
};

struct NativeParams {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* rows;
  const int32_t* lens;
  int64_t num_blocks;
  void* out;
  float* ws_o;       // [slots][G][D]
  float* ws_ml;      // [slots][G][2]
  int32_t* ctr;      // [N*Hkv] arrival counters of split units (zero between calls)
  int N, Hq, Hkv, B, W;
  int TW;            // kv heads per head unit: 4 (a workgroup's waves share tiles) or 1
  int window;        // attend to the last `window` tokens; 0 = all of them
  float scale_log2;
};

constexpr int kNativeMaxN = 4096;   // sequences per call (prefix table lives in LDS)
constexpr int kNativeThreads = 256; // 4 wavefronts
constexpr float kRescaleSlack = 8.f;

__device__ __forceinline__ int seq_len_of(const NativeParams& p, int s) {
  const int row = p.rows ? p.rows[s] : s;
  const int n = p.lens[row];
  return n > 0 ? n : 0;
}

// First token a sequence of length n attends to.
__device__ __forceinline__ int window_lo(int n, int window) { return window > 0 && n > window ? n - window : 0; }

// 16-token tiles a sequence of length n covers: from the tile of its first
// attended token to the tile of its last.
__device__ __forceinline__ int tiles_of(int n, int window) { return ((n + 15) >> 4) - (window_lo(n, window) >> 4); }

// Tile prefix over the N sequences into s_prefix[0..N]: wave 0 scans 64
// sequences at a time with DPP prefix sums; one barrier publishes it.
__device__ void tile_prefix(const NativeParams& p, int32_t* s_prefix) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    uint32_t carry = 0;
    for (int b = 0; b < p.N; b += 64) {
      const int s = b + lane;
      const uint32_t t = s < p.N ? (uint32_t)tiles_of(seq_len_of(p, s), p.window) : 0u;
      const uint32_t inc = wave_incl_scan_u32(t) + carry;
      if (s < p.N) s_prefix[s] = (int32_t)(inc - t);
      carry = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    }
    if (lane == 0) s_prefix[p.N] = (int32_t)carry;
  }
  __syncthreads();
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Wave-uniform reads through the constant address space compile to scalar
// loads (s_load, counted by lgkmcnt), so they never wait behind the vector
// loads of the K/V pipeline.
typedef const int32_t __attribute__((address_space(4)))* const_i32_ptr;
__device__ __forceinline__ int32_t scalar_load(const int32_t* p, long i) {
  return ((const_i32_ptr)p)[i];
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9 dword3). Loads at
// offsets >= bytes return zero without touching memory, so a tile can always
// be issued and is switched off by giving it a zero-sized resource.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Split units are merged inside the kernel by the wavefront whose piece
// arrives last. Pieces and counters are written and read with device-coherent
// (agent-scope) accesses, which go past the per-XCD L2 caches, so no cache-wide
// write-back or invalidate is needed: a piece's stores complete (s_waitcnt)
// before its arrival is counted, and the merging wave reads the pieces only
// after its own arrival returned the full count.
__device__ __forceinline__ void put_shared(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_shared(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The same device coherence for 16-byte pieces of partial O: buffer accesses
// with the cache policy of agent-scope atomics (sc1).
constexpr int kCoherent = 16;
typedef uint32_t pd_u32x4_t __attribute__((ext_vector_type(4)));
// Partial O of a split unit is stored row by row with column lr + 16 j at
// position 64 (j / 4) + 4 lr + j % 4: a lane's columns j .. j + 3 are one
// 16-byte store and the 16 lanes of a row write 256 contiguous bytes per
// instruction; the merge maps a position back to its column.
__device__ __forceinline__ int partial_pos(int lr, int j) { return 64 * (j >> 2) + 4 * lr + (j & 3); }
template <int D>
__device__ __forceinline__ int partial_col(int pos) {
  return ((pos >> 2) & 15) + 16 * (4 * (pos >> 6) + (pos & 3));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const NativeParams& p, int G, int D) {
  const long bytes = ((long)p.N * p.Hkv + p.W) * G * D * (long)sizeof(float);
  return make_rsrc(p.ws_o, (int)(bytes < 0x7fffffffL ? bytes : 0x7fffffffL));
}

// Pieces are the partial slots (hunit + e) * TW + wsub of the partition
// entities e = w0..w1 (waves or workgroups) that covered the unit; lane l owns
// the E = G*D/64 consecutive outputs starting at l*E of the unit's [G][D] block.
// Pieces are read in batches whose loads are all in flight together, and are
// combined in entity order, so the result does not depend on arrival order.
template <typename T, int D, int G>
__device__ __forceinline__ void merge_unit(const NativeParams& p, int seq, int head, long hunit, int wsub, int w0,
                                           int w1, int lane) {
  constexpr int E = G * D / 64;
  static_assert(E >= 1, "merge lane split");
  constexpr int KB = E >= 32 ? 1 : (E >= 16 ? 2 : 4);  // pieces per batch
  const int g = (lane * E) / D;
  const int d0 = (lane * E) - g * D;
  const int n = w1 - w0 + 1;
  const __amdgpu_buffer_rsrc_t rw = partial_rsrc(p, G, D);
  float M = kNegInf, L = 0.f, acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  for (int k0 = 0; k0 < n; k0 += KB) {
    float mk[KB], lk[KB], ok[KB][E];
    // Past-the-end entries of the last batch reload piece n-1 and are dropped.
    static_for<KB>([&](auto i) {
      const long slot = (hunit + w0 + min(k0 + (int)i, n - 1)) * p.TW + wsub;
      mk[i] = get_shared(p.ws_ml + (slot * G + g) * 2);
      lk[i] = get_shared(p.ws_ml + (slot * G + g) * 2 + 1);
      if constexpr (E % 4 == 0) {
        const int off = (int)(((slot * G + g) * D + d0) * (long)sizeof(float));
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          const pd_u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 4 * e, 0, kCoherent);
#pragma unroll
          for (int c = 0; c < 4; ++c) ok[i][e + c] = __uint_as_float(v[c]);
        }
      } else {
        const float* wo = p.ws_o + (slot * G + g) * D + d0;
#pragma unroll
        for (int e = 0; e < E; ++e) ok[i][e] = get_shared(wo + e);
      }
    });
    float Mn = M;
    static_for<KB>([&](auto i) {
      if (k0 + (int)i < n) Mn = fmaxf(Mn, mk[i]);
    });
    const float ms = (Mn == kNegInf) ? 0.f : Mn;
    const float cold = (M == kNegInf) ? 0.f : fast_exp2(M - ms);
    L *= cold;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] *= cold;
    static_for<KB>([&](auto i) {
      const float c = (k0 + (int)i < n && mk[i] != kNegInf) ? fast_exp2(mk[i] - ms) : 0.f;
      L += lk[i] * c;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += ok[i][e] * c;
    });
    M = Mn;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const long ob = ((long)seq * p.Hq + (long)head * G + g) * D;
#pragma unroll
  for (int e = 0; e < E; ++e) Elem<T>::store1(p.out, ob + partial_col<D>(d0 + e), acc[e] * inv);
}

template <typename T, int D, int G, int B>
__global__ __launch_bounds__(kNativeThreads) void paged_decode_mfma_kernel(NativeParams p) {
  static_assert(D % 32 == 0 && G >= 1 && G <= 16 && B % 16 == 0, "tile shape");
  constexpr int KS = D / 32;  // QK k-steps
  constexpr int NT = D / 16;  // PV column tiles
  constexpr int NSUB = B / 16;  // tiles per page
  using S = typename T::storage;

  __shared__ int32_t s_prefix[kNativeMaxN + 1];
  tile_prefix(p, s_prefix);

  const int TW = p.TW, HU = p.Hkv / TW;              // head units per sequence
  const int PE = p.W / TW;                           // partition entities (waves or workgroups)
  const int T_total = uniform(HU * s_prefix[p.N]);
  // Equal static ranges, one per partition entity. (Claiming a dynamic tail in
  // chunks did not pay: a chunk's first-tile latency and partial publish cost
  // 2-3 us, as much as the spread it was meant to absorb.)
  const int stat = (T_total + PE - 1) / PE;
  auto range_of = [&](int x) -> int { return x / stat; };
  const int lane = threadIdx.x & 63;
  const int wv = uniform(blockIdx.x * (kNativeThreads / 64) + (threadIdx.x >> 6));
  const int pe = TW == 1 ? wv : (int)blockIdx.x;
  const int wsub = TW == 1 ? 0 : uniform(threadIdx.x >> 6);  // this wave's head within the unit
  // Sequences without cached tokens get zeros (no tile covers them).
  for (int s = wv; s < p.N; s += p.W) {
    if (s_prefix[s + 1] == s_prefix[s]) {
      for (int e = lane; e < p.Hq * D; e += 64) Elem<T>::store1(p.out, (long)s * p.Hq * D + e, 0.f);
    }
  }
  int f = min(T_total, pe * stat);
  const int fend = min(T_total, (pe + 1) * stat);
  if (f >= fend) return;

  // Unit containing f: last s with HU*prefix[s] <= f (upper_bound - 1).
  int seq;
  {
    int lo = 0, hi = p.N;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (HU * s_prefix[mid] <= f) lo = mid + 1; else hi = mid;
    }
    seq = uniform(lo - 1);
  }
  int pre = uniform(s_prefix[seq]);
  int nt = uniform(s_prefix[seq + 1]) - pre;
  int hu = (f - HU * pre) / nt;
  int tile = (f - HU * pre) - hu * nt;
  int head = hu * TW + wsub;

  const int lr = lane & 15;  // tile row (K operand) / column (S^T, Q^T, O)
  const int lg = lane >> 4;  // 4-lane-group index
  // Lane-constant parts of the K and V addresses inside one 16-token tile.
  const int k_lane = lr * D + 8 * lg;      // K [B][D] page-head: row lr, dims 8*lg..
  const int v_lane = lr * B + 4 * lg;      // V [D][B] page-head: dim lr, tokens 4*lg..

  while (f < fend) {
    const int ustart = HU * pre + hu * nt;
    const int uend = ustart + nt;
    const int seg_end = min(fend, uend);
    const int row = p.rows ? scalar_load(p.rows, seq) : seq;
    const int len = max(scalar_load(p.lens, row), 0);
    const int lo = window_lo(len, p.window);
    const int t_first = tile + (lo >> 4);  // absolute tile ids within the sequence
    const int t_last = t_first + (seg_end - f);
    const int32_t* trow = p.tables + (long)row * p.table_stride;

    // Q^T operand: column q = lr holds Q[seq, head*G + q, 32s + 8*lg .. +8].
    uint4 qo[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (lr < G) {
        const S* qp = (const S*)p.q + ((long)seq * p.Hq + (long)head * G + lr) * D + 32 * s + 8 * lg;
        qo[s] = *(const uint4*)qp;
      } else {
        qo[s] = make_uint4(0, 0, 0, 0);
      }
    }
    float m = kNegInf, l = 0.f;
    f32x4_t o[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Issue the loads of tile t. Tiles past the segment, and pages whose id is
    // out of range, get a zero-sized resource: no memory traffic, zeros back.
    auto load_tile = [&](int t, uint4 (&kr)[KS], uint2 (&vr)[NT], bool& okb) {
      const int page = t / NSUB;
      const int sub = t - page * NSUB;
      int blk = -1;
      if (t < t_last && page < p.table_stride) blk = scalar_load(trow, page);
      okb = blk >= 0 && blk < p.num_blocks;
      const long ph = ((okb ? (long)blk : 0L) * p.Hkv + head) * (long)(B * D);
      const int bytes = okb ? B * D * (int)sizeof(S) : 0;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc((const S*)p.k + ph, bytes);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc((const S*)p.v + ph, bytes);
      const int ksub = sub * 16 * D * (int)sizeof(S);
      const int vsub = sub * 16 * (int)sizeof(S);
#pragma unroll
      for (int s = 0; s < KS; ++s)
        kr[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rk, (k_lane + 32 * s) * (int)sizeof(S), ksub, 0));
#pragma unroll
      for (int j = 0; j < NT; ++j)
        vr[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                              rv, (v_lane + 16 * j * B) * (int)sizeof(S), vsub, 0));
    };
    auto compute_tile = [&](int t, bool okb, const uint4 (&kr)[KS], const uint2 (&vr)[NT]) {
      f32x4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) st = Mfma<T>::qk(kr[s], qo[s], st);
      const int tok0 = t * 16 + 4 * lg;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = st[i] * p.scale_log2;
        if (!okb || (unsigned)(tok0 + i - lo) >= (unsigned)(len - lo)) sc[i] = kNegInf;  // outside [lo, len)
      }
      // m is uniform over the four lanes of a column; a lane compares its own
      // four scores against it, and only when some lane has outgrown it by the
      // slack is the column maximum formed (cross-lane) and the state rescaled.
      float pm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const bool grow = (m == kNegInf) ? (pm != kNegInf) : (pm > m + kRescaleSlack);
      if (__builtin_amdgcn_ballot_w64(grow)) {
        pm = fmaxf(pm, __shfl_xor(pm, 16));
        pm = fmaxf(pm, __shfl_xor(pm, 32));
        const float mn = fmaxf(m, pm);
        const float alpha = (mn == kNegInf) ? 1.f : fast_exp2(m - mn);
        l *= alpha;
        m = mn;
        // O rows are query heads 4*lg + i; their alpha sits in lane (4*lg + i).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ar = __shfl(alpha, 4 * lg + i);
#pragma unroll
          for (int j = 0; j < NT; ++j) o[j][i] *= ar;
        }
      }
      const float ms = (m == kNegInf) ? 0.f : m;
      f32x4_t pr;
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(sc[i] - ms);
      l += (pr[0] + pr[1]) + (pr[2] + pr[3]);  // per-lane partial sum, reduced after the loop
      const uint2 pa = Mfma<T>::pack(pr);
#pragma unroll
      for (int j = 0; j < NT; ++j) o[j] = Mfma<T>::pv(pa, vr[j], o[j]);
    };

    // Three-tile ring: tiles t+1 and t+2 are in flight while t is computed.
    // Every load is issued unconditionally (past-the-end tiles are switched off
    // through their resource), so the wait counts are exact on every path.
    uint4 k0[KS], k1[KS], k2[KS];
    uint2 v0[NT], v1[NT], v2[NT];
    bool ok0, ok1, ok2;
    load_tile(t_first, k0, v0, ok0);
    load_tile(t_first + 1, k1, v1, ok1);
    for (int t = t_first; t < t_last; t += 3) {
      load_tile(t + 2, k2, v2, ok2);
      compute_tile(t, ok0, k0, v0);
      if (t + 1 >= t_last) break;
      load_tile(t + 3, k0, v0, ok0);
      compute_tile(t + 1, ok1, k1, v1);
      if (t + 2 >= t_last) break;
      load_tile(t + 4, k1, v1, ok1);
      compute_tile(t + 2, ok2, k2, v2);
    }

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    // Emit: O rows (query heads) 4*lg + i, columns d = 16 j + lr.
    const bool whole = (f == ustart) && (seg_end == uend);
    const long unit = (long)seq * p.Hkv + head;
    if (whole) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qrow = 4 * lg + i;
        const float lq = __shfl(l, qrow);
        if (qrow < G) {
          const float inv = lq > 0.f ? 1.f / lq : 0.f;
          const long ob = ((long)seq * p.Hq + (long)head * G + qrow) * D + lr;
#pragma unroll
          for (int j = 0; j < NT; ++j) Elem<T>::store1(p.out, ob + 16 * j, o[j][i] * inv);
        }
      }
    } else {
      const long hunit = (long)seq * HU + hu;
      const long slot = (hunit + pe) * TW + wsub;
      const __amdgpu_buffer_rsrc_t rw = partial_rsrc(p, G, D);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qrow = 4 * lg + i;
        if (qrow < G) {
          const int off = (int)(((slot * G + qrow) * D) * (long)sizeof(float));
#pragma unroll
          for (int j = 0; j < NT; j += 4) {
            const pd_u32x4_t v = {__float_as_uint(o[j][i]), __float_as_uint(o[j + 1][i]),
                                  __float_as_uint(o[j + 2][i]), __float_as_uint(o[j + 3][i])};
            __builtin_amdgcn_raw_buffer_store_b128(v, rw, off + 4 * partial_pos(lr, j), 0, kCoherent);
          }
        }
      }
      if (lane < G) {
        put_shared(p.ws_ml + (slot * G + lane) * 2, m);
        put_shared(p.ws_ml + (slot * G + lane) * 2 + 1, l);
      }
      // Arrival: the piece's stores complete, then it is counted; the unit's
      // last piece merges them all.
      const int w0 = range_of(ustart), w1 = range_of(uend - 1);  // the ranges that hold the unit's pieces
      __builtin_amdgcn_s_waitcnt(0);
      int old = 0;
      if (lane == 0) old = __hip_atomic_fetch_add(p.ctr + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __shfl(old, 0);
      if (old == w1 - w0) {
        merge_unit<T, D, G>(p, seq, head, hunit, wsub, w0, w1, lane);
        if (lane == 0) __hip_atomic_store(p.ctr + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }

    f = seg_end;
    if (f >= fend) break;
    // Next unit (skip sequences without tokens).
    ++hu;
    tile = 0;
    if (hu == HU) {
      hu = 0;
      ++seq;
      while (seq < p.N && s_prefix[seq + 1] == s_prefix[seq]) ++seq;
      if (seq >= p.N) break;
      seq = uniform(seq);
      pre = uniform(s_prefix[seq]);
      nt = uniform(s_prefix[seq + 1]) - pre;
    }
    head = hu * TW + wsub;
  }
}

// Persistent grid size of one kernel instantiation: its resident wavefronts on
// the current device (CUs x resident workgroups x 4), cached per device.
template <typename T, int D, int G, int B>
static int persistent_waves() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, paged_decode_mfma_kernel<T, D, G, B>,
                                                   kNativeThreads, 0) != hipSuccess || blocks <= 0)
    blocks = 1;
  cached[dev] = cus * blocks * (kNativeThreads / 64);
  return cached[dev];
}

// The largest persistent grid over the instantiations a call with this head
// geometry may use; the workspace holds one partial slot per wavefront.
template <int D, int G>
static int max_persistent_waves() {
  return max(max(max(persistent_waves<BF16, D, G, 16>(), persistent_waves<BF16, D, G, 32>()),
                 persistent_waves<BF16, D, G, 64>()),
             max(max(persistent_waves<F16, D, G, 16>(), persistent_waves<F16, D, G, 32>()),
                 persistent_waves<F16, D, G, 64>()));
}
static int workspace_waves(int D, int G) {
  switch (D * 100 + G) {
    case 6401: return max_persistent_waves<64, 1>();
    case 6402: return max_persistent_waves<64, 2>();
    case 6404: return max_persistent_waves<64, 4>();
    case 6408: return max_persistent_waves<64, 8>();
    case 6416: return max_persistent_waves<64, 16>();
    case 12801: return max_persistent_waves<128, 1>();
    case 12802: return max_persistent_waves<128, 2>();
    case 12804: return max_persistent_waves<128, 4>();
    case 12808: return max_persistent_waves<128, 8>();
    case 12816: return max_persistent_waves<128, 16>();
    default: return 0;
  }
}

template <typename T, int D, int G, int B>
static int launch_native(NativeParams p, hipStream_t stream) {
  p.W = persistent_waves<T, D, G, B>();  // <= the workspace's wave count
  hipLaunchKernelGGL((paged_decode_mfma_kernel<T, D, G, B>), dim3(p.W / 4), dim3(kNativeThreads), 0, stream, p);
  return (int)hipGetLastError();
}

template <typename T, int D, int G>
static int native_b(const NativeParams& p, hipStream_t s) {
  switch (p.B) {
    case 16: return launch_native<T, D, G, 16>(p, s);
    case 32: return launch_native<T, D, G, 32>(p, s);
    case 64: return launch_native<T, D, G, 64>(p, s);
    default: return MENTAT_EUNSUP;
  }
}

template <typename T, int D>
static int native_g(int G, const NativeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return native_b<T, D, 1>(p, s);
    case 2: return native_b<T, D, 2>(p, s);
    case 4: return native_b<T, D, 4>(p, s);
    case 8: return native_b<T, D, 8>(p, s);
    case 16: return native_b<T, D, 16>(p, s);
    default: return MENTAT_EUNSUP;
  }
}

template <typename T>
static int native_d(int D, int G, const NativeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return native_g<T, 64>(G, p, s);
    case 128: return native_g<T, 128>(G, p, s);
    default: return MENTAT_EUNSUP;
  }
}

}  // namespace mentat

using namespace mentat;

// Workspace of the native path: the reserved counters, then the partial
// slots (units + waves).
size_t native_workspace_bytes(int N, int Hq, int Hkv, int D) {
  const int G = Hq / Hkv;
  const int W = workspace_waves(D, G);
  const size_t slots = (size_t)N * Hkv + W;
  return kWsReserved + slots * G * (D + 2) * sizeof(float);
}

int native_paged_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                        int64_t table_stride, const int32_t* seq_rows, const int32_t* seq_lens,
                        int64_t num_blocks, void* out, int N, int Hq, int Hkv, int D, int block_size,
                        int window_size, float scale, int dtype, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  if (N > kNativeMaxN || (long)N * Hkv > kMaxNativeUnits) return MENTAT_EUNSUP;
  if (block_size != 16 && block_size != 32 && block_size != 64) return MENTAT_EUNSUP;
  if (!block_tables || !seq_lens || table_stride <= 0 || num_blocks <= 0) return MENTAT_EINVAL;
  const size_t need = native_workspace_bytes(N, Hq, Hkv, D);
  if (!workspace || workspace_bytes < need) return MENTAT_ESPACE;
  NativeParams p;
  p.q = q; p.k = k_cache; p.v = v_cache;
  p.tables = block_tables; p.table_stride = table_stride; p.rows = seq_rows; p.lens = seq_lens;
  p.num_blocks = num_blocks; p.out = out;
  const int G = Hq / Hkv;
  p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.B = block_size; p.W = workspace_waves(D, G);
  if (p.W <= 0) return MENTAT_EUNSUP;
  p.TW = (Hkv % 4 == 0) ? 4 : 1;
  p.window = window_size;
  p.scale_log2 = scale * kLog2e;
  const size_t slots = (size_t)N * Hkv + p.W;
  p.ctr = (int32_t*)workspace;
  p.ws_o = (float*)((char*)workspace + kWsReserved);
  p.ws_ml = p.ws_o + slots * G * D;
  switch (dtype) {
    case MENTAT_BF16: return native_d<BF16>(D, G, p, stream);
    case MENTAT_F16: return native_d<F16>(D, G, p, stream);
    default: return MENTAT_EUNSUP;
  }
}
