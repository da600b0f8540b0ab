// Prefix-tree (shared-prefix) decode attention on MFMA (gfx950), native pool layout.
//
// Same result as paged decode for every query (sequence i attends to all of its
// cached tokens, core/paged_kv_cache.py:289-368 + adapters/attention_backend.py:192-229),
// but pages shared by several sequences of a branching tree are read once for
// all of them. The host plan splits the batch's contexts into segments: a run
// of 16-token tiles whose block ids are identical for a set of member queries
// (the shared prefix, internal tree edges, each leaf's private tail). A work
// item is (segment chunk, kv head, member group): up to 16/G member queries,
// i.e. one 16-column MFMA query tile (G = Hq/Hkv query heads per member).
// The host puts the member groups of one (chunk, head) next to each other; the
// wavefronts of a workgroup take consecutive items, so the groups of a shared
// chunk run on one CU and re-read its pages from that CU's caches, not HBM.
//
// Per item the wavefront runs the paged_decode_mfma tile loop
// (S^T = K.Q^T on v_mfma 16x16x32, online softmax, O += P.V on 16x16x16) over
// the chunk and writes each member's partial (m, l, O) to its slot; a merge
// kernel combines every query's partials (the LSE rule) into the output.
#include "mentat_common.h"

namespace mentat {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct TMfma;
template <> struct TMfma<BF16> {
  __device__ static f32x4_t qk(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(const uint2& a, const uint2& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  __device__ static uint2 pack(f32x4_t v) { return __builtin_bit_cast(uint2, __builtin_convertvector(v, bf16x4_t)); }
};
template <> struct TMfma<F16> {
  __device__ static f32x4_t qk(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(const uint2& a, const uint2& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
  __device__ static uint2 pack(f32x4_t v) { return __builtin_bit_cast(uint2, __builtin_convertvector(v, f16x4_t)); }
};

// Work item (int32 x kItemFields):
//   [0] table row whose page ids the chunk reads   [1] first tile   [2] tile count
//   [3] valid tokens: the chunk covers tokens [16*first, min(16*(first+count), valid))
//   [4] kv head   [5] member count   [6] first partial slot (member j -> slot + j)
//   [7] offset of the chunk's member query indices in `members`
// Items [0, n_shared) are shared tasks, one workgroup each: the chunk's K/V tiles
// are loaded once into LDS and each wavefront runs one group of 16/G members
// (at most kTreeWaves groups). Items [n_shared, n_shared + n_solo) are solo
// items, one per wavefront (at most 16/G members), reading K/V straight into
// registers.
constexpr int kItemFields = 8;

struct TreeParams {
  const void* q;       // [Nq, Hq, D]
  const void* k;       // native K store [num_blocks][Hkv][B][D]
  const void* v;       // native V store [num_blocks][Hkv][D][B]
  const int32_t* tables;
  int64_t table_stride;
  int64_t num_blocks;
  const int32_t* items;
  int n_shared, n_solo;
  const int32_t* counts;  // optional device [n_shared, n_solo] (within the host's capacities above)
  int grid_shared;        // with counts: workgroups [0, grid_shared) take the shared tasks
  const int32_t* members;
  float* ws_o;         // [slots][G][D]
  float* ws_ml;        // [slots][G][2]
  // merge
  const int32_t* q_slot_off;  // [Nq*Hkv + 1]: partial slots of (query, kv head)
  const int32_t* q_slots;
  void* out;           // [Nq, Hq, D]
  int Nq, Hq, Hkv, B;
  float scale_log2;
};

constexpr int kTreeWaves = 8;
constexpr int kTreeThreads = 64 * kTreeWaves;
constexpr int kTreePrefetch = 4;        // shared path: tiles in flight per loading thread (even)
constexpr int kTreeSharedMaxTiles = 32;  // shared path: tiles per task (host-enforced)
static_assert(kTreeSharedMaxTiles <= 64, "the task's tile mask is 64 bits");
constexpr float kTreeSlack = 8.f;

typedef const int32_t __attribute__((address_space(4)))* tconst_i32;
__device__ __forceinline__ int32_t tld(const int32_t* p, long i) { return ((tconst_i32)p)[i]; }
__device__ __forceinline__ int tuni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t trsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// LDS geometry of one stage of the shared path: two 16-token tiles, K of the
// first, K of the second, then their V as one row of 32 tokens per dim. A V
// row holds, at positions 8g .. 8g + 3, tokens 4g .. 4g + 3 of the first tile
// and at 8g + 4 .. 8g + 7 the same tokens of the second: the k index order of
// the two-tile P.V product, so a lane's V operand is one 16-byte read. K rows
// are padded by 16 bytes and V rows (64 bytes) by 16, which makes the MFMA
// operand reads (16 lanes per row group) bank-conflict free.
template <int D> struct TileLds {
  static constexpr int KRS = 2 * D + 16;
  static constexpr int KST = 16 * KRS;
  static constexpr int VRS = 80;
  static constexpr int PAIR = 2 * KST + D * VRS;
};

// Online-softmax state of one wavefront: 16 query columns (member c/G, head
// c%G), S^T = K.Q^T on v_mfma 16x16x32, O += P.V on 16x16x16.
template <typename T, int D>
struct WaveAttn {
  static constexpr int KS = D / 32, NT = D / 16;
  uint4 qo[KS];
  f32x4_t o[NT];
  float m, l;
  int lr, lg;

  __device__ __forceinline__ void init(const TreeParams& p, int lane, int qidx, int head, int G) {
    using S = typename T::storage;
    lr = lane & 15;
    lg = lane >> 4;
    const int cg = lr % G;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (qidx >= 0) {
        const S* qp = (const S*)p.q + ((long)qidx * p.Hq + (long)head * G + cg) * D + 32 * s + 8 * lg;
        qo[s] = *(const uint4*)qp;
      } else {
        qo[s] = make_uint4(0, 0, 0, 0);
      }
    }
    m = kNegInf;
    l = 0.f;
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // kr[s]: K rows (token lr, dims 32s + 8lg ..+7); vr[j]: V (dim lr + 16j, tokens 4lg ..+3).
  __device__ __forceinline__ void tile(const TreeParams& p, int t, bool okb, int valid, const uint4 (&kr)[KS],
                                       const uint2 (&vr)[NT]) {
    f32x4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) st = TMfma<T>::qk(kr[s], qo[s], st);
    float sc[4];  // raw scores; masked ones -inf
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = st[i];
    if (!(okb && (t + 1) * 16 <= valid)) {  // wave-uniform: only a chunk's last tile is partial
      const int tok0 = t * 16 + 4 * lg;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!okb || tok0 + i >= valid) sc[i] = kNegInf;
    }
    // m (log2 units, scale folded in: scale > 0, so the maximum commutes with
    // it) is uniform over the four lanes of a column; a lane compares its own
    // four scores against it, and only when some lane has outgrown it by the
    // slack is the column maximum formed (cross-lane) and the state rescaled.
    float pm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])) * p.scale_log2;
    const bool grow = (m == kNegInf) ? (pm != kNegInf) : (pm > m + kTreeSlack);
    if (__builtin_amdgcn_ballot_w64(grow)) {
      pm = fmaxf(pm, __shfl_xor(pm, 16));
      pm = fmaxf(pm, __shfl_xor(pm, 32));
      const float mn = fmaxf(m, pm);
      const float alpha = (mn == kNegInf) ? 1.f : fast_exp2(m - mn);
      l *= alpha;
      m = mn;
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
    for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(fmaf(sc[i], p.scale_log2, -ms));
    l += (pr[0] + pr[1]) + (pr[2] + pr[3]);  // per-lane partial sum, reduced in emit()
    const uint2 pa = TMfma<T>::pack(pr);
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = TMfma<T>::pv(pa, vr[j], o[j]);
  }

  // Two tiles (t, t+1) in one step: two independent S^T chains, one softmax
  // update over the 32 scores, and O += P.V on 16x16x32 with the k index
  // 8*lg + i <-> token 4*lg + i of tile t (i < 4) or of tile t+1 (i >= 4):
  // vb[j] = (V of tile t, V of tile t+1) for dims lr + 16j.
  __device__ __forceinline__ void tile2(const TreeParams& p, int t, bool ok0, bool ok1, int valid,
                                        const uint4 (&k0)[KS], const uint4 (&k1)[KS], const uint4 (&vb)[NT]) {
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      s0 = TMfma<T>::qk(k0[s], qo[s], s0);
      s1 = TMfma<T>::qk(k1[s], qo[s], s1);
    }
    float sc[8];  // raw scores; masked ones -inf
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = s0[i];
      sc[4 + i] = s1[i];
    }
    if (!(ok0 && ok1 && (t + 2) * 16 <= valid)) {  // wave-uniform: only a chunk's last step is partial
      const int tok0 = t * 16 + 4 * lg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!ok0 || tok0 + i >= valid) sc[i] = kNegInf;
        if (!ok1 || tok0 + 16 + i >= valid) sc[4 + i] = kNegInf;
      }
    }
    float pm = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]))) *
               p.scale_log2;
    const bool grow = (m == kNegInf) ? (pm != kNegInf) : (pm > m + kTreeSlack);
    if (__builtin_amdgcn_ballot_w64(grow)) {
      pm = fmaxf(pm, __shfl_xor(pm, 16));
      pm = fmaxf(pm, __shfl_xor(pm, 32));
      const float mn = fmaxf(m, pm);
      const float alpha = (mn == kNegInf) ? 1.f : fast_exp2(m - mn);
      l *= alpha;
      m = mn;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ar = __shfl(alpha, 4 * lg + i);
#pragma unroll
        for (int j = 0; j < NT; ++j) o[j][i] *= ar;
      }
    }
    const float ms = (m == kNegInf) ? 0.f : m;
    f32x4_t pa, pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pa[i] = fast_exp2(fmaf(sc[i], p.scale_log2, -ms));
      pb[i] = fast_exp2(fmaf(sc[4 + i], p.scale_log2, -ms));
    }
    l += ((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pb[0] + pb[1]) + (pb[2] + pb[3]));
    const uint2 ua = TMfma<T>::pack(pa), ub = TMfma<T>::pack(pb);
    const uint4 pk = make_uint4(ua.x, ua.y, ub.x, ub.y);
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = TMfma<T>::qk(pk, vb[j], o[j]);
  }

  // Partials of members [0, nmem) of this wave's group; member j -> slot slot0 + j.
  __device__ __forceinline__ void emit(const TreeParams& p, int nmem, int slot0, int G) {
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int mg = 16 / G;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * lg + i;  // O row = query column r: member r/G, head r%G
      const int mem = r / G, g = r % G;
      if (mem < nmem && mem < mg) {
        float* wo = p.ws_o + ((long)(slot0 + mem) * G + g) * D + lr;
#pragma unroll
        for (int j = 0; j < NT; ++j) wo[16 * j] = o[j][i];
      }
    }
    if (lg == 0 && lr / G < nmem) {
      float* ml = p.ws_ml + ((long)(slot0 + lr / G) * G + lr % G) * 2;
      ml[0] = m;
      ml[1] = l;
    }
  }
};

// Shared task: the workgroup streams the chunk's tiles through a two-stage LDS
// ring (every loading thread keeps kTreePrefetch 16-byte loads in flight), one
// barrier per tile; wave w computes member group w.
template <typename T, int D, int G, int B>
__device__ __forceinline__ void tree_shared(const TreeParams& p, const int32_t* item, char* lds) {
  using L = TileLds<D>;
  using S = typename T::storage;
  constexpr int KS = D / 32, NT = D / 16, NSUB = B / 16, MG = 16 / G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tuni(tid >> 6);
  const int row = tld(item, 0), t_first = tld(item, 1), ntile = tld(item, 2), valid = tld(item, 3);
  const int head = tld(item, 4), nmem = tld(item, 5), slot0 = tld(item, 6), moff = tld(item, 7);
  if (ntile <= 0 || ntile > kTreeSharedMaxTiles || nmem <= 0) return;  // uniform over the workgroup
  const int32_t* trow = p.tables + (long)row * p.table_stride;

  // Block ids of the task's tiles, read once into scalar registers (tiles
  // past the chunk repeat the last one and are masked).
  int blk[kTreeSharedMaxTiles];
  uint64_t okm = 0;  // bit i: tile i is inside the chunk and its page id is in range
  static_for<kTreeSharedMaxTiles>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    const int tt = t_first + (i < ntile ? i : ntile - 1);
    const int pg = min(tt / NSUB, (int)p.table_stride - 1);
    const int b = tld(trow, pg);
    const bool ok = i < ntile && b >= 0 && b < p.num_blocks;
    blk[i] = ok ? b : 0;
    okm |= ok ? (1ull << i) : 0ull;
  });

  // This thread's 16-byte piece of every tile: waves [0, 2D/64) carry K,
  // waves [2D/64, 4D/64) carry V, the rest carry nothing (D = 64).
  // A piece lands in LDS as two 8-byte halves, at loff + (tile in stage) *
  // tstep and hstep bytes apart: contiguous for K; for V (tokens 8h .. 8h + 7
  // of dim d) at row positions 16h (+ 4 for the stage's second tile) and 8 further.
  const bool loader = wave * 64 < 4 * D;
  const bool is_k = wave * 64 < 2 * D;
  int goff, loff, tstep, hstep;
  if (is_k) {
    const int tok = tid / (D / 8), dc = tid % (D / 8);
    goff = (tok * D + dc * 8) * (int)sizeof(S);
    loff = tok * L::KRS + dc * 16;
    tstep = L::KST;
    hstep = 8;
  } else {
    const int c = loader ? tid - 2 * D : 0;
    const int d = c >> 1, h = c & 1;
    goff = (d * B + h * 8) * (int)sizeof(S);
    loff = 2 * L::KST + d * L::VRS + 32 * h;
    tstep = 8;
    hstep = 16;
  }
  const S* base = (const S*)(is_k ? p.k : p.v);
  // Tile i of the task (zeros, with no memory traffic, when masked).
  auto issue = [&](auto ic) __attribute__((always_inline)) -> uint4 {
    constexpr int i = decltype(ic)::value;
    const int t = t_first + i;
    const int sub = t - (t / NSUB) * NSUB;
    const bool ok = loader && ((okm >> i) & 1ull);
    const long ph = ((long)blk[i] * p.Hkv + head) * (long)(B * D);
    const __amdgpu_buffer_rsrc_t r = trsrc(base + ph, ok ? B * D * (int)sizeof(S) : 0);
    const int soff = (is_k ? sub * 16 * D : sub * 16) * (int)sizeof(S);
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, goff, soff, 0));
  };

  // Steps of two tiles; tiles 2s, 2s+1 go to LDS stage s & 1. kTreePrefetch
  // tiles are in flight ahead of the one being written (ring of kTreePrefetch
  // + 2 registers, so a step's loads never overwrite what it writes). The
  // steps are unrolled and nested (step s + 1 sits inside step s's branch):
  // with no back edge and no join between steps, the wait before a tile's LDS
  // write counts exactly the loads issued after it. (Sibling branches would
  // join the path that skipped step s - 1, and the waits would assume it.)
  constexpr int R = kTreePrefetch + 2;
  uint4 pf[R];
  static_for<kTreePrefetch>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    pf[i] = issue(ic);
  });
  // The query loads (member index, then q) go out after the first tiles.
  const int g0 = wave * MG;
  const bool active = g0 < nmem;
  WaveAttn<T, D> w;
  {
    const int cm = (lane & 15) / G;
    const int qidx = (active && g0 + cm < nmem) ? p.members[moff + g0 + cm] : -1;
    w.init(p, lane, qidx, head, G);
  }
  auto step = [&](auto self, auto sc_) __attribute__((always_inline)) -> void {
    constexpr int st = decltype(sc_)::value;
    constexpr int i0 = 2 * st;
    {  // i0 < ntile holds here: step 0 runs for ntile >= 1, step s + 1 for 2s + 2 < ntile
      if constexpr (i0 + kTreePrefetch < kTreeSharedMaxTiles)
        pf[(i0 + kTreePrefetch) % R] = issue(std::integral_constant<int, i0 + kTreePrefetch>{});
      if constexpr (i0 + 1 + kTreePrefetch < kTreeSharedMaxTiles)
        pf[(i0 + 1 + kTreePrefetch) % R] = issue(std::integral_constant<int, i0 + 1 + kTreePrefetch>{});
      char* stg = lds + (st & 1) * L::PAIR;
      if (loader) {
        static_for<2>([&](auto hc) __attribute__((always_inline)) {
          constexpr int h = decltype(hc)::value;
          const uint4 cur = pf[(i0 + h) % R];
          char* dst = stg + loff + h * tstep;
          *(uint2*)__builtin_assume_aligned(dst, 8) = make_uint2(cur.x, cur.y);
          *(uint2*)__builtin_assume_aligned(dst + hstep, 8) = make_uint2(cur.z, cur.w);
        });
      }
      __syncthreads();
      if (active) {
        uint4 k0[KS], k1[KS], vb[NT];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          k0[s] = *(const uint4*)__builtin_assume_aligned(stg + w.lr * L::KRS + (4 * s + w.lg) * 16, 16);
          k1[s] = *(const uint4*)__builtin_assume_aligned(stg + L::KST + w.lr * L::KRS + (4 * s + w.lg) * 16, 16);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j)
          vb[j] = *(const uint4*)__builtin_assume_aligned(stg + 2 * L::KST + (w.lr + 16 * j) * L::VRS + w.lg * 16, 16);
        w.tile2(p, t_first + i0, (okm >> i0) & 1ull, (okm >> (i0 + 1)) & 1ull, valid, k0, k1, vb);
      }
    }
    if constexpr (st + 1 < kTreeSharedMaxTiles / 2) {
      if (i0 + 2 < ntile) self(self, std::integral_constant<int, st + 1>{});
    }
  };
  step(step, std::integral_constant<int, 0>{});
  if (active) w.emit(p, nmem - g0, slot0 + g0, G);
}

// Solo item: one wavefront, K/V straight into a three-tile register ring.
template <typename T, int D, int G, int B>
__device__ __forceinline__ void tree_solo(const TreeParams& p, const int32_t* item) {
  using S = typename T::storage;
  constexpr int KS = D / 32, NT = D / 16, NSUB = B / 16;
  const int lane = threadIdx.x & 63;
  const int row = tld(item, 0), t_first = tld(item, 1), ntile = tld(item, 2), valid = tld(item, 3);
  const int head = tld(item, 4), nmem = tld(item, 5), slot0 = tld(item, 6), moff = tld(item, 7);
  if (ntile <= 0 || nmem <= 0) return;
  const int t_last = t_first + ntile;
  const int32_t* trow = p.tables + (long)row * p.table_stride;
  WaveAttn<T, D> w;
  const int k_lane = (lane & 15) * D + 8 * (lane >> 4);
  const int v_lane = (lane & 15) * B + 4 * (lane >> 4);
  auto load_tile = [&](int t, uint4 (&kr)[KS], uint2 (&vr)[NT], bool& okb) __attribute__((always_inline)) {
    const int page = t / NSUB;
    const int sub = t - page * NSUB;
    int blk = -1;
    if (t < t_last && page < p.table_stride) blk = tld(trow, page);
    okb = blk >= 0 && blk < p.num_blocks;
    const long ph = ((okb ? (long)blk : 0L) * p.Hkv + head) * (long)(B * D);
    const int bytes = okb ? B * D * (int)sizeof(S) : 0;
    const __amdgpu_buffer_rsrc_t rk = trsrc((const S*)p.k + ph, bytes);
    const __amdgpu_buffer_rsrc_t rv = trsrc((const S*)p.v + ph, bytes);
    const int ksub = sub * 16 * D * (int)sizeof(S);
    const int vsub = sub * 16 * (int)sizeof(S);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kr[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, (k_lane + 32 * s) * (int)sizeof(S), ksub, 0));
#pragma unroll
    for (int j = 0; j < NT; ++j)
      vr[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, (v_lane + 16 * j * B) * (int)sizeof(S), vsub, 0));
  };
  uint4 k0[KS], k1[KS], k2[KS];
  uint2 v0[NT], v1[NT], v2[NT];
  bool ok0, ok1, ok2;
  load_tile(t_first, k0, v0, ok0);
  load_tile(t_first + 1, k1, v1, ok1);
  {  // the query loads (member index, then q) go out after the first tiles
    const int cm = (lane & 15) / G;
    w.init(p, lane, cm < nmem ? p.members[moff + cm] : -1, head, G);
  }
  for (int t = t_first; t < t_last; t += 3) {
    load_tile(t + 2, k2, v2, ok2);
    w.tile(p, t, ok0, valid, k0, v0);
    if (t + 1 >= t_last) break;
    load_tile(t + 3, k0, v0, ok0);
    w.tile(p, t + 1, ok1, valid, k1, v1);
    if (t + 2 >= t_last) break;
    load_tile(t + 4, k1, v1, ok1);
    w.tile(p, t + 2, ok2, valid, k2, v2);
  }
  w.emit(p, nmem, slot0, G);
}

template <typename T, int D, int G, int B>
__global__ __launch_bounds__(kTreeThreads) void tree_decode_kernel(TreeParams p) {
  __shared__ uint4 lds_words[2 * TileLds<D>::PAIR / 16];  // 2 stages of 2 tiles
  char* lds = (char*)lds_words;
  const int bid = blockIdx.x;
  if (p.counts) {
    // Item counts from device memory (a captured launch takes each step's
    // plan): a fixed grid, workgroups [0, grid_shared) stride over the shared
    // tasks, the others' wavefronts over the solo items.
    const int n_shared = min(max(tld(p.counts, 0), 0), p.n_shared);
    const int n_solo = min(max(tld(p.counts, 1), 0), p.n_solo);
    if (bid < p.grid_shared) {
      for (int t = bid; t < n_shared; t += p.grid_shared) {
        tree_shared<T, D, G, B>(p, p.items + (long)t * kItemFields, lds);
        __syncthreads();  // the next task restages the LDS ring
      }
      return;
    }
    const int step = ((int)gridDim.x - p.grid_shared) * kTreeWaves;
    for (int it = (bid - p.grid_shared) * kTreeWaves + tuni(threadIdx.x >> 6); it < n_solo; it += step)
      tree_solo<T, D, G, B>(p, p.items + (long)(n_shared + it) * kItemFields);
    return;
  }
  if (bid < p.n_shared) {
    tree_shared<T, D, G, B>(p, p.items + (long)bid * kItemFields, lds);
    return;
  }
  const int it = p.n_shared + (bid - p.n_shared) * kTreeWaves + tuni(threadIdx.x >> 6);
  if (it >= p.n_shared + p.n_solo) return;
  tree_solo<T, D, G, B>(p, p.items + (long)it * kItemFields);
}

// Merge: one wavefront per (query, kv head). The column maxima M_g and sums
// L_g come from a pass over the (slot, head) pairs spread across the lanes
// (lane j always has head j % G); the output pass then weights every slot's
// partial O by exp2(m - M_g), loads that do not depend on one another.
template <typename T, int D, int G>
__global__ __launch_bounds__(64) void tree_merge_kernel(TreeParams p) {
  constexpr int E = G * D / 64;  // outputs per lane
  const int u = blockIdx.x;      // query * Hkv + head
  if (u >= p.Nq * p.Hkv) return;
  const int qi = u / p.Hkv, head = u - (u / p.Hkv) * p.Hkv;
  const int lane = threadIdx.x;
  const int b = tld(p.q_slot_off, u), e = tld(p.q_slot_off, u + 1);
  const int n = e - b;
  // pass 1: per-lane max over its (slot, head lane % G) pairs, then over lanes of one head
  const int gl = lane % G;
  float mx = kNegInf;
  for (int i = lane; i < n * G; i += 64) {
    const long slot = p.q_slots[b + i / G];
    mx = fmaxf(mx, p.ws_ml[(slot * G + gl) * 2]);
  }
#pragma unroll
  for (int off = G; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  const float mref = (mx == kNegInf) ? 0.f : mx;
  float ls = 0.f;
  for (int i = lane; i < n * G; i += 64) {
    const long slot = p.q_slots[b + i / G];
    const float* ml = p.ws_ml + (slot * G + gl) * 2;
    ls += ml[1] * fast_exp2(ml[0] - mref);
  }
#pragma unroll
  for (int off = G; off < 64; off <<= 1) ls += __shfl_xor(ls, off);
  // pass 2: this lane's E outputs of head g
  const int g = (lane * E) / D, d0 = lane * E - g * D;
  const float Mg = __shfl(mref, g), Lg = __shfl(ls, g);
  float acc[E];
#pragma unroll
  for (int j = 0; j < E; ++j) acc[j] = 0.f;
#pragma unroll 4
  for (int s = b; s < e; ++s) {
    const long slot = tld(p.q_slots, s);
    const float c = fast_exp2(p.ws_ml[(slot * G + g) * 2] - Mg);
    const float* wo = p.ws_o + (slot * G + g) * D + d0;
#pragma unroll
    for (int j = 0; j < E; ++j) acc[j] += wo[j] * c;
  }
  const float inv = Lg > 0.f ? 1.f / Lg : 0.f;
  const long ob = ((long)qi * p.Hq + (long)head * G + g) * D + d0;
#pragma unroll
  for (int j = 0; j < E; ++j) Elem<T>::store1(p.out, ob + j, acc[j] * inv);
}

// Fixed grid of the counted mode: workgroups for the shared tasks and for the
// solo items, each at most what the capacities need.
constexpr int kTreeGridShared = 256;
constexpr int kTreeGridSolo = 1024;

template <typename T, int D, int G, int B>
static int tree_launch(const TreeParams& p, hipStream_t s) {
  const int blocks = p.counts ? p.grid_shared + min(kTreeGridSolo, (p.n_solo + kTreeWaves - 1) / kTreeWaves)
                              : p.n_shared + (p.n_solo + kTreeWaves - 1) / kTreeWaves;
  if (blocks > 0)
    hipLaunchKernelGGL((tree_decode_kernel<T, D, G, B>), dim3(blocks), dim3(kTreeThreads), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((tree_merge_kernel<T, D, G>), dim3(p.Nq * p.Hkv), dim3(64), 0, s, p);
  return (int)hipGetLastError();
}

template <typename T, int D, int G>
static int tree_b(const TreeParams& p, hipStream_t s) {
  switch (p.B) {
    case 16: return tree_launch<T, D, G, 16>(p, s);
    case 32: return tree_launch<T, D, G, 32>(p, s);
    case 64: return tree_launch<T, D, G, 64>(p, s);
    default: return MENTAT_EUNSUP;
  }
}
template <typename T, int D>
static int tree_g(int G, const TreeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return tree_b<T, D, 1>(p, s);
    case 2: return tree_b<T, D, 2>(p, s);
    case 4: return tree_b<T, D, 4>(p, s);
    case 8: return tree_b<T, D, 8>(p, s);
    case 16: return tree_b<T, D, 16>(p, s);
    default: return MENTAT_EUNSUP;
  }
}
template <typename T>
static int tree_d(int D, int G, const TreeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return tree_g<T, 64>(G, p, s);
    case 128: return tree_g<T, 128>(G, p, s);
    default: return MENTAT_EUNSUP;
  }
}

}  // namespace mentat

using namespace mentat;

extern "C" size_t mentat_tree_decode_workspace_bytes(int n_slots, int Hq, int Hkv, int D) {
  if (n_slots <= 0 || Hkv <= 0) return 0;
  const int G = Hq / Hkv;
  return kWsReserved + (size_t)n_slots * G * (D + 2) * sizeof(float);
}

static int tree_decode_call(const void* q, const void* k_store, const void* v_store, const int32_t* block_tables,
                            int64_t table_stride, int64_t num_blocks, const int32_t* items, int n_shared, int n_solo,
                            const int32_t* counts, const int32_t* members, const int32_t* q_slot_offsets,
                            const int32_t* q_slots, int n_slots, void* out, int Nq, int Hq, int Hkv, int D,
                            int block_size, float scale, int dtype, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (Nq == 0) return MENTAT_OK;
  if (!q || !k_store || !v_store || !block_tables || !out || !q_slot_offsets || Nq < 0 || Hq <= 0 || Hkv <= 0 ||
      Hq % Hkv != 0 || table_stride <= 0 || num_blocks <= 0 || n_shared < 0 || n_solo < 0 || n_slots < 0)
    return MENTAT_EINVAL;
  if (n_shared + n_solo > 0 && (!items || !members || !q_slots)) return MENTAT_EINVAL;
  if (!(scale > 0.f) || !std::isfinite(scale)) return MENTAT_EINVAL;  // the kernels fold a positive scale into exp2
  const size_t need = mentat_tree_decode_workspace_bytes(n_slots, Hq, Hkv, D);
  if (need && (!workspace || workspace_bytes < need)) return MENTAT_ESPACE;
  TreeParams p;
  p.q = q; p.k = k_store; p.v = v_store; p.tables = block_tables; p.table_stride = table_stride;
  p.num_blocks = num_blocks; p.items = items; p.n_shared = n_shared; p.n_solo = n_solo; p.members = members;
  p.counts = counts;
  p.grid_shared = counts ? min(kTreeGridShared, n_shared) : 0;
  const int G = Hq / Hkv;
  p.ws_o = (float*)((char*)workspace + kWsReserved);
  p.ws_ml = p.ws_o + (size_t)n_slots * G * D;
  p.q_slot_off = q_slot_offsets; p.q_slots = q_slots; p.out = out;
  p.Nq = Nq; p.Hq = Hq; p.Hkv = Hkv; p.B = block_size; p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16: return tree_d<BF16>(D, G, p, s);
    case MENTAT_F16: return tree_d<F16>(D, G, p, s);
    default: return MENTAT_EUNSUP;
  }
}

extern "C" int mentat_tree_decode(const void* q, const void* k_store, const void* v_store, const int32_t* block_tables,
                                  int64_t table_stride, int64_t num_blocks, const int32_t* items, int n_shared,
                                  int n_solo, const int32_t* members, const int32_t* q_slot_offsets,
                                  const int32_t* q_slots, int n_slots, void* out, int Nq, int Hq, int Hkv, int D,
                                  int block_size, float scale, int dtype, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  return tree_decode_call(q, k_store, v_store, block_tables, table_stride, num_blocks, items, n_shared, n_solo,
                          nullptr, members, q_slot_offsets, q_slots, n_slots, out, Nq, Hq, Hkv, D, block_size, scale,
                          dtype, workspace, workspace_bytes, stream);
}

extern "C" int mentat_tree_decode_counted(const void* q, const void* k_store, const void* v_store,
                                          const int32_t* block_tables, int64_t table_stride, int64_t num_blocks,
                                          const int32_t* items, const int32_t* counts, int max_shared, int max_solo,
                                          const int32_t* members, const int32_t* q_slot_offsets,
                                          const int32_t* q_slots, int max_slots, void* out, int Nq, int Hq, int Hkv,
                                          int D, int block_size, float scale, int dtype, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  if (!counts) return MENTAT_EINVAL;
  return tree_decode_call(q, k_store, v_store, block_tables, table_stride, num_blocks, items, max_shared, max_solo,
                          counts, members, q_slot_offsets, q_slots, max_slots, out, Nq, Hq, Hkv, D, block_size, scale,
                          dtype, workspace, workspace_bytes, stream);
}
