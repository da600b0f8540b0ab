// Causal (optionally sliding-window) prefill attention on MFMA (gfx950).
//
// The reference's prefill attention (adapters/attention_backend.py:43-96 SDPA
// path, dispatched at :175-189): q [B, S, Hq, D], k/v [B, S, Hkv, D]; query
// head h reads kv head h / G (G = Hq / Hkv); position i attends to keys
// max(0, i - window + 1) .. i (window <= 0 or >= S: all of 0 .. i); softmax
// scale 1/sqrt(D) unless given.
//
// A kv head's query rows are numbered r = position * G + g (g = head within
// the group). A workgroup takes kPfRows consecutive rows of one (batch, kv
// head): each of its 8 wavefronts owns kPfCols 16-column MFMA tiles (S^T =
// K.Q^T on v_mfma 16x16x32, online softmax in base 2 with a lazy rescale,
// O += P.V, as in the decode kernels); tiles with no visible key in a step
// skip it. The workgroup streams the kPfKeys-key K/V stages its rows need
// through a two-stage LDS ring: every thread issues four 16-byte loads of K
// and four of V (4 tokens x 8 dims) for the next stage before the current one
// is computed, and writes V to LDS transposed (one dim's keys per row, 8 bytes
// = 4 keys per write), which is the P.V operand layout. A stage is computed in
// 32-key steps (two S^T chains, one softmax update, P.V on 16x16x32). Loads
// are unconditional (the token index is clamped into the sequence) and values
// of tokens past the sequence end are replaced by zeros. Score masking runs
// only on key blocks some column cannot fully see, and the softmax scale
// rides in the exponent's fma. One tile per wavefront, 8 wavefronts and
// 64-key stages measured fastest (more tiles per wavefront raise register use
// to one wavefront per SIMD; 4 wavefronts or 32-key stages re-stage K/V for
// fewer rows; 128-key stages halve the resident workgroups). That is the
// head_dim 64 kernel; head_dim 128 runs prefill_attn32_kernel below (32
// columns per wavefront on v_mfma_f32_32x32x16).
//
// fp32 prompts run on the VALU decode kernel instead (causal_prefill_f32 in
// paged_decode.hip): one query per position over its visible keys.
#include "mentat_common.h"

namespace mentat {

namespace {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct PMfma;
template <> struct PMfma<BF16> {
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
template <> struct PMfma<F16> {
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

struct PrefillParams {
  const void* q;  // [B, S, Hq, D]
  const void* k;  // [B, S, Hkv, D]
  const void* v;  // [B, S, Hkv, D]
  void* out;      // [B, S, Hq, D]
  int S, Hq, Hkv;
  int window;     // > 0: keys max(0, i - window + 1) .. i; otherwise 0 .. i
  float scale_log2;
};

constexpr int kPfWaves = 8;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfCols = 1;                         // 16-row column tiles per wavefront
constexpr int kPfRows = 16 * kPfCols * kPfWaves;  // query rows per workgroup
constexpr float kPfSlack = 8.f;

// LDS stage of kPfKeys keys: K rows (one token, padded by 16 bytes) and V^T
// rows (one dim's kPfKeys tokens, padded by 8 bytes).
constexpr int kPfKeys = 64;
template <int D> struct PfLds {
  static constexpr int KRS = 2 * D + 16;
  static constexpr int VRS = 2 * kPfKeys + 8;
  static constexpr int KST = kPfKeys * KRS;
  static constexpr int STAGE = KST + D * VRS;
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kPfThreads) void prefill_attn_kernel(PrefillParams p) {
  using S = typename T::storage;
  using L = PfLds<D>;
  constexpr int KS = D / 32, NT = D / 16, NC = kPfCols;
  constexpr int CH = D / 8;                 // 16-byte chunks per token row
  constexpr int NQ = kPfKeys / 4;           // token quads per stage
  static_assert(NQ * CH <= kPfThreads, "one (token quad, chunk) per thread and stage");
  __shared__ __attribute__((aligned(16))) char lds[2 * L::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int rows = p.S * G;
  // Later row blocks have more keys: they get the lower block indices (start first).
  const int rb = (int)(gridDim.x - 1 - blockIdx.x);
  const int hk = blockIdx.y, b = blockIdx.z;
  const int r0 = rb * kPfRows;
  const int pos_lo = r0 / G;
  const int pos_hi = min(p.S - 1, (r0 + kPfRows - 1) / G);
  const int key_lo = p.window > 0 ? max(0, pos_lo - p.window + 1) : 0;
  const int t_lo = key_lo / kPfKeys, t_hi = pos_hi / kPfKeys;

  // Column tile c of this wave: rows rw + 16c + lr -> position, head.
  const int rw = r0 + 16 * NC * wave;
  int tpos_hi[NC], tkey_lo[NC];   // per tile (wave-uniform): last position, first key
  int tpos_lo[NC], tkmin_hi[NC];  // per tile: first position, the latest first key of its columns
  bool tfull[NC];                 // per tile: all 16 columns are rows of the sequence
  int qpos[NC], kmin[NC];         // per lane's column
  bool col_ok[NC];
  uint4 qo[NC][KS];
  f32x4_t o[NC][NT];
  float m[NC], l[NC];
  static_for<NC>([&](auto c_) {
    constexpr int c = decltype(c_)::value;
    const int rt = rw + 16 * c;
    tpos_hi[c] = rt < rows ? min((rt + 15) / G, p.S - 1) : -1;
    tkey_lo[c] = p.window > 0 ? min(rt / G, p.S - 1) - p.window + 1 : 0;
    tpos_lo[c] = rt / G;
    tkmin_hi[c] = p.window > 0 ? tpos_hi[c] - p.window + 1 : 0;
    tfull[c] = rt + 15 < rows;
    const int row = rt + lr;
    col_ok[c] = row < rows;
    qpos[c] = col_ok[c] ? row / G : 0;
    kmin[c] = p.window > 0 ? qpos[c] - p.window + 1 : 0;
    const int qhead = hk * G + (col_ok[c] ? row % G : 0);
    const S* qp = (const S*)p.q + (((long)b * p.S + qpos[c]) * p.Hq + qhead) * D + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 w = *(const uint4*)(qp + 32 * s);
      qo[c][s] = col_ok[c] ? w : make_uint4(0, 0, 0, 0);
    }
    m[c] = kNegInf;
    l[c] = 0.f;
#pragma unroll
    for (int j = 0; j < NT; ++j) o[c][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  });

  // Staging: thread tid < NQ*CH moves tokens 4*tq .. 4*tq+3, dims 8*lc .. 8*lc+7 of
  // K and V; the other threads load a copy of the last block and store nothing,
  // so every load is issued outside any branch.
  // (V with the token quad fastest over consecutive threads: see prefill_attn32_kernel.)
  const bool loader = tid < NQ * CH;
  const int lid = min(tid, NQ * CH - 1);
  const int tq = lid / CH, lc = lid - (lid / CH) * CH;
  const int tqv = lid % NQ, lcv = lid / NQ;
  uint4 kw[4], vw[4];
  auto gload = [&](int t) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tok = t * kPfKeys + 4 * tq + u;
      const int tc = min(tok, p.S - 1);
      kw[u] = *(const uint4*)((const S*)p.k + (((long)b * p.S + tc) * p.Hkv + hk) * D + 8 * lc);
      if (tok >= p.S) kw[u] = make_uint4(0, 0, 0, 0);
      const int tokv = t * kPfKeys + 4 * tqv + u;
      const int tcv = min(tokv, p.S - 1);
      vw[u] = *(const uint4*)((const S*)p.v + (((long)b * p.S + tcv) * p.Hkv + hk) * D + 8 * lcv);
      if (tokv >= p.S) vw[u] = make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](int stage) {
    char* st = lds + stage * L::STAGE;
#pragma unroll
    for (int u = 0; u < 4; ++u) *(uint4*)(st + (4 * tq + u) * L::KRS + lc * 16) = kw[u];
    // V^T row 8lc + i gets tokens 4tq .. 4tq+3 of dim 8lc + i: one 8-byte write.
    const uint32_t* w0 = (const uint32_t*)&vw[0];
    const uint32_t* w1 = (const uint32_t*)&vw[1];
    const uint32_t* w2 = (const uint32_t*)&vw[2];
    const uint32_t* w3 = (const uint32_t*)&vw[3];
    char* vt = st + L::KST + 8 * tqv;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      // dims 8lc + 2h (low halves) and 8lc + 2h + 1 (high halves)
      const uint2 lo = make_uint2(__builtin_amdgcn_perm(w1[h], w0[h], 0x05040100u),
                                  __builtin_amdgcn_perm(w3[h], w2[h], 0x05040100u));
      const uint2 hi = make_uint2(__builtin_amdgcn_perm(w1[h], w0[h], 0x07060302u),
                                  __builtin_amdgcn_perm(w3[h], w2[h], 0x07060302u));
      *(uint2*)(vt + (8 * lcv + 2 * h) * L::VRS) = lo;
      *(uint2*)(vt + (8 * lcv + 2 * h + 1) * L::VRS) = hi;
    }
  };

  gload(t_lo);
  if (loader) lstore(0);
  __syncthreads();
  for (int t = t_lo; t <= t_hi; ++t) {
    const int stage = (t - t_lo) & 1;
    const bool more = t < t_hi;
    gload(min(t + 1, t_hi));  // the last iteration reloads its own stage and stores nothing
    const char* st = lds + stage * L::STAGE;
    // Two 32-key steps: per column tile two S^T chains, one softmax update and
    // O += P.V on 16x16x32 (k = 8lg + i <-> key 4lg + i of the first 16 keys for
    // i < 4, of the second 16 for i >= 4). Each K/V operand read from LDS feeds
    // the MFMAs of every live column tile.
#pragma unroll
    for (int h2 = 0; h2 < kPfKeys / 32; ++h2) {
      const int kb = t * kPfKeys + 32 * h2;  // first key of this step
      bool live[NC];
      bool any = false;
      static_for<NC>([&](auto c_) {
        constexpr int c = decltype(c_)::value;
        live[c] = kb <= tpos_hi[c] && kb + 31 >= tkey_lo[c];
        any |= live[c];
      });
      if (!any) continue;
      const char* ks = st + (32 * h2) * L::KRS;
      f32x4_t s0[NC], s1[NC];
      static_for<NC>([&](auto c_) {
        constexpr int c = decltype(c_)::value;
        s0[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        s1[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      });
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint4 k0 = *(const uint4*)(ks + lr * L::KRS + (32 * s + 8 * lg) * 2);
        const uint4 k1 = *(const uint4*)(ks + (16 + lr) * L::KRS + (32 * s + 8 * lg) * 2);
        static_for<NC>([&](auto c_) {
          constexpr int c = decltype(c_)::value;
          if (live[c]) {
            s0[c] = PMfma<T>::qk(k0, qo[c][s], s0[c]);
            s1[c] = PMfma<T>::qk(k1, qo[c][s], s1[c]);
          }
        });
      }
      uint4 pk[NC];
      static_for<NC>([&](auto c_) {
        constexpr int c = decltype(c_)::value;
        if (!live[c]) return;
        // Raw scores; the scale is applied inside the exponent (one fma per score) and to the
        // running maximum. Masking only where some column of the tile cannot see the whole
        // 32-key block (the diagonal, the window's edge, the sequence's last rows).
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[i] = s0[c][i];
          sc[4 + i] = s1[c][i];
        }
        const bool inside = tfull[c] && kb + 31 <= tpos_lo[c] && kb >= tkmin_hi[c];
        if (!inside) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ka = kb + 4 * lg + i, kc = ka + 16;
            if (!col_ok[c] || ka > qpos[c] || ka < kmin[c]) sc[i] = kNegInf;
            if (!col_ok[c] || kc > qpos[c] || kc < kmin[c]) sc[4 + i] = kNegInf;
          }
        }
        float pm = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                         fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        pm = pm == kNegInf ? kNegInf : pm * p.scale_log2;
        const bool grow = (m[c] == kNegInf) ? (pm != kNegInf) : (pm > m[c] + kPfSlack);
        if (__builtin_amdgcn_ballot_w64(grow)) {
          pm = fmaxf(pm, __shfl_xor(pm, 16));
          pm = fmaxf(pm, __shfl_xor(pm, 32));
          const float mn = fmaxf(m[c], pm);
          const float alpha = (mn == kNegInf) ? 1.f : fast_exp2(m[c] - mn);
          l[c] *= alpha;
          m[c] = mn;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float ar = __shfl(alpha, 4 * lg + i);
#pragma unroll
            for (int j = 0; j < NT; ++j) o[c][j][i] *= ar;
          }
        }
        const float ms = (m[c] == kNegInf) ? 0.f : m[c];
        f32x4_t pa, pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pa[i] = fast_exp2(__builtin_fmaf(sc[i], p.scale_log2, -ms));
          pb[i] = fast_exp2(__builtin_fmaf(sc[4 + i], p.scale_log2, -ms));
        }
        l[c] += ((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pb[0] + pb[1]) + (pb[2] + pb[3]));
        const uint2 ua = PMfma<T>::pack(pa), ub = PMfma<T>::pack(pb);
        pk[c] = make_uint4(ua.x, ua.y, ub.x, ub.y);
      });
      const char* vs = st + L::KST + (32 * h2 + 4 * lg) * 2;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const uint2 va = *(const uint2*)(vs + (16 * j + lr) * L::VRS);
        const uint2 vb = *(const uint2*)(vs + (16 * j + lr) * L::VRS + 32);
        const uint4 vv = make_uint4(va.x, va.y, vb.x, vb.y);
        static_for<NC>([&](auto c_) {
          constexpr int c = decltype(c_)::value;
          if (live[c]) o[c][j] = PMfma<T>::qk(pk[c], vv, o[c][j]);
        });
      }
    }
    if (loader && more) lstore(stage ^ 1);
    __syncthreads();
  }

  // O rows of tile c are its columns 4lg + i; their l sits in lane 4lg + i.
  static_for<NC>([&](auto c_) {
    constexpr int c = decltype(c_)::value;
    float lt = l[c];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 4 * lg + i;
      const float lcol = __shfl(lt, col);
      const int r = rw + 16 * c + col;
      if (r < rows) {
        const int pos = r / G, head = hk * G + r % G;
        const float inv = lcol > 0.f ? 1.f / lcol : 0.f;
        const long ob = (((long)b * p.S + pos) * p.Hq + head) * D + lr;
#pragma unroll
        for (int j = 0; j < NT; ++j) Elem<T>::store1(p.out, ob + 16 * j, o[c][j][i] * inv);
      }
    }
  });
}

// ---- head_dim 128: 32 query columns per wavefront on v_mfma_f32_32x32x16 ----
// Per 32-key step a wavefront computes S^T[32 keys x 32 query columns] =
// K.Q^T (8 MFMAs over 16-dim blocks; A = K rows from LDS, B = the column's q in
// registers) and O^T[128 dims x 32 columns] += V^T.P^T (2 key chunks x 4 dim
// blocks). Each K/V operand read from LDS thus feeds 32 columns, twice the
// 16-column kernel's, which is LDS-bound at one tile per wavefront. Lane l owns
// column l % 32; its 16 accumulator values of S^T are keys 8(r/4) + 4(l/32) +
// r%4 of the step (r < 16), the other 16 keys of the column sit in lane l ^ 32,
// so the column's running maximum takes one exchange and the O rescale none.
// P^T as the B operand of chunk c is the lane's values r = 8c .. 8c+7 as they
// are: MFMA k index 8(l/32) + e is key 16c + 8(e/4) + 4(l/32) + e%4, and the
// A operand V^T reads exactly those keys of its dim (two 8-byte LDS reads).
typedef float f32x16_t __attribute__((ext_vector_type(16)));
template <typename T> struct PMfma32;
template <> struct PMfma32<BF16> {
  __device__ static f32x16_t mma(const uint4& a, const uint4& b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  __device__ static uint32_t bits(float v) { return f32_to_bf16(v); }
};
template <> struct PMfma32<F16> {
  __device__ static f32x16_t mma(const uint4& a, const uint4& b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
  __device__ static uint32_t bits(float v) { return f32_to_f16_bits(v); }
};

// W wavefronts per workgroup: 32 W query rows share each staged K/V stage.
template <typename T, int G, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_attn32_kernel(PrefillParams p) {
  constexpr int kP32Rows = 32 * W;
  using S = typename T::storage;
  constexpr int D = 128;
  using L = PfLds<D>;
  using M = PMfma32<T>;
  constexpr int CH = D / 8;        // 16-byte chunks per token row
  constexpr int NQ = kPfKeys / 4;  // token quads per stage
  static_assert(NQ * CH <= 64 * W, "one (token quad, chunk) per thread and stage");
  __shared__ __attribute__((aligned(16))) char lds[2 * L::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;
  const int rows = p.S * G;
  const int rb = (int)(gridDim.x - 1 - blockIdx.x);  // later row blocks (more keys) start first
  const int hk = blockIdx.y, b = blockIdx.z;
  const int r0 = rb * kP32Rows;
  const int pos_lo = r0 / G;
  const int pos_hi = min(p.S - 1, (r0 + kP32Rows - 1) / G);
  const int key_lo = p.window > 0 ? max(0, pos_lo - p.window + 1) : 0;
  const int t_lo = key_lo / kPfKeys, t_hi = pos_hi / kPfKeys;

  // This wavefront's columns: rows rw .. rw + 31 (position row / G, head row % G).
  const int rw = r0 + 32 * wave;
  const int tpos_hi = rw < rows ? min((rw + 31) / G, p.S - 1) : -1;
  const int tkey_lo = p.window > 0 ? min(rw / G, p.S - 1) - p.window + 1 : 0;
  const int tpos_lo = rw / G;
  const int tkmin_hi = p.window > 0 ? tpos_hi - p.window + 1 : 0;
  const bool tfull = rw + 31 < rows;
  const int row = rw + n;
  const bool col_ok = row < rows;
  const int qpos = col_ok ? row / G : 0;
  const int kmin = p.window > 0 ? qpos - p.window + 1 : 0;
  const int qhead = hk * G + (col_ok ? row % G : 0);
  uint4 qo[D / 16];  // B operand of dim block s: dims 16s + 8h .. 16s + 8h + 7 of the column
  {
    const S* qp = (const S*)p.q + (((long)b * p.S + qpos) * p.Hq + qhead) * D + 8 * h;
#pragma unroll
    for (int s2 = 0; s2 < D / 16; ++s2) {
      const uint4 w = *(const uint4*)(qp + 16 * s2);
      qo[s2] = col_ok ? w : make_uint4(0, 0, 0, 0);
    }
  }
  f32x16_t o[D / 32];
#pragma unroll
  for (int j = 0; j < D / 32; ++j) o[j] = f32x16_t{};
  float m = kNegInf, l = 0.f;

  // Staging as in prefill_attn_kernel: thread tid < NQ*CH moves tokens 4tq .. 4tq+3,
  // dims 8lc .. 8lc+7 of K and V (V written transposed); the others load a copy and
  // store nothing.
  // K: chunk fastest over consecutive threads (coalesced loads, one K row per 16
  // threads); V: token quad fastest, so that the 16 threads of a V^T write fill one
  // contiguous row segment (chunk-fastest V^T writes are 8 rows apart and meet in
  // two LDS banks).
  const bool loader = tid < NQ * CH;
  const int lid = min(tid, NQ * CH - 1);
  const int tq = lid / CH, lc = lid - (lid / CH) * CH;
  const int tqv = lid % NQ, lcv = lid / NQ;
  uint4 kw[4], vw[4];
  // Buffer loads over this (batch, kv head)'s rows: the stage's token offset rides in
  // the scalar offset, the thread's part is fixed, and tokens past the sequence lie
  // past the resource's end and read as zeros.
  const long row_bytes = (long)p.Hkv * D * (long)sizeof(S);
  const long head_off = (((long)b * p.S) * p.Hkv + hk) * D * (long)sizeof(S);
  const int rs_bytes = (int)((long)(p.S - 1) * row_bytes + D * (long)sizeof(S));
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>((const char*)p.k + head_off), (short)0, rs_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>((const char*)p.v + head_off), (short)0, rs_bytes, 0x00020000);
  const int koff = (int)(4 * tq * row_bytes) + 16 * lc;
  const int voff = (int)(4 * tqv * row_bytes) + 16 * lcv;
  auto gload = [&](int t) {
    const int so = (int)((long)t * kPfKeys * row_bytes);  // within the resource or past its end
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kw[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + (int)(u * row_bytes), so, 0));
      vw[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + (int)(u * row_bytes), so, 0));
    }
  };
  auto lstore = [&](int stage) {
    char* st = lds + stage * L::STAGE;
#pragma unroll
    for (int u = 0; u < 4; ++u) *(uint4*)(st + (4 * tq + u) * L::KRS + lc * 16) = kw[u];
    const uint32_t* w0 = (const uint32_t*)&vw[0];
    const uint32_t* w1 = (const uint32_t*)&vw[1];
    const uint32_t* w2 = (const uint32_t*)&vw[2];
    const uint32_t* w3 = (const uint32_t*)&vw[3];
    char* vt = st + L::KST + 8 * tqv;
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const uint2 lo = make_uint2(__builtin_amdgcn_perm(w1[hh], w0[hh], 0x05040100u),
                                  __builtin_amdgcn_perm(w3[hh], w2[hh], 0x05040100u));
      const uint2 hi = make_uint2(__builtin_amdgcn_perm(w1[hh], w0[hh], 0x07060302u),
                                  __builtin_amdgcn_perm(w3[hh], w2[hh], 0x07060302u));
      *(uint2*)(vt + (8 * lcv + 2 * hh) * L::VRS) = lo;
      *(uint2*)(vt + (8 * lcv + 2 * hh + 1) * L::VRS) = hi;
    }
  };

  gload(t_lo);
  if (loader) lstore(0);
  __syncthreads();
  for (int t = t_lo; t <= t_hi; ++t) {
    const int stage = (t - t_lo) & 1;
    const bool more = t < t_hi;
    gload(min(t + 1, t_hi));  // the last iteration reloads its own stage and stores nothing
    const char* st = lds + stage * L::STAGE;
#pragma unroll
    for (int h2 = 0; h2 < kPfKeys / 32; ++h2) {
      const int kb = t * kPfKeys + 32 * h2;  // first key of this step
      if (!(kb <= tpos_hi && kb + 31 >= tkey_lo)) continue;  // wave-uniform: no column sees these keys
      const char* ks = st + (32 * h2 + n) * L::KRS + 16 * h;
      f32x16_t sa = f32x16_t{};
#pragma unroll
      for (int s2 = 0; s2 < D / 16; ++s2) sa = M::mma(*(const uint4*)(ks + 32 * s2), qo[s2], sa);
      float sc[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = sa[r];
      const bool inside = tfull && kb + 31 <= tpos_lo && kb >= tkmin_hi;
      if (!inside) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 8 * (r / 4) + 4 * h + (r % 4);
          if (!col_ok || key > qpos || key < kmin) sc[r] = kNegInf;
        }
      }
      float pm = sc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) pm = fmaxf(pm, sc[r]);
      pm = fmaxf(pm, __shfl_xor(pm, 32));  // the column's other 16 keys
      pm = pm == kNegInf ? kNegInf : pm * p.scale_log2;
      const bool grow = (m == kNegInf) ? (pm != kNegInf) : (pm > m + kPfSlack);
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float mn = fmaxf(m, pm);
        const float alpha = (mn == kNegInf) ? 1.f : fast_exp2(m - mn);
        l *= alpha;
        m = mn;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) o[j] *= alpha;
      }
      const float ms = (m == kNegInf) ? 0.f : m;
      float pr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) pr[r] = fast_exp2(__builtin_fmaf(sc[r], p.scale_log2, -ms));
      float ls = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) ls += pr[r];
      l += ls;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f32x4_t a4 = {pr[8 * c], pr[8 * c + 1], pr[8 * c + 2], pr[8 * c + 3]};
        f32x4_t b4 = {pr[8 * c + 4], pr[8 * c + 5], pr[8 * c + 6], pr[8 * c + 7]};
        const uint2 ua = PMfma<T>::pack(a4), ub = PMfma<T>::pack(b4);
        const uint4 pk = make_uint4(ua.x, ua.y, ub.x, ub.y);
        // V^T of dim 32j + n, keys 16c + 4h .. +3 and 16c + 8 + 4h .. +3 of the step
        const char* vs = st + L::KST + n * L::VRS + (32 * h2 + 16 * c + 4 * h) * 2;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
          const uint2 va = *(const uint2*)(vs + 32 * j * L::VRS);
          const uint2 vb = *(const uint2*)(vs + 32 * j * L::VRS + 16);
          o[j] = M::mma(make_uint4(va.x, va.y, vb.x, vb.y), pk, o[j]);
        }
      }
    }
    if (loader && more) lstore(stage ^ 1);
    __syncthreads();
  }

  // O^T value r of block j is dim 32j + 8(r/4) + 4h + r%4 of the lane's column.
  const float lt = l + __shfl_xor(l, 32);
  if (col_ok) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    S* ob = (S*)p.out + (((long)b * p.S + qpos) * p.Hq + qhead) * D + 4 * h;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t w0 = M::bits(o[j][4 * q4] * inv) | (M::bits(o[j][4 * q4 + 1] * inv) << 16);
        const uint32_t w1 = M::bits(o[j][4 * q4 + 2] * inv) | (M::bits(o[j][4 * q4 + 3] * inv) << 16);
        *(uint2*)(ob + 32 * j + 8 * q4) = make_uint2(w0, w1);
      }
    }
  }
}

// 32-bit buffer offsets over one (batch, kv head)'s rows, the last stage's included.
template <typename T>
bool prefill32_fits(const PrefillParams& p) {
  return (long)(p.S + kPfKeys) * p.Hkv * 128 * (long)sizeof(typename T::storage) <= 0x7fffffffL;
}

template <typename T, int G, int W>
int launch_prefill32w(const PrefillParams& p, int batch, hipStream_t stream) {
  const int blocks = (p.S * G + 32 * W - 1) / (32 * W);
  hipLaunchKernelGGL((prefill_attn32_kernel<T, G, W>), dim3(blocks, p.Hkv, batch), dim3(64 * W), 0, stream, p);
  return (int)hipGetLastError();
}
// Four wavefronts (128 rows) per workgroup, two workgroups per CU: 424 TFLOP/s at
// Llama-3-8B prefill shapes against 392 with eight (one workgroup per CU).
template <typename T, int G>
int launch_prefill32(const PrefillParams& p, int batch, hipStream_t stream) {
  return launch_prefill32w<T, G, 4>(p, batch, stream);
}

template <typename T, int D, int G>
int launch_prefill(const PrefillParams& p, int batch, hipStream_t stream) {
  if constexpr (D == 128) {
    if (prefill32_fits<T>(p)) return launch_prefill32<T, G>(p, batch, stream);
  }
  // head_dim 64, or rows too long for 32-bit offsets: the 16-column kernel (64-bit addressing)
  const int blocks = (p.S * G + kPfRows - 1) / kPfRows;
  hipLaunchKernelGGL((prefill_attn_kernel<T, D, G>), dim3(blocks, p.Hkv, batch), dim3(kPfThreads), 0, stream, p);
  return (int)hipGetLastError();
}

template <typename T, int D>
int prefill_g(int G, const PrefillParams& p, int batch, hipStream_t s) {
  switch (G) {
    case 1: return launch_prefill<T, D, 1>(p, batch, s);
    case 2: return launch_prefill<T, D, 2>(p, batch, s);
    case 4: return launch_prefill<T, D, 4>(p, batch, s);
    case 8: return launch_prefill<T, D, 8>(p, batch, s);
    case 16: return launch_prefill<T, D, 16>(p, batch, s);
    default: return MENTAT_EUNSUP;
  }
}

template <typename T>
int prefill_d(int D, int G, const PrefillParams& p, int batch, hipStream_t s) {
  switch (D) {
    case 64: return prefill_g<T, 64>(G, p, batch, s);
    case 128: return prefill_g<T, 128>(G, p, batch, s);
    default: return MENTAT_EUNSUP;
  }
}

}  // namespace

int causal_prefill_f32(const void* q, const void* k, const void* v, void* out, int batch, int S, int Hq, int Hkv,
                       int D, int window, float scale, hipStream_t stream);

}  // namespace mentat

using namespace mentat;

extern "C" int mentat_prefill_attention(const void* q, const void* k, const void* v, void* out, int batch, int seqlen,
                                        int Hq, int Hkv, int D, int window, float scale, int dtype, void* stream) {
  if (!q || !k || !v || !out || batch < 0 || seqlen < 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return MENTAT_EINVAL;
  if (Hq % Hkv != 0) return MENTAT_EINVAL;
  if (batch == 0 || seqlen == 0) return 0;
  if ((long)seqlen * (Hq / Hkv) > (1L << 30) || batch > 65535 || Hkv > 65535) return MENTAT_EUNSUP;
  PrefillParams p;
  p.q = q; p.k = k; p.v = v; p.out = out;
  p.S = seqlen; p.Hq = Hq; p.Hkv = Hkv;
  p.window = window > 0 && window < seqlen ? window : 0;
  p.scale_log2 = scale * kLog2e;
  const int G = Hq / Hkv;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16: return prefill_d<BF16>(D, G, p, batch, s);
    case MENTAT_F16: return prefill_d<F16>(D, G, p, batch, s);
    case MENTAT_F32: return causal_prefill_f32(q, k, v, out, batch, seqlen, Hq, Hkv, D, p.window, scale, s);
    default: return MENTAT_EUNSUP;
  }
}
