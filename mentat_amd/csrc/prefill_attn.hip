// Causal (optionally sliding-window) prefill attention on MFMA (gfx950).
//
// The reference's prefill attention (adapters/attention_backend.py:43-96 SDPA
// path, dispatched at :175-189): q [B, S, Hq, D], k/v [B, S, Hkv, D]; query
// head h reads kv head h / G (G = Hq / Hkv); position i attends to keys
// max(0, i - window + 1) .. i (window <= 0 or >= S: all of 0 .. i); softmax
// scale 1/sqrt(D) unless given.
//
// A kv head's query rows are numbered r = position * G + g (g = head within
// the group). A workgroup takes 64 consecutive rows of one (batch, kv head):
// each of its 4 wavefronts owns 16 rows, which are the 16 columns of its MFMA
// tiles (S^T = K.Q^T on v_mfma 16x16x32, online softmax in base 2 with a lazy
// rescale, O += P.V on 16x16x16, as in the decode kernels). The workgroup
// streams the 16-token K/V tiles its rows need through a two-stage LDS ring:
// every thread issues one 16-byte load of K and one of V for the next tile
// before the current tile is computed; V is written to LDS transposed (one
// dim's 16 tokens per row), which is the P.V operand layout. Loads are
// unconditional (the token index is clamped into the sequence) and values of
// tokens past the sequence end are replaced by zeros.
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

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 16 * kPfWaves;  // query rows per workgroup
constexpr float kPfSlack = 8.f;

// LDS stage: K rows (16 tokens, padded by 16 bytes) and V^T rows (one dim's 16
// tokens, padded by 8): conflict-free 16-lane MFMA operand reads.
template <int D> struct PfLds {
  static constexpr int KRS = 2 * D + 16;
  static constexpr int VRS = 40;
  static constexpr int KST = 16 * KRS;
  static constexpr int STAGE = KST + D * VRS;
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kPfThreads) void prefill_attn_kernel(PrefillParams p) {
  using S = typename T::storage;
  using L = PfLds<D>;
  constexpr int KS = D / 32, NT = D / 16;
  constexpr int CH = D / 8;                 // 16-byte chunks per token row
  static_assert(16 * CH <= kPfThreads, "one K and one V chunk per thread and tile");
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
  const int t_lo = key_lo / 16, t_hi = pos_hi / 16;

  // This wave's 16 rows (columns of its tiles): row rw + lr -> position, head.
  const int rw = r0 + 16 * wave;
  const int wpos_lo = min(rw / G, p.S - 1);
  const int wpos_hi = min((rw + 15) / G, p.S - 1);
  const bool wave_live = rw < rows;
  const int row = rw + lr;
  const bool col_ok = row < rows;
  const int qpos = col_ok ? row / G : 0;
  const int qhead = hk * G + (col_ok ? row % G : 0);
  const int kmin = p.window > 0 ? qpos - p.window + 1 : 0;  // first key of this column

  // Q^T operand: column lr holds Q[b, qpos, qhead, 32s + 8lg .. +8].
  uint4 qo[KS];
  {
    const S* qp = (const S*)p.q + (((long)b * p.S + qpos) * p.Hq + qhead) * D + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 w = *(const uint4*)(qp + 32 * s);
      qo[s] = col_ok ? w : make_uint4(0, 0, 0, 0);
    }
  }
  float m = kNegInf, l = 0.f;
  f32x4_t o[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Staging: thread tid < 16*CH moves chunk (token tid / CH, dims 8*(tid % CH) ..+8);
  // the other threads load a copy of the last chunk and store nothing, so every
  // load is issued outside any branch.
  const bool loader = tid < 16 * CH;
  const int lid = min(tid, 16 * CH - 1);
  const int ltok = lid / CH, lch = lid - (lid / CH) * CH;
  auto gload = [&](int t, uint4& kw, uint4& vw) {
    const int tok = t * 16 + ltok;
    const int tc = min(tok, p.S - 1);
    const long off = (((long)b * p.S + tc) * p.Hkv + hk) * D + 8 * lch;
    kw = *(const uint4*)((const S*)p.k + off);
    vw = *(const uint4*)((const S*)p.v + off);
    if (tok >= p.S) { kw = make_uint4(0, 0, 0, 0); vw = make_uint4(0, 0, 0, 0); }
  };
  auto lstore = [&](int stage, const uint4& kw, const uint4& vw) {
    char* st = lds + stage * L::STAGE;
    *(uint4*)(st + ltok * L::KRS + lch * 16) = kw;
    const uint16_t* e = (const uint16_t*)&vw;
    char* vt = st + L::KST;
#pragma unroll
    for (int i = 0; i < 8; ++i) *(uint16_t*)(vt + (8 * lch + i) * L::VRS + 2 * ltok) = e[i];
  };

  uint4 kw, vw;
  gload(t_lo, kw, vw);
  if (loader) lstore(0, kw, vw);
  __syncthreads();
  for (int t = t_lo; t <= t_hi; ++t) {
    const int stage = (t - t_lo) & 1;
    const bool more = t < t_hi;
    gload(min(t + 1, t_hi), kw, vw);  // the last iteration reloads its own tile and stores nothing
    // Tiles wholly after this wave's last position or before its first key are skipped.
    const bool use = wave_live && 16 * t <= wpos_hi &&
                     (p.window <= 0 || 16 * t + 15 >= wpos_lo - p.window + 1);
    if (use) {
      const char* st = lds + stage * L::STAGE;
      uint4 kr[KS];
      uint2 vr[NT];
#pragma unroll
      for (int s = 0; s < KS; ++s) kr[s] = *(const uint4*)(st + lr * L::KRS + (32 * s + 8 * lg) * 2);
#pragma unroll
      for (int j = 0; j < NT; ++j) vr[j] = *(const uint2*)(st + L::KST + (16 * j + lr) * L::VRS + 8 * lg);
      f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) sacc = PMfma<T>::qk(kr[s], qo[s], sacc);
      const int key0 = t * 16 + 4 * lg;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = key0 + i;
        sc[i] = sacc[i] * p.scale_log2;
        if (!col_ok || kk > qpos || kk < kmin) sc[i] = kNegInf;
      }
      float pm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const bool grow = (m == kNegInf) ? (pm != kNegInf) : (pm > m + kPfSlack);
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
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(sc[i] - ms);
      l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      const uint2 pa = PMfma<T>::pack(pr);
#pragma unroll
      for (int j = 0; j < NT; ++j) o[j] = PMfma<T>::pv(pa, vr[j], o[j]);
    }
    if (loader && more) lstore(stage ^ 1, kw, vw);
    __syncthreads();
  }

  if (!wave_live) return;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  // O rows are the wave's columns 4lg + i; their l sits in lane 4lg + i.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 4 * lg + i;
    const float lc = __shfl(l, c);
    const int r = rw + c;
    if (r < rows) {
      const int pos = r / G, head = hk * G + r % G;
      const float inv = lc > 0.f ? 1.f / lc : 0.f;
      const long ob = (((long)b * p.S + pos) * p.Hq + head) * D + lr;
#pragma unroll
      for (int j = 0; j < NT; ++j) Elem<T>::store1(p.out, ob + 16 * j, o[j][i] * inv);
    }
  }
}

template <typename T, int D, int G>
int launch_prefill(const PrefillParams& p, int batch, hipStream_t stream) {
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
    default: return MENTAT_EUNSUP;
  }
}
