// Fused per-row entropy, gate, repetition penalty, argmax / top-K and
// temperature + top-p sampling over the full vocabulary (gfx950).
//
// One 1024-thread workgroup per logits row. Every pass streams the row with
// 16-byte loads in the order element = (chunk*1024 + thread)*EPV + e, eight
// loads in flight per thread. Passes: maxima; entropy sums + the first radix
// level of the sampler's masses; top-K (K passes, only when asked); the
// sampler's deeper radix levels (elements of one bin only), the last one also
// counting the chosen key's tokens per chunk, so the final index search reads
// one chunk.
//
// Per row (reference semantics, cited):
//   H_T      entropy of softmax(x / T) of the raw logits, in nats
//            (compute_entropy at the gate temperature, core/generator_utils.py:196-202,
//            called at core/generator.py:342); fp32 instead of the logits dtype.
//   gate     H_T > gate_threshold (absolute gate; the relative EMA gate of
//            core/generator.py:346-369 is applied by the host on H_T).
//   xp       repetition penalty on the row's generated ids (deduplicated, as the
//            reference's set(), core/generator_utils.py:205-230):
//            x > 0 ? x / p : x * p in fp32, rounded to the logits dtype.
//   keys     log_softmax(xp) as torch forms it: fl(fl(xp - max) - log(sum exp)),
//            rounded to the logits dtype (core/generator.py:283, :308).
//   top-K    the K largest keys, ties to the lowest index; argmax = top-1
//            (torch.argmax's first-occurrence rule; torch.topk leaves tie order
//            unspecified, this kernel fixes it) and their log-probs = keys.
//   H_pen    entropy of softmax(xp) at T = 1 (the diagnostic of core/generator.py:293).
//   sample   temperature + top-p draw from xp with a Philox4x32-10 stream; the
//            bit-exact specification (deterministic exp2, 2^40 fixed-point masses,
//            nucleus and inverse-CDF draw) is the oracle's sampling_ref.c.
#include <utility>

#include "mentat_common.h"

#pragma clang fp contract(off)

namespace mentat {

constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kMaxTopK = 8;

struct RowParams {
  const void* logits;
  int64_t row_stride;  // elements
  int R, V;
  float ent_c;         // log2(e) / T for the gate entropy
  float samp_c;        // log2(e) / T for the sampler
  float penalty;       // 1.0 = off
  const int32_t* pen_offsets;  // [R+1] or null
  const int32_t* pen_ids;
  int topk;
  uint64_t top_p_q32;  // round(top_p * 2^32)
  uint64_t seed;
  uint64_t step;
  int do_sample;
  float gate_threshold;
  float* out_entropy;      // [R]
  float* out_entropy_pen;  // [R] or null
  float* out_lse;          // [R] or null (log-sum-exp of xp)
  uint8_t* out_gate;       // [R] or null
  int32_t* out_topk;       // [R, topk] or null
  float* out_topk_lp;      // [R, topk] or null
  int32_t* out_sample;     // [R] or null
};

// ---- deterministic exp2 and Philox (must match oracle/csrc/sampling_ref.c) ----------------
__device__ __forceinline__ float det_exp2(float y) {
  if (!(y >= -64.0f)) return 0.0f;
  const float n = rintf(y);
  const float f = y - n;
  float p = 0x1.ffcbfcp-17f;
  p = fmaf(p, f, 0x1.430912p-13f);
  p = fmaf(p, f, 0x1.5d87fep-10f);
  p = fmaf(p, f, 0x1.3b2ab6p-7f);
  p = fmaf(p, f, 0x1.c6b08ep-5f);
  p = fmaf(p, f, 0x1.ebfbe0p-3f);
  p = fmaf(p, f, 0x1.62e430p-1f);
  p = fmaf(p, f, 0x1.000000p+0f);
  return ldexpf(p, (int)n);
}
__device__ __forceinline__ uint64_t det_q(float y) {
  return (uint64_t)(det_exp2(y) * 0x1p40f);
}
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
_Pragma("clang loop unroll(full)")
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[1] = (uint32_t)p1;
    c[3] = (uint32_t)p0;
    c[0] = n0;
    c[2] = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// ---- element access ---------------------------------------------------------------------
template <typename T> struct RowElem;
template <> struct RowElem<BF16> {
  static constexpr int EPV = 8;
  __device__ __forceinline__ static float get(const uint4& w, int e) {
    const uint32_t d = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
    return (e & 1) ? bf16_hi(d) : bf16_lo(d);
  }
  __device__ __forceinline__ static float round(float v) { return __uint_as_float(((uint32_t)f32_to_bf16(v)) << 16); }
  // Order-preserving 32-bit key of a value of this dtype (only the top 16 bits vary).
  __device__ __forceinline__ static uint32_t key(float v) {
    const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);  // -0 and +0 tie, as in float order
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  __device__ __forceinline__ static float scalar(const void* p, long i) { return Elem<BF16>::load1(p, i); }
  // Radix levels (bits, most significant first) covering the key bits that vary.
  static constexpr int nlevels = 2;
  static constexpr int level_bits[3] = {12, 4, 0};
};
template <> struct RowElem<F16> {
  static constexpr int EPV = 8;
  __device__ __forceinline__ static float get(const uint4& w, int e) {
    const uint32_t d = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
    return f16_bits_to_f32((uint16_t)((e & 1) ? (d >> 16) : (d & 0xffffu)));
  }
  __device__ __forceinline__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
  __device__ __forceinline__ static uint32_t key(float v) {
    const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);  // -0 and +0 tie, as in float order
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  __device__ __forceinline__ static float scalar(const void* p, long i) { return Elem<F16>::load1(p, i); }
  static constexpr int nlevels = 3;
  static constexpr int level_bits[3] = {12, 12, 8};
};
template <> struct RowElem<F32> {
  static constexpr int EPV = 4;
  __device__ __forceinline__ static float get(const uint4& w, int e) {
    return __uint_as_float(e == 0 ? w.x : e == 1 ? w.y : e == 2 ? w.z : w.w);
  }
  __device__ __forceinline__ static float round(float v) { return v; }
  __device__ __forceinline__ static uint32_t key(float v) {
    const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);  // -0 and +0 tie, as in float order
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  __device__ __forceinline__ static float scalar(const void* p, long i) { return ((const float*)p)[i]; }
  static constexpr int nlevels = 3;
  static constexpr int level_bits[3] = {12, 12, 8};
};

// Inverse of RowElem::key: the float whose ordered key is k.
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ---- block reductions (1024 threads) ----------------------------------------------------------
constexpr int kHistBins = 4096;  // widest radix level: 12 key bits

template <int NW>
struct RowSharedT {
  static constexpr int kWaves = NW;
  float f[NW * 4];
  uint64_t u[NW];
  uint64_t hist0[kHistBins];  // first radix level (shared by both selections)
  uint64_t hist1[kHistBins];  // deeper levels
  uint32_t sel[4];
  uint64_t sel64[4];
  float bk[NW];
  int32_t bi[NW];
  uint32_t chunk_tot[64];
  uint32_t cc[64 * 16];  // per-chunk counts of the last radix level's values (<= 16 of them)
  uint32_t cc2[64 * 16]; // the same for a second level-0 bin (single-pass sampler)
  uint64_t hn[16];       // level 1 of the nucleus-boundary bin (single-pass sampler)
  int32_t scan[NW * 64];
};
using RowShared = RowSharedT<kRowWaves>;

__device__ __forceinline__ float wave_max(float v) {
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o), hi = __shfl_xor((uint32_t)(v >> 32), o);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// Reduce up to 4 floats at once: op 0 = max, 1 = sum (per value).
template <int NVAL, class SH>
__device__ __forceinline__ void block_reduce(float (&v)[NVAL], const int (&op)[NVAL], SH& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
_Pragma("clang loop unroll(full)")
  for (int i = 0; i < NVAL; ++i) v[i] = op[i] == 0 ? wave_max(v[i]) : wave_sum(v[i]);
  __syncthreads();
  if (lane == 0) {
_Pragma("clang loop unroll(full)")
    for (int i = 0; i < NVAL; ++i) sh.f[wave * 4 + i] = v[i];
  }
  __syncthreads();
_Pragma("clang loop unroll(full)")
  for (int i = 0; i < NVAL; ++i) {
    float a = op[i] == 0 ? kNegInf : 0.f;
    for (int w = 0; w < SH::kWaves; ++w) a = op[i] == 0 ? fmaxf(a, sh.f[w * 4 + i]) : a + sh.f[w * 4 + i];
    v[i] = a;
  }
}
template <class SH>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, SH& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane == 0) sh.u[wave] = v;
  __syncthreads();
  uint64_t a = 0;
  for (int w = 0; w < SH::kWaves; ++w) a += sh.u[w];
  return a;
}

// Exclusive prefix sum over the threads (thread order) and the total: a
// wave-level scan, the wave totals through LDS, two barriers.
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_up((uint32_t)v, o), hi = __shfl_up((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}
template <class SH>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t& total, SH& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t inc = v;
_Pragma("clang loop unroll(full)")
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t t = shfl_up_u64(inc, o);
    if (lane >= o) inc += t;
  }
  __syncthreads();
  if (lane == 63) sh.u[wave] = inc;
  __syncthreads();
  uint64_t base = 0, tot = 0;
  for (int w = 0; w < SH::kWaves; ++w) {
    const uint64_t t = sh.u[w];
    base += w < wave ? t : 0;
    tot += t;
  }
  total = tot;
  return base + inc - v;
}

// (key, idx) ordering for top-K: larger key first, then lower index.
__device__ __forceinline__ bool tk_better(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}
// Insert (key, idx) into a sorted top-8 list, dropping the worst; every index is
// static (the carried element is swapped down the list).
__device__ __forceinline__ void tk_insert(float (&k)[kMaxTopK], int (&ix)[kMaxTopK], float key, int idx) {
  if (!tk_better(key, idx, k[kMaxTopK - 1], ix[kMaxTopK - 1])) return;
_Pragma("clang loop unroll(full)")
  for (int j = 0; j < kMaxTopK; ++j) {
    if (tk_better(key, idx, k[j], ix[j])) {
      const float tkk = k[j];
      const int tii = ix[j];
      k[j] = key;
      ix[j] = idx;
      key = tkk;
      idx = tii;
    }
  }
}

// Unaligned rows: the 16-byte group of elements i0 .. i0+EPV-1 read element by
// element (zeros past the end), packed as the aligned load would return it.
template <typename T> struct GroupLoad;
template <> struct GroupLoad<F32> {
  __device__ static uint4 scalar(const char* rp, int i0, int V) {
    const uint32_t* s = (const uint32_t*)rp;
    uint32_t w[4];
_Pragma("clang loop unroll(full)")
    for (int k = 0; k < 4; ++k) w[k] = (i0 + k < V) ? s[i0 + k] : 0u;
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <typename T> struct GroupLoad16 {
  __device__ static uint4 scalar(const char* rp, int i0, int V) {
    const uint16_t* s = (const uint16_t*)rp;
    uint32_t w[4];
_Pragma("clang loop unroll(full)")
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = (i0 + 2 * k < V) ? s[i0 + 2 * k] : 0u;
      const uint32_t hi = (i0 + 2 * k + 1 < V) ? s[i0 + 2 * k + 1] : 0u;
      w[k] = lo | (hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct GroupLoad<BF16> : GroupLoad16<BF16> {};
template <> struct GroupLoad<F16> : GroupLoad16<F16> {};

// Stream the row in steps of kRowUnroll chunks: every thread first issues its
// kRowUnroll 16-byte loads (unconditionally; bytes past the row read as zero),
// then decodes them (elements past the row become -inf) and runs the body on
// `c` (chunk) and `x` (its EPV elements). Expanded in place so that the
// accumulators stay in registers.
constexpr int kRowUnroll = 8;
#define ROW_FOR_GROUPS(...)                                                         \
  for (int c0_ = 0; c0_ < nchunks; c0_ += kRowUnroll) {                            \
    uint4 wg_[kRowUnroll];                                                          \
    _Pragma("clang loop unroll(full)") for (int u_ = 0; u_ < kRowUnroll; ++u_)     \
      wg_[u_] = load_raw(c0_ + u_);                                                 \
    _Pragma("clang loop unroll(full)") for (int u_ = 0; u_ < kRowUnroll; ++u_) {   \
      if (c0_ + u_ < nchunks) {                                                     \
        const int c = c0_ + u_;                                                     \
        float x[EPV];                                                               \
        decode(wg_[u_], c, x);                                                      \
        __VA_ARGS__                                                                 \
      }                                                                             \
    }                                                                               \
  }

constexpr int kMaxChunks = 64;                              // chunks of 1024 x EPV elements
constexpr int kMaxPenWords = kMaxChunks * kRowThreads * 8 / 32;  // penalty bits (V <= 524288)

// The multi-pass row algorithm for any dtype, with NT threads per row: `sh` and `pbits`
// (penalty bits, (V + 31) / 32 words) are LDS of the calling kernel.
template <typename T, bool AL, int NT>
__device__ __forceinline__ void rows_generic(const RowParams& p, const int row, RowSharedT<NT / 64>& sh,
                                             uint32_t* pbits) {
  constexpr int kRowThreads = NT;
  constexpr int kRowWaves = NT / 64;
  using RE = RowElem<T>;
  using S = typename T::storage;
  constexpr int EPV = RE::EPV;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const char* rp = (const char*)p.logits + (long)row * p.row_stride * (long)sizeof(S);
  const int nchunks = (p.V + kRowThreads * EPV - 1) / (kRowThreads * EPV);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(rp), (short)0, p.V * (int)sizeof(S), 0x00020000);

  // The 16-byte group of chunk c of this thread (zeros past the row end).
  auto load_raw = [&](int c) __attribute__((always_inline)) -> uint4 {
    const int i0 = (c * kRowThreads + tid) * EPV;
    if constexpr (AL) {
      return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, i0 * (int)sizeof(S), 0, 0));
    } else {
      return GroupLoad<T>::scalar(rp, i0, p.V);
    }
  };
  auto decode = [&](const uint4& w, int c, float (&x)[EPV]) __attribute__((always_inline)) {
    const int i0 = (c * kRowThreads + tid) * EPV;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      x[e] = (i0 + e < p.V) ? RE::get(w, e) : kNegInf;
    });
  };

  // ---- repetition-penalty bitmask ----
  const int nwords = (p.V + 31) / 32;
  const bool use_pen = p.penalty != 1.0f && p.pen_offsets != nullptr;
  if (use_pen) {
    for (int w = tid; w < nwords; w += kRowThreads) pbits[w] = 0u;
    __syncthreads();
    const int b = p.pen_offsets[row], e = p.pen_offsets[row + 1];
    for (int j = b + tid; j < e; j += kRowThreads) {
      const int id = p.pen_ids[j];
      if (id >= 0 && id < p.V) atomicOr(&pbits[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
  }
  auto penal = [&](int i, float x) __attribute__((always_inline)) -> float {
    if (!use_pen || i >= p.V || !((pbits[i >> 5] >> (i & 31)) & 1u)) return x;
    return RE::round(x > 0.f ? __fdiv_rn(x, p.penalty) : x * p.penalty);
  };

  // ---- pass 1: maxima of x and xp ----
  float mx[2] = {kNegInf, kNegInf};
  ROW_FOR_GROUPS(
    const int i0 = (c * kRowThreads + tid) * EPV;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      mx[0] = fmaxf(mx[0], x[e]);
      mx[1] = fmaxf(mx[1], penal(i0 + e, x[e]));
        });
    )
  { const int op[2] = {0, 0}; block_reduce<2>(mx, op, sh); }
  const float m_raw = mx[0], m_pen = mx[1];

  // ---- pass 2: entropy sums (base 2); with sampling, the first radix level of
  // the fixed-point masses (a histogram by the top 12 key bits) ----
  // The T = 1 sums of xp feed the top-K keys, the log-sum-exp and H_pen only.
  const bool need_pen_sums = p.topk > 0 || p.out_entropy_pen != nullptr || p.out_lse != nullptr;
  constexpr int L0 = RE::level_bits[0];
  if (p.do_sample) {
    for (int t = tid; t < (1 << L0); t += kRowThreads) sh.hist0[t] = 0;
    __syncthreads();
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  ROW_FOR_GROUPS(
    const int i0 = (c * kRowThreads + tid) * EPV;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      if (i0 + e >= p.V) return;
      const float y = (x[e] - m_raw) * p.ent_c;
      const float ey = fast_exp2(y);
      acc[0] += ey;
      acc[1] += ey > 0.f ? ey * y : 0.f;
      const float xp = penal(i0 + e, x[e]);
      if (need_pen_sums) {
        const float y1 = (xp - m_pen) * kLog2e;
        const float e1 = fast_exp2(y1);
        acc[2] += e1;
        acc[3] += e1 > 0.f ? e1 * y1 : 0.f;
      }
      if (p.do_sample) {
        // q = floor(det_exp2(ys) * 2^40) is exactly 0 for ys < -41
        const float ys = (xp - m_pen) * p.samp_c;
        if (ys >= -41.0f) {
          const uint64_t q = det_q(ys);
          if (q) atomicAdd((unsigned long long*)&sh.hist0[RE::key(xp) >> (32 - L0)], (unsigned long long)q);
        }
      }
        });
    )
  { const int op[4] = {1, 1, 1, 1}; block_reduce<4>(acc, op, sh); }
  const float H_T = (log2f(acc[0]) - acc[1] / acc[0]) * kLn2;
  const float H_pen = (log2f(acc[2]) - acc[3] / acc[2]) * kLn2;
  const float logsum = logf(acc[2]);  // ln(sum exp(xp - max)), as log_softmax forms it
  if (tid == 0) {
    p.out_entropy[row] = H_T;
    if (p.out_entropy_pen) p.out_entropy_pen[row] = H_pen;  // NaN-free only when computed
    if (p.out_lse) p.out_lse[row] = m_pen + logsum;
    if (p.out_gate) p.out_gate[row] = H_T > p.gate_threshold ? 1 : 0;
  }

  // ---- pass 3: top-K of the log-softmax keys ----
  // K passes; pass j takes the best (key desc, index asc) element strictly after
  // the (j-1)-th pick, so every pass is a plain compare-and-select per element.
  if (p.topk > 0) {
    float prev_k = __builtin_huge_valf();
    int prev_i = -1;
    for (int j = 0; j < p.topk; ++j) {
      float bk = kNegInf;
      int bi = 0x7fffffff;
      ROW_FOR_GROUPS(
        const int i0 = (c * kRowThreads + tid) * EPV;
        static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
          constexpr int e = decltype(ec_)::value;
          const int i = i0 + e;
          if (i >= p.V) return;
          const float key = RE::round((penal(i, x[e]) - m_pen) - logsum);
          const bool after = key < prev_k || (key == prev_k && i > prev_i);
          if (after && tk_better(key, i, bk, bi)) { bk = key; bi = i; }
                });
      )
      for (int o = 32; o >= 1; o >>= 1) {
        const float ok = __shfl_xor(bk, o);
        const int oi = __shfl_xor(bi, o);
        if (tk_better(ok, oi, bk, bi)) { bk = ok; bi = oi; }
      }
      __syncthreads();
      if (lane == 0) { sh.bk[wave] = bk; sh.bi[wave] = bi; }
      __syncthreads();
      bk = sh.bk[0];
      bi = sh.bi[0];
      for (int w = 1; w < kRowWaves; ++w)
        if (tk_better(sh.bk[w], sh.bi[w], bk, bi)) { bk = sh.bk[w]; bi = sh.bi[w]; }
      if (tid == 0) {
        if (p.out_topk) p.out_topk[(long)row * p.topk + j] = bi;
        if (p.out_topk_lp) p.out_topk_lp[(long)row * p.topk + j] = bk;
      }
      prev_k = bk;
      prev_i = bi;
    }
  }

  // ---- pass 4: exact temperature + top-p draw ----
  if (!p.do_sample) return;
  constexpr int NLEV = RE::nlevels;
  constexpr int LAST_BITS = RE::level_bits[NLEV - 1];
  constexpr bool kChunkCounts = LAST_BITS <= 4;  // the final index search rides on the last level

  // Histogram of masses by the `bits` key bits below `done` already-fixed bits
  // equal to `prefix`, into h (bins = 1 << bits); with `counts`, also the
  // number of such elements per (chunk, bin) into sh.cc.
  auto histogram = [&](uint64_t* h, int done, uint32_t prefix, int bits, bool counts) __attribute__((always_inline)) {
    const int nb = 1 << bits;
    for (int t = tid; t < nb; t += kRowThreads) h[t] = 0;
    if (counts)
      for (int t = tid; t < kMaxChunks * 16; t += kRowThreads) sh.cc[t] = 0;
    __syncthreads();
    const int shift = 32 - done - bits;
    ROW_FOR_GROUPS(
      const int i0 = (c * kRowThreads + tid) * EPV;
      static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
        constexpr int e = decltype(ec_)::value;
        if (i0 + e >= p.V) return;
        const float xp = penal(i0 + e, x[e]);
        const uint32_t k = RE::key(xp);
        if ((k >> (32 - done)) != prefix) return;
        const uint32_t bin = (k >> shift) & (uint32_t)(nb - 1);
        const float ys = (xp - m_pen) * p.samp_c;
        const uint64_t q = ys >= -41.0f ? det_q(ys) : 0;
        if (q) atomicAdd((unsigned long long*)&h[bin], (unsigned long long)q);
        if (counts) atomicAdd(&sh.cc[c * 16 + bin], 1u);
            });
    )
    __syncthreads();
  };
  // Scan of a histogram, bins in descending order: thread t owns bins
  // nb-1-t*per .. nb-per-t*per; returns the mass above its bins, and the total.
  auto scan_bins = [&](const uint64_t* h, int bits, uint64_t& total) __attribute__((always_inline)) -> uint64_t {
    const int nb = 1 << bits;
    const int per = (nb + kRowThreads - 1) / kRowThreads;
    uint64_t mine = 0;
    for (int j = 0; j < per; ++j) {
      const int b = nb - 1 - (tid * per + j);
      if (b >= 0) mine += h[b];
    }
    return block_excl_scan_u64(mine, total, sh);
  };
  // The bin holding mass position pos, given each thread's `run` (mass above its
  // bins, plus `above`); adds the mass of the bins above it to `above`.
  auto pick_bin = [&](const uint64_t* h, int bits, uint64_t run, uint64_t pos, uint64_t& above) __attribute__((always_inline)) -> uint32_t {
    const int nb = 1 << bits;
    const int per = (nb + kRowThreads - 1) / kRowThreads;
    for (int j = 0; j < per; ++j) {
      const int b = nb - 1 - (tid * per + j);
      if (b < 0) break;
      if (h[b] != 0 && run <= pos && pos < run + h[b]) {
        sh.sel[0] = (uint32_t)b;
        sh.sel64[0] = run;
      }
      run += h[b];
    }
    __syncthreads();
    const uint32_t b = sh.sel[0];
    above = sh.sel64[0];
    __syncthreads();
    return b;
  };
  // Level 0 is scanned once for both selections.
  uint64_t Z;
  const uint64_t run0 = scan_bins(sh.hist0, L0, Z);
  uint64_t need = (uint64_t)(((unsigned __int128)Z * p.top_p_q32 + 0xffffffffull) >> 32);
  if (need < 1) need = 1;
  // Key holding mass position pos (order: xp desc, index asc) and the mass above it.
  auto select = [&](uint64_t pos, bool counts, uint32_t& key_out, uint64_t& above_out) __attribute__((always_inline)) {
    uint64_t above = 0;
    uint32_t prefix = pick_bin(sh.hist0, L0, run0, pos, above);
    int done = L0;
    _Pragma("clang loop unroll(full)")
    for (int lev = 1; lev < NLEV; ++lev) {
      const int bits = RE::level_bits[lev];
      histogram(sh.hist1, done, prefix, bits, counts && lev == NLEV - 1);
      uint64_t tot;
      const uint64_t run = scan_bins(sh.hist1, bits, tot) + above;
      prefix = (prefix << bits) | pick_bin(sh.hist1, bits, run, pos, above);
      done += bits;
    }
    key_out = prefix << (32 - done);  // the full 32-bit key (low bits zero for bf16)
    above_out = above;
  };
  constexpr int kKeyBitsUsed = RE::level_bits[0] + RE::level_bits[1] + RE::level_bits[2];
  auto match = [&](float xp, uint32_t kk) {
    return (RE::key(xp) >> (32 - kKeyBitsUsed)) == (kk >> (32 - kKeyBitsUsed));
  };
  // Mass of one token with key kk (every such token has the value key_to_float(kk)).
  auto key_mass = [&](uint32_t kk) -> uint64_t { return det_q((key_to_float(kk) - m_pen) * p.samp_c); };

  uint32_t c4[4] = {(uint32_t)row, (uint32_t)p.step, (uint32_t)(p.step >> 32), 0u};
  philox4x32_10(c4, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
  const uint64_t U = ((uint64_t)c4[0] << 32) | c4[1];
  auto mulhi = [](uint64_t a, uint64_t b) -> uint64_t { return (uint64_t)(((unsigned __int128)a * b) >> 64); };

  uint32_t key_r = 0;
  uint64_t above_r = 0, r = 0;
  bool fast = false, have_cc = false;
  if constexpr (NLEV == 2 && kChunkCounts) {
    // Both selections in one data pass. The nucleus boundary lies in level-0 bin
    // bn, so the kept mass is in (above_bn, above_bn + mass(bn)] and the draw
    // position r = U*kept/2^64 in [U*above_bn, U*(above_bn + mass(bn))] / 2^64:
    // only the level-0 bins blo..bhi meeting that interval (a contiguous range of
    // bins, keys descending) can hold the draw. One pass builds the level-1
    // histogram of bn and of every bin of the range (per-chunk counts too when
    // the range has at most two bins); a range wider than kRange bins takes the
    // two-pass path below.
    constexpr int kRange = (int)(sizeof(sh.hist1) / (16 * sizeof(uint64_t)));  // 256 bins
    uint64_t* ch = sh.hist1;  // [kRange][16] level 1 of the range's bins, index bhi - b
    uint64_t above_bn;
    const uint32_t bn = pick_bin(sh.hist0, L0, run0, need - 1, above_bn);
    const uint64_t mass_bn = sh.hist0[bn];
    const uint64_t r_lo = mulhi(U, above_bn), r_hi = mulhi(U, above_bn + mass_bn);
    uint64_t a_hi, a_lo;
    const int bhi = (int)pick_bin(sh.hist0, L0, run0, r_lo, a_hi);  // the range's first bin (largest keys)
    const int blo = (int)pick_bin(sh.hist0, L0, run0, r_hi, a_lo);
    const int len = bhi - blo + 1;
    if (len <= kRange) {
      have_cc = len <= 2;
      for (int t = tid; t < len * 16; t += kRowThreads) ch[t] = 0;
      if (tid < 16) sh.hn[tid] = 0;
      if (have_cc)
        for (int t = tid; t < kMaxChunks * 16; t += kRowThreads) { sh.cc[t] = 0; sh.cc2[t] = 0; }
      __syncthreads();
      constexpr int shift1 = 32 - L0 - 4;
      ROW_FOR_GROUPS(
        const int i0 = (c * kRowThreads + tid) * EPV;
        static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
          constexpr int e = decltype(ec_)::value;
          if (i0 + e >= p.V) return;
          const float xp = penal(i0 + e, x[e]);
          const uint32_t k = RE::key(xp);
          const int b0 = (int)(k >> (32 - L0));
          const bool in_n = b0 == (int)bn, in_r = b0 >= blo && b0 <= bhi;
          if (!in_n && !in_r) return;
          const uint32_t sub = (k >> shift1) & 15u;
          const float ys = (xp - m_pen) * p.samp_c;
          const uint64_t q = ys >= -41.0f ? det_q(ys) : 0;
          if (in_n && q) atomicAdd((unsigned long long*)&sh.hn[sub], (unsigned long long)q);
          if (in_r) {
            const int ri = bhi - b0;
            if (q) atomicAdd((unsigned long long*)&ch[ri * 16 + sub], (unsigned long long)q);
            if (have_cc) atomicAdd(ri == 0 ? &sh.cc[c * 16 + sub] : &sh.cc2[c * 16 + sub], 1u);
          }
            });
      )
      __syncthreads();
      // The boundary key (level 1 of bn, keys descending), its tie index, the kept mass, r.
      uint64_t run = above_bn, above_n = above_bn;
      uint32_t sub_n = 0;
      for (int sb = 15; sb >= 0; --sb) {
        const uint64_t h = sh.hn[sb];
        if (h != 0 && run <= need - 1 && need - 1 < run + h) { sub_n = (uint32_t)sb; above_n = run; break; }
        run += h;
      }
      const uint32_t key_n = ((bn << 4) | sub_n) << shift1;
      const uint64_t qn = key_mass(key_n);
      const uint64_t jn = (need - 1 - above_n) / qn;
      r = mulhi(U, above_n + (jn + 1) * qn);
      // The range bin holding r: thread t takes bin bhi - t, the masses above by a scan.
      const uint64_t hb = tid < len ? sh.hist0[bhi - tid] : 0;
      uint64_t tot_unused;
      const uint64_t ab = a_hi + block_excl_scan_u64(hb, tot_unused, sh);
      if (tid == 0) sh.sel[2] = 0xffffffffu;
      __syncthreads();
      if (tid < len && hb != 0 && ab <= r && r < ab + hb) { sh.sel[2] = (uint32_t)tid; sh.sel64[2] = ab; }
      __syncthreads();
      const uint32_t ri = sh.sel[2];
      if (ri != 0xffffffffu) {
        run = sh.sel64[2];
        uint32_t sub_r = 0;
        above_r = run;
        for (int sb = 15; sb >= 0; --sb) {
          const uint64_t h = ch[ri * 16 + sb];
          if (h != 0 && run <= r && r < run + h) { sub_r = (uint32_t)sb; above_r = run; break; }
          run += h;
        }
        key_r = (((uint32_t)(bhi - (int)ri) << 4) | sub_r) << shift1;
        if (have_cc && ri == 1)
          for (int t = tid; t < kMaxChunks * 16; t += kRowThreads) sh.cc[t] = sh.cc2[t];
        fast = true;
      }
      __syncthreads();
    }
  }
  if (!fast) {
    uint32_t key_n;
    uint64_t above_n;
    select(need - 1, false, key_n, above_n);
    const uint64_t qn = key_mass(key_n);
    const uint64_t jn = (need - 1 - above_n) / qn;  // 0-based index of the last kept tie
    const uint64_t kept_mass = above_n + (jn + 1) * qn;
    r = mulhi(U, kept_mass);
    select(r, kChunkCounts, key_r, above_r);
  }
  const uint64_t qr = key_mass(key_r);
  const uint32_t j = (uint32_t)((r - above_r) / qr);  // the j-th (0-based) token of key_r by index

  // The j-th token with key_r in index order: per-chunk totals, then a thread scan
  // over the chunk that holds it.
  // (The single-pass sampler counted per chunk only for ranges of at most two bins.)
  if (kChunkCounts && (!fast || have_cc)) {
    const uint32_t lastv = (key_r >> (32 - kKeyBitsUsed)) & ((1u << LAST_BITS) - 1);
    if (tid < kMaxChunks) sh.chunk_tot[tid] = tid < nchunks ? sh.cc[tid * 16 + lastv] : 0u;
  } else {
    if (tid < kMaxChunks) sh.chunk_tot[tid] = 0;
    __syncthreads();
    ROW_FOR_GROUPS(
      const int i0 = (c * kRowThreads + tid) * EPV;
      uint32_t n = 0;
_Pragma("clang loop unroll(full)")
      for (int e = 0; e < EPV; ++e)
        if (i0 + e < p.V && match(penal(i0 + e, x[e]), key_r)) ++n;
      for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o);
      if (lane == 0 && n) atomicAdd(&sh.chunk_tot[c], n);
      )
  }
  __syncthreads();
  int cstar = 0;
  uint32_t before = 0;
  for (int c = 0; c < nchunks; ++c) {
    if (before + sh.chunk_tot[c] > j) { cstar = c; break; }
    before += sh.chunk_tot[c];
  }
  float xs[EPV];
  decode(load_raw(cstar), cstar, xs);
  const int is0 = (cstar * kRowThreads + tid) * EPV;
  uint32_t mine = 0;
_Pragma("clang loop unroll(full)")
  for (int e = 0; e < EPV; ++e)
    if (is0 + e < p.V && match(penal(is0 + e, xs[e]), key_r)) ++mine;
  uint64_t tot_unused;
  const uint32_t excl = before + (uint32_t)block_excl_scan_u64(mine, tot_unused, sh);
  if (mine && excl <= j && j < excl + mine) {
    uint32_t seen = excl;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      if (is0 + e < p.V && match(penal(is0 + e, xs[e]), key_r)) {
        if (seen == j && p.out_sample) p.out_sample[row] = is0 + e;
        ++seen;
      }
        });
  }
}

// ---- 16-bit logits: histogram of every value ------------------------------------------------
// Every token's 16-bit value is counted into a histogram of all 65,536 values (two 16-bit counts
// per LDS word) in one read of the row. A token's sampler mass, entropy terms and log-prob depend
// on its value alone, so the row max (largest value present), both entropies, the log-sum-exp,
// the nucleus and the draw's value and tie index are all resolved from the counts; a second read
// (mostly from the last-level cache) then finds the drawn token's index and the top-K.
// Rows with a count past 65,535 (one value repeated that often) or a non-finite value take the
// multi-pass path. Key order: sign-magnitude bits mapped to unsigned order; -0 is counted as +0,
// which compares equal to it.
template <typename T> struct Bits16;
template <> struct Bits16<BF16> {
  __device__ __forceinline__ static float val(uint32_t raw) { return __uint_as_float(raw << 16); }
  __device__ __forceinline__ static uint32_t raw(float v) { return __float_as_uint(v) >> 16; }  // v a bf16 value
  static constexpr uint32_t kPosInfRaw = 0x7f80u, kNegInfRaw = 0xff80u;
};
template <> struct Bits16<F16> {
  __device__ __forceinline__ static float val(uint32_t raw) { return f16_bits_to_f32((uint16_t)raw); }
  __device__ __forceinline__ static uint32_t raw(float v) { return f32_to_f16_bits(v); }  // v an f16 value
  static constexpr uint32_t kPosInfRaw = 0x7c00u, kNegInfRaw = 0xfc00u;
};
__host__ __device__ constexpr uint32_t key16(uint32_t raw) { return raw ^ ((raw & 0x8000u) ? 0xffffu : 0x8000u); }
__device__ __forceinline__ uint32_t raw16_of_key(uint32_t k) { return k ^ ((k & 0x8000u) ? 0x8000u : 0xffffu); }

constexpr int kFT = 1024;                                      // threads per row
constexpr int kFW = kFT / 64;
constexpr int kFastChunks = 20;                                // chunks of kFT 16-byte groups
constexpr int kFastMaxV = kFastChunks * kFT * 8;               // 163,840 (the penalty bits' LDS)
constexpr int kFastPenWords = kFastMaxV / 32;
constexpr int kHistWords = 32768;                              // 65,536 16-bit counts
constexpr int kSlabBins = 256;                                 // four bins (two words) per lane
constexpr int kSlabs = 65536 / kSlabBins;
constexpr int kCandCap = kFT;                                  // top-K candidates kept in LDS

struct FastShared {
  static constexpr int kWaves = kFW;
  uint64_t slab_mass[kSlabs];  // sampler mass per slab of 256 values
  uint32_t slab_cnt[kSlabs];   // tokens per slab
  float f[kFW * 4];
  uint64_t u[kFW];
  uint32_t g[kFW * 4];
  uint32_t sel[8];     // one slot per resolution step
  uint64_t sel64[8];
  float bk[kFW];
  int32_t bi[kFW];
  uint32_t ncand;
  uint32_t total;      // tokens counted by the sweep
  uint32_t top_pen;    // largest key a penalised token moved to
  uint32_t bad;        // a penalised value is not finite
};

__device__ __forceinline__ uint64_t shfl_down_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_down((uint32_t)v, o), hi = __shfl_down((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o));
  return v;
}

// Rows must start on 16-byte boundaries (16-byte buffer loads).
template <typename T>
__global__ __launch_bounds__(kFT) void row_stats_fast_kernel(RowParams p) {
  constexpr bool AL = true;
  using RE = RowElem<T>;
  using B16 = Bits16<T>;
  using S = typename T::storage;
  constexpr int EPV = 8;
  constexpr uint32_t kInfKey = key16(B16::kPosInfRaw), kNegInfKey = key16(B16::kNegInfRaw);
  const int row = blockIdx.x;
  if (row >= p.R) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  __shared__ __align__(16) uint32_t hist[kHistWords];
  __shared__ uint32_t pbits[kFastPenWords];
  __shared__ FastShared fs;
  static_assert(sizeof(RowSharedT<kFW>) <= sizeof(hist), "the multi-pass path reuses the histogram's LDS");
  const int V = p.V;
  const char* rp = (const char*)p.logits + (long)row * p.row_stride * (long)sizeof(S);
  const int nchunks = (V + kFT * EPV - 1) / (kFT * EPV);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(rp), (short)0, V * (int)sizeof(S), 0x00020000);
  // chunk c's group of this thread: the chunk offset rides in the scalar offset operand
  auto load_raw = [&](int c) __attribute__((always_inline)) -> uint4 {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
        rs, tid * EPV * (int)sizeof(S), c * kFT * EPV * (int)sizeof(S), 0));
  };
  auto pen_value = [&](float x) __attribute__((always_inline)) -> float {
    return RE::round(x > 0.f ? __fdiv_rn(x, p.penalty) : x * p.penalty);
  };
  auto nkey = [](float v) __attribute__((always_inline)) -> uint32_t { return key16(B16::raw(v == 0.f ? 0.f : v)); };
  auto kval = [](uint32_t k) __attribute__((always_inline)) -> float { return B16::val(raw16_of_key(k)); };

  const bool use_pen = p.penalty != 1.0f && p.pen_offsets != nullptr;
  const int nwords = (V + 31) / 32;
  {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
    for (int t = tid; t < kHistWords / 4; t += kFT) h4[t] = make_uint4(0u, 0u, 0u, 0u);
  }
  if (tid == 0) {
    fs.total = 0;
    fs.top_pen = 0;
    fs.bad = 0;
  }
  __syncthreads();
  // The draw's uniform depends only on (seed, row, step).
  uint64_t U = 0;
  if (p.do_sample) {
    uint32_t c4[4] = {(uint32_t)row, (uint32_t)p.step, (uint32_t)(p.step >> 32), 0u};
    philox4x32_10(c4, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
    U = ((uint64_t)c4[0] << 32) | c4[1];
  }

  // ---- pass A: count the raw values (kRowUnroll 16-byte loads in flight per thread); the
  // largest and smallest keys on the way ----
  auto count1 = [&](uint32_t k) __attribute__((always_inline)) { atomicAdd(&hist[k >> 1], 1u << ((k & 1u) << 4)); };
  uint32_t kmx = 0, kmn = 0xffffffffu;
  for (int c0 = 0; c0 < nchunks; c0 += kRowUnroll) {
    uint4 w[kRowUnroll];
_Pragma("clang loop unroll(full)")
    for (int u = 0; u < kRowUnroll; ++u) w[u] = load_raw(c0 + u);  // zeros past the row
_Pragma("clang loop unroll(full)")
    for (int u = 0; u < kRowUnroll; ++u) {
      const int c = c0 + u;
      const int i0 = (c * kFT + tid) * EPV;
      const uint32_t dw[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
      if (c >= nchunks) {
      } else if (i0 + EPV <= V) {
_Pragma("clang loop unroll(full)")
        for (int k = 0; k < 4; ++k) {
          // both halves' keys at once: xor 0xffff into a negative half, 0x8000 into a positive one
          const uint32_t k2 = dw[k] ^ ((((dw[k] >> 15) & 0x10001u) * 0x7fffu) | 0x80008000u);
          const uint32_t lo = k2 & 0xffffu, hi = k2 >> 16;
          count1(lo);
          count1(hi);
          kmx = max(kmx, max(lo, hi));
          kmn = min(kmn, min(lo, hi));
        }
      } else {
_Pragma("clang loop unroll(full)")
        for (int e = 0; e < EPV; ++e) {
          if (i0 + e < V) {
            const uint32_t k = key16((dw[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
            count1(k);
            kmx = max(kmx, k);
            kmn = min(kmn, k);
          }
        }
      }
    }
  }
_Pragma("clang loop unroll(full)")
  for (int o = 32; o >= 1; o >>= 1) {
    kmx = max(kmx, (uint32_t)__shfl_xor(kmx, o));
    kmn = min(kmn, (uint32_t)__shfl_xor(kmn, o));
  }
  if (lane == 0) {
    fs.g[wave * 2] = kmx;
    fs.g[wave * 2 + 1] = kmn;
  }
  __syncthreads();
  // -0 (key 0x7fff, high half of word 0x3fff) joins +0 (key 0x8000, low half of word 0x4000).
  if (tid == 0) {
    const uint32_t n = hist[0x3fff] >> 16;
    if (n) {
      hist[0x3fff] -= n << 16;
      hist[0x4000] += n;
    }
  }
  kmx = 0;
  kmn = 0xffffffffu;
  for (int w = 0; w < kFW; ++w) {
    kmx = max(kmx, fs.g[w * 2]);
    kmn = min(kmn, fs.g[w * 2 + 1]);
  }
  __syncthreads();
  const uint32_t top_raw = kmx == 0x7fffu ? 0x8000u : kmx;  // -0 counts as +0
  uint32_t top = top_raw;
  bool ok = top_raw < kInfKey && kmn > kNegInfKey;  // non-finite rows take the multi-pass path
  const float m_raw = kval(top_raw);
  float H_T = 0.f;
  if (ok && use_pen) {
    // Entropy of the raw values, then every penalised token (each distinct id once: the one
    // that clears its bit) moves to its penalised value; the bits are set again for pass B.
    float a2[2] = {0.f, 0.f};
    for (int i = 0; i < kHistWords / kFT; ++i) {
      const int w = tid + i * kFT;
      const uint32_t wd = hist[w];
      if (!wd) continue;
_Pragma("clang loop unroll(full)")
      for (int h = 0; h < 2; ++h) {
        const uint32_t n = (wd >> (16 * h)) & 0xffffu;
        if (!n) continue;
        const float y = (kval((uint32_t)(2 * w + h)) - m_raw) * p.ent_c;
        const float e = fast_exp2(y);
        a2[0] += (float)n * e;
        a2[1] += e > 0.f ? (float)n * (e * y) : 0.f;
      }
    }
    { const int op[2] = {1, 1}; block_reduce<2>(a2, op, fs); }
    H_T = (log2f(a2[0]) - a2[1] / a2[0]) * kLn2;
    // (the id list is read only now: its loads would otherwise wait for the row's)
    for (int w = tid; w < nwords; w += kFT) pbits[w] = 0u;
    __syncthreads();
    const int b = p.pen_offsets[row], e = p.pen_offsets[row + 1];
    for (int j = b + tid; j < e; j += kFT) {
      const int id = p.pen_ids[j];
      if (id >= 0 && id < V) atomicOr(&pbits[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    for (int j = b + tid; j < e; j += kFT) {
      const int id = p.pen_ids[j];
      if (id < 0 || id >= V) continue;
      const uint32_t bit = 1u << (id & 31);
      if (atomicAnd(&pbits[id >> 5], ~bit) & bit) {
        const float x = RE::scalar(rp, id);
        const uint32_t kx = nkey(x), kp = nkey(pen_value(x));
        if (kp >= kInfKey || kp <= kNegInfKey) atomicOr(&fs.bad, 1u);
        atomicMax(&fs.top_pen, kp);
        if (kx != kp) {
          atomicSub(&hist[kx >> 1], 1u << ((kx & 1u) << 4));
          atomicAdd(&hist[kp >> 1], 1u << ((kp & 1u) << 4));
        }
      }
    }
    __syncthreads();
    for (int j = b + tid; j < e; j += kFT) {
      const int id = p.pen_ids[j];
      if (id >= 0 && id < V) atomicOr(&pbits[id >> 5], 1u << (id & 31));
    }
    // The largest value now: the raw one unless all its tokens moved (then the next value
    // below it), or a moved token's.
    const bool top_left = ((hist[top_raw >> 1] >> ((top_raw & 1u) * 16)) & 0xffffu) != 0;
    if (!top_left && wave == 0) {
      uint32_t best = 0;  // key + 1 of the largest value below top_raw; 0: none
      for (int s2 = (int)(top_raw / kSlabBins); s2 >= 0; --s2) {
        const uint2 wd = reinterpret_cast<const uint2*>(hist)[s2 * (kSlabBins / 4) + lane];
_Pragma("clang loop unroll(full)")
        for (int q = 0; q < 4; ++q) {
          const uint32_t n = ((q < 2 ? wd.x : wd.y) >> ((q & 1) * 16)) & 0xffffu;
          const uint32_t k = (uint32_t)(s2 * kSlabBins + lane * 4 + q);
          if (n && k < top_raw) best = max(best, k + 1u);
        }
_Pragma("clang loop unroll(full)")
        for (int o = 32; o >= 1; o >>= 1) best = max(best, (uint32_t)__shfl_xor(best, o));
        if (best) break;
      }
      if (lane == 0) fs.sel[6] = best;
    }
    __syncthreads();
    top = max(top_left ? top_raw : (fs.sel[6] ? fs.sel[6] - 1u : 0u), fs.top_pen);
    ok = fs.bad == 0;
  }
  const float m_pen = kval(top);

  // ---- resolution: one sweep over the slabs (wave w takes slabs w, w + 16, ...; lane l the
  // four values 4l .. 4l + 3 of the slab) for the entropy sums, each slab's mass and count, and
  // the token total (a 16-bit count that overflowed leaves it short of V) ----
  const bool need_pen_sums = p.topk > 0 || p.out_entropy_pen != nullptr || p.out_lse != nullptr;
  const bool want_mass = p.do_sample != 0, want_cnt = p.topk > 0;
  auto unit_mass = [&](uint32_t k) __attribute__((always_inline)) -> uint64_t {
    const float ys = (kval(k) - m_pen) * p.samp_c;
    return ys >= -41.0f ? det_q(ys) : 0;
  };
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (ok) {
    const uint2* h2 = reinterpret_cast<const uint2*>(hist);
    uint32_t total = 0;
    uint2 nxt = h2[wave * (kSlabBins / 4) + lane];
    for (int i = 0; i < kSlabs / kFW; ++i) {
      const int s = wave + i * kFW;
      const uint2 wd = nxt;
      if (i + 1 < kSlabs / kFW) nxt = h2[(s + kFW) * (kSlabBins / 4) + lane];  // next slab's read in flight
      uint64_t mass = 0;
      uint32_t cnt = 0;
      if (__any((wd.x | wd.y) != 0u)) {
        if ((wd.x | wd.y) != 0u) {
_Pragma("clang loop unroll(full)")
          for (int b = 0; b < 4; ++b) {
            const uint32_t n = ((b < 2 ? wd.x : wd.y) >> ((b & 1) * 16)) & 0xffffu;
            if (!n) continue;
            const uint32_t k = (uint32_t)(s * kSlabBins + lane * 4 + b);
            const float v = kval(k), fn = (float)n;
            if (!use_pen) {
              const float y = (v - m_raw) * p.ent_c;
              const float e = fast_exp2(y);
              acc[0] += fn * e;
              acc[1] += e > 0.f ? fn * (e * y) : 0.f;
            }
            if (need_pen_sums) {
              const float y1 = (v - m_pen) * kLog2e;
              const float e1 = fast_exp2(y1);
              acc[2] += fn * e1;
              acc[3] += e1 > 0.f ? fn * (e1 * y1) : 0.f;
            }
            if (want_mass) {
              const float ys = (v - m_pen) * p.samp_c;
              if (ys >= -41.0f) mass += (uint64_t)n * det_q(ys);
            }
            cnt += n;
          }
        }
        total += cnt;
        if (want_mass) mass = wave_sum_u64(mass);
        if (want_cnt) cnt = wave_sum_u32(cnt);
      }
      if (lane == 0) {
        fs.slab_mass[s] = mass;
        fs.slab_cnt[s] = cnt;
      }
    }
    total = wave_sum_u32(total);
    if (lane == 0) atomicAdd(&fs.total, total);
    { const int op[4] = {1, 1, 1, 1}; block_reduce<4>(acc, op, fs); }
    ok = fs.total == (uint32_t)V;
  }
  if (!ok) {
    __syncthreads();
    rows_generic<T, AL, kFT>(p, row, *reinterpret_cast<RowSharedT<kFW>*>(hist), pbits);
    return;
  }
  if (!use_pen) H_T = (log2f(acc[0]) - acc[1] / acc[0]) * kLn2;
  const float H_pen = (log2f(acc[2]) - acc[3] / acc[2]) * kLn2;
  const float logsum = logf(acc[2]);
  if (tid == 0) {
    p.out_entropy[row] = H_T;
    if (p.out_entropy_pen) p.out_entropy_pen[row] = H_pen;
    if (p.out_lse) p.out_lse[row] = m_pen + logsum;
    if (p.out_gate) p.out_gate[row] = H_T > p.gate_threshold ? 1 : 0;
  }
  if (!p.do_sample && p.topk == 0) return;

  // Wave-level resolution (no barriers): the slab, then the value, holding position pos, keys
  // descending. Lane l holds slabs kSlabs-1-4l .. kSlabs-4-4l (largest keys in lane 0).
  auto rd64 = [](uint64_t v, int l) __attribute__((always_inline)) -> uint64_t {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  };
  auto wave_locate = [&](const uint64_t (&sm)[4], uint64_t ex, uint64_t lt, uint64_t pos, uint64_t& above) __attribute__((always_inline)) -> int {
    const int L = __ffsll((unsigned long long)__ballot(lt != 0 && ex <= pos && pos < ex + lt)) - 1;
    int slab = 0;
    uint64_t run = ex, a = 0;
_Pragma("clang loop unroll(full)")
    for (int q = 0; q < 4; ++q) {
      if (sm[q] != 0 && run <= pos && pos < run + sm[q]) { slab = kSlabs - 1 - (4 * lane + q); a = run; }
      run += sm[q];
    }
    const int l = max(L, 0);  // pos is always inside the total
    above = rd64(a, l);
    return __builtin_amdgcn_readlane(slab, l);
  };
  auto wave_pick = [&](int s, uint64_t above, uint64_t pos, bool by_mass, uint64_t& above_k) __attribute__((always_inline)) -> uint32_t {
    const uint2 wd = reinterpret_cast<const uint2*>(hist)[s * (kSlabBins / 4) + lane];
    uint64_t m[4], tot = 0;
_Pragma("clang loop unroll(full)")
    for (int b = 0; b < 4; ++b) {
      const uint32_t n = ((b < 2 ? wd.x : wd.y) >> ((b & 1) * 16)) & 0xffffu;
      const uint32_t k = (uint32_t)(s * kSlabBins + lane * 4 + b);
      m[b] = n == 0 ? 0 : by_mass ? (uint64_t)n * unit_mass(k) : (uint64_t)n;
      tot += m[b];
    }
    uint64_t inc = tot;  // suffix sum: lanes above hold larger keys
_Pragma("clang loop unroll(full)")
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t t = shfl_down_u64(inc, o);
      if (lane + o < 64) inc += t;
    }
    uint64_t run = above + (inc - tot), a = 0;
    uint32_t key = 0;
    bool hit = false;
_Pragma("clang loop unroll(full)")
    for (int b = 3; b >= 0; --b) {
      if (m[b] && run <= pos && pos < run + m[b]) {
        key = (uint32_t)(s * kSlabBins + lane * 4 + b);
        a = run;
        hit = true;
      }
      run += m[b];
    }
    const int l = max(__ffsll((unsigned long long)__ballot(hit)) - 1, 0);
    above_k = rd64(a, l);
    return (uint32_t)__builtin_amdgcn_readlane((int)key, l);
  };
  // Per-lane slab values (4 slabs, largest keys first) and their exclusive prefix over lanes.
  auto wave_slabs = [&](const uint64_t* src64, const uint32_t* src32, uint64_t (&sm)[4], uint64_t& lt) __attribute__((always_inline)) -> uint64_t {
    lt = 0;
_Pragma("clang loop unroll(full)")
    for (int q = 0; q < 4; ++q) {
      const int s = kSlabs - 1 - (4 * lane + q);
      sm[q] = src64 ? src64[s] : (uint64_t)src32[s];
      lt += sm[q];
    }
    uint64_t inc = lt;
_Pragma("clang loop unroll(full)")
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t t = shfl_up_u64(inc, o);
      if (lane >= o) inc += t;
    }
    return inc - lt;
  };

  // ---- the draw (wave 0): nucleus boundary, kept mass, r, the drawn value and its tie index ----
  if (p.do_sample && wave == 0) {
    uint64_t sm[4], lt;
    const uint64_t ex = wave_slabs(fs.slab_mass, nullptr, sm, lt);
    const uint64_t Z = rd64(ex + lt, 63);
    uint64_t need = (uint64_t)(((unsigned __int128)Z * p.top_p_q32 + 0xffffffffull) >> 32);
    if (need < 1) need = 1;
    uint64_t a_s, above_n, above_r;
    int s = wave_locate(sm, ex, lt, need - 1, a_s);
    const uint32_t key_n = wave_pick(s, a_s, need - 1, true, above_n);
    const uint64_t qn = unit_mass(key_n);
    const uint64_t jn = (need - 1 - above_n) / qn;  // 0-based index of the last kept tie
    const uint64_t kept = above_n + (jn + 1) * qn;
    const uint64_t r = (uint64_t)(((unsigned __int128)U * kept) >> 64);
    s = wave_locate(sm, ex, lt, r, a_s);
    const uint32_t key_r = wave_pick(s, a_s, r, true, above_r);
    if (lane == 0) {
      fs.sel[0] = key_r;
      fs.sel[1] = (uint32_t)((r - above_r) / unit_mass(key_r));
    }
  }
  // ---- top-K (wave 1): candidates are the values whose log-prob is at least the K-th token's ----
  if (p.topk > 0 && wave == 1) {
    uint64_t sm[4], lt, a_s, a_k;
    const uint64_t ex = wave_slabs(nullptr, fs.slab_cnt, sm, lt);
    const int s = wave_locate(sm, ex, lt, (uint64_t)(p.topk - 1), a_s);
    const uint32_t kb = wave_pick(s, a_s, (uint64_t)(p.topk - 1), false, a_k);
    const float lpK = RE::round((kval(kb) - m_pen) - logsum);
    // log-probs fall with the value: walk down from kb while they still equal lpK
    uint32_t lowest = kb;
    for (int s2 = (int)(kb / kSlabBins); s2 >= 0; --s2) {
      const uint2 wd = reinterpret_cast<const uint2*>(hist)[s2 * (kSlabBins / 4) + lane];
      bool stop = false;
_Pragma("clang loop unroll(full)")
      for (int b = 0; b < 4; ++b) {
        const uint32_t n = ((b < 2 ? wd.x : wd.y) >> ((b & 1) * 16)) & 0xffffu;
        const uint32_t k = (uint32_t)(s2 * kSlabBins + lane * 4 + b);
        if (n && k < kb) {
          if (RE::round((kval(k) - m_pen) - logsum) == lpK) lowest = min(lowest, k);
          else stop = true;
        }
      }
      lowest = wave_min_u32(lowest);
      if (__any(stop)) break;
    }
    if (lane == 0) fs.sel[2] = lowest;
  }
  __syncthreads();
  const float v_r = p.do_sample ? kval(fs.sel[0] & 0xffffu) : 0.f;
  const uint32_t j_r = p.do_sample ? fs.sel[1] : 0u;
  const float v_thr = p.topk > 0 ? kval(fs.sel[2] & 0xffffu) : __builtin_huge_valf();

  // ---- pass B (the row again): each lane's 8-bit mask of tokens equal to the drawn value per
  // chunk, and the top-K candidates ----
  uint8_t* masks = reinterpret_cast<uint8_t*>(hist);         // [kFastChunks][kFW][64 lanes]
  uint2* cand = reinterpret_cast<uint2*>(hist + 8192);       // [kCandCap] (log-prob bits, index)
  const float v_match = p.do_sample ? v_r : __builtin_nanf("");  // NaN matches nothing
  __syncthreads();
  if (tid == 0) fs.ncand = 0;
  __syncthreads();
  for (int c0 = 0; c0 < nchunks; c0 += kRowUnroll) {
    uint4 w[kRowUnroll];
_Pragma("clang loop unroll(full)")
    for (int u = 0; u < kRowUnroll; ++u) w[u] = load_raw(c0 + u);
_Pragma("clang loop unroll(full)")
    for (int u = 0; u < kRowUnroll; ++u) {
      const int c = c0 + u;
      if (c >= nchunks) continue;
      const int i0 = (c * kFT + tid) * EPV;
      const uint4 d = w[u];
      const uint32_t vm = i0 + EPV <= V ? 0xffu : i0 >= V ? 0u : (1u << (V - i0)) - 1u;  // valid elements
      const uint32_t pb = (use_pen && i0 < V) ? (pbits[i0 >> 5] >> (i0 & 31)) & vm & 0xffu : 0u;
      const uint32_t plain = vm & ~pb;
      uint32_t mt = 0, cm = 0;
_Pragma("clang loop unroll(full)")
      for (int e = 0; e < EPV; ++e) {
        const float xv = RE::get(d, e);
        const bool pl = ((plain >> e) & 1u) != 0;
        mt |= (pl && xv == v_match) ? 1u << e : 0u;
        cm |= (pl && xv >= v_thr) ? 1u << e : 0u;
      }
      // penalised elements and top-K candidates (both rare), one at a time
      for (uint32_t bits = pb | cm; bits != 0u; bits &= bits - 1u) {
        const int e = __builtin_ctz(bits);
        float xv = RE::get(d, e);
        if ((pb >> e) & 1u) {
          xv = pen_value(xv);
          if (xv == v_match) mt |= 1u << e;
          if (!(xv >= v_thr)) continue;
        }
        if (p.topk > 0) {
          const uint32_t pos = atomicAdd(&fs.ncand, 1u);
          if (pos < kCandCap)
            cand[pos] = make_uint2(__float_as_uint(RE::round((xv - m_pen) - logsum)), (uint32_t)(i0 + e));
        }
      }
      if (p.do_sample) masks[(c * kFW + wave) * 64 + lane] = (uint8_t)mt;
    }
  }
  __syncthreads();

  if (p.topk > 0) {
    auto block_best = [&](float& bk, int& bi) __attribute__((always_inline)) {
      for (int o = 32; o >= 1; o >>= 1) {
        const float ok = __shfl_xor(bk, o);
        const int oi = __shfl_xor(bi, o);
        if (tk_better(ok, oi, bk, bi)) { bk = ok; bi = oi; }
      }
      __syncthreads();
      if (lane == 0) { fs.bk[wave] = bk; fs.bi[wave] = bi; }
      __syncthreads();
      bk = fs.bk[0];
      bi = fs.bi[0];
      for (int w = 1; w < kFW; ++w)
        if (tk_better(fs.bk[w], fs.bi[w], bk, bi)) { bk = fs.bk[w]; bi = fs.bi[w]; }
    };
    const uint32_t nc = fs.ncand;
    if (nc <= (uint32_t)kCandCap) {
      float ck = kNegInf;
      int ci = 0x7fffffff;
      if ((uint32_t)tid < nc) {
        const uint2 e = cand[tid];
        ck = __uint_as_float(e.x);
        ci = (int)e.y;
      }
      for (int j = 0; j < p.topk; ++j) {
        float bk = ck;
        int bi = ci;
        block_best(bk, bi);
        if (tid == 0) {
          if (p.out_topk) p.out_topk[(long)row * p.topk + j] = bi;
          if (p.out_topk_lp) p.out_topk_lp[(long)row * p.topk + j] = bk;
        }
        if (ci == bi) { ck = kNegInf; ci = 0x7fffffff; }
      }
    } else {
      // more tied candidates than LDS holds: K selections over the row, read again
      float prev_k = __builtin_huge_valf();
      int prev_i = -1;
      for (int j = 0; j < p.topk; ++j) {
        float bk = kNegInf;
        int bi = 0x7fffffff;
        for (int c = 0; c < nchunks; ++c) {
          const int i0 = (c * kFT + tid) * EPV;
          const uint4 w = load_raw(c);
          const uint32_t pb = (use_pen && i0 < V) ? (pbits[i0 >> 5] >> (i0 & 31)) & 0xffu : 0u;
          static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
            constexpr int e = decltype(ec_)::value;
            float xv = RE::get(w, e);
            if ((pb >> e) & 1u) xv = pen_value(xv);
            if (i0 + e < V && xv >= v_thr) {
              const int i = i0 + e;
              const float key = RE::round((xv - m_pen) - logsum);
              const bool after = key < prev_k || (key == prev_k && i > prev_i);
              if (after && tk_better(key, i, bk, bi)) { bk = key; bi = i; }
            }
          });
        }
        block_best(bk, bi);
        if (tid == 0) {
          if (p.out_topk) p.out_topk[(long)row * p.topk + j] = bi;
          if (p.out_topk_lp) p.out_topk_lp[(long)row * p.topk + j] = bk;
        }
        prev_k = bk;
        prev_i = bi;
      }
    }
  }

  // ---- the drawn token: the j_r-th (by index) token of value v_r. Thread t takes the masks of
  // (chunk t / 16, wave t % 16), whose tokens follow in index order (lane, then element) ----
  if (p.do_sample) {
    const int t = tid;
    uint4 mw[4] = {};
    uint32_t v = 0;
    if (t < nchunks * kFW) {
_Pragma("clang loop unroll(full)")
      for (int q = 0; q < 4; ++q) {
        mw[q] = reinterpret_cast<const uint4*>(masks + t * 64)[q];
        v += __builtin_popcount(mw[q].x) + __builtin_popcount(mw[q].y) + __builtin_popcount(mw[q].z) +
             __builtin_popcount(mw[q].w);
      }
    }
    uint64_t tot;
    const uint64_t ex = block_excl_scan_u64((uint64_t)v, tot, fs);
    if (v && ex <= j_r && j_r < ex + v) {
      // the 16 words of lane masks (4 lanes each): popcounts, then the word, byte and bit
      // holding match j_r (static selections: no dynamic register indexing)
      const uint32_t wv[16] = {mw[0].x, mw[0].y, mw[0].z, mw[0].w, mw[1].x, mw[1].y, mw[1].z, mw[1].w,
                               mw[2].x, mw[2].y, mw[2].z, mw[2].w, mw[3].x, mw[3].y, mw[3].z, mw[3].w};
      uint32_t seen = (uint32_t)ex, wsel = 0, base = 0;
      int wi_found = -1;
      static_for<16>([&](auto wi_) __attribute__((always_inline)) {
        constexpr int wi = decltype(wi_)::value;
        const uint32_t n = (uint32_t)__builtin_popcount(wv[wi]);
        if (wi_found < 0 && seen + n > j_r) { wi_found = wi; wsel = wv[wi]; base = seen; }
        seen += n;
      });
      int found = -1;
      if (wi_found >= 0) {
        static_for<4>([&](auto bb_) __attribute__((always_inline)) {
          constexpr int bb = decltype(bb_)::value;
          uint32_t mb = (wsel >> (8 * bb)) & 0xffu;
          const uint32_t n = (uint32_t)__builtin_popcount(mb);
          if (found < 0 && base + n > j_r) {
            for (uint32_t r = j_r - base; r > 0; --r) mb &= mb - 1u;  // drop the earlier matches
            found = (wi_found * 4 + bb) * EPV + __builtin_ctz(mb);      // lane * 8 + element
          }
          base += n;
        });
      }
      if (found >= 0 && p.out_sample)
        p.out_sample[row] = ((t / kFW) * kFT + (t % kFW) * 64) * EPV + found;
    }
  }
}

template <typename T, bool AL>
__global__ __launch_bounds__(kRowThreads) void row_stats_kernel(RowParams p) {
  const int row = blockIdx.x;
  if (row >= p.R) return;
  __shared__ RowShared sh;
  __shared__ uint32_t pbits[kMaxPenWords];
  rows_generic<T, AL, kRowThreads>(p, row, sh, pbits);
}

template <typename T>
static int dispatch_rows(const RowParams& p, hipStream_t s) {
  constexpr int EPV = RowElem<T>::EPV;
  using S = typename T::storage;
  const long nchunks = ((long)p.V + kRowThreads * EPV - 1) / (kRowThreads * EPV);
  if (nchunks > kMaxChunks || (long)p.V > (long)kMaxPenWords * 32) return MENTAT_EUNSUP;
  // 16-byte loads need every row to start on a 16-byte boundary.
  const bool aligned = (((uintptr_t)p.logits) & 15u) == 0 && ((p.row_stride * (long)sizeof(S)) & 15) == 0;
  if constexpr (sizeof(S) == 2) {
    if (aligned && p.V <= kFastMaxV) {
      hipLaunchKernelGGL((row_stats_fast_kernel<T>), dim3(p.R), dim3(kFT), 0, s, p);
      return (int)hipGetLastError();
    }
  }
  if (aligned)
    hipLaunchKernelGGL((row_stats_kernel<T, true>), dim3(p.R), dim3(kRowThreads), 0, s, p);
  else
    hipLaunchKernelGGL((row_stats_kernel<T, false>), dim3(p.R), dim3(kRowThreads), 0, s, p);
  return (int)hipGetLastError();
}

}  // namespace mentat

using namespace mentat;

extern "C" int mentat_row_stats(const void* logits, int64_t row_stride, int R, int V, int dtype,
                                float temperature, float penalty, const int32_t* pen_offsets,
                                const int32_t* pen_ids, float gate_threshold, int topk, int do_sample,
                                float sample_temperature, float top_p, uint64_t seed, uint64_t step,
                                float* out_entropy, float* out_entropy_pen, float* out_lse,
                                uint8_t* out_gate, int32_t* out_topk, float* out_topk_lp,
                                int32_t* out_sample, void* stream) {
  if (R == 0) return MENTAT_OK;
  if (!logits || R < 0 || V <= 0 || row_stride < V || !out_entropy) return MENTAT_EINVAL;
  if (!(temperature > 0.f) || topk < 0 || topk > kMaxTopK || topk > V) return MENTAT_EINVAL;
  if (do_sample && (!(sample_temperature > 0.f) || !(top_p > 0.f) || top_p > 1.f || !out_sample))
    return MENTAT_EINVAL;
  if (R > 2147483647 / 2) return MENTAT_EINVAL;
  RowParams p;
  p.logits = logits; p.row_stride = row_stride; p.R = R; p.V = V;
  p.ent_c = (float)(1.4426950408889634 / (double)temperature);
  p.samp_c = do_sample ? (float)(1.4426950408889634 / (double)sample_temperature) : 0.f;
  p.penalty = penalty; p.pen_offsets = pen_offsets; p.pen_ids = pen_ids;
  p.topk = topk;
  p.top_p_q32 = (uint64_t)llrint((double)top_p * 4294967296.0);
  p.seed = seed; p.step = step; p.do_sample = do_sample; p.gate_threshold = gate_threshold;
  p.out_entropy = out_entropy; p.out_entropy_pen = out_entropy_pen; p.out_lse = out_lse;
  p.out_gate = out_gate; p.out_topk = out_topk; p.out_topk_lp = out_topk_lp; p.out_sample = out_sample;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16: return dispatch_rows<BF16>(p, s);
    case MENTAT_F16: return dispatch_rows<F16>(p, s);
    case MENTAT_F32: return dispatch_rows<F32>(p, s);
    default: return MENTAT_EUNSUP;
  }
}

namespace mentat {
__global__ void philox_kernel(const uint32_t* counters, const uint32_t* keys, uint32_t* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t c[4] = {counters[4 * i], counters[4 * i + 1], counters[4 * i + 2], counters[4 * i + 3]};
  philox4x32_10(c, keys[2 * i], keys[2 * i + 1]);
  for (int j = 0; j < 4; ++j) out[4 * i + j] = c[j];
}
}  // namespace mentat

extern "C" int mentat_philox4x32_10(const uint32_t* counters, const uint32_t* keys, uint32_t* out, int n,
                                    void* stream) {
  if (n == 0) return MENTAT_OK;
  if (!counters || !keys || !out || n < 0) return MENTAT_EINVAL;
  hipLaunchKernelGGL(philox_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, counters, keys,
                     out, n);
  return (int)hipGetLastError();
}
