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
//            called at core/generator.py:342), with the rounding chain torch's device
//            kernels give it in the logits dtype: y = rnd(x * fl(1/T)) (division by a
//            scalar is a multiply by its reciprocal), m = max y, e = exp2(fl(y - m) *
//            log2(e)), s = sum e, p = rnd(e / s), lp = rnd((y - m) - log s),
//            t = rnd(p * lp), H = -rnd(sum t); rnd rounds to the logits dtype (identity
//            for f32). Both sums are formed in double from fp32 terms and rounded to
//            float once (torch sums in float in its own order).
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
  float inv_t;         // fl(1 / T): the gate entropy's y = rnd(x * inv_t)
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
  float* out_entropy_f32;  // [R] or null: H_T with fp32 arithmetic throughout (no dtype rounding)
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
  alignas(8) float f[NW * 8];  // also four doubles per wave
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

// Butterflies within each row of 16 lanes: every lane then holds its row's total.
template <typename T, class MOVE>
__device__ __forceinline__ T row_total(T v, MOVE mv) {
  v += mv(v, std::integral_constant<int, kDppQuadXor1>{});
  v += mv(v, std::integral_constant<int, kDppQuadXor2>{});
  v += mv(v, std::integral_constant<int, kDppRowHalfMirror>{});
  v += mv(v, std::integral_constant<int, kDppRowMirror>{});
  return v;
}
// Wave totals (wave-uniform), the four row totals added in row order.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v = row_total(v, [](uint32_t x, auto c) { return dpp_u32<decltype(c)::value>(x); });
  return rl32(v, 0) + rl32(v, 16) + rl32(v, 32) + rl32(v, 48);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  v = row_total(v, [](uint64_t x, auto c) { return dpp_u64<decltype(c)::value>(x); });
  return rl64(v, 0) + rl64(v, 16) + rl64(v, 32) + rl64(v, 48);
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = row_total(v, [](double x, auto c) { return dpp_f64<decltype(c)::value>(x); });
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  return ((__builtin_bit_cast(double, rl64(u, 0)) + __builtin_bit_cast(double, rl64(u, 16))) +
          __builtin_bit_cast(double, rl64(u, 32))) + __builtin_bit_cast(double, rl64(u, 48));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppQuadXor1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppQuadXor2, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppRowHalfMirror, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppRowMirror, 0xF, 0xF, false));
  return min(min(rl32(v, 0), rl32(v, 16)), min(rl32(v, 32), rl32(v, 48)));
}
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
  const uint64_t inc = wave_incl_scan_u64(v);
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

// Sum of up to 4 doubles over the block (every thread gets the totals).
template <int NVAL, class SH>
__device__ __forceinline__ void block_sum_f64(double (&v)[NVAL], SH& sh) {
  static_assert(NVAL <= 4, "four doubles per wave slot");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
_Pragma("clang loop unroll(full)")
  for (int i = 0; i < NVAL; ++i) v[i] = wave_sum_f64(v[i]);
  __syncthreads();
  if (lane == 0) {
_Pragma("clang loop unroll(full)")
    for (int i = 0; i < NVAL; ++i) reinterpret_cast<double*>(sh.f)[wave * 4 + i] = v[i];
  }
  __syncthreads();
_Pragma("clang loop unroll(full)")
  for (int i = 0; i < NVAL; ++i) {
    double a = 0.0;
    for (int w = 0; w < SH::kWaves; ++w) a += reinterpret_cast<const double*>(sh.f)[w * 4 + i];
    v[i] = a;
  }
}

// ---- the entropy chain in the logits dtype (compute_entropy, core/generator_utils.py:196-202,
// and log_softmax, core/generator.py:283/308, as torch's device kernels round them) --------------
// A row's softmax state: its max m (a value of the dtype), s = fl(sum exp2(fl(y - m) * log2 e))
// and ln s. Keys (log-probs) are rnd(fl(y - m) - ln s).
struct ChainState {
  float m, s, logs;
};
__device__ __forceinline__ ChainState chain_state(float m, double s) {
  const float sf = (float)s;
  return ChainState{m, sf, logf(sf)};
}
__device__ __forceinline__ float chain_exp(float y, float m) { return exp2f((y - m) * kLog2e); }
// t = rnd(rnd(e / s) * rnd(fl(y - m) - ln s)) for one token of value y.
template <class RE>
__device__ __forceinline__ float chain_term(float y, const ChainState& c) {
  const float d = y - c.m;
  const float pr = RE::round(__fdiv_rn(exp2f(d * kLog2e), c.s));
  const float lp = RE::round(d - c.logs);
  const float t = RE::round(pr * lp);
  return t != t ? 0.f : t;  // torch.nan_to_num(nan=0.0): 0 * -inf for a -inf logit
}
// H = -rnd(sum t) from the double sum of the terms.
template <class RE>
__device__ __forceinline__ float chain_entropy(double S) { return -RE::round((float)S); }
// The entropy with fp32 arithmetic throughout (y = x * fl(1/T) unrounded, exact sums):
// H = ln s - (sum e * d) / s with d = fl(y - m), e = exp2(d * log2 e).
__device__ __forceinline__ float f32_entropy(double s, double sed) { return (float)(log(s) - sed / s); }

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

  // ---- pass 2: the softmax denominators in double (the gate chain on y = rnd(x * inv_t), the
  // T = 1 chain on xp); with sampling, the first radix level of the fixed-point masses (a
  // histogram by the top 12 key bits) ----
  // The T = 1 chain of xp feeds the top-K keys, the log-sum-exp and H_pen only.
  const bool need_pen_sums = p.topk > 0 || p.out_entropy_pen != nullptr || p.out_lse != nullptr;
  constexpr int L0 = RE::level_bits[0];
  if (p.do_sample) {
    for (int t = tid; t < (1 << L0); t += kRowThreads) sh.hist0[t] = 0;
    __syncthreads();
  }
  const float m_t = RE::round(m_raw * p.inv_t);  // rounding keeps the order: the largest y
  const float m_32 = m_raw * p.inv_t;
  const bool want_f32 = p.out_entropy_f32 != nullptr;
  double den[4] = {0.0, 0.0, 0.0, 0.0};
  ROW_FOR_GROUPS(
    const int i0 = (c * kRowThreads + tid) * EPV;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      if (i0 + e >= p.V) return;
      den[0] += (double)chain_exp(RE::round(x[e] * p.inv_t), m_t);
      if (want_f32) {
        const float d32 = x[e] * p.inv_t - m_32;
        const float e32 = exp2f(d32 * kLog2e);
        den[2] += (double)e32;
        den[3] += e32 > 0.f ? (double)e32 * (double)d32 : 0.0;
      }
      const float xp = penal(i0 + e, x[e]);
      if (need_pen_sums) den[1] += (double)chain_exp(xp, m_pen);
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
  block_sum_f64<4>(den, sh);
  const ChainState c_t = chain_state(m_t, den[0]), c_1 = chain_state(m_pen, den[1]);
  if (want_f32 && tid == 0) p.out_entropy_f32[row] = f32_entropy(den[2], den[3]);
  // ---- pass 2b: the entropy terms t of both chains ----
  double ent[2] = {0.0, 0.0};
  const bool want_hpen = p.out_entropy_pen != nullptr;
  ROW_FOR_GROUPS(
    const int i0 = (c * kRowThreads + tid) * EPV;
    static_for<EPV>([&](auto ec_) __attribute__((always_inline)) {
      constexpr int e = decltype(ec_)::value;
      if (i0 + e >= p.V) return;
      ent[0] += (double)chain_term<RE>(RE::round(x[e] * p.inv_t), c_t);
      if (want_hpen) ent[1] += (double)chain_term<RE>(penal(i0 + e, x[e]), c_1);
        });
    )
  block_sum_f64<2>(ent, sh);
  const float H_T = chain_entropy<RE>(ent[0]);
  const float H_pen = chain_entropy<RE>(ent[1]);
  const float logsum = c_1.logs;  // ln(sum exp(xp - max)), as log_softmax forms it
  if (tid == 0) {
    p.out_entropy[row] = H_T;
    if (p.out_entropy_pen) p.out_entropy_pen[row] = H_pen;
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

constexpr int kFT = 512;                                       // threads per row (2 waves per SIMD:
                                                               // 256 VGPRs each, room for the row)
constexpr int kFW = kFT / 64;
constexpr int kFastChunks = 40;                                // chunks of kFT 16-byte groups
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
  alignas(8) float f[kFW * 8];  // also four doubles per wave
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

// The row's registers: 32-dword vectors of 8 groups each. A group is read back with a
// wave-uniform index (GPR indexing), so the passes over the row are compact loops rather
// than one unrolled copy of their body per group.
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
__device__ __forceinline__ uint4 row_group(const u32x32& v, int g) {
  const int b = __builtin_amdgcn_readfirstlane(g) * 4;
  return make_uint4(v[b], v[b + 1], v[b + 2], v[b + 3]);
}

// Rows must start on 16-byte boundaries (16-byte buffer loads). NG: 16-byte groups per thread
// (V <= NG * kFT * 8, NG a multiple of 8); the whole row stays in registers (NG * 4 VGPRs), so
// it is read from HBM once.
template <typename T, int NG>
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
  static_assert(NG <= kFastChunks, "the penalty bits cover kFastChunks groups per thread");
  static_assert(NG % 8 == 0, "groups are held 8 to a 32-dword vector");
  constexpr int NV = NG / 8;
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

  // ---- pass A: the whole row into registers, every load in flight at once (bytes past the row
  // read as zero); each group is counted into the 65,536-value histogram as it lands, with the
  // largest and smallest keys on the way ----
  u32x32 d[NV];
  static_for<NG>([&](auto c_) __attribute__((always_inline)) {
    constexpr int c = decltype(c_)::value;
    const uint4 w = load_raw(c);
    d[c / 8][(c % 8) * 4] = w.x;
    d[c / 8][(c % 8) * 4 + 1] = w.y;
    d[c / 8][(c % 8) * 4 + 2] = w.z;
    d[c / 8][(c % 8) * 4 + 3] = w.w;
    __builtin_amdgcn_sched_barrier(0);  // issue in chunk order: groups land in order and are counted so
  });
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
  // The draw's uniform depends only on (seed, row, step).
  uint64_t U = 0;
  if (p.do_sample) {
    uint32_t c4[4] = {(uint32_t)row, (uint32_t)p.step, (uint32_t)(p.step >> 32), 0u};
    philox4x32_10(c4, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
    U = ((uint64_t)c4[0] << 32) | c4[1];
  }
  __syncthreads();
  auto count1 = [&](uint32_t k) __attribute__((always_inline)) { atomicAdd(&hist[k >> 1], 1u << ((k & 1u) << 4)); };
  uint32_t kmx = 0, kmn = 0xffffffffu;
  // (each vector's loop waits only for its own 8 loads: counting overlaps the later ones)
  static_for<NV>([&](auto v_) __attribute__((always_inline)) {
    constexpr int v = decltype(v_)::value;
#pragma clang loop unroll(disable)
    for (int g = 0; g < 8; ++g) {
    const int c = v * 8 + g;
    if (c >= nchunks) break;
    const int i0 = (c * kFT + tid) * EPV;
    const uint4 w = row_group(d[v], g);
    const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
    if (i0 + EPV <= V) {
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
  });
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
  const float m_t = RE::round(m_raw * p.inv_t);  // the largest y = rnd(x * inv_t)

  // ---- sweeps over the histogram (wave w takes slabs w, w + 16, ...; lane l the four values
  // 4l .. 4l + 3 of the slab) ----
  const bool need_pen_sums = p.topk > 0 || p.out_entropy_pen != nullptr || p.out_lse != nullptr;
  const bool want_hpen = p.out_entropy_pen != nullptr;
  const bool want_mass = p.do_sample != 0;
  // The softmax denominators (in double; slab token counts into fs.slab_cnt, the token total
  // into fs.total): the gate chain of the raw values (do_t) and the T = 1 chain (do_1).
  // With do_32, also the fp32 entropy's sums of the raw values (den[2], den[3]).
  const float m_32 = m_raw * p.inv_t;
  auto sweep_den = [&](bool do_t, bool do_1, bool do_32, bool masses, float m_1, double (&den)[4]) __attribute__((always_inline)) {
    const uint2* h2 = reinterpret_cast<const uint2*>(hist);
    uint32_t total = 0;
    den[0] = 0.0;
    den[1] = 0.0;
    den[2] = 0.0;
    den[3] = 0.0;
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
            const float v = kval((uint32_t)(s * kSlabBins + lane * 4 + b));
            const double dn = (double)n;
            if (do_t) den[0] += dn * (double)chain_exp(RE::round(v * p.inv_t), m_t);
            if (do_1) den[1] += dn * (double)chain_exp(v, m_1);
            if (do_32) {
              const float d32 = v * p.inv_t - m_32;
              const float e32 = exp2f(d32 * kLog2e);
              den[2] += dn * (double)e32;
              if (e32 > 0.f) den[3] += dn * ((double)e32 * (double)d32);
            }
            if (masses) {
              const float ys = (v - m_1) * p.samp_c;
              if (ys >= -41.0f) mass += (uint64_t)n * det_q(ys);
            }
            cnt += n;
          }
        }
        total += cnt;
        if (masses) mass = wave_sum_u64(mass);
        cnt = wave_sum_u32(cnt);
      }
      if (lane == 0) {
        fs.slab_mass[s] = mass;
        fs.slab_cnt[s] = cnt;
      }
    }
    total = wave_sum_u32(total);
    if (lane == 0) atomicAdd(&fs.total, total);
    block_sum_f64<4>(den, fs);
  };
  // The entropy terms of both chains over the slabs holding tokens (fs.slab_cnt of the last
  // sweep_den on this histogram).
  auto sweep_ent = [&](bool do_t, bool do_1, const ChainState& ct, const ChainState& c1, double (&ent)[2]) __attribute__((always_inline)) {
    const uint2* h2 = reinterpret_cast<const uint2*>(hist);
    ent[0] = 0.0;
    ent[1] = 0.0;
    for (int i = 0; i < kSlabs / kFW; ++i) {
      const int s = wave + i * kFW;
      if (fs.slab_cnt[s] == 0) continue;
      const uint2 wd = h2[s * (kSlabBins / 4) + lane];
_Pragma("clang loop unroll(full)")
      for (int b = 0; b < 4; ++b) {
        const uint32_t n = ((b < 2 ? wd.x : wd.y) >> ((b & 1) * 16)) & 0xffffu;
        if (!n) continue;
        const float v = kval((uint32_t)(s * kSlabBins + lane * 4 + b));
        const double dn = (double)n;
        if (do_t) ent[0] += dn * (double)chain_term<RE>(RE::round(v * p.inv_t), ct);
        if (do_1) ent[1] += dn * (double)chain_term<RE>(v, c1);
      }
    }
    block_sum_f64<2>(ent, fs);
  };

  const bool want_f32 = p.out_entropy_f32 != nullptr;
  float H_T = 0.f, H32 = 0.f;
  ChainState c_t{m_t, 0.f, 0.f};
  if (ok && use_pen) {
    // The gate entropy of the raw values, then every penalised token (each distinct id once: the
    // one that clears its bit) moves to its penalised value; the bits are set again for pass B.
    double den[4], ent[2];
    sweep_den(true, false, want_f32, false, m_raw, den);
    c_t = chain_state(m_t, den[0]);
    H32 = f32_entropy(den[2], den[3]);
    __syncthreads();
    sweep_ent(true, false, c_t, c_t, ent);
    H_T = chain_entropy<RE>(ent[0]);
    // (the id list is read only now: its loads would otherwise wait for the row's)
    for (int w = tid; w < nwords; w += kFT) pbits[w] = 0u;
    if (tid == 0) fs.total = 0;
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

  // ---- resolution: each slab's mass and count, the denominators and the token total (a 16-bit
  // count that overflowed leaves it short of V), then the entropy terms ----
  ChainState c_1{m_pen, 0.f, 0.f};
  if (ok) {
    double den[4];
    sweep_den(!use_pen, need_pen_sums, want_f32 && !use_pen, want_mass, m_pen, den);
    ok = fs.total == (uint32_t)V;
    if (ok) {
      if (!use_pen) {
        c_t = chain_state(m_t, den[0]);
        H32 = f32_entropy(den[2], den[3]);
      }
      c_1 = chain_state(m_pen, den[1]);
      if (!use_pen || want_hpen) {
        double ent[2];
        sweep_ent(!use_pen, want_hpen, c_t, c_1, ent);
        if (!use_pen) H_T = chain_entropy<RE>(ent[0]);
        if (want_hpen && tid == 0) p.out_entropy_pen[row] = chain_entropy<RE>(ent[1]);
      }
    }
  }
  if (!ok) {
    __syncthreads();
    rows_generic<T, AL, kFT>(p, row, *reinterpret_cast<RowSharedT<kFW>*>(hist), pbits);
    return;
  }
  const float logsum = c_1.logs;
  if (tid == 0) {
    p.out_entropy[row] = H_T;
    if (want_f32) p.out_entropy_f32[row] = H32;
    if (p.out_lse) p.out_lse[row] = m_pen + logsum;
    if (p.out_gate) p.out_gate[row] = H_T > p.gate_threshold ? 1 : 0;
  }
  if (!p.do_sample && p.topk == 0) return;

  // Wave-level resolution (no barriers): the slab, then the value, holding position pos, keys
  // descending. Lane l holds slabs kSlabs-1-4l .. kSlabs-4-4l (largest keys in lane 0).
  auto unit_mass = [&](uint32_t k) __attribute__((always_inline)) -> uint64_t {
    const float ys = (kval(k) - m_pen) * p.samp_c;
    return ys >= -41.0f ? det_q(ys) : 0;
  };
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
    // suffix sum (lanes above hold larger keys): the wave total less the exclusive prefix
    const uint64_t pre = wave_incl_scan_u64(tot);
    const uint64_t inc = rl64(pre, 63) - pre + tot;
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
    return wave_incl_scan_u64(lt) - lt;
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

  // ---- pass B (the row from registers): how many of each lane's 8 tokens of every chunk equal
  // the drawn value, and the top-K candidates. The drawn value is matched on the raw bits of a
  // dword's two values at once (a half of dw ^ (raw_r * 0x10001) is zero iff that value is the
  // drawn one; -0 is the drawn zero too). A group holds a candidate only if its largest key
  // reaches the threshold's. Penalised tokens, the row's last partial group and candidate groups
  // (all rare) are checked element by element on their values ----
  uint8_t* counts = reinterpret_cast<uint8_t*>(hist);        // [kFastChunks][kFW][64 lanes]
  uint2* cand = reinterpret_cast<uint2*>(hist + 8192);       // [kCandCap] (log-prob bits, index)
  const float v_match = p.do_sample ? v_r : __builtin_nanf("");  // NaN matches nothing
  const uint32_t raw_r = raw16_of_key(fs.sel[0] & 0xffffu);
  const uint32_t raw_r2 = raw_r * 0x10001u;
  const bool r_zero = raw_r == 0u;                             // -0 (raw 0x8000) matches as well
  const uint32_t key_thr = p.topk > 0 ? fs.sel[2] & 0xffffu : 0x10000u;  // above every key: no candidates
  const uint32_t key_thr_any = key_thr == 0x8000u ? 0x7fffu : key_thr;  // -0 reaches a +0 threshold
  // bit 15 / bit 31 set where the low / high half of x is zero (no carry crosses the halves)
  auto zero_halves = [](uint32_t x) __attribute__((always_inline)) -> uint32_t {
    return ~(((x & 0x7fff7fffu) + 0x7fff7fffu) | x) & 0x80008000u;
  };
  __syncthreads();
  if (tid == 0) {
    fs.ncand = 0;
    fs.sel[3] = 0xffffffffu;
  }
  __syncthreads();
  static_for<NV>([&](auto v_) __attribute__((always_inline)) {
    constexpr int v = decltype(v_)::value;
#pragma clang loop unroll(disable)
    for (int g = 0; g < 8; ++g) {
    const int c = v * 8 + g;
    if (c >= nchunks) break;
    const int i0 = (c * kFT + tid) * EPV;
    const uint4 dd = row_group(d[v], g);
    const uint32_t vm = i0 + EPV <= V ? 0xffu : i0 >= V ? 0u : (1u << (V - i0)) - 1u;  // valid elements
    const uint32_t pb = (use_pen && i0 < V) ? (pbits[i0 >> 5] >> (i0 & 31)) & vm & 0xffu : 0u;
    const bool exact = vm != 0xffu || pb != 0u;
    uint32_t nm = 0;
    if (p.do_sample && !exact) {
      uint32_t f0 = zero_halves(dd.x ^ raw_r2), f1 = zero_halves(dd.y ^ raw_r2);
      uint32_t f2 = zero_halves(dd.z ^ raw_r2), f3 = zero_halves(dd.w ^ raw_r2);
      if (r_zero) {
        f0 |= zero_halves(dd.x ^ 0x80008000u);
        f1 |= zero_halves(dd.y ^ 0x80008000u);
        f2 |= zero_halves(dd.z ^ 0x80008000u);
        f3 |= zero_halves(dd.w ^ 0x80008000u);
      }
      nm = __builtin_popcount(f0) + __builtin_popcount(f1) + __builtin_popcount(f2) + __builtin_popcount(f3);
    }
    uint32_t cm = 0;
    if (p.topk > 0) {
      const uint32_t dw[4] = {dd.x, dd.y, dd.z, dd.w};
      uint32_t kmax = 0;
_Pragma("clang loop unroll(full)")
      for (int k = 0; k < 4; ++k) {
        const uint32_t k2 = dw[k] ^ ((((dw[k] >> 15) & 0x10001u) * 0x7fffu) | 0x80008000u);
        kmax = max(kmax, max(k2 & 0xffffu, k2 >> 16));
      }
      cm = kmax >= key_thr_any ? vm : 0u;
    }
    // element by element: candidate groups, penalised tokens, the last partial group
    for (uint32_t bits = cm | (exact ? vm : 0u); bits != 0u; bits &= bits - 1u) {
      const int e = __builtin_ctz(bits);
      float xv = RE::get(dd, e);
      if ((pb >> e) & 1u) xv = pen_value(xv);
      if (exact && xv == v_match) ++nm;
      if (p.topk > 0 && xv >= v_thr) {
        const uint32_t pos = atomicAdd(&fs.ncand, 1u);
        if (pos < kCandCap)
          cand[pos] = make_uint2(__float_as_uint(RE::round((xv - m_pen) - logsum)), (uint32_t)(i0 + e));
      }
    }
    if (p.do_sample) counts[(c * kFW + wave) * 64 + lane] = (uint8_t)nm;
    }
  });
  __syncthreads();

  if (p.topk > 0) {
    auto block_best = [&](float& bk, int& bi) __attribute__((always_inline)) {
      for (int o = 32; o >= 1; o >>= 1) {
        const float ok2 = __shfl_xor(bk, o);
        const int oi = __shfl_xor(bi, o);
        if (tk_better(ok2, oi, bk, bi)) { bk = ok2; bi = oi; }
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
      // more tied candidates than LDS holds: K selections over the row, read again (rare:
      // the registers are not used here, so the selections add no register pressure)
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

  // ---- the drawn token: the j_r-th (by index) token of value v_r. Thread t takes the counts of
  // (chunk t / kFW, wave t % kFW), whose tokens follow in index order (lane, then element); the
  // one whose range holds j_r names the lane and the rank within its 8 tokens, and that lane finds
  // the token in its registers ----
  if (p.do_sample) {
    const int t = tid;
    uint4 cw[4] = {};
    uint32_t n = 0;
    if (t < nchunks * kFW) {
_Pragma("clang loop unroll(full)")
      for (int q = 0; q < 4; ++q) {
        cw[q] = reinterpret_cast<const uint4*>(counts + t * 64)[q];
        // counts are at most 8: the bytes of a word sum without carries
        n += ((cw[q].x * 0x01010101u) >> 24) + ((cw[q].y * 0x01010101u) >> 24) + ((cw[q].z * 0x01010101u) >> 24) +
             ((cw[q].w * 0x01010101u) >> 24);
      }
    }
    uint64_t tot;
    const uint64_t ex = block_excl_scan_u64((uint64_t)n, tot, fs);
    if (n && ex <= j_r && j_r < ex + n) {
      const uint32_t wv[16] = {cw[0].x, cw[0].y, cw[0].z, cw[0].w, cw[1].x, cw[1].y, cw[1].z, cw[1].w,
                               cw[2].x, cw[2].y, cw[2].z, cw[2].w, cw[3].x, cw[3].y, cw[3].z, cw[3].w};
      uint32_t seen = (uint32_t)ex;
      int lane_found = -1;
      uint32_t rank = 0;
      static_for<64>([&](auto l_) __attribute__((always_inline)) {
        constexpr int l = decltype(l_)::value;
        const uint32_t k = (wv[l / 4] >> (8 * (l % 4))) & 0xffu;
        if (lane_found < 0 && seen + k > j_r) { lane_found = l; rank = j_r - seen; }
        seen += k;
      });
      fs.sel[3] = (uint32_t)t;
      fs.sel[4] = (uint32_t)lane_found;
      fs.sel[5] = rank;
    }
    __syncthreads();
    const uint32_t owner = fs.sel[3];
    if (owner != 0xffffffffu && wave == (int)(owner % kFW)) {
      const int c = (int)(owner / kFW), lf = (int)fs.sel[4];
      const uint32_t rank = fs.sel[5];
      static_for<NV>([&](auto v_) __attribute__((always_inline)) {
        constexpr int v = decltype(v_)::value;
        if (v != c / 8) return;
        const uint4 dd = row_group(d[v], c % 8);
        if (lane != lf) return;
        const int i0 = (c * kFT + tid) * EPV;
        const uint32_t pb = (use_pen && i0 < V) ? (pbits[i0 >> 5] >> (i0 & 31)) & 0xffu : 0u;
        uint32_t seen = 0;
        int found = -1;
        static_for<EPV>([&](auto e_) __attribute__((always_inline)) {
          constexpr int e = decltype(e_)::value;
          float xv = RE::get(dd, e);
          if ((pb >> e) & 1u) xv = pen_value(xv);
          if (i0 + e < V && xv == v_match) {
            if (found < 0 && seen == rank) found = i0 + e;
            ++seen;
          }
        });
        if (found >= 0 && p.out_sample) p.out_sample[row] = found;
      });
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
      // the smallest register-resident instantiation that holds the row
      const long groups = ((long)p.V + kFT * 8 - 1) / (kFT * 8);
      if (groups <= 16)
        hipLaunchKernelGGL((row_stats_fast_kernel<T, 16>), dim3(p.R), dim3(kFT), 0, s, p);
      else if (groups <= 32)
        hipLaunchKernelGGL((row_stats_fast_kernel<T, 32>), dim3(p.R), dim3(kFT), 0, s, p);
      else
        hipLaunchKernelGGL((row_stats_fast_kernel<T, kFastChunks>), dim3(p.R), dim3(kFT), 0, s, p);
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
                                float* out_entropy, float* out_entropy_f32, float* out_entropy_pen, float* out_lse,
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
  p.inv_t = 1.0f / temperature;
  p.samp_c = do_sample ? (float)(1.4426950408889634 / (double)sample_temperature) : 0.f;
  p.penalty = penalty; p.pen_offsets = pen_offsets; p.pen_ids = pen_ids;
  p.topk = topk;
  p.top_p_q32 = (uint64_t)llrint((double)top_p * 4294967296.0);
  p.seed = seed; p.step = step; p.do_sample = do_sample; p.gate_threshold = gate_threshold;
  p.out_entropy = out_entropy; p.out_entropy_f32 = out_entropy_f32; p.out_entropy_pen = out_entropy_pen;
  p.out_lse = out_lse;
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
