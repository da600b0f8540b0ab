// Shared device helpers for the gfx950 kernels of libmentat_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "../../include/mentat_capi.h"

namespace mentat {

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1, so
// register arrays indexed by i stay in registers.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Every workspace passed to this library begins with MENTAT_WORKSPACE_RESERVED
// bytes of arrival counters for the native paged decode (one int32 per
// (sequence, kv head) unit). They must be zero before a workspace's first use;
// every call leaves them zero, and every entry point keeps its own data after
// them, so one workspace can serve all entry points on a stream.
constexpr size_t kWsReserved = MENTAT_WORKSPACE_RESERVED;
constexpr int kMaxNativeUnits = (int)(kWsReserved / sizeof(int32_t));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// ---- element conversions ------------------------------------------------------------
struct F32 {
  using storage = float;
  static constexpr int code = MENTAT_F32;
};
struct F16 {
  using storage = uint16_t;
  static constexpr int code = MENTAT_F16;
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int code = MENTAT_BF16;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <typename T> struct Elem;
template <> struct Elem<F32> {
  static constexpr int per16 = 4;  // elements per 16-byte load
  __device__ static void unpack(const uint4& w, float* f) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  }
  __device__ static float load1(const void* p, long i) { return ((const float*)p)[i]; }
  __device__ static void store1(void* p, long i, float v) { ((float*)p)[i] = v; }
};
template <> struct Elem<BF16> {
  static constexpr int per16 = 8;
  __device__ static void unpack(const uint4& w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x); f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z); f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
  }
  __device__ static float load1(const void* p, long i) {
    return __uint_as_float(((uint32_t)((const uint16_t*)p)[i]) << 16);
  }
  __device__ static void store1(void* p, long i, float v) { ((uint16_t*)p)[i] = f32_to_bf16(v); }
};
template <> struct Elem<F16> {
  static constexpr int per16 = 8;
  __device__ static void unpack(const uint4& w, float* f) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = f16_bits_to_f32((uint16_t)(ws[i] & 0xffffu));
      f[2 * i + 1] = f16_bits_to_f32((uint16_t)(ws[i] >> 16));
    }
  }
  __device__ static float load1(const void* p, long i) {
    return f16_bits_to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static void store1(void* p, long i, float v) { ((uint16_t*)p)[i] = f32_to_f16_bits(v); }
};

// 16-bit values as torch's elementwise kernels round them: lo/hi unpack a
// packed pair, rnd rounds an fp32 result to the dtype (one rounding per torch
// op), bits gives the rounded value's 16 bits.
template <typename T> struct G16;
template <> struct G16<BF16> {
  __device__ static float lo(uint32_t w) { return bf16_lo(w); }
  __device__ static float hi(uint32_t w) { return bf16_hi(w); }
  __device__ static uint32_t bits(float v) { return f32_to_bf16(v); }
  __device__ static float rnd(float v) { return __uint_as_float((uint32_t)f32_to_bf16(v) << 16); }
};
// The empty asm makes the float value exist before it is narrowed (no fused
// mixed-precision instruction that would round once).
template <> struct G16<F16> {
  __device__ static float lo(uint32_t w) { return f16_bits_to_f32((uint16_t)(w & 0xffffu)); }
  __device__ static float hi(uint32_t w) { return f16_bits_to_f32((uint16_t)(w >> 16)); }
  __device__ static uint32_t bits(float v) {
    asm volatile("" : "+v"(v));
    return f32_to_f16_bits(v);
  }
  __device__ static float rnd(float v) {
    asm volatile("" : "+v"(v));
    return f16_bits_to_f32(f32_to_f16_bits(v));
  }
};

// RoPE of one (a, b) = (t[i], t[i + D/2]) pair as the adapters' torch code
// rounds it, t' = rnd(rnd(t * cos) + rnd(rotate_half(t) * sin)):
// a' = rnd(rnd(a c_i) + rnd(-b s_i)), b' = rnd(rnd(b c_{i+D/2}) + rnd(a s_{i+D/2})).
template <typename T>
__device__ __forceinline__ void rope_pair(float a, float b, float ci, float si, float ch, float sh, float& ya,
                                          float& yb) {
  using E = G16<T>;
  ya = E::rnd(E::rnd(a * ci) + E::rnd(-b * si));
  yb = E::rnd(E::rnd(b * ch) + E::rnd(a * sh));
}

// ---- 16-byte dot products: q (kept in its packed form) · k -----------------------------
// For 16-bit types the packed pairs go straight into v_dot2 (fp32 accumulate).
template <typename T> struct Dot16;
template <> struct Dot16<BF16> {
  __device__ static float dot(const uint4& q, const uint4& k, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.x),
                                          __builtin_bit_cast(bf16x2_t, k.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.y),
                                          __builtin_bit_cast(bf16x2_t, k.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.z),
                                          __builtin_bit_cast(bf16x2_t, k.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.w),
                                          __builtin_bit_cast(bf16x2_t, k.w), acc, false);
    return acc;
  }
};
template <> struct Dot16<F16> {
  __device__ static float dot(const uint4& q, const uint4& k, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.x), __builtin_bit_cast(f16x2_t, k.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.y), __builtin_bit_cast(f16x2_t, k.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.z), __builtin_bit_cast(f16x2_t, k.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.w), __builtin_bit_cast(f16x2_t, k.w), acc, false);
    return acc;
  }
};
template <> struct Dot16<F32> {
  __device__ static float dot(const uint4& q, const uint4& k, float acc) {
    acc = fmaf(__uint_as_float(q.x), __uint_as_float(k.x), acc);
    acc = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), acc);
    acc = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), acc);
    acc = fmaf(__uint_as_float(q.w), __uint_as_float(k.w), acc);
    return acc;
  }
};

// ---- cross-lane helpers ------------------------------------------------------------------
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LANES consecutive lanes (LANES in {1,2,4,8,16,32,64});
// every lane of the group receives the group total.
template <int LANES>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LANES >= 2) v += dpp_f<kDppQuadXor1>(v);
  if constexpr (LANES >= 4) v += dpp_f<kDppQuadXor2>(v);
  if constexpr (LANES >= 8) v += dpp_f<kDppRowHalfMirror>(v);
  if constexpr (LANES >= 16) v += dpp_f<kDppRowMirror>(v);
  if constexpr (LANES >= 32) v += __shfl_xor(v, 16);
  if constexpr (LANES >= 64) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- wave-wide sums, minima and prefix sums through DPP (register moves, no LDS round trip) ----
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr3 = 0x113, kDppRowShr4 = 0x114,
              kDppRowShr8 = 0x118, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
// Lanes whose row / bank is masked off, or that have no source lane, read 0.
template <int CTRL, int RM = 0xF, int BM = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, RM, BM, true);
}
template <int CTRL, int RM = 0xF, int BM = 0xF>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL, RM, BM>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL, RM, BM>((uint32_t)v);
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  return __builtin_bit_cast(double, dpp_u64<CTRL>(__builtin_bit_cast(uint64_t, v)));
}
__device__ __forceinline__ uint32_t rl32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ uint64_t rl64(uint64_t v, int l) {
  return ((uint64_t)rl32((uint32_t)(v >> 32), l) << 32) | rl32((uint32_t)v, l);
}
// Inclusive prefix sum over the wave's lanes (lane order): window sums within rows, then the
// row totals carried across rows by row broadcasts.
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const uint64_t v0 = v;
  v += dpp_u64<kDppRowShr1>(v0);
  v += dpp_u64<kDppRowShr2>(v0);
  v += dpp_u64<kDppRowShr3>(v0);
  v += dpp_u64<kDppRowShr4, 0xF, 0xE>(v);
  v += dpp_u64<kDppRowShr8, 0xF, 0xC>(v);
  v += dpp_u64<kDppRowBcast15, 0xA, 0xF>(v);
  v += dpp_u64<kDppRowBcast31, 0xC, 0xF>(v);
  return v;
}

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const uint32_t v0 = v;
  v += dpp_u32<kDppRowShr1>(v0);
  v += dpp_u32<kDppRowShr2>(v0);
  v += dpp_u32<kDppRowShr3>(v0);
  v += dpp_u32<kDppRowShr4, 0xF, 0xE>(v);
  v += dpp_u32<kDppRowShr8, 0xF, 0xC>(v);
  v += dpp_u32<kDppRowBcast15, 0xA, 0xF>(v);
  v += dpp_u32<kDppRowBcast31, 0xC, 0xF>(v);
  return v;
}


}  // namespace mentat
