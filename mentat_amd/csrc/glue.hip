// Fused per-layer glue of the captured decode step (gfx950), 16-bit models:
// residual add + RMSNorm, rotary embedding of Q and K, SiLU(gate) * up.
//
// Reference: the decode loop of core/generator_utils.py:340-418 runs each
// layer as input_layernorm -> q/k/v projections -> RoPE (the adapters'
// rotate_half form, adapters/llama_adapter.py:70-113) -> attention -> o_proj
// -> residual add -> post_attention_layernorm -> MLP -> residual add, with
// the model's own modules (HF LlamaRMSNorm / Qwen3RMSNorm, LlamaMLP), each a
// handful of torch kernels. Here each group is one launch, rounding as those
// torch kernels do (one rounding to the tensor dtype per torch op):
//   add:     h = rnd(residual + x)
//   RMSNorm: y = rnd(w * rnd(h * rsqrt(mean(h^2) + eps)))   (h in fp32)
//   RoPE:    t' = rnd(rnd(t * cos) + rnd(rotate_half(t) * sin))
//   MLP act: m = rnd(rnd(silu(g)) * u),  silu(g) = g / (1 + exp(-g)) in fp32
// Only the fp32 summation order of the norm's mean differs from torch.
#include "mentat_common.h"

namespace mentat {

namespace {

constexpr int kNormThreads = 256;

// One workgroup per row; each thread owns 8-element groups g = tid, tid + 256, ...
// (H % 8 == 0, H <= 8 * 256 * kNormGroups). NG: groups per thread; FULL: every
// thread owns NG groups (H a multiple of 2048), so no load sits under a branch.
// The weight is loaded with the row, before the block reduction, so the row
// costs one memory round trip.
// NP > 0: x is not given; each element is the sum of NP fp32 partials (xp + s *
// pstride, the slices of a split-K product) rounded once to the dtype, the value a
// single product would have stored.
constexpr int kNormGroups = 4;
template <typename T, int NG, bool FULL, int NP = 0>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const uint16_t* x, const uint16_t* res_in,
                                                               uint16_t* res_out, const uint16_t* w, uint16_t* y,
                                                               int H, float eps, const float* xp = nullptr,
                                                               long pstride = 0) {
  using E = G16<T>;
  const int row = blockIdx.x, tid = threadIdx.x;
  const long base = (long)row * H;
  const int ng = H / 8;
  float h[NG][8];
  uint4 wv[NG];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    const int g = tid + k * kNormThreads;
    if (FULL || g < ng) {
      uint4 xv;
      if constexpr (NP > 0) {
        float4 pa[NP], pb[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          pa[q] = *(const float4*)(xp + q * pstride + base + 8 * g);
          pb[q] = *(const float4*)(xp + q * pstride + base + 8 * g + 4);
        }
        float a8[8] = {pa[0].x, pa[0].y, pa[0].z, pa[0].w, pb[0].x, pb[0].y, pb[0].z, pb[0].w};
#pragma unroll
        for (int q = 1; q < NP; ++q) {
          a8[0] += pa[q].x; a8[1] += pa[q].y; a8[2] += pa[q].z; a8[3] += pa[q].w;
          a8[4] += pb[q].x; a8[5] += pb[q].y; a8[6] += pb[q].z; a8[7] += pb[q].w;
        }
        xv = make_uint4(E::bits(a8[0]) | (E::bits(a8[1]) << 16), E::bits(a8[2]) | (E::bits(a8[3]) << 16),
                        E::bits(a8[4]) | (E::bits(a8[5]) << 16), E::bits(a8[6]) | (E::bits(a8[7]) << 16));
      } else {
        xv = *(const uint4*)(x + base + 8 * g);
      }
      wv[k] = *(const uint4*)(w + 8 * g);
      const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
      if (res_in) {
        const uint4 rv = *(const uint4*)(res_in + base + 8 * g);
        const uint32_t rs[4] = {rv.x, rv.y, rv.z, rv.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h[k][2 * j] = E::rnd(E::lo(rs[j]) + E::lo(xs[j]));
          h[k][2 * j + 1] = E::rnd(E::hi(rs[j]) + E::hi(xs[j]));
          o[j] = E::bits(h[k][2 * j]) | (E::bits(h[k][2 * j + 1]) << 16);
        }
        *(uint4*)(res_out + base + 8 * g) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h[k][2 * j] = E::lo(xs[j]);
          h[k][2 * j + 1] = E::hi(xs[j]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(h[k][e], h[k][e], ss);
    }
  }
  __shared__ float red[kNormThreads / 64];
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float r = __frsqrt_rn(tot / (float)H + eps);
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    const int g = tid + k * kNormThreads;
    if (FULL || g < ng) {
      const uint32_t ws[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = E::rnd(E::lo(ws[j]) * E::rnd(h[k][2 * j] * r));
        const float b = E::rnd(E::hi(ws[j]) * E::rnd(h[k][2 * j + 1] * r));
        o[j] = E::bits(a) | (E::bits(b) << 16);
      }
      *(uint4*)(y + base + 8 * g) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

template <typename T, int NG>
void launch_rmsnorm(int rows, int H, hipStream_t s, const uint16_t* xi, const uint16_t* ri, uint16_t* ro,
                    const uint16_t* wi, uint16_t* yo, float eps) {
  if ((H / 8) % kNormThreads == 0)
    hipLaunchKernelGGL((rmsnorm_kernel<T, NG, true>), dim3(rows), dim3(kNormThreads), 0, s, xi, ri, ro, wi, yo, H,
                       eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, NG, false>), dim3(rows), dim3(kNormThreads), 0, s, xi, ri, ro, wi, yo,
                       H, eps);
}

template <typename T>
void launch_rmsnorm_t(int rows, int H, hipStream_t s, const uint16_t* xi, const uint16_t* ri, uint16_t* ro,
                      const uint16_t* wi, uint16_t* yo, float eps) {
  switch ((H / 8 + kNormThreads - 1) / kNormThreads) {
    case 1: launch_rmsnorm<T, 1>(rows, H, s, xi, ri, ro, wi, yo, eps); break;
    case 2: launch_rmsnorm<T, 2>(rows, H, s, xi, ri, ro, wi, yo, eps); break;
    case 3: launch_rmsnorm<T, 3>(rows, H, s, xi, ri, ro, wi, yo, eps); break;
    default: launch_rmsnorm<T, 4>(rows, H, s, xi, ri, ro, wi, yo, eps); break;
  }
}

// Rotary embedding of q (Hq heads) and k (Hk heads) with cos/sin [rows][D]: head h of
// row r is read at qi/ki + r * in_stride + h * D and written at qo/ko + (r * H + h) * D
// (in place when the pointers agree and in_stride = H * D); with vi/vo, the row's Hk v
// heads are copied the same way. One thread per (row, head, i < D/2) rotates the pair
// (i, i + D/2). Grid: rows x ceil((Hq + 2 Hk) * D/2 / 256).
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* qi, uint16_t* qo, const uint16_t* ki, uint16_t* ko,
                                                   const uint16_t* vi, uint16_t* vo, long q_stride, long k_stride,
                                                   long v_stride, const uint16_t* cs, const uint16_t* sn, int Hq,
                                                   int Hk, int D) {
  using E = G16<T>;
  const int row = blockIdx.x;
  const int half = D / 2;
  const int idx = blockIdx.y * 256 + threadIdx.x;
  const int nv = vi ? Hk : 0;
  if (idx >= (Hq + Hk + nv) * half) return;
  const int hd = idx / half, i = idx - hd * half;
  if (hd >= Hq + Hk) {  // v: copied
    const int h = hd - Hq - Hk;
    const uint16_t* src = vi + (long)row * v_stride + (long)h * D;
    uint16_t* dst = vo + ((long)row * Hk + h) * D;
    dst[i] = src[i];
    dst[i + half] = src[i + half];
    return;
  }
  const uint16_t* src;
  uint16_t* dst;
  if (hd < Hq) {
    src = qi + (long)row * q_stride + (long)hd * D;
    dst = qo + ((long)row * Hq + hd) * D;
  } else {
    src = ki + (long)row * k_stride + (long)(hd - Hq) * D;
    dst = ko + ((long)row * Hk + (hd - Hq)) * D;
  }
  auto ld = [](const uint16_t* p, int j) { return E::lo((uint32_t)p[j]); };
  const uint16_t* c = cs + (long)row * D;
  const uint16_t* s = sn + (long)row * D;
  const float a = ld(src, i), b = ld(src, i + half);
  float ya, yb;
  rope_pair<T>(a, b, ld(c, i), ld(s, i), ld(c, i + half), ld(s, i + half), ya, yb);
  dst[i] = (uint16_t)E::bits(ya);
  dst[i + half] = (uint16_t)E::bits(yb);
}

// m[r][j] = rnd(rnd(silu(g[r][j])) * u[r][j]) for rows r and j < F (F % 8 == 0): g and u rows
// in_stride elements apart, m dense; 8 elements per thread, grid ceil(rows * F / 8 / 256).
// With split = S > 1, m is [S][rows][F / S] instead (column j of row r at
// ((j / (F/S)) * rows + r) * (F/S) + j % (F/S)): the K slices of a split-K
// product with the next projection, each slice dense.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, const uint16_t* u, uint16_t* m, long n8,
                                                       int F8, long in_stride, long rows, int split) {
  using E = G16<T>;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const long r = i / F8, c = i - r * F8;
  long mo = 8 * i;
  if (split > 1) {
    const int fs8 = F8 / split;
    const long sl = c / fs8;
    mo = 8 * ((sl * rows + r) * fs8 + (c - sl * fs8));
  }
  const long io = r * in_stride + 8 * c;
  const uint4 gv = *(const uint4*)(g + io), uv = *(const uint4*)(u + io);
  const uint32_t gs[4] = {gv.x, gv.y, gv.z, gv.w}, us[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g0 = E::lo(gs[j]), g1 = E::hi(gs[j]);
    const float a = E::rnd(E::rnd(g0 / (1.f + expf(-g0))) * E::lo(us[j]));
    const float b = E::rnd(E::rnd(g1 / (1.f + expf(-g1))) * E::hi(us[j]));
    o[j] = E::bits(a) | (E::bits(b) << 16);
  }
  *(uint4*)(m + mo) = make_uint4(o[0], o[1], o[2], o[3]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

}  // namespace mentat

using namespace mentat;

extern "C" int mentat_rmsnorm(const void* x, const void* residual_in, void* residual_out, const void* weight, void* out,
                              int rows, int H, float eps, int dtype, void* stream) {
  if (rows < 0 || H <= 0) return MENTAT_EINVAL;
  if (rows == 0) return MENTAT_OK;
  if (!x || !weight || !out || (residual_in && !residual_out)) return MENTAT_EINVAL;
  if (H % 8 != 0 || H > 8 * kNormThreads * kNormGroups) return MENTAT_EUNSUP;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (residual_in && (!aligned16(residual_in) ||
                                                                               !aligned16(residual_out))))
    return MENTAT_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const auto* xi = (const uint16_t*)x;
  const auto* ri = (const uint16_t*)residual_in;
  auto* ro = (uint16_t*)residual_out;
  const auto* wi = (const uint16_t*)weight;
  auto* yo = (uint16_t*)out;
  switch (dtype) {
    case MENTAT_BF16:
      launch_rmsnorm_t<BF16>(rows, H, s, xi, ri, ro, wi, yo, eps);
      break;
    case MENTAT_F16:
      launch_rmsnorm_t<F16>(rows, H, s, xi, ri, ro, wi, yo, eps);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}

template <typename T, int NP>
static void launch_rmsnorm_parts(int rows, int H, hipStream_t s, const float* xp, const uint16_t* ri, uint16_t* ro,
                                 const uint16_t* wi, uint16_t* yo, float eps) {
  const long ps = (long)rows * H;
  switch ((H / 8 + kNormThreads - 1) / kNormThreads) {
#define MENTAT_NORM_PARTS(NGV)                                                                                   \
  if ((H / 8) % kNormThreads == 0)                                                                               \
    hipLaunchKernelGGL((rmsnorm_kernel<T, NGV, true, NP>), dim3(rows), dim3(kNormThreads), 0, s, nullptr, ri, ro, \
                       wi, yo, H, eps, xp, ps);                                                                  \
  else                                                                                                           \
    hipLaunchKernelGGL((rmsnorm_kernel<T, NGV, false, NP>), dim3(rows), dim3(kNormThreads), 0, s, nullptr, ri, ro, \
                       wi, yo, H, eps, xp, ps);
    case 1: MENTAT_NORM_PARTS(1) break;
    case 2: MENTAT_NORM_PARTS(2) break;
    case 3: MENTAT_NORM_PARTS(3) break;
    default: MENTAT_NORM_PARTS(4) break;
#undef MENTAT_NORM_PARTS
  }
}

template <typename T>
static int rmsnorm_parts_t(int n_parts, int rows, int H, hipStream_t s, const float* xp, const uint16_t* ri,
                           uint16_t* ro, const uint16_t* wi, uint16_t* yo, float eps) {
  switch (n_parts) {
    case 2: launch_rmsnorm_parts<T, 2>(rows, H, s, xp, ri, ro, wi, yo, eps); break;
    case 4: launch_rmsnorm_parts<T, 4>(rows, H, s, xp, ri, ro, wi, yo, eps); break;
    case 8: launch_rmsnorm_parts<T, 8>(rows, H, s, xp, ri, ro, wi, yo, eps); break;
    default: return MENTAT_EUNSUP;
  }
  return MENTAT_OK;
}

extern "C" int mentat_rmsnorm_partials(const float* parts, int n_parts, const void* residual_in, void* residual_out,
                                       const void* weight, void* out, int rows, int H, float eps, int dtype,
                                       void* stream) {
  if (rows < 0 || H <= 0 || n_parts < 1) return MENTAT_EINVAL;
  if (rows == 0) return MENTAT_OK;
  if (!parts || !weight || !out || (residual_in && !residual_out)) return MENTAT_EINVAL;
  if (H % 8 != 0 || H > 8 * kNormThreads * kNormGroups) return MENTAT_EUNSUP;
  if (!aligned16(parts) || !aligned16(weight) || !aligned16(out) ||
      (residual_in && (!aligned16(residual_in) || !aligned16(residual_out))))
    return MENTAT_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const auto* ri = (const uint16_t*)residual_in;
  auto* ro = (uint16_t*)residual_out;
  const auto* wi = (const uint16_t*)weight;
  auto* yo = (uint16_t*)out;
  int st;
  switch (dtype) {
    case MENTAT_BF16: st = rmsnorm_parts_t<BF16>(n_parts, rows, H, s, parts, ri, ro, wi, yo, eps); break;
    case MENTAT_F16: st = rmsnorm_parts_t<F16>(n_parts, rows, H, s, parts, ri, ro, wi, yo, eps); break;
    default: return MENTAT_EUNSUP;
  }
  if (st != MENTAT_OK) return st;
  return (int)hipGetLastError();
}

static int rope_launch(const void* qi, void* qo, const void* ki, void* ko, const void* vi, void* vo, int64_t qs,
                       int64_t ks, int64_t vs, const void* cos, const void* sin, int rows, int Hq, int Hk, int D,
                       int dtype, void* stream) {
  const int nh = Hq + Hk + (vi ? Hk : 0);
  const dim3 grid(rows, (nh * (D / 2) + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  const auto* c = (const uint16_t*)cos;
  const auto* sn = (const uint16_t*)sin;
  switch (dtype) {
    case MENTAT_BF16:
      hipLaunchKernelGGL(rope_kernel<BF16>, grid, dim3(256), 0, s, (const uint16_t*)qi, (uint16_t*)qo,
                         (const uint16_t*)ki, (uint16_t*)ko, (const uint16_t*)vi, (uint16_t*)vo, (long)qs, (long)ks,
                         (long)vs, c, sn, Hq, Hk, D);
      break;
    case MENTAT_F16:
      hipLaunchKernelGGL(rope_kernel<F16>, grid, dim3(256), 0, s, (const uint16_t*)qi, (uint16_t*)qo,
                         (const uint16_t*)ki, (uint16_t*)ko, (const uint16_t*)vi, (uint16_t*)vo, (long)qs, (long)ks,
                         (long)vs, c, sn, Hq, Hk, D);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}

extern "C" int mentat_rope(void* q, void* k, const void* cos, const void* sin, int rows, int Hq, int Hk, int D,
                           int dtype, void* stream) {
  if (rows < 0 || Hq < 0 || Hk < 0 || D <= 0 || D % 2 != 0) return MENTAT_EINVAL;
  if (rows == 0 || Hq + Hk == 0) return MENTAT_OK;
  if ((Hq && !q) || (Hk && !k) || !cos || !sin) return MENTAT_EINVAL;
  return rope_launch(q, q, k, k, nullptr, nullptr, (int64_t)Hq * D, (int64_t)Hk * D, 0, cos, sin, rows, Hq, Hk, D,
                     dtype, stream);
}

extern "C" int mentat_rope_qkv(const void* qkv, int64_t row_stride, void* q, void* k, void* v, const void* cos,
                               const void* sin, int rows, int Hq, int Hk, int D, int dtype, void* stream) {
  if (rows < 0 || Hq <= 0 || Hk <= 0 || D <= 0 || D % 2 != 0 || row_stride < (int64_t)(Hq + 2 * Hk) * D)
    return MENTAT_EINVAL;
  if (rows == 0) return MENTAT_OK;
  if (!qkv || !q || !k || !v || !cos || !sin) return MENTAT_EINVAL;
  const auto* b = (const uint16_t*)qkv;
  return rope_launch(b, q, b + (long)Hq * D, k, b + (long)(Hq + Hk) * D, v, row_stride, row_stride, row_stride, cos,
                     sin, rows, Hq, Hk, D, dtype, stream);
}

extern "C" int mentat_silu_mul(const void* gate, const void* up, void* out, int rows, int F, int64_t in_row_stride,
                               int dtype, void* stream) {
  if (rows < 0 || F < 0 || in_row_stride < F) return MENTAT_EINVAL;
  if (rows == 0 || F == 0) return MENTAT_OK;
  if (!gate || !up || !out) return MENTAT_EINVAL;
  if (F % 8 != 0 || in_row_stride % 8 != 0 || !aligned16(gate) || !aligned16(up) || !aligned16(out))
    return MENTAT_EUNSUP;
  hipStream_t s = (hipStream_t)stream;
  const long n8 = (long)rows * (F / 8);
  const dim3 grid((unsigned)((n8 + 255) / 256));
  switch (dtype) {
    case MENTAT_BF16:
      hipLaunchKernelGGL(silu_mul_kernel<BF16>, grid, dim3(256), 0, s, (const uint16_t*)gate, (const uint16_t*)up,
                         (uint16_t*)out, n8, F / 8, (long)in_row_stride, (long)rows, 1);
      break;
    case MENTAT_F16:
      hipLaunchKernelGGL(silu_mul_kernel<F16>, grid, dim3(256), 0, s, (const uint16_t*)gate, (const uint16_t*)up,
                         (uint16_t*)out, n8, F / 8, (long)in_row_stride, (long)rows, 1);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}

extern "C" int mentat_silu_mul_split(const void* gate, const void* up, void* out, int rows, int F, int64_t in_row_stride,
                                     int split, int dtype, void* stream) {
  if (rows < 0 || F < 0 || in_row_stride < F || split < 1) return MENTAT_EINVAL;
  if (rows == 0 || F == 0) return MENTAT_OK;
  if (!gate || !up || !out) return MENTAT_EINVAL;
  if (F % (8 * split) != 0 || in_row_stride % 8 != 0 || !aligned16(gate) || !aligned16(up) || !aligned16(out))
    return MENTAT_EUNSUP;
  hipStream_t s = (hipStream_t)stream;
  const long n8 = (long)rows * (F / 8);
  const dim3 grid((unsigned)((n8 + 255) / 256));
  switch (dtype) {
    case MENTAT_BF16:
      hipLaunchKernelGGL(silu_mul_kernel<BF16>, grid, dim3(256), 0, s, (const uint16_t*)gate, (const uint16_t*)up,
                         (uint16_t*)out, n8, F / 8, (long)in_row_stride, (long)rows, split);
      break;
    case MENTAT_F16:
      hipLaunchKernelGGL(silu_mul_kernel<F16>, grid, dim3(256), 0, s, (const uint16_t*)gate, (const uint16_t*)up,
                         (uint16_t*)out, n8, F / 8, (long)in_row_stride, (long)rows, split);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}
