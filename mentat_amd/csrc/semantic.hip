// Semantic-diversity prune on the device (gfx950): the per-step EMA of every
// live leaf's semantic vector in one launch, and the pairwise cosine
// similarity mask of the prune candidates in two launches.
//
// Reference: core/generator.py:376-398 (_update_semantic_vectors: a new leaf
// clones its hidden state, an existing one does v.mul_(1 - alpha).add_(h,
// alpha=alpha) in the model dtype) and :400-460 (_prune_similar:
// F.normalize(stack(v), p=2, dim=1), sim = mm(vn, vn^T), upper triangle,
// sibling pairs masked, sim > threshold).
//
// Rounding follows torch's kernels for 16-bit tensors (float arithmetic,
// one rounding per op): mul_ rounds x*(1-alpha); add_ rounds
// fma(alpha, h, that); the norm is the float norm rounded; clamp_min(1e-12)
// is taken in float and rounded; the division is a float divide rounded; the
// product matrix is a float dot product rounded to the dtype, compared with
// the threshold rounded to the dtype (torch converts the scalar operand of a
// comparison to the tensor's dtype). Only the float summation order of the norm and
// the dot product differs from the library routines.
#include "mentat_common.h"

namespace mentat {

namespace {

template <typename T> struct SemElem;
template <> struct SemElem<BF16> {
  __device__ static float ld(const void* p, long i) { return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16); }
  __device__ static void st(void* p, long i, float v) { ((uint16_t*)p)[i] = f32_to_bf16(v); }
  __device__ static float rnd(float v) { return __uint_as_float((uint32_t)f32_to_bf16(v) << 16); }
};
// The empty asm makes the float value exist before it is narrowed: without it the
// compiler may fuse the float op and the narrowing into one mixed-precision
// instruction that rounds once, where torch's kernels round to float first.
template <> struct SemElem<F16> {
  __device__ static float ld(const void* p, long i) { return f16_bits_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void st(void* p, long i, float v) {
    asm volatile("" : "+v"(v));
    ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  }
  __device__ static float rnd(float v) {
    asm volatile("" : "+v"(v));
    return f16_bits_to_f32(f32_to_f16_bits(v));
  }
};
template <> struct SemElem<F32> {
  __device__ static float ld(const void* p, long i) { return ((const float*)p)[i]; }
  __device__ static void st(void* p, long i, float v) { ((float*)p)[i] = v; }
  __device__ static float rnd(float v) { return v; }
};

constexpr int kSemThreads = 256;

// Row i: dst[i] <- h[i] (init[i] != 0) or rnd(fma(add_scale, h, rnd(dst * mul_scale))).
template <typename T>
__global__ __launch_bounds__(kSemThreads) void semantic_ema_kernel(const int64_t* dst_ptrs, const void* hidden,
                                                                   const int32_t* init, int H, long h_stride,
                                                                   float mul_scale, float add_scale) {
  using E = SemElem<T>;
  const int i = blockIdx.x;
  void* dst = (void*)dst_ptrs[i];
  const bool fresh = init[i] != 0;
  const long hb = (long)i * h_stride;
  for (int k = threadIdx.x; k < H; k += kSemThreads) {
    const float h = E::ld(hidden, hb + k);
    float v;
    if (fresh) {
      v = h;
    } else {
      const float x = E::rnd(E::ld(dst, k) * mul_scale);
      v = __builtin_fmaf(add_scale, h, x);
    }
    E::st(dst, k, v);
  }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int k = 0; k < kSemThreads / 64; ++k) s += red[k];
  return s;
}

// Row i of the candidates: scratch[i] <- rnd(v / rnd(max(rnd(||v||), 1e-12))).
template <typename T>
__global__ __launch_bounds__(kSemThreads) void semantic_normalize_kernel(const int64_t* ptrs, int H, void* scratch) {
  using E = SemElem<T>;
  __shared__ float red[kSemThreads / 64];
  const int i = blockIdx.x;
  const void* src = (const void*)ptrs[i];
  float ss = 0.f;
  for (int k = threadIdx.x; k < H; k += kSemThreads) {
    const float x = E::ld(src, k);
    ss = __builtin_fmaf(x, x, ss);
  }
  const float norm = E::rnd(__builtin_sqrtf(block_sum(ss, red)));
  const float denom = E::rnd(fmaxf(norm, 1e-12f));
  for (int k = threadIdx.x; k < H; k += kSemThreads) E::st(scratch, (long)i * H + k, E::ld(src, k) / denom);
}

// mask[i][j] = 1 iff i < j, group[i] == group[j], parent_key[i] != parent_key[j]
// and rnd(dot(n_i, n_j)) > rnd(threshold); one workgroup per row i, one wavefront per j.
template <typename T>
__global__ __launch_bounds__(kSemThreads) void semantic_similar_kernel(const void* scratch, const int32_t* parent_key,
                                                                       const int32_t* group, int M, int H,
                                                                       float threshold, uint8_t* mask) {
  using E = SemElem<T>;
  const int i = blockIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float thr = E::rnd(threshold);  // torch compares in the tensor's dtype: the scalar is rounded to it
  for (int j = w; j < M; j += kSemThreads / 64) {
    bool keep = j > i && group[j] == group[i] && parent_key[j] != parent_key[i];
    if (keep) {
      float d = 0.f;
      for (int k = lane; k < H; k += 64)
        d = __builtin_fmaf(E::ld(scratch, (long)i * H + k), E::ld(scratch, (long)j * H + k), d);
      for (int o = 32; o >= 1; o >>= 1) d += __shfl_xor(d, o);
      keep = E::rnd(d) > thr;
    }
    if (lane == 0) mask[(long)i * M + j] = keep ? 1 : 0;
  }
}

}  // namespace

}  // namespace mentat

using namespace mentat;

extern "C" int mentat_semantic_ema(const int64_t* dst_ptrs, const void* hidden, const int32_t* init, int n, int H,
                                   int64_t hidden_stride, float mul_scale, float add_scale, int dtype, void* stream) {
  if (n < 0 || H <= 0 || hidden_stride < H) return MENTAT_EINVAL;
  if (n == 0) return 0;
  if (!dst_ptrs || !hidden || !init) return MENTAT_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16:
      hipLaunchKernelGGL(semantic_ema_kernel<BF16>, dim3(n), dim3(kSemThreads), 0, s, dst_ptrs, hidden, init, H,
                         (long)hidden_stride, mul_scale, add_scale);
      break;
    case MENTAT_F16:
      hipLaunchKernelGGL(semantic_ema_kernel<F16>, dim3(n), dim3(kSemThreads), 0, s, dst_ptrs, hidden, init, H,
                         (long)hidden_stride, mul_scale, add_scale);
      break;
    case MENTAT_F32:
      hipLaunchKernelGGL(semantic_ema_kernel<F32>, dim3(n), dim3(kSemThreads), 0, s, dst_ptrs, hidden, init, H,
                         (long)hidden_stride, mul_scale, add_scale);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}

extern "C" int mentat_semantic_similar(const int64_t* ptrs, const int32_t* parent_key, const int32_t* group, int M,
                                       int H, float threshold, int dtype, void* scratch, size_t scratch_bytes,
                                       uint8_t* mask, void* stream) {
  if (M < 0 || H <= 0) return MENTAT_EINVAL;
  if (M == 0) return 0;
  if (!ptrs || !parent_key || !group || !scratch || !mask) return MENTAT_EINVAL;
  const size_t esz = dtype == MENTAT_F32 ? 4 : 2;
  if (scratch_bytes < (size_t)M * H * esz) return MENTAT_ESPACE;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MENTAT_BF16:
      hipLaunchKernelGGL(semantic_normalize_kernel<BF16>, dim3(M), dim3(kSemThreads), 0, s, ptrs, H, scratch);
      hipLaunchKernelGGL(semantic_similar_kernel<BF16>, dim3(M), dim3(kSemThreads), 0, s, (const void*)scratch,
                         parent_key, group, M, H, threshold, mask);
      break;
    case MENTAT_F16:
      hipLaunchKernelGGL(semantic_normalize_kernel<F16>, dim3(M), dim3(kSemThreads), 0, s, ptrs, H, scratch);
      hipLaunchKernelGGL(semantic_similar_kernel<F16>, dim3(M), dim3(kSemThreads), 0, s, (const void*)scratch,
                         parent_key, group, M, H, threshold, mask);
      break;
    case MENTAT_F32:
      hipLaunchKernelGGL(semantic_normalize_kernel<F32>, dim3(M), dim3(kSemThreads), 0, s, ptrs, H, scratch);
      hipLaunchKernelGGL(semantic_similar_kernel<F32>, dim3(M), dim3(kSemThreads), 0, s, (const void*)scratch,
                         parent_key, group, M, H, threshold, mask);
      break;
    default:
      return MENTAT_EUNSUP;
  }
  return (int)hipGetLastError();
}
