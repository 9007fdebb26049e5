// Softmax cross-entropy over f32 logits, for gfx950.
//
// Reference: src/ferrite/model/gpt.py:147-152 (loss_fn: log_softmax in f32,
// negative log-likelihood of the target, mean over tokens) and its autodiff
// backward, d logits = (softmax - onehot(target)) * dloss / N.
//
// HBM-bound on the [N, V] logits (1 GiB at N = 8192, V = 32768): the forward
// reads them once, keeping an online (max, sum of exp) pair per thread, and
// writes only the per-row logsumexp and loss; the backward reads them once
// more and writes the gradient directly in the dtype its consumer (the LM-head
// products) reads. Neither materialises log-probabilities or a one-hot.
#include <math.h>

#include "common.h"

namespace ferrite {
namespace {

constexpr int kCeThreads = 256;

// Merge two (max, sum of exp(x - max)) pairs.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  if (m2 > m) {
    s = s * __expf(m - m2) + s2;
    m = m2;
  } else if (m2 > -INFINITY) {
    s += s2 * __expf(m2 - m);
  }
}

__device__ __forceinline__ void ms_add(float& m, float& s, float x) {
  if (x > m) {
    s = s * __expf(m - x) + 1.f;
    m = x;
  } else if (x > -INFINITY) {  // (-inf) - (-inf) would be NaN
    s += __expf(x - m);
  }
}

// One workgroup per row: lse[row] = max + log(sum exp(x - max)), loss[row] = lse - x[target].
// VEC: the row is 16-byte aligned and V % 4 == 0 (f32x4 loads).
template <bool VEC>
__global__ __launch_bounds__(kCeThreads) void ce_fwd_kernel(const float* __restrict__ logits,
                                                           const int64_t* __restrict__ targets,
                                                           float* __restrict__ loss, float* __restrict__ lse,
                                                           int64_t V) {
  __shared__ float sm[kCeThreads / 64], ss[kCeThreads / 64];
  const int64_t row = blockIdx.x;
  const float* x = logits + row * V;
  float m = -INFINITY, s = 0.f;
  if constexpr (VEC) {
    const int64_t nv = V / 4;
    for (int64_t i = threadIdx.x; i < nv; i += kCeThreads) {
      const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x) + i);
      ms_add(m, s, v[0]);
      ms_add(m, s, v[1]);
      ms_add(m, s, v[2]);
      ms_add(m, s, v[3]);
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kCeThreads) ms_add(m, s, x[i]);
  }
  // wave, then workgroup merge (fixed order)
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
    ms_merge(m, s, m2, s2);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[wave] = m;
    ss[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int w = 1; w < kCeThreads / 64; ++w) ms_merge(M, S, sm[w], ss[w]);
    const float l = M + logf(S);
    lse[row] = l;
    const int64_t t = targets[row];
    loss[row] = (t >= 0 && t < V) ? l - x[t] : NAN;
  }
}

// grad[row, j] = (exp(x - lse[row]) - [j == target]) * (*dloss) * scale.
template <typename TO, bool VEC>
__global__ __launch_bounds__(kCeThreads) void ce_bwd_kernel(const float* __restrict__ logits,
                                                           const int64_t* __restrict__ targets,
                                                           const float* __restrict__ lse,
                                                           const float* __restrict__ dloss, float scale,
                                                           TO* __restrict__ grad, int64_t V) {
  const int64_t row = blockIdx.x;
  const float* x = logits + row * V;
  TO* gr = grad + row * V;
  const float l = lse[row];
  const float c = *dloss * scale;
  const int64_t t = targets[row];
  if constexpr (VEC) {
    const int64_t nv = V / 4;
    for (int64_t i = threadIdx.x; i < nv; i += kCeThreads) {
      const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x) + i);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (__expf(v[e] - l) - (4 * i + e == t ? 1.f : 0.f)) * c;
      if constexpr (sizeof(TO) == 2) {
        *reinterpret_cast<bf16x4*>(gr + 4 * i) = bf16x4{(bf16)o[0], (bf16)o[1], (bf16)o[2], (bf16)o[3]};
      } else {
        *reinterpret_cast<f32x4*>(gr + 4 * i) = f32x4{o[0], o[1], o[2], o[3]};
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kCeThreads)
      gr[i] = Elem<TO>::from_f32((__expf(x[i] - l) - (i == t ? 1.f : 0.f)) * c);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace ferrite

extern "C" int ferrite_hip_cross_entropy_fwd(const float* logits, const int64_t* targets, float* loss, float* lse,
                                             int64_t n, int64_t v, void* stream) {
  using namespace ferrite;
  if (n < 0 || v < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_fwd: need n >= 0, v >= 1");
  if (n > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_fwd: too many rows");
  if (n == 0) return FERRITE_OK;
  if (!logits || !targets || !loss || !lse)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_fwd: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (v % 4 == 0 && aligned16(logits))
    hipLaunchKernelGGL((ce_fwd_kernel<true>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets, loss, lse, v);
  else
    hipLaunchKernelGGL((ce_fwd_kernel<false>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets, loss, lse,
                       v);
  return check_launch("ferrite_cross_entropy_fwd");
}

extern "C" int ferrite_hip_cross_entropy_bwd(const float* logits, const int64_t* targets, const float* lse,
                                             const float* dloss, float scale, void* grad, int64_t n, int64_t v,
                                             int grad_dtype, void* stream) {
  using namespace ferrite;
  if (!valid_dtype(grad_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_bwd: dtype must be FERRITE_F32 or FERRITE_BF16");
  if (n < 0 || v < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_bwd: need n >= 0, v >= 1");
  if (n > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_bwd: too many rows");
  if (n == 0) return FERRITE_OK;
  if (!logits || !targets || !lse || !dloss || !grad)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_cross_entropy_bwd: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = v % 4 == 0 && aligned16(logits) && aligned16(grad);
  if (grad_dtype == FERRITE_BF16) {
    bf16* g = static_cast<bf16*>(grad);
    if (vec)
      hipLaunchKernelGGL((ce_bwd_kernel<bf16, true>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets, lse,
                         dloss, scale, g, v);
    else
      hipLaunchKernelGGL((ce_bwd_kernel<bf16, false>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets,
                         lse, dloss, scale, g, v);
  } else {
    float* g = static_cast<float*>(grad);
    if (vec)
      hipLaunchKernelGGL((ce_bwd_kernel<float, true>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets,
                         lse, dloss, scale, g, v);
    else
      hipLaunchKernelGGL((ce_bwd_kernel<float, false>), dim3((unsigned)n), dim3(kCeThreads), 0, s, logits, targets,
                         lse, dloss, scale, g, v);
  }
  return check_launch("ferrite_cross_entropy_bwd");
}
