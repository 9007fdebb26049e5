// Fused AdamW step over a list of parameter tensors, for gfx950.
//
// Reference: src/ferrite/model/train.py:59-74 (adamw_update), which XLA runs as
// fusions over the parameter tree:
//   gnorm = sqrt(sum over all tensors of sum(g^2));  scale = min(1, clip / (gnorm + 1e-6))
//   g = g * scale
//   m = b1 * m + (1 - b1) * g;   v = b2 * v + (1 - b2) * g * g
//   p = p - lr * ((m / bc1) / (sqrt(v / bc2) + eps) + decay * p)
// with decay = weight_decay for tensors of rank >= 2, else 0.
//
// HBM-bound: per element the update reads g, p, m, v and writes p, m, v once
// (22 bytes for bf16 p/g with f32 moments), after one read of g for the norm.
// Three kernels, no host synchronisation: per-block partial sums of g^2, one
// block that sums them in a fixed order (deterministic) into the norm and the
// clip scale, and the element-wise update that reads the scale from device
// memory. Tensor pointers travel in the kernel arguments, up to
// kAdamGroup tensors per launch, so a step needs no device-side tables.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace ferrite {
namespace {

constexpr int kAdamGroup = 32;                // tensors per launch (kernel-argument table)
constexpr int kAdamThreads = 256;
constexpr int kAdamTile = kAdamThreads * 8;   // elements per block iteration (8 per thread)
constexpr int kAdamNormBlocks = 2048;         // partial sums per group (enough loads in flight to stream g)

struct AdamGroup {
  void* p[kAdamGroup];
  const void* g[kAdamGroup];
  float* m[kAdamGroup];
  float* v[kAdamGroup];
  int64_t n[kAdamGroup];
  int64_t tile0[kAdamGroup + 1];  // prefix sums of tiles per tensor
  float decay[kAdamGroup];        // weight_decay or 0 per tensor
  uint32_t aligned;               // bit i: tensor i's four pointers are 16-byte aligned
  int count;
};

// The tensor holding tile t (tile0 is increasing; the loop is wave-uniform).
__device__ __forceinline__ int tensor_of(const AdamGroup& grp, int64_t t) {
  int i = 0;
  while (i + 1 < grp.count && grp.tile0[i + 1] <= t) ++i;
  return i;
}

__device__ __forceinline__ void load8f(const bf16* p, float* o) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (float)v[e];
}
__device__ __forceinline__ void load8f(const float* p, float* o) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = a[e];
    o[4 + e] = b[e];
  }
}
__device__ __forceinline__ void store8f(bf16* p, const float* x) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (bf16)x[e];
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ __forceinline__ void store8f(float* p, const float* x) {
  *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
}

// Block-wide sum (256 threads), result valid in every thread.
__device__ __forceinline__ float block_sum(float x, float* lds) {
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[wave] = x;
  __syncthreads();
  return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

template <typename TG>
__global__ __launch_bounds__(kAdamThreads) void adamw_sqnorm_kernel(AdamGroup grp, float* __restrict__ partial) {
  __shared__ float lds[4];
  const int64_t total = grp.tile0[grp.count];
  float acc = 0.f;
  for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
    const int i = tensor_of(grp, t);
    const TG* g = static_cast<const TG*>(grp.g[i]);
    const int64_t e0 = (t - grp.tile0[i]) * kAdamTile + threadIdx.x * 8;
    const int64_t n = grp.n[i];
    if (((grp.aligned >> i) & 1) && e0 + 8 <= n) {
      float x[8];
      load8f(g + e0, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += x[e] * x[e];
    } else {
      for (int64_t e = e0; e < std::min<int64_t>(e0 + 8, n); ++e) {
        const float x = Elem<TG>::to_f32(g[e]);
        acc += x * x;
      }
    }
  }
  acc = block_sum(acc, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = acc;
}

// One block: norm = sqrt(sum of the partials), summed in a fixed order; the
// clip scale goes next to the partials for the update kernels.
__global__ __launch_bounds__(kAdamThreads) void adamw_finalize_kernel(const float* __restrict__ partial, int nparts,
                                                                     float max_norm, float* __restrict__ scale_out,
                                                                     float* __restrict__ norm_out) {
  __shared__ float lds[4];
  float acc = 0.f;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) acc += partial[i];
  acc = block_sum(acc, lds);
  if (threadIdx.x == 0) {
    const float norm = sqrtf(acc);
    const float scale = fminf(1.0f, max_norm / (norm + 1e-6f));
    *scale_out = scale;
    if (norm_out) *norm_out = norm;
  }
}

struct AdamHyper {
  float lr, b1, one_minus_b1, b2, one_minus_b2, eps, bc1, bc2;
};

template <typename TP>
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, float decay, const AdamHyper& hp) {
  m = hp.b1 * m + hp.one_minus_b1 * g;
  v = hp.b2 * v + hp.one_minus_b2 * g * g;
  p = p - hp.lr * ((m / hp.bc1) / (sqrtf(v / hp.bc2) + hp.eps) + decay * p);
}

template <typename TP, typename TG>
__global__ __launch_bounds__(kAdamThreads) void adamw_update_kernel(AdamGroup grp, const float* __restrict__ scale_ptr,
                                                                   AdamHyper hp, const float* __restrict__ step_scalars) {
  const float scale = *scale_ptr;
  if (step_scalars) {  // per-step values from device memory (a captured graph replays fixed arguments)
    hp.lr = step_scalars[0];
    hp.bc1 = step_scalars[1];
    hp.bc2 = step_scalars[2];
  }
  const int64_t total = grp.tile0[grp.count];
  for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
    const int i = tensor_of(grp, t);
    TP* p = static_cast<TP*>(grp.p[i]);
    const TG* g = static_cast<const TG*>(grp.g[i]);
    float* m = grp.m[i];
    float* v = grp.v[i];
    const float decay = grp.decay[i];
    const int64_t e0 = (t - grp.tile0[i]) * kAdamTile + threadIdx.x * 8;
    const int64_t n = grp.n[i];
    if (((grp.aligned >> i) & 1) && e0 + 8 <= n) {
      float pv[8], gv[8], mv[8], vv[8];
      load8f(p + e0, pv);
      load8f(g + e0, gv);
      load8f(m + e0, mv);
      load8f(v + e0, vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) adam_elem<TP>(pv[e], gv[e] * scale, mv[e], vv[e], decay, hp);
      store8f(p + e0, pv);
      store8f(m + e0, mv);
      store8f(v + e0, vv);
    } else {
      for (int64_t e = e0; e < std::min<int64_t>(e0 + 8, n); ++e) {
        float pe = Elem<TP>::to_f32(p[e]), me = m[e], ve = v[e];
        adam_elem<TP>(pe, Elem<TG>::to_f32(g[e]) * scale, me, ve, decay, hp);
        p[e] = Elem<TP>::from_f32(pe);
        m[e] = me;
        v[e] = ve;
      }
    }
  }
}

inline bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

int64_t adam_groups(int64_t n) { return cdiv(n, kAdamGroup); }

// Fill the kernel-argument table of tensors [first, first + count).
AdamGroup make_group(int64_t first, int count, void* const* params, const void* const* grads, float* const* m,
                     float* const* v, const int64_t* numel, const int32_t* decay, float weight_decay) {
  AdamGroup grp{};
  grp.count = count;
  grp.tile0[0] = 0;
  for (int j = 0; j < count; ++j) {
    const int64_t i = first + j;
    grp.p[j] = params[i];
    grp.g[j] = grads[i];
    grp.m[j] = m[i];
    grp.v[j] = v[i];
    grp.n[j] = numel[i];
    grp.decay[j] = decay[i] ? weight_decay : 0.f;
    grp.tile0[j + 1] = grp.tile0[j] + cdiv(numel[i], kAdamTile);
    if (al16(params[i]) && al16(grads[i]) && al16(m[i]) && al16(v[i])) grp.aligned |= 1u << j;
  }
  return grp;
}

template <typename TP, typename TG>
int adamw_launch(int64_t nt, void* const* params, const void* const* grads, float* const* m, float* const* v,
                 const int64_t* numel, const int32_t* decay, const AdamHyper& hp, const float* step_scalars,
                 float weight_decay, float max_norm, float* norm_out, float* ws, hipStream_t stream) {
  const int64_t ng = adam_groups(nt);
  float* partial = ws;
  float* scale = ws + ng * kAdamNormBlocks;
  for (int64_t gi = 0; gi < ng; ++gi) {
    const int count = (int)std::min<int64_t>(kAdamGroup, nt - gi * kAdamGroup);
    const AdamGroup grp = make_group(gi * kAdamGroup, count, params, grads, m, v, numel, decay, weight_decay);
    // Every block writes its partial (zero when it has no tile), so the
    // finalize kernel sums exactly ng * kAdamNormBlocks values.
    hipLaunchKernelGGL((adamw_sqnorm_kernel<TG>), dim3(kAdamNormBlocks), dim3(kAdamThreads), 0, stream, grp,
                       partial + gi * kAdamNormBlocks);
  }
  hipLaunchKernelGGL(adamw_finalize_kernel, dim3(1), dim3(kAdamThreads), 0, stream, partial,
                     (int)(ng * kAdamNormBlocks), max_norm, scale, norm_out);
  for (int64_t gi = 0; gi < ng; ++gi) {
    const int count = (int)std::min<int64_t>(kAdamGroup, nt - gi * kAdamGroup);
    const AdamGroup grp = make_group(gi * kAdamGroup, count, params, grads, m, v, numel, decay, weight_decay);
    const int64_t tiles = grp.tile0[count];
    if (tiles == 0) continue;
    const unsigned blocks = (unsigned)std::min<int64_t>(tiles, 2048);
    hipLaunchKernelGGL((adamw_update_kernel<TP, TG>), dim3(blocks), dim3(kAdamThreads), 0, stream, grp, scale, hp,
                       step_scalars);
  }
  return check_launch("ferrite_adamw");
}

}  // namespace
}  // namespace ferrite

extern "C" int64_t ferrite_hip_adamw_workspace(int64_t n_tensors) {
  if (n_tensors < 0) return -1;
  return (ferrite::adam_groups(n_tensors) * ferrite::kAdamNormBlocks + 4) * (int64_t)sizeof(float);
}

extern "C" int ferrite_hip_adamw(int64_t n_tensors, void* const* params, const void* const* grads,
                                 float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                                 const int32_t* decay, int param_dtype, int grad_dtype, float lr, float beta1,
                                 float beta2, float eps, float weight_decay, float max_grad_norm, int64_t step,
                                 const float* step_scalars, float* grad_norm, void* workspace, void* stream) {
  using namespace ferrite;
  const char* name = "ferrite_hip_adamw";
  if (!valid_dtype(param_dtype) || !valid_dtype(grad_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (n_tensors < 0 || (step < 1 && !step_scalars))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need n_tensors >= 0 and step >= 1");
  if (!workspace || (n_tensors > 0 && (!params || !grads || !exp_avg || !exp_avg_sq || !numel || !decay)))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  for (int64_t i = 0; i < n_tensors; ++i) {
    if (numel[i] < 0) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": negative numel");
    if (numel[i] > 0 && (!params[i] || !grads[i] || !exp_avg[i] || !exp_avg_sq[i]))
      return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null tensor pointer");
  }
  // Bias corrections 1 - beta^step, evaluated in double and rounded once.
  AdamHyper hp;
  hp.lr = lr;
  hp.b1 = beta1;
  hp.one_minus_b1 = (float)(1.0 - (double)beta1);
  hp.b2 = beta2;
  hp.one_minus_b2 = (float)(1.0 - (double)beta2);
  hp.eps = eps;
  hp.bc1 = step_scalars ? 1.f : (float)(1.0 - pow((double)beta1, (double)step));
  hp.bc2 = step_scalars ? 1.f : (float)(1.0 - pow((double)beta2, (double)step));
  float* ws = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define FERRITE_ADAMW_LAUNCH(TP, TG)                                                                           \
  return adamw_launch<TP, TG>(n_tensors, params, grads, exp_avg, exp_avg_sq, numel, decay, hp, step_scalars,   \
                              weight_decay, max_grad_norm, grad_norm, ws, s)
  if (param_dtype == FERRITE_BF16) {
    if (grad_dtype == FERRITE_BF16) FERRITE_ADAMW_LAUNCH(bf16, bf16);
    FERRITE_ADAMW_LAUNCH(bf16, float);
  }
  if (grad_dtype == FERRITE_BF16) FERRITE_ADAMW_LAUNCH(float, bf16);
  FERRITE_ADAMW_LAUNCH(float, float);
#undef FERRITE_ADAMW_LAUNCH
}
