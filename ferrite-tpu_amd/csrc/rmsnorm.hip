// Fused residual-add + RMSNorm and plain RMSNorm for gfx950.
//
// Reference: src/ferrite/kernels/rmsnorm.py:39-56 (kernel bodies) and :77-110
// (_call: row blocking and padding). The reference pads rows to a block multiple
// and the feature dim to a multiple of 128, then slices back. Here each wave
// owns whole rows and predicates its loads and stores, which gives the same
// values without the copies.
//
// Memory-bound: per row it reads x, residual (and the weight, which stays in
// L2) once and writes h and y once. Each lane holds 8-element chunks of the row
// in registers between the sum-of-squares reduction and the output pass, so the
// kernel is a single HBM pass. Statistics are f32 whatever the storage type:
//   h   = f32(x) + f32(residual)            (stored rounded to x's dtype)
//   inv = rsqrt(sum(h*h) * (1/dim) + eps)
//   y   = (h * inv) * f32(w)                (from the unrounded f32 h)
#include "common.h"

namespace ferrite {
namespace {

constexpr int kChunk = 8;         // elements per lane per chunk
constexpr int kRowsPerBlock = 4;  // one wave per row, 4 waves per workgroup

__device__ __forceinline__ void load8(const bf16* p, float* out) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}
__device__ __forceinline__ void load8(const float* p, float* out) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = a[e];
    out[4 + e] = b[e];
  }
}
__device__ __forceinline__ void store8(bf16* p, const float* in) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (bf16)in[e];
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ __forceinline__ void store8(float* p, const float* in) {
  f32x4 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = in[e];
    b[e] = in[4 + e];
  }
  *reinterpret_cast<f32x4*>(p) = a;
  *reinterpret_cast<f32x4*>(p + 4) = b;
}

// Fast path: dim % 8 == 0, 16-byte aligned rows, dim <= 64 * 8 * VPL. Lane l
// owns chunks c = l + 64 * i (i < VPL) of its row.
template <typename TX, typename TW, bool RES, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const TX* __restrict__ x, const TX* __restrict__ r,
                                                          const TW* __restrict__ w, TX* __restrict__ h,
                                                          TX* __restrict__ y, int64_t rows, int dim, float inv_dim,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * dim;
  const int nchunks = dim / kChunk;

  float hv[VPL][kChunk];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) {
      float xv[kChunk];
      load8(x + base + c * kChunk, xv);
      if constexpr (RES) {
        float rv[kChunk];
        load8(r + base + c * kChunk, rv);
#pragma unroll
        for (int e = 0; e < kChunk; ++e) hv[i][e] = xv[e] + rv[e];
      } else {
#pragma unroll
        for (int e = 0; e < kChunk; ++e) hv[i][e] = xv[e];
      }
#pragma unroll
      for (int e = 0; e < kChunk; ++e) ss += hv[i][e] * hv[i][e];
    }
  }
  if constexpr (RES) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunks) store8(h + base + c * kChunk, hv[i]);
    }
  }
  ss = wave_sum(ss);
  const float inv = __builtin_amdgcn_rsqf(ss * inv_dim + eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) {
      float wv[kChunk], yv[kChunk];
      load8(w + c * kChunk, wv);
#pragma unroll
      for (int e = 0; e < kChunk; ++e) yv[e] = (hv[i][e] * inv) * wv[e];
      store8(y + base + c * kChunk, yv);
    }
  }
}

// General path: any dim and alignment. Two sweeps over the row; the second
// recomputes h = x + r from the same inputs (bitwise the same f32 values).
template <typename TX, typename TW, bool RES>
__global__ __launch_bounds__(256) void rmsnorm_rows_generic_kernel(const TX* __restrict__ x, const TX* __restrict__ r,
                                                                  const TW* __restrict__ w, TX* __restrict__ h,
                                                                  TX* __restrict__ y, int64_t rows, int64_t dim,
                                                                  float inv_dim, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * dim;
  float ss = 0.f;
  for (int64_t e = lane; e < dim; e += 64) {
    float hv = Elem<TX>::to_f32(x[base + e]);
    if constexpr (RES) {
      hv += Elem<TX>::to_f32(r[base + e]);
      h[base + e] = Elem<TX>::from_f32(hv);
    }
    ss += hv * hv;
  }
  ss = wave_sum(ss);
  const float inv = __builtin_amdgcn_rsqf(ss * inv_dim + eps);
  for (int64_t e = lane; e < dim; e += 64) {
    float hv = Elem<TX>::to_f32(x[base + e]);
    if constexpr (RES) hv += Elem<TX>::to_f32(r[base + e]);
    y[base + e] = Elem<TX>::from_f32((hv * inv) * Elem<TW>::to_f32(w[e]));
  }
}

template <typename TX, typename TW, bool RES>
int launch(const void* x, const void* r, const void* w, void* h, void* y, int64_t rows, int64_t dim, float eps,
           hipStream_t stream) {
  if (rows == 0) return FERRITE_OK;
  const float inv_dim = (float)(1.0 / (double)dim);
  const int64_t blocks = cdiv(rows, kRowsPerBlock);
  if (blocks > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "rmsnorm: too many rows");
  const TX* xp = static_cast<const TX*>(x);
  const TX* rp = static_cast<const TX*>(r);
  const TW* wp = static_cast<const TW*>(w);
  TX* hp = static_cast<TX*>(h);
  TX* yp = static_cast<TX*>(y);
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool fast = dim % kChunk == 0 && aligned16(x) && aligned16(y) && aligned16(w) &&
                    (!RES || (aligned16(r) && aligned16(h))) && dim <= 64 * kChunk * 8;
  dim3 grid((unsigned)blocks), block(256);
  if (fast) {
    const int nchunks = (int)(dim / kChunk);
    const int vpl = (int)cdiv(nchunks, 64);
#define FERRITE_RMS_CASE(V)                                                                                     \
  hipLaunchKernelGGL((rmsnorm_rows_kernel<TX, TW, RES, V>), grid, block, 0, stream, xp, rp, wp, hp, yp, rows, \
                     (int)dim, inv_dim, eps)
    if (vpl <= 1)
      FERRITE_RMS_CASE(1);
    else if (vpl <= 2)
      FERRITE_RMS_CASE(2);
    else if (vpl <= 4)
      FERRITE_RMS_CASE(4);
    else
      FERRITE_RMS_CASE(8);
#undef FERRITE_RMS_CASE
  } else {
    hipLaunchKernelGGL((rmsnorm_rows_generic_kernel<TX, TW, RES>), grid, block, 0, stream, xp, rp, wp, hp, yp, rows,
                       dim, inv_dim, eps);
  }
  return check_launch(RES ? "ferrite_add_rmsnorm" : "ferrite_rmsnorm");
}

template <bool RES>
int dispatch(const void* x, const void* r, const void* w, void* h, void* y, int64_t rows, int64_t dim, int x_dtype,
             int w_dtype, float eps, void* stream) {
  const char* name = RES ? "ferrite_hip_add_rmsnorm" : "ferrite_hip_rmsnorm";
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (rows < 0 || dim < 1)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need rows >= 0 and dim >= 1");
  if (rows > 0 && (!x || !w || !y || (RES && (!r || !h))))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == FERRITE_BF16) {
    if (w_dtype == FERRITE_BF16) return launch<bf16, bf16, RES>(x, r, w, h, y, rows, dim, eps, s);
    return launch<bf16, float, RES>(x, r, w, h, y, rows, dim, eps, s);
  }
  if (w_dtype == FERRITE_BF16) return launch<float, bf16, RES>(x, r, w, h, y, rows, dim, eps, s);
  return launch<float, float, RES>(x, r, w, h, y, rows, dim, eps, s);
}

}  // namespace
}  // namespace ferrite

extern "C" int ferrite_hip_add_rmsnorm(const void* x, const void* residual, const void* weight, void* h, void* y,
                                       int64_t rows, int64_t dim, int x_dtype, int w_dtype, float eps,
                                       void* stream) {
  return ferrite::dispatch<true>(x, residual, weight, h, y, rows, dim, x_dtype, w_dtype, eps, stream);
}

extern "C" int ferrite_hip_rmsnorm(const void* x, const void* weight, void* y, int64_t rows, int64_t dim,
                                   int x_dtype, int w_dtype, float eps, void* stream) {
  return ferrite::dispatch<false>(x, nullptr, weight, nullptr, y, rows, dim, x_dtype, w_dtype, eps, stream);
}
