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
#include <algorithm>
#include <mutex>
#include <string>

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

// Streaming 16-byte loads/stores with the non-temporal hint: every byte of x,
// residual, h and y is touched exactly once, so keeping them out of the caches
// leaves the memory system to the stream (measured: ~15% faster than plain
// loads at [4096, 1024], and the only way past a plain copy's bandwidth there).
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p)); }

// 8 elements of T as raw 16-byte words (one word for bf16, two for f32).
template <typename T>
struct Raw8 {
  u32x4 w[sizeof(T) / 2];
};
template <typename T>
__device__ __forceinline__ void ld8_nt(const T* p, Raw8<T>& r) {
#pragma unroll
  for (int i = 0; i < (int)sizeof(T) / 2; ++i) r.w[i] = ld16_nt(reinterpret_cast<const char*>(p) + 16 * i);
}
template <typename T>
__device__ __forceinline__ void unpack8(const Raw8<T>& r, float* out) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 v = __builtin_bit_cast(bf16x8, r.w[0]);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x4 v = __builtin_bit_cast(f32x4, r.w[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[4 * i + e] = v[e];
    }
  }
}
template <typename T>
__device__ __forceinline__ void st8_nt(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)in[e];
    st16_nt(p, __builtin_bit_cast(u32x4, v));
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x4 v = {in[4 * i], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]};
      st16_nt(reinterpret_cast<char*>(p) + 16 * i, __builtin_bit_cast(u32x4, v));
    }
  }
}

// One batch of up to DEPTH consecutive rows starting at `base` for one wave.
// With CHECK = false every row and chunk is in range (the common case: full
// batches of rows whose width is exactly 512 * VPL), so all loads of the batch
// are issued back to back with no branches.
template <typename TX, typename TW, bool RES, int VPL, int DEPTH, bool CHECK>
__device__ __forceinline__ void rms_batch(const TX* __restrict__ x, const TX* __restrict__ r, TX* __restrict__ h,
                                          TX* __restrict__ y, const float (&wv)[VPL][kChunk], int64_t base,
                                          int64_t rows, int dim, int nchunks, float inv_dim, float eps) {
  const int lane = threadIdx.x & 63;
  Raw8<TX> xr[DEPTH][VPL], rr[DEPTH][VPL];
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) {
    if (CHECK && base + k >= rows) break;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (!CHECK || c < nchunks) {
        ld8_nt(x + (base + k) * dim + c * kChunk, xr[k][i]);
        if constexpr (RES) ld8_nt(r + (base + k) * dim + c * kChunk, rr[k][i]);
      }
    }
  }
  // Keep every load of the batch ahead of the arithmetic (the scheduler would
  // otherwise sink them next to their uses and leave few bytes in flight).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) {
    if (CHECK && base + k >= rows) break;
    const int64_t off = (base + k) * dim;
    float hv[VPL][kChunk];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      if (!CHECK || lane + 64 * i < nchunks) {
        unpack8(xr[k][i], hv[i]);
        if constexpr (RES) {
          float rv[kChunk];
          unpack8(rr[k][i], rv);
#pragma unroll
          for (int e = 0; e < kChunk; ++e) hv[i][e] += rv[e];
        }
#pragma unroll
        for (int e = 0; e < kChunk; ++e) ss += hv[i][e] * hv[i][e];
      }
    }
    if constexpr (RES) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = lane + 64 * i;
        if (!CHECK || c < nchunks) st8_nt(h + off + c * kChunk, hv[i]);
      }
    }
    ss = wave_sum(ss);
    const float inv = __builtin_amdgcn_rsqf(ss * inv_dim + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (!CHECK || c < nchunks) {
        float yv[kChunk];
#pragma unroll
        for (int e = 0; e < kChunk; ++e) yv[e] = (hv[i][e] * inv) * wv[i][e];
        st8_nt(y + off + c * kChunk, yv);
      }
    }
  }
}

// Fast path: dim % 8 == 0, 16-byte aligned rows, dim <= 64 * 8 * VPL (FULL:
// dim == 64 * 8 * VPL). Lane l owns chunks c = l + 64 * i (i < VPL) of its row.
// The grid is persistent: each wave takes DEPTH consecutive rows at a time and
// issues all of their loads before any arithmetic, so it keeps DEPTH rows of x
// and residual in flight; waves then stride over the remaining rows.
template <typename TX, typename TW, bool RES, int VPL, int DEPTH, bool FULL>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const TX* __restrict__ x, const TX* __restrict__ r,
                                                          const TW* __restrict__ w, TX* __restrict__ h,
                                                          TX* __restrict__ y, int64_t rows, int dim, float inv_dim,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
  const int nchunks = dim / kChunk;

  float wv[VPL][kChunk];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (FULL || c < nchunks) load8(w + c * kChunk, wv[i]);
  }

  for (int64_t base = ((int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * DEPTH; base < rows;
       base += nwaves * DEPTH) {
    if (FULL && base + DEPTH <= rows)
      rms_batch<TX, TW, RES, VPL, DEPTH, false>(x, r, h, y, wv, base, rows, dim, nchunks, inv_dim, eps);
    else
      rms_batch<TX, TW, RES, VPL, DEPTH, true>(x, r, h, y, wv, base, rows, dim, nchunks, inv_dim, eps);
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
    // DEPTH rows in flight per wave (fewer for wide rows, to bound registers);
    // at most one workgroup per (CU x 4) so small problems run in one pass.
    auto pgrid = [&](int depth) {
      return dim3((unsigned)std::min<int64_t>(cdiv(rows, (int64_t)kRowsPerBlock * depth), 1024));
    };
#define FERRITE_RMS_CASE(V, DEPTH)                                                                                 \
  do {                                                                                                             \
    if (nchunks == 64 * (V))                                                                                       \
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TX, TW, RES, V, DEPTH, true>), pgrid(DEPTH), block, 0, stream, xp, rp, \
                         wp, hp, yp, rows, (int)dim, inv_dim, eps);                                                \
    else                                                                                                           \
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TX, TW, RES, V, DEPTH, false>), pgrid(DEPTH), block, 0, stream, xp,    \
                         rp, wp, hp, yp, rows, (int)dim, inv_dim, eps);                                            \
  } while (0)
    // Rows of up to 1024 elements: two rows in flight per wave and two workgroups per
    // CU where the rows allow (at [4096, 1024]: 6.73 -> 6.58 us; at [65536, 1024]
    // 100.1 -> 92.4 us, the rate of a plain two-buffer streaming copy; four rows
    // per wave with one workgroup per CU, or one row with four, are slower).
    if (vpl <= 1)
      FERRITE_RMS_CASE(1, 4);
    else if (vpl <= 2)
      FERRITE_RMS_CASE(2, 2);
    else if (vpl <= 4)
      FERRITE_RMS_CASE(4, 2);
    else
      FERRITE_RMS_CASE(8, 1);
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


// ---------------------------------------------------------------------------
// Backward (rmsnorm.py:159-166, and :148-153 for the fused add):
//   inv = rsqrt(mean(h^2) + eps),  xhat = h * inv,  dxhat = dy * w
//   dh  = inv * (dxhat - xhat * mean(dxhat * xhat))  [+ dh_direct]
//   dw  = sum over rows of dy * xhat
// mean(dxhat * xhat) is evaluated as inv * mean(dxhat * h), so one pass with two
// wave reductions per row gives both statistics. All arithmetic is f32.
//
// dw is deterministic: each workgroup accumulates its rows' dy * xhat in
// registers (every lane owns the same columns on every row), its four waves
// combine through LDS into one partial row of the workspace, and a second
// kernel sums the partial rows in a fixed order.
// ---------------------------------------------------------------------------

constexpr int kBwdMaxParts = 512;  // partial dw rows (workgroups of the row pass)

template <typename TX, typename TW, typename TO, bool DIRECT, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_bwd_rows_kernel(const TX* __restrict__ h, const TW* __restrict__ w,
                                                              const TX* __restrict__ dy, const TX* __restrict__ dd,
                                                              TO* __restrict__ dh, float* __restrict__ partial,
                                                              int64_t rows, int dim, float inv_dim, float eps) {
  extern __shared__ float red[];  // [4][dim]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = dim / kChunk;
  float wv[VPL][kChunk], acc[VPL][kChunk];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) load8(w + c * kChunk, wv[i]);
#pragma unroll
    for (int e = 0; e < kChunk; ++e) acc[i][e] = 0.f;
  }
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + wave; row < rows; row += (int64_t)gridDim.x * kRowsPerBlock) {
    const int64_t off = row * dim;
    Raw8<TX> hr[VPL], gr[VPL], dr[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunks) {
        ld8_nt(h + off + c * kChunk, hr[i]);
        ld8_nt(dy + off + c * kChunk, gr[i]);
        if constexpr (DIRECT) ld8_nt(dd + off + c * kChunk, dr[i]);
      }
    }
    float hv[VPL][kChunk], gv[VPL][kChunk];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      if (lane + 64 * i < nchunks) {
        unpack8(hr[i], hv[i]);
        unpack8(gr[i], gv[i]);
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          s1 += hv[i][e] * hv[i][e];
          s2 += (gv[i][e] * wv[i][e]) * hv[i][e];
        }
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float inv = __builtin_amdgcn_rsqf(s1 * inv_dim + eps);
    const float mean = inv * s2 * inv_dim;  // mean(dxhat * xhat)
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunks) {
        float dv[kChunk], out[kChunk];
        if constexpr (DIRECT) unpack8(dr[i], dv);
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          const float xh = hv[i][e] * inv;
          out[e] = inv * (gv[i][e] * wv[i][e] - xh * mean);
          if constexpr (DIRECT) out[e] += dv[e];
          acc[i][e] += gv[i][e] * xh;
        }
        st8_nt(dh + off + c * kChunk, out);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) store8(red + wave * dim + c * kChunk, acc[i]);
  }
  __syncthreads();
  for (int col = threadIdx.x; col < dim; col += blockDim.x)
    partial[(int64_t)blockIdx.x * dim + col] = (red[col] + red[dim + col]) + (red[2 * dim + col] + red[3 * dim + col]);
}

// General row pass (any dim or alignment): one wave per row, two sweeps. The
// per-row inv goes to the workspace for the column pass below.
template <typename TX, typename TW, typename TO, bool DIRECT>
__global__ __launch_bounds__(256) void rmsnorm_bwd_rows_generic_kernel(const TX* __restrict__ h,
                                                                      const TW* __restrict__ w,
                                                                      const TX* __restrict__ dy,
                                                                      const TX* __restrict__ dd, TO* __restrict__ dh,
                                                                      float* __restrict__ inv_rows, int64_t rows,
                                                                      int64_t dim, float inv_dim, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t off = row * dim;
  float s1 = 0.f, s2 = 0.f;
  for (int64_t e = lane; e < dim; e += 64) {
    const float hv = Elem<TX>::to_f32(h[off + e]);
    s1 += hv * hv;
    s2 += (Elem<TX>::to_f32(dy[off + e]) * Elem<TW>::to_f32(w[e])) * hv;
  }
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
  const float inv = __builtin_amdgcn_rsqf(s1 * inv_dim + eps);
  const float mean = inv * s2 * inv_dim;
  if (lane == 0) inv_rows[row] = inv;
  for (int64_t e = lane; e < dim; e += 64) {
    const float xh = Elem<TX>::to_f32(h[off + e]) * inv;
    float o = inv * (Elem<TX>::to_f32(dy[off + e]) * Elem<TW>::to_f32(w[e]) - xh * mean);
    if constexpr (DIRECT) o += Elem<TX>::to_f32(dd[off + e]);
    dh[off + e] = Elem<TO>::from_f32(o);
  }
}

// Column pass of the general path: partial[p, col] = sum over rows r = p (mod P)
// of dy[r, col] * h[r, col] * inv[r]. Threads own columns, so each row read is
// coalesced.
template <typename TX>
__global__ __launch_bounds__(256) void rmsnorm_bwd_cols_kernel(const TX* __restrict__ h, const TX* __restrict__ dy,
                                                              const float* __restrict__ inv_rows,
                                                              float* __restrict__ partial, int64_t rows,
                                                              int64_t dim) {
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= dim) return;
  float acc = 0.f;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y)
    acc += Elem<TX>::to_f32(dy[r * dim + col]) * (Elem<TX>::to_f32(h[r * dim + col]) * inv_rows[r]);
  partial[(int64_t)blockIdx.y * dim + col] = acc;
}

// dw[col] = sum of the partial rows; cast to the weight's dtype. A block owns
// 64 columns; its 16 waves each sum every 16th partial row (in increasing
// order), and wave 0 adds the 16 results in order, so the sum is deterministic
// and every wave keeps several independent loads in flight.
constexpr int kDwCols = 64, kDwGroups = 16;

template <typename TW>
__global__ __launch_bounds__(kDwCols* kDwGroups) void rmsnorm_bwd_dw_kernel(const float* __restrict__ partial,
                                                                           TW* __restrict__ dw, int nparts,
                                                                           int64_t dim) {
  __shared__ float red[kDwGroups][kDwCols];
  const int c = threadIdx.x % kDwCols, grp = threadIdx.x / kDwCols;
  const int64_t col = (int64_t)blockIdx.x * kDwCols + c;
  float acc = 0.f;
  if (col < dim) {
#pragma unroll 8
    for (int p = grp; p < nparts; p += kDwGroups) acc += partial[(int64_t)p * dim + col];
  }
  red[grp][c] = acc;
  __syncthreads();
  if (grp == 0 && col < dim) {
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < kDwGroups; ++g) sum += red[g][c];
    dw[col] = Elem<TW>::from_f32(sum);
  }
}

// Workspace of the backward: nparts partial rows of dim floats (nparts <= kBwdMaxParts),
// then, on the general path only, one float per row. The size query of the C ABI
// returns the bound over every path; bwd_plan gives what one call really uses.
int64_t bwd_workspace_bytes(int64_t rows, int64_t dim) { return ((int64_t)kBwdMaxParts * dim + rows) * 4; }

struct BwdPlan {
  bool fast;      // the one-pass row kernel (else the general row + column passes)
  int nparts;     // partial dw rows
  int64_t bytes;  // workspace bytes this call uses
};

BwdPlan bwd_plan(const void* h, const void* w, const void* dy, const void* dd, const void* dh, int64_t rows,
                 int64_t dim) {
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  BwdPlan p{};
  p.fast = dim % kChunk == 0 && dim <= 64 * kChunk * 8 && aligned16(h) && aligned16(dy) && aligned16(w) &&
           aligned16(dh) && (!dd || aligned16(dd));
  if (rows <= 0)
    p.nparts = 0;
  else if (p.fast)  // at least 4 rows per wave; at most kBwdMaxParts workgroups (two per CU)
    p.nparts = (int)std::min<int64_t>(cdiv(rows, (int64_t)kRowsPerBlock * 4), kBwdMaxParts);
  else
    p.nparts = (int)std::min<int64_t>(rows, kBwdMaxParts);
  p.bytes = ((int64_t)p.nparts * dim + (p.fast || rows <= 0 ? 0 : rows)) * 4;
  return p;
}

template <typename TX, typename TW, typename TO, bool DIRECT>
int bwd_launch(const void* h, const void* w, const void* dy, const void* dd, void* dh, void* dw, void* ws,
               int64_t rows, int64_t dim, float eps, hipStream_t stream) {
  const float inv_dim = (float)(1.0 / (double)dim);
  const TX* hp = static_cast<const TX*>(h);
  const TX* gp = static_cast<const TX*>(dy);
  const TX* dp = static_cast<const TX*>(dd);
  const TW* wp = static_cast<const TW*>(w);
  TO* op = static_cast<TO*>(dh);
  float* partial = static_cast<float*>(ws);
  const BwdPlan plan = bwd_plan(h, w, dy, DIRECT ? dd : nullptr, dh, rows, dim);
  const int nparts = plan.nparts;
  if (rows > 0 && plan.fast) {
    const int vpl = (int)cdiv(dim / kChunk, 64);
    const size_t lds = (size_t)kRowsPerBlock * dim * sizeof(float);
#define FERRITE_RMS_BWD_CASE(V)                                                                                    \
  hipLaunchKernelGGL((rmsnorm_bwd_rows_kernel<TX, TW, TO, DIRECT, V>), dim3(nparts), dim3(256), lds, stream, hp, wp, \
                     gp, dp, op, partial, rows, (int)dim, inv_dim, eps)
    if (vpl <= 1)
      FERRITE_RMS_BWD_CASE(1);
    else if (vpl <= 2)
      FERRITE_RMS_BWD_CASE(2);
    else if (vpl <= 4)
      FERRITE_RMS_BWD_CASE(4);
    else
      FERRITE_RMS_BWD_CASE(8);
#undef FERRITE_RMS_BWD_CASE
  } else if (rows > 0) {
    float* inv_rows = partial + (int64_t)nparts * dim;
    const int64_t blocks = cdiv(rows, kRowsPerBlock);
    if (blocks > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: too many rows");
    hipLaunchKernelGGL((rmsnorm_bwd_rows_generic_kernel<TX, TW, TO, DIRECT>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, hp, wp, gp, dp, op, inv_rows, rows, dim, inv_dim, eps);
    const int64_t cblocks = cdiv(dim, 256);
    if (cblocks > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: dim too large");
    hipLaunchKernelGGL((rmsnorm_bwd_cols_kernel<TX>), dim3((unsigned)cblocks, (unsigned)nparts), dim3(256), 0, stream,
                       hp, gp, inv_rows, partial, rows, dim);
  }
  hipLaunchKernelGGL((rmsnorm_bwd_dw_kernel<TW>), dim3((unsigned)cdiv(dim, kDwCols)), dim3(kDwCols * kDwGroups), 0,
                     stream, partial, static_cast<TW*>(dw), nparts, dim);
  return check_launch("ferrite_rmsnorm_bwd");
}

template <typename TX, typename TW>
int bwd_dispatch_out(const void* h, const void* w, const void* dy, const void* dd, void* dh, void* dw, void* ws,
                     int64_t rows, int64_t dim, int dh_dtype, float eps, hipStream_t s) {
  if (dh_dtype == FERRITE_F32) {
    return dd ? bwd_launch<TX, TW, float, true>(h, w, dy, dd, dh, dw, ws, rows, dim, eps, s)
              : bwd_launch<TX, TW, float, false>(h, w, dy, dd, dh, dw, ws, rows, dim, eps, s);
  }
  if constexpr (sizeof(TX) == 2) {
    return dd ? bwd_launch<TX, TW, TX, true>(h, w, dy, dd, dh, dw, ws, rows, dim, eps, s)
              : bwd_launch<TX, TW, TX, false>(h, w, dy, dd, dh, dw, ws, rows, dim, eps, s);
  }
  return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_rmsnorm_bwd: a bf16 dh needs bf16 inputs");
}

// ---------------------------------------------------------------------------
// Streaming copy of two buffers (a -> a_out, b -> b_out): add+RMSNorm's access
// pattern (two 16-byte non-temporal loads and two stores per lane and 2 KB
// unit) with no arithmetic, to measure the HBM ceiling a kernel of that shape
// can reach. Persistent grid: wave w copies units w, w + waves, ... (one unit =
// 2 KB of each buffer, two 16-byte words per lane).
// ---------------------------------------------------------------------------
constexpr int kCopyUnit = 2048;

__global__ __launch_bounds__(256) void stream_copy2_kernel(const char* __restrict__ a, const char* __restrict__ b,
                                                           char* __restrict__ a_out, char* __restrict__ b_out,
                                                           int64_t units, int64_t tail_words) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += nwaves) {
    const int64_t o0 = u * kCopyUnit + lane * 16, o1 = o0 + 1024;
    const u32x4 a0 = ld16_nt(a + o0), a1 = ld16_nt(a + o1), b0 = ld16_nt(b + o0), b1 = ld16_nt(b + o1);
    st16_nt(a_out + o0, a0);
    st16_nt(a_out + o1, a1);
    st16_nt(b_out + o0, b0);
    st16_nt(b_out + o1, b1);
  }
  // The last partial unit: 16-byte words, one per thread of block 0.
  if (blockIdx.x == 0 && threadIdx.x < tail_words) {
    const int64_t o = units * kCopyUnit + (int64_t)threadIdx.x * 16;
    st16_nt(a_out + o, ld16_nt(a + o));
    st16_nt(b_out + o, ld16_nt(b + o));
  }
}

// One-direction streams, the read-only and write-only halves of the ceiling:
// persistent grids in which wave w takes 4 KB units w, w + waves, ... (four
// 16-byte non-temporal accesses per lane and unit). The read stream folds every
// word it loads with XOR so that no load is dead, and each workgroup leaves one
// word in sink[blockIdx.x]; the fill stream stores `value` in every word.
constexpr int kStreamUnit = 4096;

__global__ __launch_bounds__(256) void stream_read_kernel(const char* __restrict__ a, uint32_t* __restrict__ sink,
                                                          int64_t units, int64_t tail_words) {
  __shared__ uint32_t part[4];
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  u32x4 x = {0u, 0u, 0u, 0u};
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += nwaves) {
    const int64_t o = u * kStreamUnit + lane * 16;
    const u32x4 a0 = ld16_nt(a + o), a1 = ld16_nt(a + o + 1024), a2 = ld16_nt(a + o + 2048), a3 = ld16_nt(a + o + 3072);
    x ^= (a0 ^ a1) ^ (a2 ^ a3);
  }
  if (blockIdx.x == 0 && threadIdx.x < tail_words) x ^= ld16_nt(a + units * kStreamUnit + (int64_t)threadIdx.x * 16);
  uint32_t w = (x[0] ^ x[1]) ^ (x[2] ^ x[3]);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) w ^= (uint32_t)__shfl_xor((int)w, off, kWave);
  if (lane == 0) part[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = (part[0] ^ part[1]) ^ (part[2] ^ part[3]);
}

__global__ __launch_bounds__(256) void stream_fill_kernel(char* __restrict__ out, uint32_t value, int64_t units,
                                                          int64_t tail_words) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const u32x4 v = {value, value, value, value};
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += nwaves) {
    const int64_t o = u * kStreamUnit + lane * 16;
    st16_nt(out + o, v);
    st16_nt(out + o + 1024, v);
    st16_nt(out + o + 2048, v);
    st16_nt(out + o + 3072, v);
  }
  if (blockIdx.x == 0 && threadIdx.x < tail_words) st16_nt(out + units * kStreamUnit + (int64_t)threadIdx.x * 16, v);
}

// Workgroups of a stream launch: `blocks` if given (1 .. 65536), else 512 (two per CU), and
// never more than there are units for.
int64_t stream_blocks(int blocks, int64_t units) {
  const int64_t want = blocks > 0 ? blocks : 512;
  return std::max<int64_t>(1, std::min<int64_t>(want, cdiv(units, 4)));
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free backward (ferrite_hip_rmsnorm_bwd_noalloc):
// the partial dw rows (and inverse RMS per row) live in this file-scope device
// array instead of a caller's workspace. Each device that loads the library
// holds its own copy until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in symbol): the
// device address is looked up once per device with hipGetSymbolAddress, with
// that device current, and that address is what the kernels receive.
// ---------------------------------------------------------------------------
constexpr int kMaxDevices = 64;
static_assert(FERRITE_RMSNORM_BWD_SCRATCH_BYTES % 256 == 0, "scratch size");

static __device__ __align__(256) float scratch[FERRITE_RMSNORM_BWD_SCRATCH_BYTES / sizeof(float)];

struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

// Device address of `scratch` on the stream's device (looked up on the first
// call per device, with that device current), or nullptr with the error message
// set.
void* scratch_on_device(hipStream_t stream) {
  const int dev = stream_device(stream);
  if (dev < 0 || dev >= kMaxDevices) {
    fail(FERRITE_ERR_LAUNCH, "ferrite_hip_rmsnorm_bwd_noalloc: cannot tell the stream's HIP device");
    return nullptr;
  }
  ScratchSlot& slot = g_scratch[dev];
  std::call_once(slot.once, [&slot, dev] {
    DeviceGuard on(dev);
    void* p = nullptr;
    slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    slot.ptr = slot.err == hipSuccess ? p : nullptr;
  });
  if (!slot.ptr) {
    fail(FERRITE_ERR_LAUNCH, std::string("ferrite_hip_rmsnorm_bwd_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                                 hipGetErrorString(slot.err));
    return nullptr;
  }
  return slot.ptr;
}

int bwd_entry(const char* name, const void* h, const void* weight, const void* dy, const void* dh_direct, void* dh,
              void* dweight, void* workspace, bool noalloc, int64_t rows, int64_t dim, int x_dtype, int w_dtype,
              int dh_dtype, float eps, void* stream) {
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype) || !valid_dtype(dh_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (rows < 0 || dim < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need rows >= 0 and dim >= 1");
  if (!weight || !dweight || (!noalloc && !workspace) || (rows > 0 && (!h || !dy || !dh)))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  if (noalloc) {
    const BwdPlan plan = bwd_plan(h, weight, dy, dh_direct, dh, rows, dim);
    if (plan.bytes > (int64_t)FERRITE_RMSNORM_BWD_SCRATCH_BYTES)
      return fail(FERRITE_ERR_INVALID_ARGUMENT,
                  std::string(name) + ": rows=" + std::to_string(rows) + ", dim=" + std::to_string(dim) + " need " +
                      std::to_string(plan.bytes) + " bytes of scratch, more than its fixed " +
                      std::to_string((long long)FERRITE_RMSNORM_BWD_SCRATCH_BYTES) +
                      " (use ferrite_hip_rmsnorm_bwd with a workspace)");
    workspace = scratch_on_device(static_cast<hipStream_t>(stream));
    if (!workspace) return FERRITE_ERR_LAUNCH;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == FERRITE_BF16) {
    if (w_dtype == FERRITE_BF16)
      return bwd_dispatch_out<bf16, bf16>(h, weight, dy, dh_direct, dh, dweight, workspace, rows, dim, dh_dtype, eps, s);
    return bwd_dispatch_out<bf16, float>(h, weight, dy, dh_direct, dh, dweight, workspace, rows, dim, dh_dtype, eps, s);
  }
  if (w_dtype == FERRITE_BF16)
    return bwd_dispatch_out<float, bf16>(h, weight, dy, dh_direct, dh, dweight, workspace, rows, dim, dh_dtype, eps, s);
  return bwd_dispatch_out<float, float>(h, weight, dy, dh_direct, dh, dweight, workspace, rows, dim, dh_dtype, eps, s);
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

extern "C" int64_t ferrite_hip_rmsnorm_bwd_workspace(int64_t rows, int64_t dim) {
  if (rows < 0 || dim < 1) return -1;
  return ferrite::bwd_workspace_bytes(rows, dim);
}

extern "C" int ferrite_hip_rmsnorm_bwd(const void* h, const void* weight, const void* dy, const void* dh_direct,
                                       void* dh, void* dweight, void* workspace, int64_t rows, int64_t dim,
                                       int x_dtype, int w_dtype, int dh_dtype, float eps, void* stream) {
  return ferrite::bwd_entry("ferrite_hip_rmsnorm_bwd", h, weight, dy, dh_direct, dh, dweight, workspace, false, rows,
                            dim, x_dtype, w_dtype, dh_dtype, eps, stream);
}

extern "C" int ferrite_hip_rmsnorm_bwd_noalloc(const void* h, const void* weight, const void* dy,
                                               const void* dh_direct, void* dh, void* dweight, int64_t rows,
                                               int64_t dim, int x_dtype, int w_dtype, int dh_dtype, float eps,
                                               void* stream) {
  return ferrite::bwd_entry("ferrite_hip_rmsnorm_bwd_noalloc", h, weight, dy, dh_direct, dh, dweight, nullptr, true,
                            rows, dim, x_dtype, w_dtype, dh_dtype, eps, stream);
}

extern "C" int ferrite_hip_stream_copy2(const void* a, const void* b, void* a_out, void* b_out, int64_t bytes,
                                        void* stream) {
  using namespace ferrite;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_copy2: bytes must be a multiple of 16");
  if (bytes == 0) return FERRITE_OK;
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a || !b || !a_out || !b_out || !aligned16(a) || !aligned16(b) || !aligned16(a_out) || !aligned16(b_out))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_copy2: null or unaligned pointer");
  const int64_t units = bytes / kCopyUnit, tail = (bytes % kCopyUnit) / 16;
  // 512 workgroups (two per CU) measured best at 33.5 MB and at 537 MB per buffer pair.
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(512, cdiv(units, 4)));
  hipLaunchKernelGGL(stream_copy2_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char*>(a), static_cast<const char*>(b), static_cast<char*>(a_out),
                     static_cast<char*>(b_out), units, tail);
  return check_launch("ferrite_hip_stream_copy2");
}

extern "C" int ferrite_hip_stream_read(const void* a, int64_t bytes, void* sink, int blocks, void* stream) {
  using namespace ferrite;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_read: bytes must be a multiple of 16");
  if (blocks < 0 || blocks > 65536)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_read: blocks must be 0 (default) or 1 .. 65536");
  if (bytes == 0) return FERRITE_OK;
  if (!a || !sink || (reinterpret_cast<uintptr_t>(a) & 15) || (reinterpret_cast<uintptr_t>(sink) & 3))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_read: null or unaligned pointer");
  const int64_t units = bytes / kStreamUnit, tail = (bytes % kStreamUnit) / 16;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)stream_blocks(blocks, units)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(a), static_cast<uint32_t*>(sink), units,
                     tail);
  return check_launch("ferrite_hip_stream_read");
}

extern "C" int ferrite_hip_stream_fill(void* out, int64_t bytes, uint32_t value, int blocks, void* stream) {
  using namespace ferrite;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_fill: bytes must be a multiple of 16");
  if (blocks < 0 || blocks > 65536)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_fill: blocks must be 0 (default) or 1 .. 65536");
  if (bytes == 0) return FERRITE_OK;
  if (!out || (reinterpret_cast<uintptr_t>(out) & 15))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_stream_fill: null or unaligned pointer");
  const int64_t units = bytes / kStreamUnit, tail = (bytes % kStreamUnit) / 16;
  hipLaunchKernelGGL(stream_fill_kernel, dim3((unsigned)stream_blocks(blocks, units)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<char*>(out), value, units, tail);
  return check_launch("ferrite_hip_stream_fill");
}
