// Blocked matmul out[M,N] = x[M,K] @ y[K,N] with f32 accumulation, gfx950 MFMA.
//
// Reference: src/ferrite/kernels/matmul.py:27-38 (kernel body: f32 accumulator
// over the K grid axis, cast on the last step) and :41-86 (block choice, zero
// padding of ragged shapes, slice back). Here a workgroup owns one BM x BN
// output macro-tile and loops over K in BK steps through double-buffered LDS;
// out-of-range rows/columns are zero-filled on load and skipped on store,
// which is the same arithmetic as the reference's zero padding.
//
// Operand layouts for v_mfma_f32_32x32x16_bf16 (and the f32 32x32x2 form):
// lane l supplies row (l % 32) of A and column (l % 32) of B with k running
// along the lane's 8 elements, so both operands want k contiguous. x is
// row-major [M][K] (k contiguous); y is [K][N] and is transposed on its way
// into LDS (a thread loads 4 k-rows x 16 bytes and writes 4-element k runs).
// The kernel computes C^T tiles (A operand = y^T, B operand = x): each lane then
// owns 4 consecutive output columns of one output row per register quad, which
// the epilogue writes as one 8- or 16-byte store.
//
// LDS rows are 128 bytes (BK elements) split into eight 16-byte chunks; chunk
// c of row n lives at chunk c ^ ((n ^ (n >> 3)) & 7). Fragment reads (32
// consecutive rows, same chunk) and the transposed staging writes (rows 8
// apart, same chunk) both land on distinct banks.
#include "common.h"

namespace ferrite {
namespace {

__device__ __forceinline__ int swz(int n) { return (n ^ (n >> 3)) & 7; }

// Byte offset of element k (multiple of the 16-byte vector) of LDS row n.
template <typename T>
__device__ __forceinline__ int lds_off(int n, int k) {
  constexpr int kVec = Elem<T>::kVec;
  const int chunk = k / kVec;
  return n * 128 + ((chunk ^ swz(n)) << 4) + (k % kVec) * (int)sizeof(T);
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::frag read_frag(const char* lds, int n, int k0) {
  typename Elem<T>::frag f;
  if constexpr (sizeof(T) == 2) {
    f = *reinterpret_cast<const bf16x8*>(lds + lds_off<T>(n, k0));
  } else {
    f32x4 a = *reinterpret_cast<const f32x4*>(lds + lds_off<T>(n, k0));
    f32x4 b = *reinterpret_cast<const f32x4*>(lds + lds_off<T>(n, k0 + 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = a[e];
      f[4 + e] = b[e];
    }
  }
  return f;
}

template <typename T, typename TO, int BM, int BN, int BK, int WM, int WN, bool ALIGNED>
struct Gemm {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int kVec = Elem<T>::kVec;
  static constexpr int kWTM = BM / WM, kWTN = BN / WN;
  static constexpr int kTM = kWTM / 32, kTN = kWTN / 32;
  static constexpr int kKC = BK / 16;
  static constexpr int kAVecs = BM * BK / kVec / kThreads;          // x vectors per thread
  static constexpr int kBJobs = (BK / 4) * (BN / kVec) / kThreads;  // 4 x kVec y blocks per thread
  static constexpr int kStageBytes = (BM + BN) * 128;
  static_assert(BK * sizeof(T) == 128, "LDS rows are 128 bytes");
  static_assert(kAVecs * kThreads * kVec == BM * BK, "x tile split");
  static_assert(kBJobs * kThreads * kVec * 4 == BN * BK, "y tile split");
  typedef typename Elem<T>::vec vec;

  struct Stage {
    vec a[kAVecs];
    vec b[kBJobs][4];
  };

  static __device__ __forceinline__ vec load_vec(const T* p, int64_t row, int64_t col, int64_t rows, int64_t cols,
                                                 int64_t ld) {
    vec v;
    if constexpr (ALIGNED) {
      if (row < rows && col < cols)
        v = *reinterpret_cast<const vec*>(p + row * ld + col);
      else
        for (int e = 0; e < kVec; ++e) v[e] = (T)0.f;
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = (row < rows && col + e < cols) ? p[row * ld + col + e] : (T)0.f;
    }
    return v;
  }

  static __device__ __forceinline__ void load(Stage& s, const T* x, const T* y, int64_t m0, int64_t n0, int64_t k0,
                                              int64_t M, int64_t N, int64_t K) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAVecs; ++i) {
      const int idx = t + kThreads * i;
      const int row = idx / (BK / kVec), cv = idx % (BK / kVec);
      s.a[i] = load_vec(x, m0 + row, k0 + cv * kVec, M, K, K);
    }
#pragma unroll
    for (int j = 0; j < kBJobs; ++j) {
      const int job = t + kThreads * j;
      const int cg = job % (BN / kVec), kg = job / (BN / kVec);
#pragma unroll
      for (int r = 0; r < 4; ++r) s.b[j][r] = load_vec(y, k0 + kg * 4 + r, n0 + cg * kVec, K, N, N);
    }
  }

  static __device__ __forceinline__ void store(const Stage& s, char* lds) {
    const int t = threadIdx.x;
    char* as = lds;
    char* bs = lds + BM * 128;
#pragma unroll
    for (int i = 0; i < kAVecs; ++i) {
      const int idx = t + kThreads * i;
      const int row = idx / (BK / kVec), cv = idx % (BK / kVec);
      *reinterpret_cast<vec*>(as + lds_off<T>(row, cv * kVec)) = s.a[i];
    }
#pragma unroll
    for (int j = 0; j < kBJobs; ++j) {
      const int job = t + kThreads * j;
      const int cg = job % (BN / kVec), kg = job / (BN / kVec);
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        const int n = cg * kVec + e;
        if constexpr (sizeof(T) == 2) {
          bf16x4 w4 = {s.b[j][0][e], s.b[j][1][e], s.b[j][2][e], s.b[j][3][e]};
          *reinterpret_cast<bf16x4*>(bs + lds_off<T>(n, kg * 4)) = w4;
        } else {
          f32x4 w4 = {s.b[j][0][e], s.b[j][1][e], s.b[j][2][e], s.b[j][3][e]};
          *reinterpret_cast<f32x4*>(bs + lds_off<T>(n, kg * 4)) = w4;
        }
      }
    }
  }

  static __device__ __forceinline__ void compute(const char* lds, f32x16 (&acc)[kTN][kTM], int wm0, int wn0) {
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const char* as = lds;
    const char* bs = lds + BM * 128;
#pragma unroll
    for (int kk = 0; kk < kKC; ++kk) {
      typename Elem<T>::frag fa[kTM], fb[kTN];
#pragma unroll
      for (int i = 0; i < kTM; ++i) fa[i] = read_frag<T>(as, wm0 + i * 32 + l32, kk * 16 + g * 8);
#pragma unroll
      for (int j = 0; j < kTN; ++j) fb[j] = read_frag<T>(bs, wn0 + j * 32 + l32, kk * 16 + g * 8);
#pragma unroll
      for (int j = 0; j < kTN; ++j)
#pragma unroll
        for (int i = 0; i < kTM; ++i) mma32(fb[j], fa[i], acc[j][i]);
    }
  }
};

template <typename T, typename TO, int BM, int BN, int BK, int WM, int WN, bool ALIGNED>
__global__ __launch_bounds__((WM * WN * 64), 1) void gemm_kernel(const T* __restrict__ x, const T* __restrict__ y,
                                                              TO* __restrict__ out, int64_t M, int64_t N, int64_t K,
                                                              int tiles_n) {
  typedef Gemm<T, TO, BM, BN, BK, WM, WN, ALIGNED> G;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / tiles_n) * BM;
  const int64_t n0 = (int64_t)(tile % tiles_n) * BN;
  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave / WN) * G::kWTM, wn0 = (wave % WN) * G::kWTN;

  f32x16 acc[G::kTN][G::kTM];
#pragma unroll
  for (int j = 0; j < G::kTN; ++j)
#pragma unroll
    for (int i = 0; i < G::kTM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  const int nk = (int)((K + BK - 1) / BK);
  typename G::Stage st;
  G::load(st, x, y, m0, n0, 0, M, N, K);
  G::store(st, smem);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = smem + (kt & 1) * G::kStageBytes;
    if (kt + 1 < nk) G::load(st, x, y, m0, n0, (int64_t)(kt + 1) * BK, M, N, K);
    G::compute(cur, acc, wm0, wn0);
    if (kt + 1 < nk) G::store(st, smem + ((kt + 1) & 1) * G::kStageBytes);
    __syncthreads();
  }

  // Epilogue: acc[j][i] is the C^T tile (rows n, cols m). Register r of lane
  // (l32, g) is C[m = .. + l32][n = .. + (r/4)*8 + g*4 + r%4].
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
#pragma unroll
  for (int j = 0; j < G::kTN; ++j) {
#pragma unroll
    for (int i = 0; i < G::kTM; ++i) {
      const int64_t m = m0 + wm0 + i * 32 + l32;
      if (m >= M) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn0 + j * 32 + q * 8 + g * 4;
        TO* dst = out + m * N + n;
        if (ALIGNED && n + 3 < N) {
          if constexpr (sizeof(TO) == 2) {
            bf16x4 v = {(bf16)acc[j][i][q * 4 + 0], (bf16)acc[j][i][q * 4 + 1], (bf16)acc[j][i][q * 4 + 2],
                        (bf16)acc[j][i][q * 4 + 3]};
            *reinterpret_cast<bf16x4*>(dst) = v;
          } else {
            f32x4 v = {acc[j][i][q * 4 + 0], acc[j][i][q * 4 + 1], acc[j][i][q * 4 + 2], acc[j][i][q * 4 + 3]};
            *reinterpret_cast<f32x4*>(dst) = v;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) dst[e] = Elem<TO>::from_f32(acc[j][i][q * 4 + e]);
        }
      }
    }
  }
}

template <typename T, typename TO, int BM, int BN, int BK, int WM, int WN>
int launch_gemm(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  typedef Gemm<T, TO, BM, BN, BK, WM, WN, true> G;
  const int64_t tiles_m = cdiv(M, BM), tiles_n = cdiv(N, BN);
  if (tiles_m * tiles_n > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "matmul: output too large");
  const size_t lds = 2 * (size_t)G::kStageBytes;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool aligned = K % Elem<T>::kVec == 0 && N % Elem<T>::kVec == 0 && N % 4 == 0 && a16(x) && a16(y) && a16(out);
  dim3 grid((unsigned)(tiles_m * tiles_n)), block(WM * WN * 64);
  if (aligned) {
    auto k = gemm_kernel<T, TO, BM, BN, BK, WM, WN, true>;
    (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k, grid, block, lds, stream, static_cast<const T*>(x), static_cast<const T*>(y),
                       static_cast<TO*>(out), M, N, K, (int)tiles_n);
  } else {
    auto k = gemm_kernel<T, TO, BM, BN, BK, WM, WN, false>;
    (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k, grid, block, lds, stream, static_cast<const T*>(x), static_cast<const T*>(y),
                       static_cast<TO*>(out), M, N, K, (int)tiles_n);
  }
  return check_launch("ferrite_matmul");
}

}  // namespace
}  // namespace ferrite

extern "C" int ferrite_hip_matmul(const void* x, const void* y, void* out, int64_t m, int64_t n, int64_t k,
                                  int in_dtype, int out_dtype, void* stream) {
  using namespace ferrite;
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: dtype must be FERRITE_F32 or FERRITE_BF16");
  if (m < 1 || n < 1 || k < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: need M, N, K >= 1");
  if (!x || !y || !out) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype == FERRITE_BF16) {
    if (out_dtype == FERRITE_BF16) return launch_gemm<bf16, bf16, 256, 256, 64, 2, 2>(x, y, out, m, n, k, s);
    return launch_gemm<bf16, float, 256, 256, 64, 2, 2>(x, y, out, m, n, k, s);
  }
  if (out_dtype == FERRITE_BF16) return launch_gemm<float, bf16, 128, 128, 32, 2, 2>(x, y, out, m, n, k, s);
  return launch_gemm<float, float, 128, 128, 32, 2, 2>(x, y, out, m, n, k, s);
}
