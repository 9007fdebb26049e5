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
#include <algorithm>

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
      // Zero, then the load when in range (a zeroing loop in the else branch was kept
      // as a scratch array by the compiler: 48 bytes per lane of spill).
      v = __builtin_bit_cast(vec, u32x4{0u, 0u, 0u, 0u});
      if (row < rows && col < cols) v = *reinterpret_cast<const vec*>(p + row * ld + col);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = (row < rows && col + e < cols) ? p[row * ld + col + e] : (T)0.f;
    }
    return v;
  }

  // Thread t of the tile's kThreads loads its share of the k-step from k0; k from
  // kend on (the end of K, or of the caller's K slice) reads as zero.
  static __device__ __forceinline__ void load(Stage& s, const T* x, const T* y, int64_t m0, int64_t n0, int64_t k0,
                                              int64_t M, int64_t N, int64_t K, int64_t kend, int t) {
#pragma unroll
    for (int i = 0; i < kAVecs; ++i) {
      const int idx = t + kThreads * i;
      const int row = idx / (BK / kVec), cv = idx % (BK / kVec);
      s.a[i] = load_vec(x, m0 + row, k0 + cv * kVec, M, kend, K);
    }
#pragma unroll
    for (int j = 0; j < kBJobs; ++j) {
      const int job = t + kThreads * j;
      const int cg = job % (BN / kVec), kg = job / (BN / kVec);
#pragma unroll
      for (int r = 0; r < 4; ++r) s.b[j][r] = load_vec(y, k0 + kg * 4 + r, n0 + cg * kVec, kend, N, N);
    }
  }
  static __device__ __forceinline__ void load(Stage& s, const T* x, const T* y, int64_t m0, int64_t n0, int64_t k0,
                                              int64_t M, int64_t N, int64_t K) {
    load(s, x, y, m0, n0, k0, M, N, K, K, threadIdx.x);
  }

  static __device__ __forceinline__ void store(const Stage& s, char* lds, int t = threadIdx.x) {
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
          // Element e of the four k-rows, gathered from 32-bit words with shifts and
          // masks (element extraction from bf16 vectors went through scratch memory).
          uint32_t w[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) w[r] = __builtin_bit_cast(u32x4, s.b[j][r])[e >> 1];
          const uint32_t lo = (e & 1) ? (w[0] >> 16) | (w[1] & 0xffff0000u) : (w[0] & 0xffffu) | (w[1] << 16);
          const uint32_t hi = (e & 1) ? (w[2] >> 16) | (w[3] & 0xffff0000u) : (w[2] & 0xffffu) | (w[3] << 16);
          *reinterpret_cast<u32x2*>(bs + lds_off<T>(n, kg * 4)) = u32x2{lo, hi};
        } else {
          f32x4 w4 = {s.b[j][0][e], s.b[j][1][e], s.b[j][2][e], s.b[j][3][e]};
          *reinterpret_cast<f32x4*>(bs + lds_off<T>(n, kg * 4)) = w4;
        }
      }
    }
  }

  // One of the f32 stage's eight LDS writes: x vector p (p < kAVecs), else column
  // p - kAVecs of the y job, written as its four k values (the same places store() writes).
  static __device__ __forceinline__ void store_part(const Stage& s, char* lds, int t, int p) {
    static_assert(sizeof(T) == 4 && kAVecs == 4 && kBJobs == 1, "f32 64 x 64 x 32 stages");
    if (p < kAVecs) {
      const int idx = t + kThreads * p;
      const int row = idx / (BK / kVec), cv = idx % (BK / kVec);
      *reinterpret_cast<vec*>(lds + lds_off<T>(row, cv * kVec)) = s.a[p];
    } else {
      const int e = p - kAVecs;
      const int cg = t % (BN / kVec), kg = t / (BN / kVec);
      *reinterpret_cast<f32x4*>(lds + BM * 128 + lds_off<T>(cg * kVec + e, kg * 4)) =
          f32x4{s.b[0][0][e], s.b[0][1][e], s.b[0][2][e], s.b[0][3][e]};
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
      if constexpr (sizeof(T) == 4) {
        // f32: the eight k-steps of every accumulator in turn, so that consecutive
        // 32x32x2 products go to different accumulators.
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int j = 0; j < kTN; ++j)
#pragma unroll
            for (int i = 0; i < kTM; ++i)
              acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[j][e], fa[i][e], acc[j][i], 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int i = 0; i < kTM; ++i) mma32(fb[j], fa[i], acc[j][i]);
      }
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

// f32 products with few output tiles (1000^3 has 256 tiles of 64 x 64): S slices of
// K for one tile in one workgroup of 2S waves, each pair of waves running the
// two-wave 64 x 64 loop above over its slice from its own pair of LDS stages. At
// the end slices 1 .. S-1 leave their accumulators in LDS and slice 0 adds them
// in slice order, so the K split needs no partial slabs in HBM and no second
// kernel, and the sum's order does not depend on timing. With still fewer tiles,
// blockIdx.y selects one of several groups of S slices, whose sums go to the f32
// partial slab blockIdx.y of `out` for gemm_splitk_reduce_kernel.
//
// The k-steps are software-pipelined: two register
// stages, the loads of step kt + 2 and the LDS writes of step kt + 1 (loaded a
// whole step earlier) issued one at a time between step kt's products, so that
// neither waits in a burst at the step's edge (loads issued together after the
// barrier queue in the CU's address path and hold up the products). The loads
// are bounds-checked buffer loads with per-lane offsets fixed for the kernel and
// the descriptor's base moved per step on the scalar unit; the y descriptor's
// range ends at the slice's last k row, and x columns past it read as zeros
// through the offset of a partial step. 16-byte rows (ALIGNED) load 4-float
// vectors, other rows single floats. Measured on one MI355X against the loop
// with one register stage (both bitwise equal): 1000^3 26.7 -> 23.8 us with the
// two stages, -> 21.4 us (at K = 1024) with the loads spread and their offsets
// fixed; 1000 x 1000 x 8192 147 -> 130 us; 1000 x 1003 x 999 40.0 -> 30.9 us.
//
// BMN = 128 runs the same loop on 128 x 128 tiles of four waves (64 x 64 each), one slice:
// the f32 products with enough tiles for every CU.
template <typename TO, int S, bool ALIGNED, int BMN = 64>
__global__ __launch_bounds__((BMN == 64 ? 128 : 256) * S, 1) void gemm_f32_slices_kernel(
    const float* __restrict__ x, const float* __restrict__ y, TO* __restrict__ out, int64_t M, int64_t N, int64_t K,
    int tiles_n, int64_t kslice) {
  constexpr int WM = BMN / 64;
  typedef Gemm<float, TO, BMN, BMN, 32, WM, 2, ALIGNED> G;
  constexpr int kT = G::kThreads, kTM = G::kTM, kTN = G::kTN;
  static_assert(G::kAVecs == 4 && G::kBJobs == 1, "four x vectors and one y job per thread and stage");
  static_assert((BMN == 64 && kT == 128 && kTM == 2 && kTN == 1) || (BMN == 128 && S == 1 && kT == 256 && kTM == 2 && kTN == 2),
                "two waves of 64 x 32 per slice, or four of 64 x 64 and one slice");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // Blocks are dealt to the 8 XCDs round robin: the tiles of one XCD are made
  // consecutive and walked in groups of 4 tile rows, so that an XCD's L2 holds
  // the x and y panels of a compact block of tiles (1000^3: 4 x 8 tiles, 3 MB
  // of panels per XCD instead of 16 x 2, 4.5 MB).
  const int ntiles = (int)gridDim.x;
  int v = blockIdx.x;
  if (ntiles % 8 == 0) v = (v % 8) * (ntiles / 8) + v / 8;
  constexpr int kGroup = 4;
  const int tiles_m = ntiles / tiles_n;
  const int first_m = v / (kGroup * tiles_n) * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int64_t m0 = (int64_t)(first_m + (v % (kGroup * tiles_n)) % gsize) * BMN;
  const int64_t n0 = (int64_t)((v % (kGroup * tiles_n)) / gsize) * BMN;
  const int slice = threadIdx.x / kT, t = threadIdx.x % kT;
  const int ws = t >> 6;  // the wave within its slice
  const int wm0 = (ws / 2) * G::kWTM, wn0 = (ws % 2) * G::kWTN;
  char* const lds = smem + slice * 2 * G::kStageBytes;

  f32x16 acc[kTN][kTM];
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  // Every slice runs the same number of k-steps (the workgroup's barriers are
  // shared); a short last slice reads zeros past K.
  const int64_t kbeg = kslice * ((int64_t)blockIdx.y * S + slice), kend = std::min(K, kbeg + kslice);
  out += (int64_t)blockIdx.y * M * N;
  const int nk = (int)(kslice / 32);
  // Offsets in bytes from the slice's first x column of row m0 and first y row at column n0
  // (the launcher keeps them under 2^31); rows past M and columns past N get an offset past
  // every range and read zeros. With 16-byte rows (ALIGNED) a load moves a 4-float vector,
  // otherwise one float (8 or 32 loads per thread and stage).
  constexpr int kPer = ALIGNED ? 1 : 4, kLoads = 8 * kPer;
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  uint32_t xv[4], yv[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {  // x vector p: row (t + kT p) / 8, columns 4 (t % 8) ..
    const int row = (t + kT * p) >> 3;
    xv[p] = m0 + row < M ? (uint32_t)((row * K + (t & 7) * 4) * 4) : 0x80000000u;
  }
  const int ycol = (t % (BMN / 4)) * 4, yrow = (t / (BMN / 4)) * 4;  // y job: k rows yrow .. + 3, columns ycol ..
#pragma unroll
  for (int r = 0; r < 4; ++r) yv[r] = n0 + ycol < N ? (uint32_t)(((yrow + r) * N + ycol) * 4) : 0x80000000u;
  const int ycols = (int)std::min<int64_t>(N - n0 - ycol, 4);  // columns of the job inside N
  // The slice is wave-uniform; readfirstlane says so, and the per-step bases stay scalar.
  auto uni = [](const float* ptr) {
    const uint64_t a = reinterpret_cast<uint64_t>(ptr);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return reinterpret_cast<const float*>(((uint64_t)hi << 32) | lo);
  };
  const float* const xs = uni(x + m0 * K + kbeg);
  const float* const ys = uni(y + kbeg * N + n0);
  const int klen = __builtin_amdgcn_readfirstlane((int)(kend - kbeg));  // k rows of the slice (<= 0 past K)
  // Load i of stage kt: x vector i / kPer (below 4) or y row yrow + i / kPer - 4; element
  // i % kPer of it without ALIGNED. The y descriptor's range ends at the slice's last k row.
  auto load_one = [&](typename G::Stage& st, int kt, int i) {
    const int rem = klen - kt * 32;
    const int vi = i / kPer, e = i % kPer;
    if (vi < 4) {
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(xs + kt * 32), 0, 0x7ffffff0, 0x00020000);
      const uint32_t off = rem >= 32 || (t & 7) * 4 + e < rem ? xv[vi] + 4 * e : 0x80000000u;
      if constexpr (ALIGNED)
        st.a[vi] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
      else
        st.a[vi][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
    } else {
      // readfirstlane: the clamp would otherwise become a VALU med3, and the descriptor a VGPR.
      const int rows = __builtin_amdgcn_readfirstlane(rem < 0 ? 0 : rem < 32 ? rem : 32);
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc((void*)(ys + (int64_t)kt * 32 * N), 0, rows * (int)N * 4, 0x00020000);
      if constexpr (ALIGNED)
        st.b[0][vi - 4] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)yv[vi - 4], 0, 0));
      else
        st.b[0][vi - 4][e] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(r, e < ycols ? (int)(yv[vi - 4] + 4 * e) : (int)0x80000000, 0, 0));
    }
  };
  typename G::Stage st0, st1;
#pragma unroll
  for (int i = 0; i < kLoads; ++i) load_one(st0, 0, i);
  G::store(st0, lds, t);
#pragma unroll
  for (int i = 0; i < kLoads; ++i) load_one(st1, 1, i);
  __syncthreads();
  // Step kt: products from LDS stage kt & 1 in four groups of 4 k pairs (k = 16 (q / 2) +
  // 8 g + 4 (q % 2) + e for lane group g, the order G::compute uses), the next group's
  // fragments read ahead; between the 16 product pairs, the loads of stage kt + 2 into
  // `refill` (one per pair, or two) and the 8 LDS writes of stage kt + 1 from `next`.
  auto step = [&](int kt, typename G::Stage& refill, const typename G::Stage& next) {
    const char* cur = lds + (kt & 1) * G::kStageBytes;
    char* nxt = lds + ((kt + 1) & 1) * G::kStageBytes;
    f32x4 fa[2][kTM], fb[2][kTN];
    auto rd = [&](int q) {
      const int k0 = (q >> 1) * 16 + g * 8 + (q & 1) * 4;
#pragma unroll
      for (int i = 0; i < kTM; ++i) fa[q & 1][i] = *reinterpret_cast<const f32x4*>(cur + lds_off<float>(wm0 + 32 * i + l32, k0));
#pragma unroll
      for (int j = 0; j < kTN; ++j)
        fb[q & 1][j] = *reinterpret_cast<const f32x4*>(cur + BMN * 128 + lds_off<float>(wn0 + 32 * j + l32, k0));
    };
    rd(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q + 1 < 4) rd(q + 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int i = 0; i < kTM; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[q & 1][j][e], fa[q & 1][i][e], acc[j][i], 0, 0, 0);
        const int pi = q * 4 + e;
        if constexpr (ALIGNED) {
          if ((pi & 1) == 0)
            load_one(refill, kt + 2, pi >> 1);
          else
            G::store_part(next, nxt, t, pi >> 1);
        } else {
          load_one(refill, kt + 2, 2 * pi);
          load_one(refill, kt + 2, 2 * pi + 1);
          if (pi & 1) G::store_part(next, nxt, t, pi >> 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
  };
  // kslice is a multiple of 64, so nk is even and every pass runs both steps (a step behind a
  // branch would leave the wait counts at the loop head unsettled). Stages past the slice
  // read zeros and are never multiplied.
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, st0, st1);
    step(kt + 1, st1, st0);
  }

  // Slice s > 0 writes register r of accumulator i of its lane to dword
  // (i * 16 + r) * 128 + t of its exchange area; slice 0 reads the same places
  // (S > 1 runs 64 x 64 tiles only: kTN = 1, 128 threads per slice).
  float* const xch = reinterpret_cast<float*>(smem);
  if (slice > 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) xch[((slice - 1) * 32 + i * 16 + r) * 128 + t] = acc[0][i][r];
  }
  __syncthreads();
  if (slice > 0) return;
#pragma unroll
  for (int s2 = 1; s2 < S; ++s2)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[0][i][r] += xch[((s2 - 1) * 32 + i * 16 + r) * 128 + t];

  // Register r of accumulator (j, i) of lane (l32, g):
  // C[m0 + wm0 + i*32 + l32][n0 + wn0 + j*32 + (r/4)*8 + g*4 + r%4].
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
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
            *reinterpret_cast<f32x4*>(dst) =
                f32x4{acc[j][i][q * 4 + 0], acc[j][i][q * 4 + 1], acc[j][i][q * 4 + 2], acc[j][i][q * 4 + 3]};
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) dst[e] = Elem<TO>::from_f32(acc[j][i][q * 4 + e]);
        }
      }
    }
}

// ===========================================================================
// GELU epilogues (the MLP of model/gpt.py:141: jax.nn.gelu(approximate=True))
// ===========================================================================
// gelu(u) = u/2 (1 + tanh(z)), z = b (u + c u^3), b = sqrt(2/pi), c = 0.044715,
// written as u s with s = (1 + tanh z)/2 = 1 / (1 + 2^(-2 z log2 e)): one exp2
// and one reciprocal instead of a libm tanh (the epilogue runs once per output
// element, after the products, with nothing to hide it behind), and no
// cancellation in 1 + tanh z at negative u. gelu'(u) = s + 2 u s (1 - s) b (1 + 3 c u^2).
// Both in f32 from the bf16-rounded u, as an elementwise pass over the rounded
// product computes them.
constexpr int kEpiNone = 0, kEpiGelu = 1, kEpiGeluGrad = 2;
constexpr float kGeluB = 0.7978845608028654f, kGeluC = 0.044715f;
constexpr float kGeluE = -2.0f * kGeluB * 1.4426950408889634f;  // -2 b log2(e)

__device__ __forceinline__ float gelu_gate(float u) {  // s = (1 + tanh z) / 2
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(kGeluE * (u + kGeluC * u * u * u)));
}
__device__ __forceinline__ float gelu_tanh(float u) { return u * gelu_gate(u); }
__device__ __forceinline__ float gelu_tanh_grad(float u) {
  const float s = gelu_gate(u);
  return s + 2.f * u * s * (1.f - s) * kGeluB * (1.f + 3.f * kGeluC * u * u);
}

// Four consecutive outputs v = bf16(x . y) of one row. kEpiGelu: aux <- v (the
// pre-activation), out <- bf16(gelu(v)). kEpiGeluGrad: u is the pre-activation
// (read from aux); out <- bf16(v * gelu'(u)) (v is the incoming gradient).
__device__ __forceinline__ void gelu_store(const bf16x4& v, bf16* out, bf16* aux) {
  *reinterpret_cast<bf16x4*>(aux) = v;
  bf16x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (bf16)gelu_tanh((float)v[e]);
  *reinterpret_cast<bf16x4*>(out) = r;
}
__device__ __forceinline__ void gelu_grad_store(const bf16x4& v, const bf16x4& u, bf16* out) {
  bf16x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (bf16)((float)v[e] * gelu_tanh_grad((float)u[e]));
  *reinterpret_cast<bf16x4*>(out) = r;
}
template <int EPI>
__device__ __forceinline__ void gelu_epilogue(const bf16x4& v, bf16* out, bf16* aux) {
  if constexpr (EPI == kEpiGelu)
    gelu_store(v, out, aux);
  else
    gelu_grad_store(v, *reinterpret_cast<const bf16x4*>(aux), out);
}

// The same epilogue as a pass of its own, for products the DMA kernel does not
// take: kEpiGelu reads the pre-activation from aux, kEpiGeluGrad the gradient
// from out (both written there by the plain product).
template <int EPI>
__global__ __launch_bounds__(256) void gelu_pass_kernel(bf16* __restrict__ out, bf16* __restrict__ aux, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if constexpr (EPI == kEpiGelu)
    out[i] = (bf16)gelu_tanh((float)aux[i]);
  else
    out[i] = (bf16)((float)out[i] * gelu_tanh_grad((float)aux[i]));
}

// ===========================================================================
// bf16 GEMM on DMA-fed LDS tiles (K % 64 == 0, N % 8 == 0, 16-byte aligned)
// ===========================================================================
// 256 x 256 output tile per workgroup of 8 waves, 64 k per step through two
// LDS stages filled by buffer_load ... lds. Wave w owns output rows
// 128 (w / 4) .. +127 and columns 64 (w % 4) .. +63, computed as C^T tiles:
// A = y^T fragments (transposed reads of the y tile), B = x row fragments.
//
// x tile (256 rows of 64 k, 128 bytes each): four 64-row subtiles; row r of a
// subtile sits in 1 KB block r % 8 at position r / 8, blocks 1040 bytes apart,
// so a 16-lane row read (16 consecutive rows, one 16-byte chunk) covers 16
// different bank slots.
struct GemmXTile {
  static constexpr int kRowBytes = 128, kStride = 1040;
  static constexpr int kSubBytes = 8 * kStride;
  static constexpr int kBytes = 4 * kSubBytes;
  static __host__ __device__ constexpr int off(int row, int byte) {
    return (row >> 6) * kSubBytes + (row & 7) * kStride + ((row >> 3) & 7) * kRowBytes + byte;
  }
  // Instruction i = 8 s + b fills block b of subtile s: lane L takes row
  // 64 s + b + 8 (L / 8), 16-byte chunk L % 8.
  static __device__ __forceinline__ int dma_row(int i, int L) { return 64 * (i >> 3) + (i & 7) + 8 * (L >> 3); }
  static __host__ __device__ constexpr int block_off(int i) { return (i >> 3) * kSubBytes + (i & 7) * kStride; }
};

// y tile (64 k-rows of 256 columns, 512 bytes each): block 4p + m holds rows
// m + 8p and m + 8p + 4, blocks 1088 bytes apart, so the four consecutive rows
// of a transposed read lie in the four 64-byte bank groups.
struct GemmYTile {
  static constexpr int kRowBytes = 512, kStride = 1088;
  static constexpr int kBytes = 32 * kStride;
  static __host__ __device__ constexpr int off(int row, int byte) {
    return ((row & 3) + 4 * (row >> 3)) * kStride + ((row >> 2) & 1) * kRowBytes + byte;
  }
  static __device__ __forceinline__ int dma_row(int b, int L) { return (b & 3) + 8 * (b >> 2) + 4 * (L >> 5); }
  static __host__ __device__ constexpr int block_off(int b) { return b * kStride; }
};

struct Gemm2 {
  static constexpr int kWaves = 8, kThreads = 64 * kWaves;
  static constexpr int BM = 256, BN = 256, BK = 64;
  static constexpr int kDma = 32 / kWaves;  // instructions per wave per stage, for x and for y
};

// Each operand tile is 256 free indices (m for x, n for y) by 64 k. An operand
// stored k-contiguous (x as [M,K], or y given transposed as [N,K]) is staged in
// the GemmXTile layout and read with plain 16-byte reads; one stored
// free-index-contiguous (y as [K,N], or x given transposed as [K,M]) is staged
// in the GemmYTile layout and read with transposing reads. Both reads hand the
// MFMA the same fragment: lane l32 = free index, lane group g = 8 k values.
template <bool KCONTIG>
struct OperandTile {
  static constexpr int kBytes = KCONTIG ? GemmXTile::kBytes : GemmYTile::kBytes;
  static constexpr int kReads = KCONTIG ? 1 : 2;  // LDS read instructions per fragment
  static __host__ __device__ constexpr int block_off(int i) {
    return KCONTIG ? GemmXTile::block_off(i) : GemmYTile::block_off(i);
  }
  // Lane's byte offset for DMA instruction i, relative to the tile's first element in
  // global memory (ld = leading dimension in elements); 0x80000000 (past any buffer
  // range, so the lane writes zeros) for free indices past `nfree`.
  static __device__ __forceinline__ uint32_t dma_off(int i, int lane, int ld, int free0, int nfree) {
    if constexpr (KCONTIG) {
      const int r = GemmXTile::dma_row(i, lane);
      return free0 + r < nfree ? (uint32_t)(((int64_t)r * ld + (lane & 7) * 8) * 2) : 0x80000000u;
    } else {
      const int r = GemmYTile::dma_row(i, lane);
      const int c = (lane & 31) * 8;
      return free0 + c < nfree ? (uint32_t)(((int64_t)r * ld + c) * 2) : 0x80000000u;
    }
  }
  // Lane base for fragment reads.
  static __device__ __forceinline__ int lane_base(int lane) {
    const int l32 = lane & 31, g = lane >> 5;
    if constexpr (KCONTIG)
      return GemmXTile::off(l32, 16 * g);
    else
      return GemmYTile::off(8 * g + ((lane & 15) >> 2), 2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));
  }
  // Fragment of free indices f0 .. f0 + 31 (f0 % 32 == 0) and k = 16 kk + (0..15).
  static __device__ __forceinline__ bf16x8 read(const char* base, int kk, int f0) {
    if constexpr (KCONTIG)
      return *reinterpret_cast<const bf16x8*>(base + GemmXTile::off(f0, 32 * kk));
    else
      return tr_frag(base + GemmYTile::off(16 * kk, 2 * f0), GemmYTile::off(4, 0));
  }
};

// out[M,N] (or, with a K split, the f32 partial slab of K slice blockIdx.x / tiles)
// = x . y over this slice. XT: x is given transposed, stored [K,M]; YT: y is given
// transposed, stored [N,K]. BM = 256 or 128 output rows per workgroup (128 only
// with a k-contiguous x, whose tile is then the first two 64-row subtiles).
template <typename TO, bool XT, bool YT, int BM = 256, int SLOTS = 2, int EPI = kEpiNone, int W = 8>
__global__ __launch_bounds__(64 * W, W == 8 ? 2 : 1) void gemm_dma_kernel(const bf16* __restrict__ x, const bf16* __restrict__ y,
                                                          TO* __restrict__ out, int M, int N, int K, int tiles_m,
                                                          int tiles_n, int kslice, bf16* __restrict__ aux) {
  typedef Gemm2 G;
  typedef OperandTile<!XT> XTl;
  typedef OperandTile<YT> YTl;
  static_assert(BM == 256 || (BM == 128 && !XT), "128-row tiles need a k-contiguous x");
  static_assert(SLOTS == 2 || (SLOTS == 3 && BM == 128), "three LDS stages fit 128-row tiles only");
  static_assert(EPI == kEpiNone || sizeof(TO) == 2, "the GELU epilogues write bf16");
  static_assert(W == 8 || (W == 4 && BM == 256), "four waves own 128 x 128 each of a 256-row tile");
  // W = 8: wave w owns rows (w / 4) BM/2 .., columns (w % 4) 64 ..; W = 4: wave w owns
  // rows (w / 2) 128 .., columns (w % 2) 128 .. (one wave per SIMD, accumulators in AGPRs).
  constexpr int YF = W == 8 ? 2 : 4;         // y fragments (32 columns each) per wave and k-step
  constexpr int XF = W == 8 ? BM / 64 : 4;   // x fragments (32 rows each) per wave and k-step
  constexpr int kDmaX = BM / 8 / W;          // x DMA instructions per wave and stage
  constexpr int kDmaY = 32 / W;              // y DMA instructions per wave and stage
  constexpr int kXBytes = BM == 256 ? XTl::kBytes : 2 * GemmXTile::kSubBytes;
  constexpr int kStageBytes = kXBytes + YTl::kBytes;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lane = threadIdx.x & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // K slice (slowest-varying block index), then the tile. Tiles of one XCD
  // (blocks are dealt to the 8 XCDs round robin) are made consecutive and ordered
  // in groups of 4 tile rows, so an XCD's L2 holds few x and y panels.
  const int ntiles = tiles_m * tiles_n;
  const int slice = blockIdx.x / ntiles;
  int v = blockIdx.x - slice * ntiles;
  if (ntiles % 8 == 0) v = (v % 8) * (ntiles / 8) + v / 8;
  constexpr int kGroup = 4;
  const int group = v / (kGroup * tiles_n);
  const int first_m = group * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int tm = first_m + (v % (kGroup * tiles_n)) % gsize;
  const int tn = (v % (kGroup * tiles_n)) / gsize;
  const int m0 = tm * BM, n0 = tn * G::BN;
  const int wm0 = W == 8 ? (wave >> 2) * (BM / 2) : (wave >> 1) * 128;
  const int wn0 = W == 8 ? (wave & 3) * 64 : (wave & 1) * 128;
  const int kbeg = slice * kslice;
  const int nk = min(K - kbeg, kslice) / G::BK;
  out += (int64_t)slice * M * N;

  // Per-lane DMA offsets; free indices past M or N read as zeros.
  uint32_t xoff[kDmaX], yoff[kDmaY];
#pragma unroll
  for (int i = 0; i < kDmaX; ++i) xoff[i] = XTl::dma_off(wave + W * i, lane, XT ? M : K, m0, M);
#pragma unroll
  for (int i = 0; i < kDmaY; ++i) yoff[i] = YTl::dma_off(wave + W * i, lane, YT ? K : N, n0, N);
  // DMA instruction q (x instructions first, then y) of stage kt. A stage past
  // the slice gets an empty buffer range: its instructions read nothing and
  // write zeros into a slot that no later stage reads.
  auto issue_one = [&](int kt, int q) {
    char* st = smem + (kt % SLOTS) * kStageBytes;
    const int k0 = kbeg + kt * G::BK;
    const uint32_t range = kt < nk ? 0x7ffffff0u : 0u;
    if (q < kDmaX) {
      const u32x4 rx = buffer_rsrc(XT ? x + (int64_t)k0 * M + m0 : x + (int64_t)m0 * K + k0, range);
      dma16(rx, st + XTl::block_off(wave + W * q), xoff[q]);
    } else {
      const u32x4 ry = buffer_rsrc(YT ? y + (int64_t)n0 * K + k0 : y + (int64_t)k0 * N + n0, range);
      dma16(ry, st + kXBytes + YTl::block_off(wave + W * (q - kDmaX)), yoff[q - kDmaX]);
    }
  };
  constexpr int kDmaWave = kDmaX + kDmaY;  // DMA instructions per wave and stage
  auto issue = [&](int kt) {
#pragma unroll
    for (int q = 0; q < kDmaWave; ++q) issue_one(kt, q);
  };

  f32x16 acc[YF][XF];
#pragma unroll
  for (int j = 0; j < YF; ++j)
#pragma unroll
    for (int i = 0; i < XF; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  const int xb = XTl::lane_base(lane);
  const int yb = YTl::lane_base(lane);
  // Per k-step of 16: NM products over YF y fragments (A operand) and XF x
  // fragments (B).
  constexpr int NM = YF * XF;
  constexpr int NFR = YF + XF;
  static_assert(NFR <= NM, "one fragment read per product slot at most");
  constexpr int NSLOT = 4 * NM;  // product slots per 64-deep stage

  // SLOTS stages in a ring: stage kt + SLOTS - 1 is loaded while stage kt is
  // multiplied, into the slot that stage kt - 1 left at this step's barrier.
  // The program order is the schedule: product slot i holds one MFMA, at most
  // one fragment read for the next k-step and at most one DMA instruction, and
  // a scheduling fence closes it. The DMA instructions go out one at a time
  // between products (issued together after the barrier, the eight waves
  // queue in the CU's address path and stall their products): over the first
  // half of the stage with two slots, so the last lands before the next
  // barrier, and over the whole stage with three.
  constexpr int kDmaSpan = SLOTS == 3 ? NSLOT : NSLOT / 2;
  issue(0);
  if (SLOTS == 3 && nk > 1) issue(1);
  for (int kt = 0; kt < nk; ++kt) {
    if (SLOTS == 3 && kt + 1 < nk)
      wait_vmem<kDmaWave>();  // stage kt has landed; stage kt + 1 may be in flight
    else
      wait_vmem<0>();
    lds_barrier();
    const int kload = kt + SLOTS - 1;
    const char* xs = smem + (kt % SLOTS) * kStageBytes + xb;
    const char* ys = smem + (kt % SLOTS) * kStageBytes + kXBytes + yb;
    bf16x8 fa[2][YF], fb[2][XF];
    // Fragment f of k-step kk in the order of first use by the products
    // (j, i) = (r / XF, r % XF): y 0, x 0 .. XF - 1, then y 1 .. YF - 1.
    auto read = [&](int kk, int f) {
      if (f == 0)
        fa[kk & 1][0] = YTl::read(ys, kk, wn0);
      else if (f <= XF)
        fb[kk & 1][f - 1] = XTl::read(xs, kk, wm0 + 32 * (f - 1));
      else
        fa[kk & 1][f - XF] = YTl::read(ys, kk, wn0 + 32 * (f - XF));
    };
#pragma unroll
    for (int f = 0; f < NFR; ++f) read(0, f);
    __builtin_amdgcn_sched_barrier(0);
#pragma clang loop unroll(full)
    for (int i = 0; i < NSLOT; ++i) {
      const int kk = i / NM, r = i % NM, c = kk & 1;
      if (kk + 1 < 4 && r < NFR) read(kk + 1, r);
#pragma unroll
      for (int q = 0; q < kDmaWave; ++q)
        if (i == (2 * q + 1) * kDmaSpan / (2 * kDmaWave)) issue_one(kload, q);
      mma32(fa[c][r / XF], fb[c][r % XF], acc[r / XF][r % XF]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vmem<0>();  // the empty loads past the slice have landed too

  // Epilogue: acc[j][i] is a C^T tile; register r of lane (l32, g) is
  // C[m0 + wm0 + 32 i + l32][n0 + wn0 + 32 j + (r / 4) * 8 + g * 4 + r % 4].
  // Stored straight from there, every store instruction would touch 32 rows
  // (32 cache lines for 512 bytes). Each 32-row group of the wave's outputs
  // goes through the wave's own part of the (now idle) stage ring instead:
  // written as 16-byte chunks XOR-swizzled by row, read back 16 bytes per lane,
  // so that each store instruction writes whole row segments of the wave's
  // YF * 32 columns. The barrier: every wave has finished its fragment reads
  // and every DMA has landed (each wave waited for its own just above).
  constexpr int kEs = sizeof(TO), kRowBytes = YF * 32 * kEs, kCh = kRowBytes / 16, kRowsPerInst = 64 / kCh;
  constexpr int kPer = 16 / kEs;  // outputs per 16-byte chunk
  static_assert(W * 32 * kRowBytes <= SLOTS * kStageBytes, "every wave's row group fits the stage ring");
  lds_barrier();
  char* const ep = smem + wave * (32 * kRowBytes);
#pragma unroll
  for (int i = 0; i < XF; ++i) {
#pragma unroll
    for (int j = 0; j < YF; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (kEs == 2) {
          const int ch = 4 * j + q;  // columns 32 j + 8 q .. + 7; this lane's half 4 g .. + 3
          *reinterpret_cast<bf16x4*>(ep + l32 * kRowBytes + ((ch ^ (l32 & (kCh - 1))) * 16) + 8 * g) =
              bf16x4{(bf16)acc[j][i][4 * q], (bf16)acc[j][i][4 * q + 1], (bf16)acc[j][i][4 * q + 2],
                     (bf16)acc[j][i][4 * q + 3]};
        } else {
          const int ch = 8 * j + 2 * q + g;  // columns 32 j + 8 q + 4 g .. + 3
          *reinterpret_cast<f32x4*>(ep + l32 * kRowBytes + ((ch ^ (l32 & (kCh - 1))) * 16)) =
              f32x4{acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
        }
      }
    const int mg = m0 + wm0 + 32 * i;
#pragma unroll
    for (int rr = 0; rr < 32 / kRowsPerInst; ++rr) {
      const int r = rr * kRowsPerInst + lane / kCh, c = lane % kCh;
      const int m = mg + r, n = n0 + wn0 + c * kPer;
      const u32x4 w4 = *reinterpret_cast<const u32x4*>(ep + r * kRowBytes + ((c ^ (r & (kCh - 1))) * 16));
      // N % 8 == 0: a chunk is either all in or all out.
      if (m < M && n < N) {
        TO* dst = out + (int64_t)m * N + n;
        if constexpr (EPI == kEpiNone) {
          *reinterpret_cast<u32x4*>(dst) = w4;
        } else {
          const bf16x8 v = __builtin_bit_cast(bf16x8, w4);
          const bf16x4 lo = {v[0], v[1], v[2], v[3]}, hi = {v[4], v[5], v[6], v[7]};
          bf16* const a = aux + (int64_t)m * N + n;
          if constexpr (EPI == kEpiGelu) {
            gelu_store(lo, reinterpret_cast<bf16*>(dst), a);
            gelu_store(hi, reinterpret_cast<bf16*>(dst) + 4, a + 4);
          } else {
            const bf16x8 u = *reinterpret_cast<const bf16x8*>(a);
            gelu_grad_store(lo, bf16x4{u[0], u[1], u[2], u[3]}, reinterpret_cast<bf16*>(dst));
            gelu_grad_store(hi, bf16x4{u[4], u[5], u[6], u[7]}, reinterpret_cast<bf16*>(dst) + 4);
          }
        }
      }
    }
  }
}

// out = sum over the K slices of the f32 partial slabs, in slice order
// (deterministic), cast to TO. MN % 4 == 0.
// The part's bf16 MFMA ceiling: every wave streams v_mfma_f32_32x32x16_bf16
// over eight independent accumulators (a product waits for its own
// accumulator only every eighth instruction, past the instruction's latency)
// with register operands, no memory traffic and no other work. Operands are
// varied bf16 values (not zeros or constants), so the matrix pipes switch as
// they do on real data; the clock that load sustains sets the rate. Each wave
// writes one float of its accumulators to sink so nothing is dead code.
__global__ __launch_bounds__(512, 1) void mfma_ceiling_kernel(float* __restrict__ sink, int iters) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t hsh = (uint32_t)(lane * 8 + e + 1) * 2654435761u;
    a[e] = (bf16)((float)((hsh >> 8) & 0xffff) * (1.0f / 65536.0f) - 0.5f);
    b[e] = (bf16)((float)((hsh >> 16) & 0xff) * (1.0f / 256.0f) - 0.5f);
  }
  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) t += acc[j][r];
  if (lane == 0) sink[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = t;
}

template <typename TO, int EPI = kEpiNone>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part, TO* __restrict__ out,
                                                                int64_t mn, int slices, bf16* __restrict__ aux) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= mn) return;
  f32x4 acc = *reinterpret_cast<const f32x4*>(part + i);
  for (int s = 1; s < slices; ++s) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(part + (int64_t)s * mn + i);
    acc += v;
  }
  if constexpr (EPI != kEpiNone)
    gelu_epilogue<EPI>(bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]}, reinterpret_cast<bf16*>(out + i),
                       aux + i);
  else if constexpr (sizeof(TO) == 2)
    *reinterpret_cast<bf16x4*>(out + i) = bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
  else
    *reinterpret_cast<f32x4*>(out + i) = acc;
}

template <typename T, typename TO, int BM, int BN, int BK, int WM, int WN, bool AL>
void launch_gemm_kernel(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, int64_t tiles,
                        int64_t tiles_n, size_t lds, hipStream_t stream) {
  auto k = gemm_kernel<T, TO, BM, BN, BK, WM, WN, AL>;
  (void)allow_lds((const void*)k, (int)lds, stream, "ferrite_matmul");  // a failure resurfaces as the launch's error
  hipLaunchKernelGGL(k, dim3((unsigned)tiles), dim3(WM * WN * 64), lds, stream, static_cast<const T*>(x),
                     static_cast<const T*>(y), static_cast<TO*>(out), M, N, K, (int)tiles_n);
}

template <typename T, typename TO, int BM, int BN, int BK, int WM, int WN>
int launch_gemm(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  typedef Gemm<T, TO, BM, BN, BK, WM, WN, true> G;
  const int64_t tiles_m = cdiv(M, BM), tiles_n = cdiv(N, BN);
  if (tiles_m * tiles_n > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "matmul: output too large");
  const size_t lds = 2 * (size_t)G::kStageBytes;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool aligned =
      K % Elem<T>::kVec == 0 && N % Elem<T>::kVec == 0 && N % 4 == 0 && a16(x) && a16(y) && a16(out);
  if (aligned)
    launch_gemm_kernel<T, TO, BM, BN, BK, WM, WN, true>(x, y, out, M, N, K, tiles_m * tiles_n, tiles_n, lds, stream);
  else
    launch_gemm_kernel<T, TO, BM, BN, BK, WM, WN, false>(x, y, out, M, N, K, tiles_m * tiles_n, tiles_n, lds, stream);
  return check_launch("ferrite_matmul");
}

// The K split of an f32 product with few output tiles (64 x 64 each): S slices per
// workgroup (gemm_f32_slices_kernel), 4 or 2 while the workgroups' waves stay within
// two per SIMD and each slice is at least 128 deep (1000^3: 256 tiles x 4 slices x 2
// waves = two waves per SIMD); when that still fills under half the SIMDs, G groups
// of S slices in G workgroups per tile, summed by a second pass (512 x 512 x 2048:
// 64 tiles, S = 4, G = 4).
struct F32Split {
  int s, g;
};
F32Split f32_split(int64_t M, int64_t N, int64_t K, int64_t cus) {
  const int64_t tiles = cdiv(M, (int64_t)64) * cdiv(N, (int64_t)64);
  const int64_t waves = 8 * cus;  // two per SIMD
  int s = K >= 512 ? 4 : K >= 256 ? 2 : 1;
  while (s > 1 && tiles * 2 * s > waves) s /= 2;
  int64_t g = 1;
  if (2 * tiles * 2 * s <= waves && (M * N) % 4 == 0)
    g = std::min<int64_t>({cdiv(waves, tiles * 2 * s), K / (128 * s), (int64_t)8});
  return {s, (int)std::max<int64_t>(g, 1)};
}
int64_t f32_workspace(int64_t M, int64_t N, int64_t K, int64_t cus) {
  const F32Split sp = f32_split(M, N, K, cus);
  return sp.g > 1 ? (int64_t)sp.g * M * N * (int64_t)sizeof(float) : 0;
}

template <typename TO, int S, int BMN = 64>
void launch_gemm_f32_slices(const float* x, const float* y, TO* out, int64_t M, int64_t N, int64_t K, int groups,
                            hipStream_t stream) {
  typedef Gemm<float, TO, BMN, BMN, 32, BMN / 64, 2, true> G;
  const int64_t tiles_n = cdiv(N, (int64_t)BMN), tiles = cdiv(M, (int64_t)BMN) * tiles_n;
  const size_t lds = (size_t)S * 2 * G::kStageBytes;
  static_assert((S - 1) * 32 * 128 * 4 <= S * 2 * G::kStageBytes, "the slices' accumulators fit the stages");
  const int64_t kslice = cdiv(cdiv(K, (int64_t)S * groups), (int64_t)64) * 64;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool aligned = K % 4 == 0 && N % 4 == 0 && a16(x) && a16(y) && a16(out);
  auto go = [&](auto kern) {
    (void)allow_lds((const void*)kern, (int)lds, stream, "ferrite_matmul");  // a failure resurfaces as the launch's error
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)groups), dim3(G::kThreads * S), lds, stream, x, y, out, M,
                       N, K, (int)tiles_n, kslice);
  };
  if (aligned)
    go(gemm_f32_slices_kernel<TO, S, true, BMN>);
  else
    go(gemm_f32_slices_kernel<TO, S, false, BMN>);
}

// f32 products with at least a CU's worth of 128 x 128 tiles: the pipelined loop on those
// tiles (four waves, no K split), while its lane offsets (128 x rows of K floats, 32 y rows
// of N) stay under 2^31 bytes; else the register-staged 128 x 128 kernel.
template <typename TO>
int launch_gemm_f32_big(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (128 * K * 4 < 0x7ffffff0 && 32 * N * 4 < 0x7ffffff0) {
    launch_gemm_f32_slices<TO, 1, 128>(static_cast<const float*>(x), static_cast<const float*>(y), static_cast<TO*>(out),
                                       M, N, K, 1, stream);
    return check_launch("ferrite_matmul");
  }
  return launch_gemm<float, TO, 128, 128, 32, 2, 2>(x, y, out, M, N, K, stream);
}

template <typename TO, int S>
int launch_gemm_f32_split(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, int groups,
                          void* ws, hipStream_t stream) {
  const float* xf = static_cast<const float*>(x);
  const float* yf = static_cast<const float*>(y);
  if (groups > 1) {
    launch_gemm_f32_slices<float, S>(xf, yf, static_cast<float*>(ws), M, N, K, groups, stream);
    const int64_t mn = M * N;
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<TO>), dim3((unsigned)cdiv(mn / 4, 256)), dim3(256), 0, stream,
                       static_cast<const float*>(ws), static_cast<TO*>(out), mn, groups, nullptr);
  } else {
    launch_gemm_f32_slices<TO, S>(xf, yf, static_cast<TO*>(out), M, N, K, 1, stream);
  }
  return check_launch("ferrite_matmul");
}

template <typename TO>
int launch_gemm_f32_small(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, void* ws,
                          int64_t ws_bytes, hipStream_t stream) {
  const int64_t cus = cu_count(stream);
  F32Split sp = f32_split(M, N, K, cus);
  if (sp.g > 1 && (ws == nullptr || ws_bytes < f32_workspace(M, N, K, cus) || (reinterpret_cast<uintptr_t>(ws) & 15)))
    sp.g = 1;
  // The sliced kernel's lane offsets (64 x rows of K, 32 y rows of N bytes) stay under 2^31.
  const bool offsets_fit = 64 * K * 4 < 0x7ffffff0 && 32 * N * 4 < 0x7ffffff0;
  if (offsets_fit && sp.s == 4) return launch_gemm_f32_split<TO, 4>(x, y, out, M, N, K, sp.g, ws, stream);
  if (offsets_fit && sp.s == 2) return launch_gemm_f32_split<TO, 2>(x, y, out, M, N, K, sp.g, ws, stream);
  return launch_gemm<float, TO, 64, 64, 32, 1, 2>(x, y, out, M, N, K, stream);
}

// K slices for a problem with few output tiles: as many slices as keep every
// workgroup in one round (one per CU), each at least 512 deep; 1 when the tiles
// already fill most CUs or the f32 partials would outweigh the work. A round
// that spills over by a few workgroups costs a whole second round: 36 tiles in
// 8 slices (288 workgroups on 256 CUs) take longer than in 7.
int splitk_slices(int64_t M, int64_t N, int64_t K, int64_t cus) {
  const int64_t tiles = cdiv(M, (int64_t)Gemm2::BM) * cdiv(N, (int64_t)Gemm2::BN);
  // Up to half the CUs busy and a long K (the 8192 x 768 outputs of a 768-wide model): two
  // slices fill 3/4 of the CUs, and the two f32 partial slabs stay in the Infinity Cache.
  if (tiles >= cus / 4) return (2 * tiles <= cus && K >= 2048) ? 2 : 1;
  int64_t s = std::min<int64_t>({cus / tiles, K / 512, (int64_t)16});
  if (s < 2) return 1;
  const int64_t kslice = cdiv(cdiv(K, s), (int64_t)Gemm2::BK) * Gemm2::BK;
  return (int)cdiv(K, kslice);
}

int64_t splitk_workspace(int64_t M, int64_t N, int64_t K, int64_t cus) {
  const int s = splitk_slices(M, N, K, cus);
  return s > 1 ? (int64_t)s * M * N * (int64_t)sizeof(float) : 0;
}

// f32 products too small for 128 x 128 tiles on every CU run 64 x 64 tiles
// (launch_gemm_f32_small).
bool f32_small(int64_t M, int64_t N, int64_t cus) { return cdiv(M, (int64_t)128) * cdiv(N, (int64_t)128) < cus; }

// Output rows per workgroup. 128-row tiles (k-contiguous x only) halve the work of a
// tile, so a problem whose 256-row tiles spill into a mostly empty round, or fill
// less than half the CUs, runs in fewer or shorter rounds: 8192 x 2304 takes 288
// 256-row tiles (two rounds on 256 CUs) but 576 128-row ones (three rounds of half
// the work), and 8192 x 768 one round of 192 tiles instead of 96 tiles or a K split.
// A 128-row tile moves more bytes per product, costed at 0.55 of a 256-row one.
// With fewer than a quarter of the CUs' worth of 256-row tiles the K split is used.
int pick_bm(int64_t M, int64_t N, bool xt, int64_t cus) {
  if (xt) return 256;
  const int64_t t256 = cdiv(M, (int64_t)256) * cdiv(N, (int64_t)Gemm2::BN);
  const int64_t t128 = cdiv(M, (int64_t)128) * cdiv(N, (int64_t)Gemm2::BN);
  if (t256 < cus / 4) return 256;
  return 11 * cdiv(t128, cus) < 20 * cdiv(t256, cus) ? 128 : 256;
}

// Four waves of 128 x 128 outputs per 256 x 256 tile (one per SIMD, accumulators in
// AGPRs) read a third fewer LDS bytes per product than eight waves of 128 x 64, but
// have no second wave to cover a workgroup's start and end. They pay from four
// rounds of workgroups on: 8192^3 1244 -> 1372 TFLOP/s, 8192 x 4096 x 4096 level,
// 4096^3 (one round) 2-5% slower. Both give bitwise the same output.
bool use_four_waves(int64_t M, int64_t N, int64_t cus) {
  return cdiv(M, (int64_t)256) * cdiv(N, (int64_t)256) >= 4 * cus;
}

template <typename TO, bool XT, bool YT, int EPI = kEpiNone>
int launch_gemm_dma_t(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, void* ws,
                      int64_t ws_bytes, hipStream_t stream, void* aux = nullptr) {
  typedef Gemm2 G;
  bf16* const ax = static_cast<bf16*>(aux);
  const int64_t cus = cu_count(stream);
  if constexpr (!XT) {
    if (pick_bm(M, N, XT, cus) == 128) {
      constexpr int kLds128 = 3 * (2 * GemmXTile::kSubBytes + OperandTile<YT>::kBytes);
      static_assert(kLds128 <= 160 * 1024, "three stages of a 128-row tile fit the LDS");
      const int64_t tiles_m = cdiv(M, (int64_t)128), tiles_n = cdiv(N, G::BN);
      auto kern = gemm_dma_kernel<TO, false, YT, 128, 3, EPI>;
      if (int rc = allow_lds((const void*)kern, kLds128, stream, "ferrite_matmul")) return rc;
      hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n)), dim3(G::kThreads), kLds128, stream,
                         static_cast<const bf16*>(x), static_cast<const bf16*>(y), static_cast<TO*>(out), (int)M,
                         (int)N, (int)K, (int)tiles_m, (int)tiles_n, (int)K, ax);
      return check_launch("ferrite_matmul");
    }
  }
  const int64_t tiles_m = cdiv(M, G::BM), tiles_n = cdiv(N, G::BN);
  int slices = splitk_slices(M, N, K, cus);
  if (slices > 1 && (ws == nullptr || ws_bytes < splitk_workspace(M, N, K, cus) || (M * N) % 4 != 0 ||
                     (reinterpret_cast<uintptr_t>(ws) & 15) != 0))
    slices = 1;
  const int kslice = slices > 1 ? (int)(cdiv(cdiv(K, slices), (int64_t)G::BK) * G::BK) : (int)K;
  constexpr int kLds = 2 * (OperandTile<!XT>::kBytes + OperandTile<YT>::kBytes);
  const dim3 grid((unsigned)(tiles_m * tiles_n * slices));
  if (slices == 1) {
    // The GELU epilogues keep eight waves: with four, the 128 x 128 accumulators of a wave
    // and the epilogue's operands do not fit its registers (12 bytes per lane spilled).
    const bool w4 = EPI == kEpiNone && use_four_waves(M, N, cus);
    auto kern = gemm_dma_kernel<TO, XT, YT, 256, 2, EPI, 8>;
    if constexpr (EPI == kEpiNone)
      if (w4) kern = gemm_dma_kernel<TO, XT, YT, 256, 2, EPI, 4>;
    if (int rc = allow_lds((const void*)kern, kLds, stream, "ferrite_matmul")) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(w4 ? 256 : G::kThreads), kLds, stream, static_cast<const bf16*>(x),
                       static_cast<const bf16*>(y), static_cast<TO*>(out), (int)M, (int)N, (int)K, (int)tiles_m,
                       (int)tiles_n, kslice, ax);
  } else {
    auto kern = gemm_dma_kernel<float, XT, YT>;
    if (int rc = allow_lds((const void*)kern, kLds, stream, "ferrite_matmul")) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(G::kThreads), kLds, stream, static_cast<const bf16*>(x),
                       static_cast<const bf16*>(y), static_cast<float*>(ws), (int)M, (int)N, (int)K, (int)tiles_m,
                       (int)tiles_n, kslice, nullptr);
    const int64_t mn = M * N;
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<TO, EPI>), dim3((unsigned)cdiv(mn / 4, 256)), dim3(256), 0, stream,
                       static_cast<const float*>(ws), static_cast<TO*>(out), mn, slices, ax);
  }
  return check_launch("ferrite_matmul");
}

template <typename TO, int EPI = kEpiNone>
int launch_gemm_dma(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K, bool xt, bool yt,
                    void* ws, int64_t ws_bytes, hipStream_t stream, void* aux = nullptr) {
  if (xt && yt) return launch_gemm_dma_t<TO, true, true, EPI>(x, y, out, M, N, K, ws, ws_bytes, stream, aux);
  if (xt) return launch_gemm_dma_t<TO, true, false, EPI>(x, y, out, M, N, K, ws, ws_bytes, stream, aux);
  if (yt) return launch_gemm_dma_t<TO, false, true, EPI>(x, y, out, M, N, K, ws, ws_bytes, stream, aux);
  return launch_gemm_dma_t<TO, false, false, EPI>(x, y, out, M, N, K, ws, ws_bytes, stream, aux);
}

// Whether the DMA-fed kernel takes this problem: whole 64-deep k steps, N % 8 == 0 (and
// M % 8 == 0 for a transposed x), 16-byte pointers, and every lane offset inside the 31-bit
// buffer range (256 free rows of a k-contiguous operand, 64 k-rows of the other).
bool dma_ok(const void* x, const void* y, const void* out, int64_t m, int64_t n, int64_t k, bool xt, bool yt) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  auto fits = [](int64_t bytes) { return bytes < 0x7ffffff0; };
  return k % Gemm2::BK == 0 && n % 8 == 0 && (!xt || m % 8 == 0) && a16(x) && a16(y) && a16(out) &&
         m <= 0x7fffffff && n <= 0x7fffffff && k <= 0x7fffffff && fits(xt ? 64 * m * 2 : 256 * k * 2) &&
         fits(yt ? 256 * k * 2 : 64 * n * 2) && cdiv(m, (int64_t)128) * cdiv(n, (int64_t)Gemm2::BN) * 16 <= 0x7fffffff;
}

}  // namespace
}  // namespace ferrite

extern "C" int64_t ferrite_hip_matmul_workspace(int64_t m, int64_t n, int64_t k, int in_dtype) {
  if (m < 1 || n < 1 || k < 1) return -1;
  // No stream here: the workspace is sized for the current device's CU count.
  const int64_t cus = ferrite::cu_count_of(-1);
  if (in_dtype == FERRITE_BF16) return ferrite::splitk_workspace(m, n, k, cus);
  return ferrite::f32_small(m, n, cus) ? ferrite::f32_workspace(m, n, k, cus) : 0;
}

extern "C" int ferrite_hip_matmul_ex(const void* x, const void* y, void* out, int64_t m, int64_t n, int64_t k,
                                     int x_t, int y_t, int in_dtype, int out_dtype, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  using namespace ferrite;
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: dtype must be FERRITE_F32 or FERRITE_BF16");
  if (m < 1 || n < 1 || k < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: need M, N, K >= 1");
  if (!x || !y || !out) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_matmul: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xt = x_t != 0, yt = y_t != 0;
  if (in_dtype == FERRITE_BF16 && dma_ok(x, y, out, m, n, k, xt, yt)) {
    if (out_dtype == FERRITE_BF16) return launch_gemm_dma<bf16>(x, y, out, m, n, k, xt, yt, workspace, workspace_bytes, s);
    return launch_gemm_dma<float>(x, y, out, m, n, k, xt, yt, workspace, workspace_bytes, s);
  }
  if (xt || yt)
    return fail(FERRITE_ERR_INVALID_ARGUMENT,
                "ferrite_hip_matmul: transposed operands need bf16, K % 64 == 0, N % 8 == 0, M % 8 == 0 for a "
                "transposed x, and 16-byte aligned pointers");
  if (in_dtype == FERRITE_BF16) {
    // Shapes the DMA kernel does not take (ragged K, unaligned rows or pointers): four waves
    // of 64 x 64 outputs per 128 x 128 tile (256 x 256 tiles spilled 48 bytes per lane).
    if (out_dtype == FERRITE_BF16) return launch_gemm<bf16, bf16, 128, 128, 64, 2, 2>(x, y, out, m, n, k, s);
    return launch_gemm<bf16, float, 128, 128, 64, 2, 2>(x, y, out, m, n, k, s);
  }
  // f32: 128 x 128 tiles of four waves reach ~80% of the fp32 MFMA peak at 4096^3; a
  // problem with fewer such tiles than CUs (1000^3 has 64) runs 64 x 64 tiles instead,
  // with K split inside the workgroup while SIMDs would stay idle.
  if (f32_small(m, n, cu_count(s))) {
    if (out_dtype == FERRITE_BF16) return launch_gemm_f32_small<bf16>(x, y, out, m, n, k, workspace, workspace_bytes, s);
    return launch_gemm_f32_small<float>(x, y, out, m, n, k, workspace, workspace_bytes, s);
  }
  if (out_dtype == FERRITE_BF16) return launch_gemm_f32_big<bf16>(x, y, out, m, n, k, s);
  return launch_gemm_f32_big<float>(x, y, out, m, n, k, s);
}

extern "C" int ferrite_hip_matmul_gelu(const void* x, const void* y, void* out, void* aux, int64_t m, int64_t n,
                                       int64_t k, int x_t, int y_t, int mode, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  using namespace ferrite;
  const char* name = "ferrite_hip_matmul_gelu";
  if (mode != FERRITE_GELU && mode != FERRITE_GELU_GRAD)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": mode must be FERRITE_GELU or FERRITE_GELU_GRAD");
  if (m < 1 || n < 1 || k < 1) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need M, N, K >= 1");
  if (!x || !y || !out || !aux) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  if (aux == out) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": aux and out must differ");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xt = x_t != 0, yt = y_t != 0;
  auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; };
  if (dma_ok(x, y, out, m, n, k, xt, yt) && a8(aux)) {
    if (mode == FERRITE_GELU)
      return launch_gemm_dma<bf16, kEpiGelu>(x, y, out, m, n, k, xt, yt, workspace, workspace_bytes, s, aux);
    return launch_gemm_dma<bf16, kEpiGeluGrad>(x, y, out, m, n, k, xt, yt, workspace, workspace_bytes, s, aux);
  }
  // Other shapes: the plain product (into aux for the forward, into out for the
  // gradient), then the GELU as a pass of its own.
  void* prod = mode == FERRITE_GELU ? aux : out;
  if (int rc = ferrite_hip_matmul_ex(x, y, prod, m, n, k, x_t, y_t, FERRITE_BF16, FERRITE_BF16, workspace,
                                     workspace_bytes, stream))
    return rc;
  const int64_t mn = m * n;
  if (cdiv(mn, 256) > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": output too large");
  if (mode == FERRITE_GELU)
    hipLaunchKernelGGL(gelu_pass_kernel<kEpiGelu>, dim3((unsigned)cdiv(mn, 256)), dim3(256), 0, s,
                       static_cast<bf16*>(out), static_cast<bf16*>(aux), mn);
  else
    hipLaunchKernelGGL(gelu_pass_kernel<kEpiGeluGrad>, dim3((unsigned)cdiv(mn, 256)), dim3(256), 0, s,
                       static_cast<bf16*>(out), static_cast<bf16*>(aux), mn);
  return check_launch(name);
}

extern "C" int ferrite_hip_matmul(const void* x, const void* y, void* out, int64_t m, int64_t n, int64_t k,
                                  int in_dtype, int out_dtype, void* stream) {
  return ferrite_hip_matmul_ex(x, y, out, m, n, k, 0, 0, in_dtype, out_dtype, nullptr, 0, stream);
}

extern "C" int ferrite_hip_mfma_ceiling(float* sink, int blocks, int waves, int iters, void* stream) {
  using namespace ferrite;
  if (blocks < 1 || blocks > 65536 || (waves != 4 && waves != 8) || iters < 1 || iters > (1 << 24))
    return fail(FERRITE_ERR_INVALID_ARGUMENT,
                "ferrite_hip_mfma_ceiling: need 1 <= blocks <= 65536, waves 4 or 8, 1 <= iters <= 2^24");
  if (!sink || (reinterpret_cast<uintptr_t>(sink) & 3))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_mfma_ceiling: null or unaligned sink");
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3((unsigned)blocks), dim3(64 * waves), 0, static_cast<hipStream_t>(stream),
                     sink, iters);
  return check_launch("ferrite_hip_mfma_ceiling");
}
