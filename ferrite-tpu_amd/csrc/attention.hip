// Causal / non-causal flash attention for gfx950: forward, delta, dK/dV, dQ.
//
// Reference: src/ferrite/kernels/flash_attention.py
//   :91-127  _fwd_kernel      online softmax over kv blocks, f32 m/l/acc
//   :130-175 _flash_forward   grid (b, h, q blocks, kv blocks), causal skipping
//   :184-194 _recompute_p_ds  P = exp(S - lse), dS = P * (dP - delta)
//   :197-221 _bwd_dkv_kernel  dV += P^T dO, dK += dS^T Q, dK *= scale
//   :224-243 _bwd_dq_kernel   dQ += dS K, dQ *= scale
//   :326-330 _flash_bwd       delta = rowsum(f32 dO * f32 O)
//
// Design (MI355X-first, not a translation of the Pallas grid):
//  * A workgroup is 4 waves. The forward and dQ kernels give each wave 32 query
//    rows; the dK/dV kernel gives each wave 32 key rows. The sweep over the other
//    sequence axis runs inside the workgroup through double-buffered LDS, and
//    causally invisible tiles are neither loaded nor computed.
//  * All products use 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16, or eight
//    v_mfma_f32_32x32x2_f32 for f32 inputs = true fp32, the reference's
//    Precision.HIGHEST). The score tile is computed transposed where that makes
//    the row statistics lane-local: S^T = K Q^T puts one query row in each lane
//    (plus its partner 32 lanes away), so row max / row sum need one
//    v_permlane32_swap, and P^T is already the B operand of O^T = V^T P^T. P
//    never leaves registers.
//  * Tiles staged "row-major" in LDS are stored with rows permuted inside each
//    32-row block so that MFMA output register r of lane group g is row
//    g*16 + r; 8 consecutive registers are then 8 consecutive rows, which the
//    next product reads as one 16-byte fragment. Tiles staged "transposed" (V^T,
//    K^T, Q^T, dO^T) have 128-byte rows with XOR-swizzled 16-byte chunks.
//  * Softmax runs in the exp2 domain with scale*log2(e) folded into one
//    multiply. The running max is only raised when a row's max grows by more
//    than 2^8 (lazy rescaling): the result is the same exact-arithmetic
//    quantity, p stays <= 256, and the O rescale is skipped on almost every
//    tile.
//  * lse and delta are compact f32 [B, H, S].
#include <mutex>

#include "common.h"

namespace ferrite {
namespace {

constexpr int kThreads = 256;
constexpr float kRescaleThreshold = 8.0f;  // log2 domain

// Physical LDS row (inside a 32-row block) of logical row `r`, see above.
__device__ __forceinline__ int perm_row(int r) {
  const int g = (r >> 4) & 1, rr = r & 15;
  return (r & ~31) | ((rr >> 2) << 3) | (g << 2) | (rr & 3);
}

// Inverse of perm_row: the logical row held by physical row `p` (bits 4,3,2 of
// the row inside its 32-row block rotate the other way).
__device__ __forceinline__ int perm_src(int p) {
  return (p & ~31) | (((p >> 2) & 1) << 4) | (((p >> 4) & 1) << 3) | (((p >> 3) & 1) << 2) | (p & 3);
}

__device__ __forceinline__ int swz(int n) { return (n ^ (n >> 3)) & 7; }

// ---- tile geometry -------------------------------------------------------
// Row-major tile: ROWS x D elements, pitch D*sizeof(T) + 16 bytes.
template <typename T, int D>
struct RowTile {
  static constexpr int kPitch = D * (int)sizeof(T) + 16;
  static __device__ __forceinline__ int off(int prow, int k) { return prow * kPitch + k * (int)sizeof(T); }
  // Fragment of 8 elements (k0 .. k0+7) of physical row prow.
  static __device__ __forceinline__ typename Elem<T>::frag frag(const char* base, int prow, int k0) {
    typename Elem<T>::frag f;
    if constexpr (sizeof(T) == 2) {
      f = *reinterpret_cast<const bf16x8*>(base + off(prow, k0));
    } else {
      f32x4 a = *reinterpret_cast<const f32x4*>(base + off(prow, k0));
      f32x4 b = *reinterpret_cast<const f32x4*>(base + off(prow, k0 + 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[e] = a[e];
        f[4 + e] = b[e];
      }
    }
    return f;
  }
};

// Transposed tile: D rows of 128 bytes (kCols = 128 / sizeof(T) elements).
template <typename T>
struct TrTile {
  static constexpr int kCols = 128 / (int)sizeof(T);
  static constexpr int kVec = Elem<T>::kVec;
  static __device__ __forceinline__ int off(int n, int k) {
    return n * 128 + (((k / kVec) ^ swz(n)) << 4) + (k % kVec) * (int)sizeof(T);
  }
  static __device__ __forceinline__ typename Elem<T>::frag frag(const char* base, int n, int k0) {
    typename Elem<T>::frag f;
    if constexpr (sizeof(T) == 2) {
      f = *reinterpret_cast<const bf16x8*>(base + off(n, k0));
    } else {
      f32x4 a = *reinterpret_cast<const f32x4*>(base + off(n, k0));
      f32x4 b = *reinterpret_cast<const f32x4*>(base + off(n, k0 + 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[e] = a[e];
        f[4 + e] = b[e];
      }
    }
    return f;
  }
};

// Global -> register staging of a ROWS x D tile as 4-row x 16-byte jobs, with
// stores to a row-major (permuted) and/or a transposed LDS tile.
template <typename T, int D, int ROWS, bool ALIGNED>
struct Stager {
  static constexpr int kVec = Elem<T>::kVec;
  static constexpr int kColGroups = D / kVec;
  static constexpr int kJobs = (ROWS / 4) * kColGroups;
  static constexpr int kJobsPerThread = (kJobs + kThreads - 1) / kThreads;
  static constexpr uint32_t kOutOfRange = 0x80000000u;  // >= any num_records (heads are < 2 GiB)
  typedef typename Elem<T>::vec vec;
  vec v[kJobsPerThread][4];
  uint32_t voff[kJobsPerThread][4];  // byte offset of each job row inside a tile (aligned path)

  // Aligned rows use raw buffer loads: the tile's first row is folded into the
  // buffer base, each lane's offset inside the tile is fixed, and the hardware
  // range check returns zeros for rows past the end and for padded columns
  // (whose offset is kOutOfRange), so the staging has no branches.
  __device__ __forceinline__ explicit Stager(int d) {
    if constexpr (ALIGNED) {
      const int t = threadIdx.x;
#pragma unroll
      for (int j = 0; j < kJobsPerThread; ++j) {
        const int job = t + kThreads * j;
        const int cg = job % kColGroups, rg = job / kColGroups;
        const int c0 = cg * kVec;
        const bool ok = job < kJobs && c0 < d;
#pragma unroll
        for (int i = 0; i < 4; ++i) voff[j][i] = ok ? (uint32_t)(((rg * 4 + i) * d + c0) * (int)sizeof(T)) : kOutOfRange;
      }
    }
  }

  // Rows [r0, r0 + ROWS) of a [nrows, d] matrix (row stride d) at `base`.
  __device__ __forceinline__ void load(const T* __restrict__ base, int r0, int nrows, int d) {
    const int t = threadIdx.x;
    if constexpr (ALIGNED) {
      const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<T*>(base) + (int64_t)r0 * d, (short)0, rows_left * d * (int)sizeof(T), 0x00020000);
#pragma unroll
      for (int j = 0; j < kJobsPerThread; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[j][i] = __builtin_bit_cast(vec, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)voff[j][i], 0, 0));
      return;
    }
#pragma unroll
    for (int j = 0; j < kJobsPerThread; ++j) {
      const int job = t + kThreads * j;
      const int cg = job % kColGroups, rg = job / kColGroups;
      const int c0 = cg * kVec;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = r0 + rg * 4 + i;
        const bool rok = job < kJobs && row < nrows;
#pragma unroll
        for (int e = 0; e < kVec; ++e) v[j][i][e] = (rok && c0 + e < d) ? base[row * d + c0 + e] : (T)0.f;
      }
    }
  }

  __device__ __forceinline__ void store_rows(char* lds) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < kJobsPerThread; ++j) {
      const int job = t + kThreads * j;
      if (job >= kJobs) continue;
      const int cg = job % kColGroups, rg = job / kColGroups;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<vec*>(lds + RowTile<T, D>::off(perm_row(rg * 4 + i), cg * kVec)) = v[j][i];
    }
  }

  __device__ __forceinline__ void store_transposed(char* lds) const {
    static_assert(ROWS == TrTile<T>::kCols, "transposed tiles have 128-byte rows");
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < kJobsPerThread; ++j) {
      const int job = t + kThreads * j;
      if (job >= kJobs) continue;
      const int cg = job % kColGroups, rg = job / kColGroups;
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        const int n = cg * kVec + e;
        if constexpr (sizeof(T) == 2) {
          bf16x4 w4 = {v[j][0][e], v[j][1][e], v[j][2][e], v[j][3][e]};
          *reinterpret_cast<bf16x4*>(lds + TrTile<T>::off(n, rg * 4)) = w4;
        } else {
          f32x4 w4 = {v[j][0][e], v[j][1][e], v[j][2][e], v[j][3][e]};
          *reinterpret_cast<f32x4*>(lds + TrTile<T>::off(n, rg * 4)) = w4;
        }
      }
    }
  }
};

// Q / dO fragments of one wave's 32 rows held in registers as the B operand:
// lane (l32, g) holds row r0 + l32, elements kk*16 + g*8 .. +8. With NEG the
// fragments are negated (used for a negative softmax scale).
template <typename T, int D, bool ALIGNED, bool NEG = false>
__device__ __forceinline__ void load_row_frags(typename Elem<T>::frag (&f)[D / 16], const T* __restrict__ base,
                                               int r0, int nrows, int d) {
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int row = r0 + l32;
  if constexpr (ALIGNED) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), (short)0, nrows * d * (int)sizeof(T), 0x00020000);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const int c0 = kk * 16 + g * 8;
      if constexpr (sizeof(T) == 2) {
        const int off = c0 < d ? (row * d + c0) * 2 : 0x7ffffff0;
        f[kk] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
      } else {
        const int off0 = c0 < d ? (row * d + c0) * 4 : 0x7ffffff0;
        const int off1 = c0 + 4 < d ? (row * d + c0 + 4) * 4 : 0x7ffffff0;
        const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off0, 0, 0));
        const f32x4 b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off1, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[kk][e] = a[e];
          f[kk][4 + e] = b[e];
        }
      }
    }
  } else {
    const bool rok = row < nrows;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const int c0 = kk * 16 + g * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[kk][e] = (rok && c0 + e < d) ? base[row * d + c0 + e] : (T)0.f;
    }
  }
  if constexpr (NEG) {
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) f[kk][e] = -f[kk][e];
  }
}

// Store a transposed 32 x D accumulator set (acc[u] register r = row-of-D
// u*32 + (r/4)*8 + g*4 + r%4 for the lane's column) as rows of `out`:
// out[row0 + l32][d] = acc * mul.
template <typename T, int D, bool ALIGNED>
__device__ __forceinline__ void store_acc_rows(const f32x16 (&acc)[D / 32], T* __restrict__ out, int64_t row,
                                               int64_t nrows, int d, float mul) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;
  if (row >= nrows) return;
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = u * 32 + q * 8 + g * 4;
      T* dst = out + row * d + c;
      const float a0 = acc[u][q * 4 + 0] * mul, a1 = acc[u][q * 4 + 1] * mul;
      const float a2 = acc[u][q * 4 + 2] * mul, a3 = acc[u][q * 4 + 3] * mul;
      if (ALIGNED && c + 3 < d) {
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<bf16x4*>(dst) = bf16x4{(bf16)a0, (bf16)a1, (bf16)a2, (bf16)a3};
        } else {
          *reinterpret_cast<f32x4*>(dst) = f32x4{a0, a1, a2, a3};
        }
      } else {
        const float a[4] = {a0, a1, a2, a3};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < d) dst[e] = Elem<T>::from_f32(a[e]);
      }
    }
  }
}

// N products acc(i) += A(i) * B(i) whose A operands come from LDS: the reads
// run kAhead products ahead of the MFMAs and the scheduler is asked to
// alternate one MFMA with one LDS read, so the read latency hides behind the
// matrix pipe instead of stalling each product.
constexpr int kAhead = 4;

template <int N, typename Read, typename Mma>
__device__ __forceinline__ void lds_mfma_pipeline(Read read, Mma mma) {
  typedef decltype(read(0)) FragT;
  FragT buf[N];
#pragma unroll
  for (int i = 0; i < kAhead && i < N; ++i) buf[i] = read(i);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + kAhead < N) buf[i + kAhead] = read(i + kAhead);
    mma(i, buf[i]);
  }
  if constexpr (sizeof(FragT) == 16) {  // bf16: one LDS read and one MFMA per product
#pragma unroll
    for (int i = 0; i < kAhead && i < N; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kAhead < N) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
}

template <typename T>
struct AttnTiles {
  // kv rows per forward / dQ step, q rows per dK/dV step: one 128-byte
  // transposed row.
  static constexpr int kStep = 128 / (int)sizeof(T);
};

// ===========================================================================
// Forward
// ===========================================================================
template <typename T, int D, bool ALIGNED>
struct Fwd {
  static constexpr int BQ = 128;
  static constexpr int BK = AttnTiles<T>::kStep;
  static constexpr int NT = BK / 32;  // S^T subtiles per step
  static constexpr int KS = D / 16;   // k-chunks of q.k
  static constexpr int DT = D / 32;   // O^T output tiles
  static constexpr int kKBytes = BK * RowTile<T, D>::kPitch;
  static constexpr int kVBytes = D * 128;
  static constexpr int kStageBytes = kKBytes + kVBytes;
  static constexpr int kLds = 2 * kStageBytes;
  static constexpr int kMinBlocks = (D <= 128 && sizeof(T) == 2) ? 2 : 1;
};

// `scale_log2` = |scale| * log2(e) (> 0); a negative scale arrives as neg_q = 1
// and is applied by negating the query fragments.
template <typename T, int D, bool ALIGNED>
__global__ __launch_bounds__(kThreads, (Fwd<T, D, ALIGNED>::kMinBlocks)) void attn_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
    float* __restrict__ lse, int bh_count, int Sq, int Sk, int d, int causal, float scale_log2, int neg_q,
    int n_qtiles) {
  typedef Fwd<T, D, ALIGNED> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Heaviest (last) query tiles first; all tiles of one head share an XCD
  // when bh_count is a multiple of 8.
  const int bh = blockIdx.x % bh_count;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / bh_count);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * F::BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + l32;

  const T* qb = q + (int64_t)bh * Sq * d;
  const T* kb = k + (int64_t)bh * Sk * d;
  const T* vb = v + (int64_t)bh * Sk * d;

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const int n_tiles = causal ? min(q_last, Sk - 1) / F::BK + 1 : (Sk + F::BK - 1) / F::BK;
  const bool wave_active = q0w < Sq;
  const int wave_tiles = !wave_active ? 0 : causal ? min(q0w + 31, Sq - 1) / F::BK + 1 : n_tiles;

  frag qf[F::KS];
  if (neg_q)
    load_row_frags<T, D, ALIGNED, true>(qf, qb, q0w, Sq, d);
  else
    load_row_frags<T, D, ALIGNED, false>(qf, qb, q0w, Sq, d);

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  float m = -INFINITY;
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};

  Stager<T, D, F::BK, ALIGNED> ks(d), vs(d);
  ks.load(kb, 0, Sk, d);
  vs.load(vb, 0, Sk, d);

  for (int j = 0; j < n_tiles; ++j) {
    char* st = smem + (j & 1) * F::kStageBytes;
    char* kl = st;
    char* vl = st + F::kKBytes;
    ks.store_rows(kl);
    vs.store_transposed(vl);
    __syncthreads();
    if (j + 1 < n_tiles) {
      ks.load(kb, (j + 1) * F::BK, Sk, d);
      vs.load(vb, (j + 1) * F::BK, Sk, d);
    }
    if (j >= wave_tiles) continue;

    const int kv0 = j * F::BK;
    // S^T = K Q^T: s[t][r] is key kv0 + t*32 + g*16 + r, query qrow. All K
    // fragments of the tile are read before the products so the LDS latency
    // overlaps the MFMA chain; the two subtiles alternate accumulators.
    f32x16 s[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
    lds_mfma_pipeline<F::KS * F::NT>(
        [&](int i) { return RowTile<T, D>::frag(kl, (i % F::NT) * 32 + l32, (i / F::NT) * 16 + g * 8); },
        [&](int i, const frag& a) { mma32(a, qf[i / F::NT], s[i % F::NT]); });

    // Mask on the raw scores (diagonal and ragged tiles only), then the row max.
    if ((causal && kv0 + F::BK - 1 > q0w) || kv0 + F::BK > Sk) {
      const int lim = causal ? min(qrow, Sk - 1) : Sk - 1;
#pragma unroll
      for (int t = 0; t < F::NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = (kv0 + t * 32 + g * 16 + r > lim) ? -INFINITY : s[t][r];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    mx = lane32_max(mx) * scale_log2;
    if (__any(mx > m + kRescaleThreshold)) {
      const float m_new = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
      for (int i = 0; i < 4; ++i) lsum[i] *= alpha;
#pragma unroll
      for (int u = 0; u < F::DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[u][r] *= alpha;
      m = m_new;
    }
    const float neg_m = -m;
    frag pf[F::NT][2];
#pragma unroll
    for (int t = 0; t < F::NT; ++t) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][r], scale_log2, neg_m));
        lsum[r & 3] += p[r];
      }
      to_frag(p, pf[t][0]);
      to_frag(p + 8, pf[t][1]);
    }
    // O^T += V^T P^T: all V^T fragments first, then the products with the
    // output tiles innermost (independent accumulators back to back).
    // Product i uses chunk c = i / DT of the 16-key chunks (t, h) and output tile u = i % DT.
    lds_mfma_pipeline<F::DT * F::NT * 2>(
        [&](int i) {
          const int c = i / F::DT;
          return TrTile<T>::frag(vl, (i % F::DT) * 32 + l32, (c >> 1) * 32 + g * 16 + (c & 1) * 8);
        },
        [&](int i, const frag& a) {
          const int c = i / F::DT;
          mma32(a, pf[c >> 1][c & 1], acc[i % F::DT]);
        });
  }

  if (!wave_active) return;
  const float l = lane32_sum((lsum[0] + lsum[1]) + (lsum[2] + lsum[3]));
  const float inv = 1.0f / l;
  store_acc_rows<T, D, ALIGNED>(acc, o + (int64_t)bh * Sq * d, qrow, Sq, d, inv);
  if (g == 0 && qrow < Sq) lse[(int64_t)bh * Sq + qrow] = (m + __builtin_amdgcn_logf(l)) * kLn2;
}

// ===========================================================================
// Forward, bf16 with D in {64, 128}: K and V staged by LDS DMA
// ===========================================================================
// Same decomposition as attn_fwd_kernel (4 waves x 32 query rows, 64-key
// tiles, double-buffered LDS), but the K and V tiles reach LDS through
// buffer_load ... lds (gfx950 direct-to-LDS loads): no staging registers, no
// LDS writes, and rows past the end or padded columns arrive as zeros from the
// buffer range check. Both tiles are plain row-major with 16-byte chunks
// XOR-swizzled per row; V^T fragments come from ds_read_b64_tr_b16, which
// transposes 4x4 blocks of 16-bit elements across each 16-lane group.
template <int D>
struct SwzTile {
  static constexpr int kRowBytes = D * 2;
  static constexpr int kChunks = kRowBytes / 16;       // 16-byte chunks per row
  static constexpr int kRowsPer256 = 256 / kRowBytes;  // rows sharing one pass of the 64 banks
  // Chunk swizzle: an odd multiplier makes it a bijection over any kChunks
  // consecutive rows (conflict-free 16-byte fragment reads down 16 rows), and
  // 5 also separates the 4-row x 4-chunk footprint of a transposed read.
  static __device__ __forceinline__ int swz(int r) { return (5 * (r / kRowsPer256)) & (kChunks - 1); }
  static __device__ __forceinline__ int off(int r, int col) {
    return r * kRowBytes + (((col >> 3) ^ swz(r)) << 4) + (col & 7) * 2;
  }
  static __device__ __forceinline__ bf16x8 frag(const char* base, int r, int col) {
    return *reinterpret_cast<const bf16x8*>(base + off(r, col));
  }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));

// A-operand fragment of V^T (32 d x 16 keys) from a row-major V tile: lane
// (l32, g) gets V[kv0 + g*16 + e][dcol0 + l32] for e = 0..7, as two transposed
// 8-byte reads (e = 0..3 and 4..7). Within each 16-lane group, slot s = lane %
// 16 supplies the address of keys kv0 + g*16 + half*4 + s/4, columns
// dcol0 + 16*((lane/16) % 2) + 4*(s % 4); the instruction hands lane 4a + b of
// the group element b of the pieces supplied by slots a, a+4, a+8, a+12.
template <int D>
__device__ __forceinline__ bf16x8 vt_frag(const char* vl, int kv0, int dcol0) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 15;
  const int row = kv0 + (lane >> 5) * 16 + (s >> 2);
  const int col = dcol0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const lds_i16x4* p0 = reinterpret_cast<const lds_i16x4*>(
      reinterpret_cast<uintptr_t>(vl + SwzTile<D>::off(row, col)));
  const lds_i16x4* p1 = reinterpret_cast<const lds_i16x4*>(
      reinterpret_cast<uintptr_t>(vl + SwzTile<D>::off(row + 4, col)));
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p1));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// DMA of one 64-row tile of a [nrows, d] bf16 matrix into a swizzled LDS tile.
// Each wave instruction fills 1 KB of LDS (64 lanes x 16 bytes, lane order);
// lane (row R, physical chunk c) loads logical chunk c ^ swz(R) of source row
// src_row(R). PERM applies the 32-row permutation of the MFMA output order.
template <int D, bool PERM>
struct TileDma {
  static constexpr int kRows = 64;
  static constexpr int kRowsPerInst = 64 / SwzTile<D>::kChunks;
  static constexpr int kInsts = kRows / kRowsPerInst;  // per tile, all waves
  static constexpr int kPerWave = kInsts / 4;
  uint32_t voff[kPerWave];

  __device__ __forceinline__ explicit TileDma(int d) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int inst = wave + 4 * i;
      const int R = inst * kRowsPerInst + lane / SwzTile<D>::kChunks;
      const int c = lane % SwzTile<D>::kChunks;
      const int col = (c ^ SwzTile<D>::swz(R)) * 8;
      const int src = PERM ? perm_src(R) : R;
      voff[i] = col < d ? (uint32_t)((src * d + col) * 2) : 0x80000000u;
    }
  }

  // Rows [r0, r0 + 64) of `base`; rows past nrows read as zeros.
  __device__ __forceinline__ void issue(const bf16* base, int r0, int nrows, int d, char* lds) const {
    const int wave = threadIdx.x >> 6;
    const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(base) + (int64_t)r0 * d, (short)0, rows_left * d * 2, 0x00020000);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      char* dst = lds + (wave + 4 * i) * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(dst)), 16,
          (int)voff[i], 0, 0, 0);
    }
  }
};

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int D>
struct FwdDma {
  static constexpr int BQ = 128, BK = 64, NT = 2, KS = D / 16, DT = D / 32;
  static constexpr int kTileBytes = BK * D * 2;
  static constexpr int kStageBytes = 2 * kTileBytes;  // K then V
  static constexpr int kLds = 2 * kStageBytes;
};

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_dma_kernel(const bf16* __restrict__ q,
                                                                  const bf16* __restrict__ k,
                                                                  const bf16* __restrict__ v, bf16* __restrict__ o,
                                                                  float* __restrict__ lse, int bh_count, int Sq,
                                                                  int Sk, int d, int causal, float scale_log2,
                                                                  int neg_q, int n_qtiles) {
  typedef FwdDma<D> F;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int bh = blockIdx.x % bh_count;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / bh_count);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * F::BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + l32;

  const bf16* qb = q + (int64_t)bh * Sq * d;
  const bf16* kb = k + (int64_t)bh * Sk * d;
  const bf16* vb = v + (int64_t)bh * Sk * d;

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const int n_tiles = causal ? min(q_last, Sk - 1) / F::BK + 1 : (Sk + F::BK - 1) / F::BK;
  const bool wave_active = q0w < Sq;
  const int wave_tiles = !wave_active ? 0 : causal ? min(q0w + 31, Sq - 1) / F::BK + 1 : n_tiles;

  TileDma<D, true> kdma(d);
  TileDma<D, false> vdma(d);
  kdma.issue(kb, 0, Sk, d, smem);
  vdma.issue(vb, 0, Sk, d, smem + F::kTileBytes);

  bf16x8 qf[F::KS];
  if (neg_q)
    load_row_frags<bf16, D, true, true>(qf, qb, q0w, Sq, d);
  else
    load_row_frags<bf16, D, true, false>(qf, qb, q0w, Sq, d);

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  float m = -INFINITY;
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};

  for (int j = 0; j < n_tiles; ++j) {
    wait_dma();
    __syncthreads();
    const char* kl = smem + (j & 1) * F::kStageBytes;
    const char* vl = kl + F::kTileBytes;
    if (j + 1 < n_tiles) {
      char* nxt = smem + ((j + 1) & 1) * F::kStageBytes;
      kdma.issue(kb, (j + 1) * F::BK, Sk, d, nxt);
      vdma.issue(vb, (j + 1) * F::BK, Sk, d, nxt + F::kTileBytes);
    }
    if (j >= wave_tiles) continue;

    const int kv0 = j * F::BK;
    f32x16 s[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
    lds_mfma_pipeline<F::KS * F::NT>(
        [&](int i) { return SwzTile<D>::frag(kl, (i % F::NT) * 32 + l32, (i / F::NT) * 16 + g * 8); },
        [&](int i, const bf16x8& a) { mma32(a, qf[i / F::NT], s[i % F::NT]); });

    if ((causal && kv0 + F::BK - 1 > q0w) || kv0 + F::BK > Sk) {
      const int lim = causal ? min(qrow, Sk - 1) : Sk - 1;
#pragma unroll
      for (int t = 0; t < F::NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = (kv0 + t * 32 + g * 16 + r > lim) ? -INFINITY : s[t][r];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    mx = lane32_max(mx) * scale_log2;
    if (__any(mx > m + kRescaleThreshold)) {
      const float m_new = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
      for (int i = 0; i < 4; ++i) lsum[i] *= alpha;
#pragma unroll
      for (int u = 0; u < F::DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[u][r] *= alpha;
      m = m_new;
    }
    const float neg_m = -m;
    bf16x8 pf[F::NT][2];
#pragma unroll
    for (int t = 0; t < F::NT; ++t) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][r], scale_log2, neg_m));
        lsum[r & 3] += p[r];
      }
      to_frag(p, pf[t][0]);
      to_frag(p + 8, pf[t][1]);
    }
    // O^T += V^T P^T. Product i uses key chunk c = i / DT (subtile c/2, half
    // c%2) and output tile u = i % DT.
#pragma unroll
    for (int i = 0; i < F::DT * F::NT * 2; ++i) {
      const int c = i / F::DT, u = i % F::DT;
      mma32(vt_frag<D>(vl, (c >> 1) * 32 + (c & 1) * 8, u * 32), pf[c >> 1][c & 1], acc[u]);
    }
  }

  if (!wave_active) return;
  const float l = lane32_sum((lsum[0] + lsum[1]) + (lsum[2] + lsum[3]));
  store_acc_rows<bf16, D, true>(acc, o + (int64_t)bh * Sq * d, qrow, Sq, d, 1.0f / l);
  if (g == 0 && qrow < Sq) lse[(int64_t)bh * Sq + qrow] = (m + __builtin_amdgcn_logf(l)) * kLn2;
}

// ===========================================================================
// delta = rowsum(f32 dO * f32 O)
// ===========================================================================
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_delta_kernel(const T* __restrict__ o, const T* __restrict__ dout,
                                                             float* __restrict__ delta, int64_t rows, int d) {
  // 16 lanes per row, 16 rows per workgroup.
  const int sub = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  float acc = 0.f;
  if (row < rows) {
    const T* op = o + row * d;
    const T* dp = dout + row * d;
    for (int c = sub * 8; c < d; c += 128) {
      if (c + 8 <= d && (d % Elem<T>::kVec) == 0) {
        typename Elem<T>::vec a0 = *reinterpret_cast<const typename Elem<T>::vec*>(op + c);
        typename Elem<T>::vec b0 = *reinterpret_cast<const typename Elem<T>::vec*>(dp + c);
#pragma unroll
        for (int e = 0; e < Elem<T>::kVec; ++e) acc += Elem<T>::to_f32(b0[e]) * Elem<T>::to_f32(a0[e]);
        if constexpr (Elem<T>::kVec == 4) {
          typename Elem<T>::vec a1 = *reinterpret_cast<const typename Elem<T>::vec*>(op + c + 4);
          typename Elem<T>::vec b1 = *reinterpret_cast<const typename Elem<T>::vec*>(dp + c + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc += Elem<T>::to_f32(b1[e]) * Elem<T>::to_f32(a1[e]);
        }
      } else {
        for (int e = c; e < c + 8 && e < d; ++e) acc += Elem<T>::to_f32(dp[e]) * Elem<T>::to_f32(op[e]);
      }
    }
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) delta[row] = acc;
}

// ===========================================================================
// dQ: per query tile, sweep key tiles up to the diagonal.
// ===========================================================================
template <typename T, int D, bool ALIGNED>
struct Dq {
  static constexpr int BQ = 128;
  static constexpr int BK = AttnTiles<T>::kStep;
  static constexpr int NT = BK / 32;
  static constexpr int KS = D / 16;
  static constexpr int DT = D / 32;
  static constexpr int kRowBytes = BK * RowTile<T, D>::kPitch;
  static constexpr int kStageBytes = 2 * kRowBytes + D * 128;  // K rows, V rows, K^T
  static constexpr int kLds = 2 * kStageBytes;
};

template <typename T, int D, bool ALIGNED>
__global__ __launch_bounds__(kThreads, 1) void attn_dq_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                             const T* __restrict__ v, const T* __restrict__ dout,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ delta, T* __restrict__ dq,
                                                             int bh_count, int64_t Sq, int64_t Sk, int d, int causal,
                                                             float scale, float scale_log2, int n_qtiles) {
  typedef Dq<T, D, ALIGNED> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int bh = blockIdx.x % bh_count;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / bh_count);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t q0 = (int64_t)qt * F::BQ;
  const int64_t q0w = q0 + wave * 32;
  const int64_t qrow = q0w + l32;

  const T* qb = q + (int64_t)bh * Sq * d;
  const T* dob = dout + (int64_t)bh * Sq * d;
  const T* kb = k + (int64_t)bh * Sk * d;
  const T* vb = v + (int64_t)bh * Sk * d;

  const int64_t q_last = (q0 + F::BQ < Sq ? q0 + F::BQ : Sq) - 1;
  const int n_tiles = causal ? (int)((q_last < Sk - 1 ? q_last : Sk - 1) / F::BK + 1) : (int)cdiv(Sk, F::BK);
  const bool wave_active = q0w < Sq;
  const int64_t wq_last = (q0w + 31 < Sq ? q0w + 31 : Sq - 1);
  const int wave_tiles = !wave_active ? 0 : causal ? (int)(wq_last / F::BK + 1) : n_tiles;

  frag qf[F::KS], dof[F::KS];
  load_row_frags<T, D, ALIGNED>(qf, qb, q0w, Sq, d);
  load_row_frags<T, D, ALIGNED>(dof, dob, q0w, Sq, d);
  const bool qok = qrow < Sq;
  const float lse2 = qok ? lse[(int64_t)bh * Sq + qrow] * kLog2e : 0.f;
  const float dl = qok ? delta[(int64_t)bh * Sq + qrow] : 0.f;

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;

  Stager<T, D, F::BK, ALIGNED> ks(d), vs(d);
  ks.load(kb, 0, Sk, d);
  vs.load(vb, 0, Sk, d);

  for (int j = 0; j < n_tiles; ++j) {
    char* st = smem + (j & 1) * F::kStageBytes;
    char* kl = st;
    char* vl = st + F::kRowBytes;
    char* ktl = st + 2 * F::kRowBytes;
    ks.store_rows(kl);
    ks.store_transposed(ktl);
    vs.store_rows(vl);
    __syncthreads();
    if (j + 1 < n_tiles) {
      ks.load(kb, (int64_t)(j + 1) * F::BK, Sk, d);
      vs.load(vb, (int64_t)(j + 1) * F::BK, Sk, d);
    }
    if (j >= wave_tiles) continue;

    const int64_t kv0 = (int64_t)j * F::BK;
    f32x16 s[F::NT], dp[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = 0.f;
        dp[t][r] = 0.f;
      }
#pragma unroll
    for (int kk = 0; kk < F::KS; ++kk)
#pragma unroll
      for (int t = 0; t < F::NT; ++t) {
        mma32(RowTile<T, D>::frag(kl, t * 32 + l32, kk * 16 + g * 8), qf[kk], s[t]);   // S^T = K Q^T
        mma32(RowTile<T, D>::frag(vl, t * 32 + l32, kk * 16 + g * 8), dof[kk], dp[t]);  // dP^T = V dO^T
      }
    const bool need_mask = (causal && kv0 + F::BK - 1 > q0w) || (kv0 + F::BK > Sk);
    frag dsf[F::NT][2];
#pragma unroll
    for (int t = 0; t < F::NT; ++t) {
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(s[t][r] * scale_log2 - lse2);
        if (need_mask) {
          const int64_t kv = kv0 + t * 32 + g * 16 + r;
          if (kv >= Sk || (causal && kv > qrow)) p = 0.f;
        }
        ds[r] = p * (dp[t][r] - dl);
      }
      to_frag(ds, dsf[t][0]);
      to_frag(ds + 8, dsf[t][1]);
    }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int u = 0; u < F::DT; ++u)
#pragma unroll
      for (int t = 0; t < F::NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          mma32(TrTile<T>::frag(ktl, u * 32 + l32, t * 32 + g * 16 + h * 8), dsf[t][h], acc[u]);
  }
  if (!wave_active) return;
  store_acc_rows<T, D, ALIGNED>(acc, dq + (int64_t)bh * Sq * d, qrow, Sq, d, scale);
}

// ===========================================================================
// dK, dV: per key tile (128 keys, 32 per wave), sweep query tiles from the
// diagonal down. K and V fragments stay in registers (B operands).
// ===========================================================================
template <typename T, int D, bool ALIGNED>
struct Dkv {
  static constexpr int BKV = 128;
  static constexpr int BQ = AttnTiles<T>::kStep;  // query rows per step
  static constexpr int NT = BQ / 32;
  static constexpr int KS = D / 16;
  static constexpr int DT = D / 32;
  static constexpr int kRowBytes = BQ * RowTile<T, D>::kPitch;
  static constexpr int kTrBytes = D * 128;
  static constexpr int kStatBytes = BQ * 4;
  static constexpr int kStageBytes = 2 * kRowBytes + 2 * kTrBytes + 2 * kStatBytes;
  static constexpr int kLds = 2 * kStageBytes;
};

template <typename T, int D, bool ALIGNED>
__global__ __launch_bounds__(kThreads, 1) void attn_dkv_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                              const T* __restrict__ v, const T* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta, T* __restrict__ dk,
                                                              T* __restrict__ dv, int bh_count, int64_t Sq,
                                                              int64_t Sk, int d, int causal, float scale,
                                                              float scale_log2) {
  typedef Dkv<T, D, ALIGNED> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Heaviest (first) key tiles first.
  const int bh = blockIdx.x % bh_count;
  const int kt = (int)(blockIdx.x / bh_count);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t k0 = (int64_t)kt * F::BKV;
  const int64_t k0w = k0 + wave * 32;
  const int64_t kvrow = k0w + l32;

  const T* qb = q + (int64_t)bh * Sq * d;
  const T* dob = dout + (int64_t)bh * Sq * d;
  const T* kb = k + (int64_t)bh * Sk * d;
  const T* vb = v + (int64_t)bh * Sk * d;
  const float* lseb = lse + (int64_t)bh * Sq;
  const float* db = delta + (int64_t)bh * Sq;

  const int first = causal ? (int)(k0 / F::BQ) : 0;
  const int n_qt = (int)cdiv(Sq, F::BQ);
  const bool wave_active = k0w < Sk;

  frag kf[F::KS], vf[F::KS];
  load_row_frags<T, D, ALIGNED>(kf, kb, k0w, Sk, d);
  load_row_frags<T, D, ALIGNED>(vf, vb, k0w, Sk, d);

  f32x16 dka[F::DT], dva[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dka[u][r] = 0.f;
      dva[u][r] = 0.f;
    }

  Stager<T, D, F::BQ, ALIGNED> qs(d), dos(d);
  float st_lse = 0.f, st_d = 0.f;
  auto load_q = [&](int it) {
    const int64_t r0 = (int64_t)it * F::BQ;
    qs.load(qb, r0, Sq, d);
    dos.load(dob, r0, Sq, d);
    if (threadIdx.x < F::BQ) {
      const int64_t row = r0 + threadIdx.x;
      // Rows past Sq get lse = +inf so that P = 0 there.
      st_lse = row < Sq ? lseb[row] * kLog2e : INFINITY;
      st_d = row < Sq ? db[row] : 0.f;
    }
  };
  if (first < n_qt) load_q(first);

  for (int it = first; it < n_qt; ++it) {
    char* st = smem + ((it - first) & 1) * F::kStageBytes;
    char* ql = st;
    char* dol = st + F::kRowBytes;
    char* qtl = st + 2 * F::kRowBytes;
    char* dotl = qtl + F::kTrBytes;
    float* lsel = reinterpret_cast<float*>(dotl + F::kTrBytes);
    float* dll = lsel + F::BQ;
    qs.store_rows(ql);
    qs.store_transposed(qtl);
    dos.store_rows(dol);
    dos.store_transposed(dotl);
    if (threadIdx.x < F::BQ) {
      lsel[threadIdx.x] = st_lse;
      dll[threadIdx.x] = st_d;
    }
    __syncthreads();
    if (it + 1 < n_qt) load_q(it + 1);

    const int64_t qs0 = (int64_t)it * F::BQ;
    // Causal: this wave's keys see queries >= k0w only.
    if (!wave_active || (causal && qs0 + F::BQ - 1 < k0w)) continue;

    // S = Q K^T and dP = dO V^T: s[t][r] is query qs0 + t*32 + g*16 + r, key kvrow.
    f32x16 s[F::NT], dp[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = 0.f;
        dp[t][r] = 0.f;
      }
#pragma unroll
    for (int kk = 0; kk < F::KS; ++kk)
#pragma unroll
      for (int t = 0; t < F::NT; ++t) {
        mma32(RowTile<T, D>::frag(ql, t * 32 + l32, kk * 16 + g * 8), kf[kk], s[t]);
        mma32(RowTile<T, D>::frag(dol, t * 32 + l32, kk * 16 + g * 8), vf[kk], dp[t]);
      }
    const bool need_mask = causal && qs0 < k0w + 31;
    frag pf[F::NT][2], dsf[F::NT][2];
#pragma unroll
    for (int t = 0; t < F::NT; ++t) {
      float p[16], ds[16];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 ls = *reinterpret_cast<const f32x4*>(lsel + t * 32 + g * 16 + r4 * 4);
        const f32x4 dd = *reinterpret_cast<const f32x4*>(dll + t * 32 + g * 16 + r4 * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r4 * 4 + e;
          float pv = __builtin_amdgcn_exp2f(s[t][r] * scale_log2 - ls[e]);
          if (need_mask) {
            const int64_t qq = qs0 + t * 32 + g * 16 + r;
            if (kvrow > qq) pv = 0.f;
          }
          p[r] = pv;
          ds[r] = pv * (dp[t][r] - dd[e]);
        }
      }
      to_frag(p, pf[t][0]);
      to_frag(p + 8, pf[t][1]);
      to_frag(ds, dsf[t][0]);
      to_frag(ds + 8, dsf[t][1]);
    }
    // dV^T += dO^T P ; dK^T += Q^T dS
#pragma unroll
    for (int u = 0; u < F::DT; ++u)
#pragma unroll
      for (int t = 0; t < F::NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          mma32(TrTile<T>::frag(dotl, u * 32 + l32, t * 32 + g * 16 + h * 8), pf[t][h], dva[u]);
          mma32(TrTile<T>::frag(qtl, u * 32 + l32, t * 32 + g * 16 + h * 8), dsf[t][h], dka[u]);
        }
  }
  if (!wave_active) return;
  store_acc_rows<T, D, ALIGNED>(dka, dk + (int64_t)bh * Sk * d, kvrow, Sk, d, scale);
  store_acc_rows<T, D, ALIGNED>(dva, dv + (int64_t)bh * Sk * d, kvrow, Sk, d, 1.0f);
}

// ===========================================================================
// Host side
// ===========================================================================
template <typename K>
void set_lds(K kernel, int bytes) {
  // Idempotent; called on every launch because the attribute is per device.
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct Shape {
  int64_t b, h, sq, sk, d;
};

int check_shape(const char* name, const Shape& s, int dtype, int causal, bool bwd) {
  if (!valid_dtype(dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (s.b < 1 || s.h < 1 || s.sq < 1 || s.sk < 1 || s.d < 1)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need b, h, sq, sk, d >= 1");
  if (causal && s.sq != s.sk)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": causal attention needs sq == sk");
  const int64_t dmax = bwd ? 128 : 256;
  if (s.d > dmax || (s.d > 128 && s.d != 256))
    return fail(FERRITE_ERR_INVALID_ARGUMENT,
                std::string(name) + ": head_dim " + std::to_string(s.d) +
                    (bwd ? " not supported (backward supports head_dim <= 128)"
                         : " not supported (head_dim <= 128 or == 256)"));
  if (s.b * s.h > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": b*h too large");
  // In-kernel offsets within one (b, h) head are 32-bit byte offsets.
  const int64_t head_bytes = (s.sq > s.sk ? s.sq : s.sk) * s.d * (dtype == FERRITE_BF16 ? 2 : 4);
  if (head_bytes > 0x7fff0000)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": one (b, h) head must be under 2 GiB");
  return FERRITE_OK;
}

int pad_dim(int64_t d) { return d <= 64 ? 64 : d <= 128 ? 128 : 256; }

template <int D>
int fwd_dma_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, int causal,
                   float c, int neg_q, hipStream_t stream) {
  typedef FwdDma<D> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  auto kern = attn_fwd_dma_kernel<D>;
  set_lds(kern, F::kLds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(kThreads), F::kLds, stream, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<bf16*>(o), lse, (int)bh,
                     (int)s.sq, (int)s.sk, (int)s.d, causal, c, neg_q, (int)nq);
  return check_launch("ferrite_flash_attention_fwd");
}

template <typename T, int D, bool AL>
int fwd_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, int causal,
               float scale, hipStream_t stream) {
  typedef Fwd<T, D, AL> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  auto kern = attn_fwd_kernel<T, D, AL>;
  set_lds(kern, F::kLds);
  // The kernel takes the row max on raw scores, which needs a positive
  // multiplier: a negative scale negates q instead, and a zero scale becomes a
  // tiny positive one (uniform weights either way).
  float c = scale * kLog2e;
  const int neg_q = c < 0.f;
  c = fmaxf(fabsf(c), 1e-30f);
  if constexpr (sizeof(T) == 2 && AL && D <= 128) return fwd_dma_launch<D>(q, k, v, o, lse, s, causal, c, neg_q, stream);
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o), lse, (int)bh, (int)s.sq,
                     (int)s.sk, (int)s.d, causal, c, neg_q, (int)nq);
  return check_launch("ferrite_flash_attention_fwd");
}

template <typename T, int D, bool AL>
int dq_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
              void* dq, const Shape& s, int causal, float scale, hipStream_t stream) {
  typedef Dq<T, D, AL> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: grid too large");
  auto kern = attn_dq_kernel<T, D, AL>;
  set_lds(kern, F::kLds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<const T*>(dout), lse, delta,
                     static_cast<T*>(dq), (int)bh, s.sq, s.sk, (int)s.d, causal, scale, scale * kLog2e, (int)nq);
  return check_launch("ferrite_flash_attention_bwd_dq");
}

template <typename T, int D, bool AL>
int dkv_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
               void* dk, void* dv, const Shape& s, int causal, float scale, hipStream_t stream) {
  typedef Dkv<T, D, AL> F;
  const int64_t nk = cdiv(s.sk, F::BKV);
  const int64_t bh = s.b * s.h;
  if (nk * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: grid too large");
  auto kern = attn_dkv_kernel<T, D, AL>;
  set_lds(kern, F::kLds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<const T*>(dout), lse, delta,
                     static_cast<T*>(dk), static_cast<T*>(dv), (int)bh, s.sq, s.sk, (int)s.d, causal, scale,
                     scale * kLog2e);
  return check_launch("ferrite_flash_attention_bwd_dkv");
}

// Dispatch over (dtype, padded D, aligned) for a launcher template L.
#define FERRITE_DISPATCH(LAUNCH, s, dtype, aligned, ...)                                        \
  do {                                                                                          \
    const int dp_ = pad_dim((s).d);                                                             \
    if ((dtype) == FERRITE_BF16) {                                                              \
      if (dp_ == 64) return (aligned) ? LAUNCH<bf16, 64, true>(__VA_ARGS__)                     \
                                      : LAUNCH<bf16, 64, false>(__VA_ARGS__);                   \
      if (dp_ == 128) return (aligned) ? LAUNCH<bf16, 128, true>(__VA_ARGS__)                   \
                                       : LAUNCH<bf16, 128, false>(__VA_ARGS__);                 \
      FERRITE_DISPATCH_256(LAUNCH, bf16, aligned, __VA_ARGS__);                                 \
    } else {                                                                                    \
      if (dp_ == 64) return (aligned) ? LAUNCH<float, 64, true>(__VA_ARGS__)                    \
                                      : LAUNCH<float, 64, false>(__VA_ARGS__);                  \
      if (dp_ == 128) return (aligned) ? LAUNCH<float, 128, true>(__VA_ARGS__)                  \
                                       : LAUNCH<float, 128, false>(__VA_ARGS__);                \
      FERRITE_DISPATCH_256(LAUNCH, float, aligned, __VA_ARGS__);                                \
    }                                                                                           \
  } while (0)

}  // namespace
}  // namespace ferrite

using namespace ferrite;

extern "C" int ferrite_hip_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t b,
                                    int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                    void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_fwd", s, dtype, causal, false)) return rc;
  if (!q || !k || !v || !o || !lse) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: null pointer");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(o);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return (aligned) ? LAUNCH<T, 256, true>(__VA_ARGS__) : LAUNCH<T, 256, false>(__VA_ARGS__)
  FERRITE_DISPATCH(fwd_launch, s, dtype, al, q, k, v, o, lse, s, causal, scale, st);
#undef FERRITE_DISPATCH_256
}

extern "C" int ferrite_hip_attn_bwd_delta(const void* o, const void* dout, float* delta, int64_t b, int64_t h,
                                          int64_t s, int64_t d, int dtype, void* stream) {
  if (!valid_dtype(dtype))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: dtype must be FERRITE_F32 or FERRITE_BF16");
  if (b < 1 || h < 1 || s < 1 || d < 1)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: need b, h, s, d >= 1");
  if (!o || !dout || !delta) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: null pointer");
  if (d > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: d too large");
  const int64_t rows = b * h * s;
  const int64_t blocks = cdiv(rows, 16);
  if (blocks > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool al = aligned16(o) && aligned16(dout);
  if (!al) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_delta: o and dout must be 16-byte aligned");
  if (dtype == FERRITE_BF16)
    hipLaunchKernelGGL(attn_delta_kernel<bf16>, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       static_cast<const bf16*>(o), static_cast<const bf16*>(dout), delta, rows, (int)d);
  else
    hipLaunchKernelGGL(attn_delta_kernel<float>, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       static_cast<const float*>(o), static_cast<const float*>(dout), delta, rows, (int)d);
  return check_launch("ferrite_flash_attention_bwd_delta");
}

extern "C" int ferrite_hip_attn_bwd_dkv(const void* q, const void* k, const void* v, const void* dout,
                                        const float* lse, const float* delta, void* dk, void* dv, int64_t b,
                                        int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                        float scale, void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_bwd_dkv", s, dtype, causal, true)) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: null pointer");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(dout) && aligned16(dk) && aligned16(dv);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return fail(FERRITE_ERR_INVALID_ARGUMENT, "unreachable head_dim")
  FERRITE_DISPATCH(dkv_launch, s, dtype, al, q, k, v, dout, lse, delta, dk, dv, s, causal, scale, st);
#undef FERRITE_DISPATCH_256
}

extern "C" int ferrite_hip_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                                       const float* lse, const float* delta, void* dq, int64_t b, int64_t h,
                                       int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                       void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_bwd_dq", s, dtype, causal, true)) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dq)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: null pointer");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(dout) && aligned16(dq);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return fail(FERRITE_ERR_INVALID_ARGUMENT, "unreachable head_dim")
  FERRITE_DISPATCH(dq_launch, s, dtype, al, q, k, v, dout, lse, delta, dq, s, causal, scale, st);
#undef FERRITE_DISPATCH_256
}
