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
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "attn_sched.h"

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
__host__ __device__ constexpr int perm_src(int p) {
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
  int ld;                            // element stride between rows (d, or more for a column slab)

  // Aligned rows use raw buffer loads: the tile's first row is folded into the
  // buffer base, each lane's offset inside the tile is fixed, and the hardware
  // range check returns zeros for rows past the end and for padded columns
  // (whose offset is kOutOfRange), so the staging has no branches.
  // `d` columns are valid; rows lie `ld_` elements apart (0: ld = d).
  __device__ __forceinline__ explicit Stager(int d, int ld_ = 0) : ld(ld_ ? ld_ : d) {
    if constexpr (ALIGNED) {
      const int t = threadIdx.x;
#pragma unroll
      for (int j = 0; j < kJobsPerThread; ++j) {
        const int job = t + kThreads * j;
        const int cg = job % kColGroups, rg = job / kColGroups;
        const int c0 = cg * kVec;
        const bool ok = job < kJobs && c0 < d;
#pragma unroll
        for (int i = 0; i < 4; ++i) voff[j][i] = ok ? (uint32_t)(((rg * 4 + i) * ld + c0) * (int)sizeof(T)) : kOutOfRange;
      }
    }
  }

  // Rows [r0, r0 + ROWS) of a [nrows, d] matrix (row stride ld) at `base`.
  __device__ __forceinline__ void load(const T* __restrict__ base, int r0, int nrows, int d) {
    const int t = threadIdx.x;
    if constexpr (ALIGNED) {
      const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<T*>(base) + (int64_t)r0 * ld, (short)0, rows_left * ld * (int)sizeof(T), 0x00020000);
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
        for (int e = 0; e < kVec; ++e) v[j][i][e] = (rok && c0 + e < d) ? base[(int64_t)row * ld + c0 + e] : (T)0.f;
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
// ld: element stride between rows (d for a dense [rows, d] tensor; larger for a head
// of a token-major [rows, heads, d] one).
template <typename T, int D, bool ALIGNED, bool NEG = false>
__device__ __forceinline__ void load_row_frags(typename Elem<T>::frag (&f)[D / 16], const T* __restrict__ base,
                                               int r0, int nrows, int d, int ld = 0) {
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int row = r0 + l32;
  if (ld == 0) ld = d;
  if constexpr (ALIGNED) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), (short)0, nrows * ld * (int)sizeof(T), 0x00020000);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const int c0 = kk * 16 + g * 8;
      if constexpr (sizeof(T) == 2) {
        const int off = c0 < d ? (row * ld + c0) * 2 : 0x7ffffff0;
        f[kk] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
      } else {
        const int off0 = c0 < d ? (row * ld + c0) * 4 : 0x7ffffff0;
        const int off1 = c0 + 4 < d ? (row * ld + c0 + 4) * 4 : 0x7ffffff0;
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
      for (int e = 0; e < 8; ++e) f[kk][e] = (rok && c0 + e < d) ? base[row * ld + c0 + e] : (T)0.f;
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
                                               int64_t nrows, int d, float mul, int64_t ld = 0) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;
  if (row >= nrows) return;
  if (ld == 0) ld = d;
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = u * 32 + q * 8 + g * 4;
      T* dst = out + row * ld + c;
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

// 32 full-width rows (row0 .. row0 + 31; rows at or past nrows arrive as
// zeros) of a bf16 operand with D columns and row pitch ld, by DMA into LDS at
// dst as whole rows: a row per D / 8 lanes and 1 KB per instruction, 16-byte
// chunks XOR-swizzled by row. Loaded straight into fragments, every load
// instruction touches 32 rows (32 cache lines for 1 KB). row_frags_lds reads
// back the fragments load_row_frags would load.
template <int D>
__device__ __forceinline__ void dma_rows32(const bf16* base, int row0, int nrows, int ld, char* dst) {
  constexpr int kRow = 2 * D, kCh = kRow / 16, kRpi = 1024 / kRow;
  const int lane = threadIdx.x & 63;
  const u32x4 rs = buffer_rsrc(base + (int64_t)row0 * ld, row0 < nrows ? (uint32_t)((nrows - row0) * ld * 2) : 0u);
#pragma unroll
  for (int i = 0; i < 32 / kRpi; ++i) {
    const int rr = kRpi * i + lane / kCh, c = (lane % kCh) ^ (rr & (kCh - 1));
    dma16(rs, dst + 1024 * i, (uint32_t)((rr * ld + 8 * c) * 2));
  }
}
template <int D>
__device__ __forceinline__ void row_frags_lds(bf16x8 (&f)[D / 16], const char* src) {
  constexpr int kRow = 2 * D, kCh = kRow / 16;
  const int lane = threadIdx.x & 63, l32 = lane & 31, g = lane >> 5;
#pragma unroll
  for (int kc = 0; kc < D / 16; ++kc) {
    const int c = 2 * kc + g;
    f[kc] = *reinterpret_cast<const bf16x8*>(src + l32 * kRow + ((c ^ (l32 & (kCh - 1))) * 16));
  }
}

// Full-width (d == D) bf16 rows of a wave's accumulators through LDS. A lane's
// accumulator registers hold 4-column pieces of one row (register r of tile u
// is column 32 u + 8 (r / 4) + 4 g + r % 4 of row l32), so stored directly
// every store instruction touches 32 rows (32 cache lines for 512 bytes; the
// stores of one forward workgroup took ~4000 cycles on MI355X). The rows go
// into this wave's 32 x 2D-byte LDS region (16-byte chunks XOR-swizzled by
// row) and come back 16 bytes per lane, so that each store instruction writes
// whole rows, 2D / 16 lanes per row. The caller keeps other waves' reads and
// DMA off the region; one wave's LDS writes and reads are processed in order.
// Rows row0 + r at or past nrows are skipped.
// FRESH: the lane from lane_id() (see there), for kernels at their register
// limit whose lane terms would otherwise cross their stage loop.
template <int D, bool FRESH = false>
__device__ __forceinline__ void store_acc_rows_lds(const f32x16 (&acc)[D / 32], char* lds, bf16* __restrict__ out,
                                                   int64_t row0, int64_t nrows, float mul, int64_t ld) {
  constexpr int kRowBytes = 2 * D, kCh = kRowBytes / 16, kRowsPerInst = 64 / kCh;
  const int lane = FRESH ? lane_id() : (int)(threadIdx.x & 63), l32 = lane & 31, g = lane >> 5;
#pragma unroll
  for (int u = 0; u < D / 32; ++u)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<bf16x4*>(lds + l32 * kRowBytes + (((4 * u + qq) ^ (l32 & (kCh - 1))) * 16) + 8 * g) =
          bf16x4{(bf16)(acc[u][4 * qq] * mul), (bf16)(acc[u][4 * qq + 1] * mul), (bf16)(acc[u][4 * qq + 2] * mul),
                 (bf16)(acc[u][4 * qq + 3] * mul)};
#pragma unroll
  for (int i = 0; i < 32 / kRowsPerInst; ++i) {
    const int r = i * kRowsPerInst + lane / kCh, c = lane % kCh;
    const bf16x8 val = *reinterpret_cast<const bf16x8*>(lds + r * kRowBytes + ((c ^ (r & (kCh - 1))) * 16));
    if (row0 + r < nrows) *reinterpret_cast<bf16x8*>(out + (row0 + r) * ld + 8 * c) = val;
  }
}

// Element strides of one tensor seen as [B, H, rows, d] with contiguous columns:
// between batches, heads and rows. A dense [B, H, S, d] tensor has (H S d, S d, d);
// the q part of a token-major [B, S, 3, H, d] projection has (3 S H d, d, 3 H d).
struct View {
  int64_t b, h, r;
  __host__ __device__ int64_t at(int bh, int heads) const { return (int64_t)(bh / heads) * b + (int64_t)(bh % heads) * h; }
};
struct AttnViews {
  View q, k, v, o, dout, dq, dk, dv;
  int heads;
};

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
// Forward, bf16 with D in {64, 128}: ping-pong schedule over LDS DMA
// ===========================================================================
// 8 waves and 256 query rows per workgroup, 32 rows per wave. Waves w and
// w + 4 run on the same SIMD and belong to opposite groups. Each tile step
// has two phases separated by a workgroup barrier; in every phase one group
// issues its matrix products (S^T = K Q^T for tile t and O^T += V^T P^T for
// tile t - 1) while the other runs the softmax of its scores, so each SIMD's
// MFMA pipe is fed by one wave while the other one works on the VALU.
//
// K and V tiles of 64 keys reach LDS through buffer_load ... lds (one 1 KB
// block per instruction, no staging registers) in three-slot rings, K two
// steps and V one step ahead of use. Rows past the end of the keys read as
// zeros from the buffer range check.

// K tile for the A operand of S^T = K Q^T: 16-byte reads in which lane
// (l32, g) takes physical row 32t + l32, 16-byte chunk 2kc + g. Row r sits in
// 1 KB block r % kBlocks at position r / kBlocks. The 16-byte gap between
// blocks puts the 16 rows of each 16-lane quarter in 16 different bank
// groups, and the address of (32t + l32, chunk) is a per-lane base plus a
// constant, so the reads need no address arithmetic.
template <int D>
struct PpKTile {
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kChunks = kRowBytes / 16;
  static constexpr int kBlocks = 64 * kRowBytes / 1024;  // 16 (D = 128) or 8 (D = 64)
  static constexpr int kStride = 1024 + 16;
  static constexpr int kBytes = kBlocks * kStride;
  static __host__ __device__ constexpr int off(int r, int byte) {
    return (r % kBlocks) * kStride + (r / kBlocks) * kRowBytes + byte;
  }
  static __host__ __device__ constexpr int block_off(int b) { return b * kStride; }
  // Row that lane L of the instruction filling block b loads.
  static __host__ __device__ constexpr int dma_row(int b, int L) { return b + (L / kChunks) * kBlocks; }
  static __host__ __device__ constexpr int dma_chunk(int L) { return L % kChunks; }
  static __device__ __forceinline__ bool dma_lane(int) { return true; }
};

// V tile for V^T fragments read with ds_read_b64_tr_b16, in which lanes 0-31
// take 64 bytes from each of rows r..r+3 (r % 4 == 0). Row r sits in block
// (r % 4) + 4 * (r / (4 * kRowsPerBlock)) at position (r / 4) % kRowsPerBlock:
// the 64-byte gap between blocks puts those four rows in the four 64-byte
// bank groups, and addresses again split into a lane base plus a constant.
template <int D>
struct PpVTile {
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kChunks = kRowBytes / 16;
  static constexpr int kRowsPerBlock = 1024 / kRowBytes;  // 4 or 8
  static constexpr int kBlocks = 64 / kRowsPerBlock;
  static constexpr int kStride = 1024 + 64;
  static constexpr int kBytes = kBlocks * kStride;
  static __host__ __device__ constexpr int off(int r, int byte) {
    return ((r & 3) + 4 * (r / (4 * kRowsPerBlock))) * kStride + ((r >> 2) % kRowsPerBlock) * kRowBytes + byte;
  }
  static __host__ __device__ constexpr int block_off(int b) { return b * kStride; }
  static __host__ __device__ constexpr int dma_row(int b, int L) {
    return (b & 3) + 4 * (L / kChunks) + 4 * kRowsPerBlock * (b >> 2);
  }
  static __host__ __device__ constexpr int dma_chunk(int L) { return L % kChunks; }
  static __device__ __forceinline__ bool dma_lane(int) { return true; }
};

// One wave's share of the DMA of a 64-row bf16 tile with d == D: GROUP waves
// split the blocks, wave gw taking blocks gw + GROUP i. PERM loads physical
// row r from logical row perm_src(r). A lane's source row for instruction i is
// its row for instruction 0 plus a wave- and lane-independent delta (the bits
// that i sets are disjoint from the wave's and the lane's, and perm_src only
// permutes bits), so one VGPR offset serves all instructions; instruction i
// moves the buffer window instead: base + delta, range - delta.
template <class Layout, bool PERM, int GROUP = 4>
struct PpDma {
  static constexpr int kPerWave = Layout::kBlocks / GROUP;
  uint32_t voff;
  int gw;

  static constexpr int delta_rows(int i) {
    return PERM ? perm_src(Layout::dma_row(GROUP * i, 0)) - perm_src(Layout::dma_row(0, 0))
                : Layout::dma_row(GROUP * i, 0) - Layout::dma_row(0, 0);
  }

  __device__ __forceinline__ PpDma(int gw_, int d) : gw(gw_) {
    const int lane = threadIdx.x & 63;
    const int r = Layout::dma_row(gw, lane);
    const int src = PERM ? perm_src(r) : r;
    voff = Layout::dma_lane(lane) ? (uint32_t)((src * d + Layout::dma_chunk(lane) * 8) * 2) : 0x80000000u;
  }

  // Buffer descriptor of rows [r0, nrows) of `base` (rows past nrows read as zeros).
  static __device__ __forceinline__ u32x4 rsrc_of(const bf16* base, int r0, int nrows, int d) {
    const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
    const uint64_t addr = reinterpret_cast<uint64_t>(base + (int64_t)r0 * d);
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffffu)),
                 (uint32_t)__builtin_amdgcn_readfirstlane(rows_left * d * 2), 0x00020000u};
  }
  // The i-th of this wave's instructions for rows [r0, r0 + 64) of `base`
  // into the tile at `lds`: the window starts delta_rows(i) rows later.
  __device__ __forceinline__ void issue_one(const bf16* base, int r0, int nrows, int d, char* lds, int i) const {
    const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)reinterpret_cast<uintptr_t>(lds + Layout::block_off(gw + GROUP * i)));
    const u32x4 rs = rsrc_of(base, r0 + delta_rows(i), nrows, d);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rs)
                 : "memory", "m0");
  }

  // Rows [r0, r0 + 64) of `base` into the tile at `lds`; rows at or past
  // nrows arrive as zeros. Issued as inline assembly so that the compiler's
  // wait insertion does not tie every later LDS read to these loads; the
  // kernel orders them itself with explicit vmcnt waits and barriers.
  __device__ __forceinline__ void issue(const bf16* base, int r0, int nrows, int d, char* lds) const {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) issue_one(base, r0, nrows, d, lds, i);
  }
};


template <int D>
struct FwdPp {
  static constexpr int kWaves = 8, kThreads = 64 * kWaves;
  static constexpr int BQ = 32 * kWaves, BK = 64, NT = 2, KS = D / 16, DT = D / 32;
  typedef PpKTile<D> KT;
  typedef PpVTile<D> VT;
  static constexpr int kSlots = 3;
  static constexpr int kLds = kSlots * (KT::kBytes + VT::kBytes);
  static constexpr int kDma = KT::kBlocks / 4;  // DMA instructions per tile for each wave of the loading group
  static_assert(KT::kBlocks == VT::kBlocks, "K and V tiles take the same number of DMA blocks");
};

// The matrix phase: S^T = K_t Q^T into s (QK) and O^T += V_{t-1}^T P^T (PV).
// kp / vp are the lane's base addresses inside the K and V slots. Reads run
// kPpAhead products ahead of the MFMAs: four matrix waves share the LDS, so
// its latency is longer than in a lone wave.
constexpr int kPpAhead = 8;

template <int D, bool QK, bool PV>
__device__ __forceinline__ void pp_gemm(const char* kp, const char* vp, const bf16x8 (&qf)[D / 16],
                                        const bf16x8 (&pf)[2][2], f32x16 (&s)[2], f32x16 (&acc)[D / 32]) {
  typedef FwdPp<D> F;
  typedef typename F::KT KT;
  typedef typename F::VT VT;
  constexpr int NQ = QK ? F::KS * F::NT : 0;
  constexpr int NP = PV ? F::DT * 4 : 0;
  constexpr int N = NQ + NP;
  if constexpr (QK) {
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
  }
  // Product i < NQ: subtile i % NT, k-chunk i / NT. Product NQ + j: key chunk
  // c = j / DT (subtile c / 2, half c % 2), output tile u = j % DT.
  auto read = [&](int i) -> bf16x8 {
    if (i < NQ) {
      return *reinterpret_cast<const bf16x8*>(kp + KT::off(32 * (i % F::NT), (i / F::NT) * 32));
    } else {
      const int j = i - NQ, c = j / F::DT, u = j % F::DT;
      return tr_frag(vp + VT::off((c >> 1) * 32 + (c & 1) * 8, u * 64), VT::off(4, 0));
    }
  };
  bf16x8 buf[N];
#pragma unroll
  for (int i = 0; i < kPpAhead && i < N; ++i) buf[i] = read(i);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + kPpAhead < N) buf[i + kPpAhead] = read(i + kPpAhead);
    if (i < NQ) {
      mma32(buf[i], qf[i / F::NT], s[i % F::NT]);
    } else {
      const int j = i - NQ, c = j / F::DT;
      mma32(buf[i], pf[c >> 1][c & 1], acc[j % F::DT]);
    }
  }
  // One MFMA, then the LDS reads of the product kPpAhead further on (one for
  // a K fragment, two for a V^T fragment).
  auto reads = [](int i) {
    if (i < NQ)
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    else
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  };
#pragma unroll
  for (int i = 0; i < kPpAhead && i < N; ++i) reads(i);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i + kPpAhead < N) reads(i + kPpAhead);
  }
}

template <int D>
__global__ __launch_bounds__(512, 2) void attn_fwd_pp_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                             const bf16* __restrict__ v, bf16* __restrict__ o,
                                                             float* __restrict__ lse, int bh_count, int Sq, int Sk,
                                                             int d, int causal, float scale_log2, int neg_q,
                                                             int n_qtiles) {
  typedef FwdPp<D> F;
  typedef typename F::KT KT;
  typedef typename F::VT VT;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const kring = smem;
  char* const vring = smem + F::kSlots * KT::kBytes;

  // Heaviest (last) query tiles first; all tiles of one head share an XCD
  // when bh_count is a multiple of 8.
  const int bh = blockIdx.x % bh_count;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / bh_count);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int group = wave >> 2;
  // SIMD w % 4 holds row blocks 2 (w % 4) and 2 (w % 4) + 1, one per group,
  // so both groups see the same share of the causal diagonal.
  const int q0 = qt * F::BQ;
  const int q0w = q0 + 32 * (2 * (wave & 3) + group);
  const int qrow = q0w + l32;

  const bf16* qb = q + (int64_t)bh * Sq * d;
  const bf16* kb = k + (int64_t)bh * Sk * d;
  const bf16* vb = v + (int64_t)bh * Sk * d;

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const int n = causal ? min(q_last, Sk - 1) / F::BK + 1 : (Sk + F::BK - 1) / F::BK;
  const bool wave_active = q0w < Sq;
  const int n_w = !wave_active ? 0 : causal ? min(min(q0w + 31, Sq - 1), Sk - 1) / F::BK + 1 : n;

  // Group 1 loads the K tiles and group 0 the V tiles, each at the start of
  // its softmax phase, so that a wave about to run its matrix products never
  // waits behind the DMA issue.
  const PpDma<KT, true> kdma(wave & 3, d);
  const PpDma<VT, false> vdma(wave & 3, d);

  bf16x8 qf[F::KS];
  if (neg_q)
    load_row_frags<bf16, D, true, true>(qf, qb, q0w, Sq, d);
  else
    load_row_frags<bf16, D, true, false>(qf, qb, q0w, Sq, d);

  // Ring prologue: K_0 and K_1 into K slots 0 and 1, V_0 into V slot 0.
  if (group == 1) {
    kdma.issue(kb, 0, Sk, d, kring);
    if (1 < n) kdma.issue(kb, F::BK, Sk, d, kring + KT::kBytes);
  } else {
    vdma.issue(vb, 0, Sk, d, vring);
  }

  // Lane bases inside a K / V slot.
  const int kbase = KT::off(l32, g * 16);
  const int vbase = VT::off((lane >> 5) * 16 + ((lane & 15) >> 2), 2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  f32x16 s[F::NT];
  bf16x8 pf[F::NT][2];
  float m = -INFINITY;
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};

  auto kslot = [&](int t) { return kring + (t % F::kSlots) * KT::kBytes + kbase; };
  auto vslot = [&](int t) { return vring + (t % F::kSlots) * VT::kBytes + vbase; };

  auto softmax = [&](int t) {
    const int kv0 = t * F::BK;
    // Mask on the raw scores (diagonal and ragged tiles only), then the row max.
    if ((causal && kv0 + F::BK - 1 > q0w) || kv0 + F::BK > Sk) {
      const int lim = causal ? min(qrow, Sk - 1) : Sk - 1;
#pragma unroll
      for (int u = 0; u < F::NT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[u][r] = (kv0 + u * 32 + g * 16 + r > lim) ? -INFINITY : s[u][r];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < F::NT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[u][r]);
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
#pragma unroll
    for (int u = 0; u < F::NT; ++u) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][r], scale_log2, neg_m));
        lsum[r & 3] += p[r];
      }
      to_frag(p, pf[u][0]);
      to_frag(p + 8, pf[u][1]);
    }
  };

  // Step st has two phases, each opened by a workgroup barrier. Group 0 runs
  // the products of tile st (and PV of st - 1) in the first phase and the
  // softmax of tile st in the second; group 1 runs the softmax of st - 1 in
  // the first and the products of st in the second. K_{st+2} goes out from
  // group 1 after the first barrier of step st and V_{st+1} from group 0
  // after the second, once every wave has left the slots they overwrite.
  // Both groups pass 2 (n + 1) barriers.
  auto open_step = [&](int st) {
    // The loads of K_st (group 1, issued in step st - 2) and V_{st-1}
    // (group 0, step st - 2) are complete; the group's loads from step
    // st - 1 may still be in flight.
    if (group == 1 ? st + 1 < n : st < n)
      wait_vmem<F::kDma>();
    else
      wait_vmem<0>();
    lds_barrier();
    if (group == 1 && st + 2 < n) kdma.issue(kb, (st + 2) * F::BK, Sk, d, kring + ((st + 2) % F::kSlots) * KT::kBytes);
  };
  auto mid_step = [&](int st) {
    lds_barrier();
    if (group == 0 && st + 1 < n) vdma.issue(vb, (st + 1) * F::BK, Sk, d, vring + ((st + 1) % F::kSlots) * VT::kBytes);
  };
  // The wave in its matrix phase takes issue priority over the one in its
  // softmax, which fills the remaining VALU cycles; without it the older wave
  // of the pair wins every tie and starves the other's MFMAs.
  auto gemm_phase = [&](auto&& body) {
    __builtin_amdgcn_s_setprio(1);
    body();
    __builtin_amdgcn_s_setprio(0);
  };
  int st = 0;
  if (n_w > 0) {
    if (group == 0) {
      open_step(0);
      gemm_phase([&] { pp_gemm<D, true, false>(kslot(0), vslot(0), qf, pf, s, acc); });
      mid_step(0);
      softmax(0);
      for (st = 1; st < n_w; ++st) {
        open_step(st);
        gemm_phase([&] { pp_gemm<D, true, true>(kslot(st), vslot(st - 1), qf, pf, s, acc); });
        mid_step(st);
        softmax(st);
      }
      open_step(n_w);
      gemm_phase([&] { pp_gemm<D, false, true>(kslot(n_w), vslot(n_w - 1), qf, pf, s, acc); });
      mid_step(n_w);
    } else {
      open_step(0);
      mid_step(0);
      gemm_phase([&] { pp_gemm<D, true, false>(kslot(0), vslot(0), qf, pf, s, acc); });
      for (st = 1; st < n_w; ++st) {
        open_step(st);
        softmax(st - 1);
        mid_step(st);
        gemm_phase([&] { pp_gemm<D, true, true>(kslot(st), vslot(st - 1), qf, pf, s, acc); });
      }
      open_step(n_w);
      softmax(n_w - 1);
      mid_step(n_w);
      gemm_phase([&] { pp_gemm<D, false, true>(kslot(n_w), vslot(n_w - 1), qf, pf, s, acc); });
    }
    st = n_w + 1;
  }
  for (; st <= n; ++st) {
    open_step(st);
    mid_step(st);
  }

  if (!wave_active) return;
  const float l = lane32_sum((lsum[0] + lsum[1]) + (lsum[2] + lsum[3]));
  store_acc_rows<bf16, D, true>(acc, o + (int64_t)bh * Sq * d, qrow, Sq, d, 1.0f / l);
  if (g == 0 && qrow < Sq) lse[(int64_t)bh * Sq + qrow] = (m + __builtin_amdgcn_logf(l)) * kLn2;
}

// ===========================================================================
// Forward, bf16, causal, D in {64, 128}, S % 64 == 0: software-pipelined waves
// ===========================================================================
// 256 query rows per workgroup; each wave owns RB blocks of 32 rows (RB = 1:
// 8 waves, two per SIMD; RB = 2: 4 waves, one per SIMD). Instead of trading
// phases with a partner wave, every wave overlaps its own work: stage j issues
// the products S^T = K_{j+1} Q^T and O^T += V_{j-1}^T P_{j-1}^T, and the
// softmax of tile j runs between those MFMAs on the VALU. One workgroup
// barrier per stage orders the K and V rings, which use the ping-pong
// kernel's LDS layouts and DMA.
//
// The softmax takes no per-tile row max: p = exp2(s c - m) with the running
// m, and the lane's partial row sums double as the overflow test. When one
// exceeds 2^8 or is not finite (always on the first tile, where m = -inf),
// the wave redoes that tile: row max, m raised to it, O and l rescaled, p
// recomputed. Every p that is kept is <= 2^8, the bound of the lazy rescale.

// An empty asm that takes and returns `f`: the value is computed at this
// point of the program, and later code may not be merged with its producer.
__device__ __forceinline__ void pin(bf16x8& f) {
  u32x4 w = __builtin_bit_cast(u32x4, f);
  asm volatile("" : "+v"(w));
  f = __builtin_bit_cast(bf16x8, w);
}

// ---- the pair exchange of the split causal kernels --------------------------
// Blocks A and B of a pair each leave their share of a shared tile in the
// workspace; the second to arrive merges the two. The shares cross between
// workgroups through device memory with agent-scope accesses (each store and
// load goes past the caches a CU does not share), not through agent-scope
// fences: a fence writes back or invalidates the whole L2 of its XCD, which
// every other workgroup there then refills (a split forward ran 2.5x slower
// with them). Pairs of floats, lane-contiguous: register pair r / 2 of a
// wave's 64 lanes fills 512 consecutive bytes, whole cache lines.
__device__ __forceinline__ void xput2(float* p, float x, float y) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, f32x2{x, y}), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x2 xget2(const float* p) {
  return __builtin_bit_cast(f32x2, __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
// Offset (floats) of register pair r2 of accumulator tile `tile` (a wave's
// f32x16 tiles numbered by the caller) in a share laid out as above, for the
// wave's lane `lane`.
__device__ __forceinline__ int xat(int tile, int r2, int lane) { return (tile * 8 + r2) * 128 + 2 * lane; }
// Every wave's stores of its share have reached memory; then one count per
// workgroup (the pair's count is even before a launch and each launch adds
// two). True for the second of the pair to arrive, which merges; called by
// every wave of the workgroup.
__device__ __forceinline__ bool pair_arrive_second(int* count) {
  __shared__ int arrival;
  wait_vmem<0>();
  lds_barrier();
  if (threadIdx.x == 0) arrival = atomicAdd(count, 1);
  lds_barrier();
  return (arrival & 1) != 0;
}

// Workspace of the split backward kernels: one count per pair, rounded up to
// 256 bytes, then the pairs' shares.
__host__ __device__ constexpr int64_t split_counts_bytes(int64_t pairs) { return (pairs * 4 + 255) / 256 * 256; }

// KSPLIT = 2: the waves form pairs on one SIMD (waves w and w + W / 2) that
// take the same rows and split every 64-key tile, keys 0-31 and 32-63; the
// pair merges its softmax states at the end.
template <int D, int RB, int W, int KSPLIT = 1>
struct FwdW {
  static constexpr int kWaves = W, kThreads = 64 * kWaves;
  static constexpr int BQ = 32 * RB * W / KSPLIT, BK = 64;
  static constexpr int KS = D / 16, DT = D / 32;
  typedef PpKTile<D> KT;
  typedef PpVTile<D> VT;
  // D = 256: a slot of 64-key K and V tiles takes 68 KB, so two slots.
  static constexpr int kSlots = D > 128 ? 2 : 3;
  static constexpr int kLds = kSlots * (KT::kBytes + VT::kBytes);
  static constexpr int kDma = KT::kBlocks / kWaves;  // DMA instructions per tile and wave
  static constexpr int kAhead = 3;                   // fragments read ahead of their MFMAs
  static_assert(KT::kBlocks == VT::kBlocks && kDma >= 1, "K and V tiles split evenly over the waves");
};

// SPLIT (a resident grid, ZIG pairing, 128-row tiles, an even number of them): the
// long tile L = n_qtiles - 1 - p and the short tile p of pair p have
// 2 (L + 1) + 2 (p + 1) = 2 (n_qtiles + 1) key tiles between them, and a whole
// long tile keeps its workgroup busy long after its partner is done. Instead
// blocks A and B of the pair cut that sequence of key tiles at `cut`
// (sched::split_segments): the tile the cut falls in is shared, and A and B
// leave their states of it (unnormalised O, row max, row sum) in the
// workspace `ws`; the second to get there (an atomic count per pair, kept even
// between launches) merges the two in a fixed order and writes O and lse.
template <int D, int RB, int W, bool ZIG, int KSPLIT = 1, bool SPLIT = false>
__global__ __launch_bounds__((FwdW<D, RB, W, KSPLIT>::kThreads), (KSPLIT > 1 ? 4 : W == 4 && D <= 128 ? 2 : 1)) void attn_fwd_sw_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, bf16* __restrict__ o,
    float* __restrict__ lse, int bh_count, int S, int d, float scale_log2, int neg_q, int n_qtiles, AttnViews vw,
    char* __restrict__ ws, int cut) {
  typedef FwdW<D, RB, W, KSPLIT> F;
  typedef typename F::KT KT;
  typedef typename F::VT VT;
  constexpr int KS = F::KS, DT = F::DT;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const kring = smem;
  char* const vring = smem + F::kSlots * KT::kBytes;

  // Heaviest (last) query tiles first; all tiles of one head share an XCD
  // when bh_count is a multiple of 8.
  // ZIG: the second half of the tiles in rising order, for a grid that is
  // resident all at once (block b and block b + grid / 2 share a CU).
  const int bh = blockIdx.x % bh_count;
  const int blk = (int)(blockIdx.x / bh_count);
  const int half_q = n_qtiles / 2;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  // Row block of the wave and, with KSPLIT = 2, its key subtile of every tile
  // (NKT subtiles of 32 keys per tile and wave).
  constexpr int WR = W / KSPLIT, NKT = 2 / KSPLIT;
  const int wr = wave % WR;
  const int kh = KSPLIT == 1 ? 0 : wave / WR;

  // Row pitches (elements): d for dense [B, H, S, d] tensors.
  const int ldq = (int)vw.q.r, ldk = (int)vw.k.r, ldv = (int)vw.v.r;
  const bf16* qb = q + vw.q.at(bh, vw.heads);

  // The workgroup's segments: key tiles [t0, t1) of query tile qt. One whole
  // tile without SPLIT; with it, block A's share of the long tile L (role 0),
  // or block B's share of L (role 1) and then the whole short tile.
  static_assert(!SPLIT || (ZIG && KSPLIT == 2 && RB == 1 && F::BQ == 2 * F::BK), "the split pairs 128-row tiles");
  // One segment, inlined once per call below (a loop over the segments left
  // the register allocation of the key-split kernel with spills).
  auto segment = [&](const int qt, const int t0, const int t1, const int role) __attribute__((always_inline)) {
  // With SPLIT (two segments, 128 VGPRs), the lane terms are formed per
  // segment: nothing lane-derived from the first segment stays live (or
  // spills) across the second one's stage loop.
  const int lane = SPLIT ? lane_id() : (int)(threadIdx.x & 63), l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * F::BQ;
  const int q0w = q0 + 32 * RB * wr;
  // Tiles of 64 keys: n for the workgroup, n_w for this wave, whose last
  // tile (keys from 64 (nwf - 1)) is its diagonal, both counted from t0. The
  // upper key half of 32 rows starting a key tile sees no key of that tile:
  // that wave computes nothing in a segment that begins with its diagonal tile
  // (the first 32 rows of the sequence, and with SPLIT the start of B's share).
  int n, n_w, nwf, tt1, nkv;
  const bf16* kb = k + vw.k.at(bh, vw.heads);
  const bf16* vb = v + vw.v.at(bh, vw.heads);
  if constexpr (SPLIT) {
    tt1 = min(t1, (min(q0 + F::BQ, S) - 1) / F::BK + 1);
    n = tt1 - t0;
    nwf = q0w < S ? (q0w + 32 * RB - 1) / F::BK + 1 : 0;
    n_w = kh == 1 && q0w % F::BK == 0 && t0 == nwf - 1 ? 0 : max(min(nwf, tt1) - t0, 0);
    // K and V rows of the segment; the DMA reads nothing past them.
    kb += (int64_t)t0 * F::BK * ldk;
    vb += (int64_t)t0 * F::BK * ldv;
    nkv = n * F::BK;
  } else {
    (void)t0, (void)t1, (void)role;
    n = (min(q0 + F::BQ, S) - 1) / F::BK + 1;
    n_w = q0w < S && !(kh == 1 && q0w == 0) ? (q0w + 32 * RB - 1) / F::BK + 1 : 0;
    nwf = tt1 = 0;
    nkv = S;
  }

  // K_0 and K_1 go out first; stage j then loads K_{j+3} and V_{j+1}.
  const PpDma<KT, true, F::kWaves> kdma(wave, ldk);
  const PpDma<VT, false, F::kWaves> vdma(wave, ldv);
  // Full-width (d == D) Q rows come by DMA as whole rows (a row per D / 8 lanes,
  // 16-byte chunks XOR-swizzled by row) into K slot 2 and the V slots, which
  // the DMA reaches only from stage -1 on; loaded into registers directly,
  // every load instruction touches 32 rows (32 cache lines for 1 KB). Each
  // wave reads its own rows back after sync(-1).
  constexpr int kQRow = 2 * D;
  constexpr int kQStage = sched::fwd_prologue_k(F::kSlots) * KT::kBytes;  // past the prologue's K tiles
  static_assert(kQStage + F::kWaves * 32 * RB * kQRow <= F::kLds, "the Q rows fit the idle ring slots");
  const bool q_lds = d == D;
  char* const qst = smem + kQStage + wave * (32 * RB * kQRow);
  kdma.issue(kb, 0, nkv, ldk, kring);
  if (q_lds) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) dma_rows32<D>(qb, q0w + 32 * rb, S, ldq, qst + rb * 32 * kQRow);
  }
  if constexpr (sched::fwd_prologue_k(F::kSlots) > 1) kdma.issue(kb, F::BK, nkv, ldk, kring + KT::kBytes);

  bf16x8 qf[RB][KS];
  if (!q_lds) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (neg_q)
        load_row_frags<bf16, D, true, true>(qf[rb], qb, q0w + 32 * rb, S, d, ldq);
      else
        load_row_frags<bf16, D, true, false>(qf[rb], qb, q0w + 32 * rb, S, d, ldq);
    }
  }

  const int kbase = KT::off(32 * kh + l32, g * 16);
  const int vbase = VT::off((lane >> 5) * 16 + ((lane & 15) >> 2), 2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));
  // Diagonal tile: key kt*32 + g*16 + r of the tile is invisible to row
  // rb*32 + l32 of the wave when r > lim_at(lane, rb, kt).
  // With SPLIT, a wave whose last tile of the segment lies below its diagonal
  // sees all of it: a uniform offset lifts every limit out of reach (nwf and
  // tt1 are 0 without SPLIT).
  // With SPLIT the limits are formed in the masked stage from lane_id()
  // (formed here, they would stay live across the stage loop and spill).
  const int lim_lift = SPLIT && nwf > tt1 ? 1 << 20 : 0;
  int lim[RB][2];
  if constexpr (!SPLIT) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) lim[rb][kt] = q0w % F::BK + rb * 32 + l32 - kt * 32 - g * 16;
  }
  auto lim_at = [&](int ln, int rb, int kt) {
    if constexpr (SPLIT)
      return q0w % F::BK + rb * 32 + (ln & 31) - kt * 32 - (ln >> 5) * 16 + lim_lift;
    else
      return lim[rb][kt];
  };

  f32x16 acc[RB][DT];  // O^T per row block: register r of tile u = dim u*32 + (r/4)*8 + g*4 + r%4
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][u][r] = 0.f;
  f32x16 s[2][NKT][RB];       // [buffer][key subtile][row block]: S^T of one tile
  bf16x8 pf[2][RB][2 * NKT];  // [buffer][row block][16-key chunk]: P^T fragments
  float m[RB], neg_m[RB], lsum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -INFINITY;
    neg_m[rb] = INFINITY;
    lsum[rb] = 0.f;
  }

  // Stage j loads K_{j+3} and V_{j+1} into the slots that K_j and V_{j-2}
  // left at its barrier (both were last read in stage j - 1); this wave's
  // instruction qd is block qd of its K share, then block qd - kDma of its V
  // share. Issued unconditionally: a tile past the end has an empty buffer
  // range, so its instructions read nothing and write zeros into a slot nobody
  // reads again.
  auto dma_part = [&](int j, int qd) {
    const int tk = sched::fwd_k_loaded(j, F::kSlots), tv = sched::fwd_v_loaded(j, F::kSlots);
    if (qd < F::kDma) {
      kdma.issue_one(kb, tk * F::BK, nkv, ldk, kring + (tk % F::kSlots) * KT::kBytes, qd);
    } else {
      // Two slots load no V at stage -1: tile 0 with an empty range, which
      // reads nothing (a select, not a branch, in the fenced slots).
      const bool vl = sched::fwd_v_loads(j, F::kSlots);
      const int tvc = vl ? tv : 0;
      vdma.issue_one(vb, tvc * F::BK, vl ? nkv : 0, ldv, vring + (tvc % F::kSlots) * VT::kBytes, qd - F::kDma);
    }
  };
  auto dma = [&](int j) {
#pragma unroll
    for (int qd = 0; qd < 2 * F::kDma; ++qd) dma_part(j, qd);
  };

  // Stage j with parity P = j & 1 (tile t lives in s[t & 1] and pf[t & 1]).
  auto stage = [&](auto P_, auto QK_, auto SM_, auto MASK_, auto PV_, int j) __attribute__((always_inline)) {
    constexpr int P = decltype(P_)::value;
    constexpr bool QK = decltype(QK_)::value, SM = decltype(SM_)::value;
    constexpr bool MASK = decltype(MASK_)::value, PV = decltype(PV_)::value;
    f32x16(&sn)[NKT][RB] = s[1 - P];
    f32x16(&sc)[NKT][RB] = s[P];
    bf16x8(&pc)[RB][2 * NKT] = pf[P];
    bf16x8(&pp)[RB][2 * NKT] = pf[1 - P];
    // Stage j reads K_{j+1} and V_{j-1}. The slot offsets pass through an
    // empty asm: where the compiler can fold them to constants (the unrolled
    // stage pairs), it hoists a separate lane address for every fragment read
    // out of the stage loop (the reads' 16-bit offsets cannot reach past 64 KB
    // of ring), and those addresses spill: the D = 64 key-split kernel wrote
    // 12 bytes of scratch per lane without this.
    int koff = (sched::fwd_k_read(j) % F::kSlots) * KT::kBytes;
    int voff = ((sched::fwd_v_read(j) + F::kSlots) % F::kSlots) * VT::kBytes;
    asm volatile("" : "+s"(koff), "+s"(voff));
    const char* kp = kring + koff + kbase;
    const char* vp = vring + voff + vbase;
    // K fragments: key subtile f % NKT (with KSPLIT = 2 the wave's own, whose
    // rows kbase already points at), k-chunk f / NKT.
    constexpr int NFQ = QK ? NKT * KS : 0;
    // V^T fragments: the wave's key chunk i / DT of 16 keys (chunk 2 kh + i / DT
    // of the tile with KSPLIT = 2), dim tile i % DT.
    constexpr int NFV = PV ? 2 * NKT * DT : 0;
    constexpr int NF = NFQ + NFV;
    auto read = [&](int f) -> bf16x8 {
      if (f < NFQ) return *reinterpret_cast<const bf16x8*>(kp + KT::off(32 * (f % NKT), (f / NKT) * 32));
      const int i = f - NFQ, c = 2 * kh + i / DT, u = i % DT;
      return tr_frag(vp + VT::off((c >> 1) * 32 + (c & 1) * 8, u * 64), VT::off(4, 0));
    };
    // Product rb of fragment f.
    auto prod1 = [&](int f, int rb, const bf16x8& a) {
      if (f < NFQ) {
        const int kt = f % NKT, kc = f / NKT;
        if (kc == 0)
          sn[kt][rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[rb][0], f32x16{}, 0, 0, 0);
        else
          mma32(a, qf[rb][kc], sn[kt][rb]);
      } else {
        const int i = f - NFQ, cl = i / DT, u = i % DT;
        mma32(a, pp[rb][cl], acc[rb][u]);
      }
    };
    const int ln_mask = SPLIT && MASK ? lane_id() : 0;  // the lane for the diagonal's limits
    float t[RB][2];  // [row block][partial] sums of this tile's p in the lane
    // Softmax element e of the lane: row block e / (16 NKT), key subtile
    // (e / 16) % NKT of the wave's (kt + kh of the tile), register e % 16.
    // Every 8 elements make one P^T fragment.
    float p[8];
    auto softmax_elem = [&](int e, const float(&nm)[RB]) {
      const int rb = e / (16 * NKT), kt = (e >> 4) % NKT, r = e & 15;
      float x = sc[kt][rb][r];
      if constexpr (MASK) x = r > lim_at(ln_mask, rb, kt + kh) ? -INFINITY : x;
      p[r & 7] = __builtin_amdgcn_exp2f(__builtin_fmaf(x, scale_log2, nm[rb]));
      t[rb][r & 1] += p[r & 7];
      if ((r & 7) == 7) {
        bf16x8& f = pc[rb][2 * kt + (r >> 3)];
        to_frag(p, f);
        // Keep the conversion here: without the fence the compiler sinks it
        // below the rare redo branch, which holds all p values live across it.
        pin(f);
      }
    };
    constexpr int NE = 16 * NKT * RB;  // softmax elements per lane
    auto softmax = [&](const float(&nm)[RB]) {
#pragma unroll
      for (int e = 0; e < NE; ++e) softmax_elem(e, nm);
    };
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) t[rb][0] = t[rb][1] = 0.f;

    if constexpr (NF > 0) {
      // The program order is the schedule: MFMA slot i carries the product
      // i % RB of fragment i / RB, the LDS read of the fragment kAhead
      // further on (at the fragment's first product) and an equal share of
      // the softmax elements, fenced so that the scheduler keeps it so.
      // The stage's DMA instructions go out one at a time between products
      // (issued together, the eight waves queue behind each other in the
      // CU's vector memory path), with no branch in the fenced slots, spread
      // over the S products when the stage also has P V products (1.5% faster
      // than over all of them).
      constexpr int NM = NF * RB;
      constexpr int NQ = 2 * F::kDma;
      static_assert(!SM || NE % NM == 0 || NM % NE == 0, "softmax elements spread evenly over the products");
      bf16x8 buf[NF];
#pragma unroll
      for (int f = 0; f < F::kAhead && f < NF; ++f) buf[f] = read(f);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        const int f = i / RB, rb = i % RB;
        if (rb == 0 && f + F::kAhead < NF) buf[f + F::kAhead] = read(f + F::kAhead);
#pragma unroll
        for (int qd = 0; qd < NQ; ++qd)
          if (i == (2 * qd + 1) * (NFQ > 0 && NFV > 0 ? NM / 2 : NM) / (2 * NQ)) dma_part(j, qd);
        prod1(f, rb, buf[f]);
        if constexpr (SM) {
          if constexpr (NE >= NM) {
#pragma unroll
            for (int e = i * (NE / NM); e < (i + 1) * (NE / NM); ++e) softmax_elem(e, neg_m);
          } else {
            if (i % (NM / NE) == 0) softmax_elem(i / (NM / NE), neg_m);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      dma(j);
      if constexpr (SM) softmax(neg_m);
    }

    if constexpr (SM) {
      bool bad = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) bad = bad || !(t[rb][0] + t[rb][1] <= 256.f);
      if (__builtin_amdgcn_ballot_w64(bad)) {
        // Redo the tile from the row max: raise m, rescale O and l.
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float mx = -INFINITY;
#pragma unroll
          for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              float x = sc[kt][rb][r];
              if constexpr (MASK) x = r > lim_at(ln_mask, rb, kt + kh) ? -INFINITY : x;
              mx = fmaxf(mx, x);
            }
          const float m_new = fmaxf(m[rb], lane32_max(mx) * scale_log2);
          const float alpha = __builtin_amdgcn_exp2f(m[rb] - m_new);
          m[rb] = m_new;
          neg_m[rb] = -m_new;
          lsum[rb] *= alpha;
#pragma unroll
          for (int u = 0; u < DT; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[rb][u][r] *= alpha;
          t[rb][0] = t[rb][1] = 0.f;
        }
        softmax(neg_m);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) lsum[rb] += t[rb][0] + t[rb][1];
    }
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // The workgroup passes stages j = -1 .. n; sync(j) opens stage j.
  auto sync = [&](int j) {
    // This wave's parts of K_{j+1} and V_{j-1} have landed; with three slots
    // the loads issued by stage j - 1 (or K_1 of the prologue) may still be in
    // flight, with two none is.
    if (j >= 0)
      wait_vmem<sched::fwd_in_flight(0, F::kDma, F::kSlots)>();
    else
      wait_vmem<sched::fwd_in_flight(-1, F::kDma, F::kSlots)>();
    // Every wave's parts have landed and every wave has left stage j - 1.
    lds_barrier();
  };
  // This wave's stages: QK of tile 0; QK + softmax for tiles 0 .. n_w - 2
  // (with PV from tile 1 on); the diagonal tile's masked softmax; the last PV.
  sync(-1);
  if (q_lds) {
    // This wave's Q rows have landed (sync(-1) waited for them); the barrier
    // keeps stage -1's DMA (K_2 and V_0, or with two slots K_1) off the staging until every wave has
    // read its rows.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      row_frags_lds<D>(qf[rb], qst + rb * 32 * kQRow);
      if (neg_q) {
#pragma unroll
        for (int kc = 0; kc < KS; ++kc) {
          u32x4 w = __builtin_bit_cast(u32x4, qf[rb][kc]);
          w ^= 0x80008000u;
          qf[rb][kc] = __builtin_bit_cast(bf16x8, w);
        }
      }
    }
    lds_barrier();
  }
  if (n_w > 0)
    stage(P1(), T_(), F_(), F_(), F_(), -1);
  else
    dma(-1);
  int j = 0;
  if (n_w >= 2) {
    sync(0);
    stage(P0(), T_(), T_(), F_(), F_(), 0);
    for (j = 1; j + 2 < n_w; j += 2) {
      sync(j);
      stage(P1(), T_(), T_(), F_(), T_(), j);
      sync(j + 1);
      stage(P0(), T_(), T_(), F_(), T_(), j + 1);
    }
    if (j + 1 < n_w) {
      sync(j);
      stage(P1(), T_(), T_(), F_(), T_(), j);
      ++j;
    }
  }
  if (n_w == 1) {
    sync(0);
    stage(P0(), F_(), T_(), T_(), F_(), 0);
    sync(1);
    stage(P1(), F_(), F_(), F_(), T_(), 1);
    j = 2;
  } else if (n_w >= 2) {
    if (j & 1) {
      sync(j);
      stage(P1(), F_(), T_(), T_(), T_(), j);
      sync(j + 1);
      stage(P0(), F_(), F_(), F_(), T_(), j + 1);
    } else {
      sync(j);
      stage(P0(), F_(), T_(), T_(), T_(), j);
      sync(j + 1);
      stage(P1(), F_(), F_(), F_(), T_(), j + 1);
    }
    j += 2;
  }
  for (; j <= n; ++j) {
    sync(j);
    dma(j);
  }
  wait_vmem<0>();

  // With SPLIT, the epilogue's lane terms from lane_id() (nothing lane-derived
  // stays live across the stage loop).
  const int lane_e = SPLIT ? lane_id() : lane, l32_e = lane_e & 31, g_e = lane_e >> 5;
  if constexpr (KSPLIT > 1) {
    // The upper key half hands its accumulators, maxima and partial sums to
    // the lower half of its rows through the (now idle) rings; the lower half
    // rescales both to the larger maximum. A wave that computed nothing hands
    // over zeros and -inf, which weigh nothing.
    constexpr int kXs = (16 * DT + 2) * 64;  // floats per row block
    static_assert(RB == 1 && WR * kXs * 4 <= F::kLds, "the upper halves' states fit the rings");
    float* const xs = reinterpret_cast<float*>(smem) + wr * kXs;
    lds_barrier();
    if (kh == 1) {
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<f32x4*>(xs + ((u * 4 + r4) * 64 + lane_e) * 4) =
              f32x4{acc[0][u][4 * r4], acc[0][u][4 * r4 + 1], acc[0][u][4 * r4 + 2], acc[0][u][4 * r4 + 3]};
      xs[16 * DT * 64 + lane_e] = m[0];
      xs[16 * DT * 64 + 64 + lane_e] = lsum[0];
    }
    lds_barrier();
    if (kh == 0) {
      const float m1 = xs[16 * DT * 64 + lane_e];
      const float l1 = xs[16 * DT * 64 + 64 + lane_e];
      const float mm = fmaxf(m[0], m1);
      float a0 = __builtin_amdgcn_exp2f(m[0] - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
      if (SPLIT && mm == -INFINITY) a0 = a1 = 0.f;  // neither half saw a key of the segment
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 o1 = *reinterpret_cast<const f32x4*>(xs + ((u * 4 + r4) * 64 + lane_e) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[0][u][4 * r4 + e] = acc[0][u][4 * r4 + e] * a0 + o1[e] * a1;
        }
      lsum[0] = lsum[0] * a0 + l1 * a1;
      m[0] = mm;
    }
  }
  // The lower key half of each row block writes (every wave without KSPLIT).
  const bool writer = kh == 0 && q0w < S;
  float lrow[RB];  // the rows' sums of p (the lane's and its partner's 32 lanes away)
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) lrow[rb] = lane32_sum(lsum[rb]);

  if constexpr (SPLIT) {
    if (role >= 0) {
      // This share of the long tile: the writers' (O, m, l) into the pair's
      // slot, role-major, then one count per workgroup.
      const int slot = bh * half_q + blk % half_q;
      constexpr int kAccFloats = WR * DT * 16 * 64;
      constexpr int kPartBytes = (kAccFloats + 2 * F::BQ) * 4;
      float* const part = reinterpret_cast<float*>(ws + (int64_t)(2 * slot + role) * kPartBytes);
      float* const other = reinterpret_cast<float*>(ws + (int64_t)(2 * slot + 1 - role) * kPartBytes);
      int* const count = reinterpret_cast<int*>(ws + (int64_t)2 * bh_count * half_q * kPartBytes) + slot;
      if (writer) {
#pragma unroll
        for (int u = 0; u < DT; ++u)
#pragma unroll
          for (int r2 = 0; r2 < 8; ++r2) xput2(part + xat(wr * DT + u, r2, lane_e), acc[0][u][2 * r2], acc[0][u][2 * r2 + 1]);
        if (g_e == 0) xput2(part + kAccFloats + 2 * (32 * wr + l32_e), m[0], lrow[0]);
      }
      // The first of A and B to arrive is done with the long tile.
      if (!pair_arrive_second(count)) return;
      if (writer) {
        // Merge in role order whichever block runs it: A (keys before the
        // split), then B.
        const f32x2 st = xget2(other + kAccFloats + 2 * (32 * wr + l32_e));
        const float mo = st[0], lo = st[1];
        const float ma = role == 0 ? m[0] : mo, mb = role == 0 ? mo : m[0];
        const float la = role == 0 ? lrow[0] : lo, lb = role == 0 ? lo : lrow[0];
        const float mm = fmaxf(ma, mb);  // A's rows all see key 0: finite
        const float ca = __builtin_amdgcn_exp2f(ma - mm), cb = __builtin_amdgcn_exp2f(mb - mm);
#pragma unroll
        for (int u = 0; u < DT; ++u)
#pragma unroll
          for (int r2 = 0; r2 < 8; ++r2) {
            const f32x2 oo = xget2(other + xat(wr * DT + u, r2, lane_e));
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const float mine = acc[0][u][2 * r2 + e];
              const float xa = role == 0 ? mine : oo[e], xb = role == 0 ? oo[e] : mine;
              // Spelled out: A and B inline this merge separately, and left to
              // itself the compiler contracts it into an fma on different sides
              // in the two copies (results that differ in the last bit).
              acc[0][u][2 * r2 + e] = __builtin_fmaf(xa, ca, xb * cb);
            }
          }
        lrow[0] = __builtin_fmaf(la, ca, lb * cb);
        m[0] = mm;
      }
    }
  }

  if (d < D) {
    if (!writer) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = q0w + 32 * rb + l32_e;
      const float l = lrow[rb];
      store_acc_rows<bf16, D, true>(acc[rb], o + vw.o.at(bh, vw.heads), row, S, d, 1.0f / l, vw.o.r);
      if (g_e == 0 && row < S) lse[(int64_t)bh * S + row] = (m[rb] + __builtin_amdgcn_logf(l)) * kLn2;
    }
    return;
  }
  // Full-width rows go out through LDS (store_acc_rows_lds), each wave in its
  // own part of the (now idle) rings. The barrier: every wave has left its last
  // stage and its ring reads, and every DMA (this wave's waited above) has
  // landed.
  static_assert(F::kWaves * 32 * RB * 2 * D <= F::kLds, "every wave's rows fit the rings");
  lds_barrier();
  if (!writer) return;
  char* const ot = smem + wave * (32 * RB * 2 * D);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = q0w + 32 * rb + l32_e;
    const float l = lrow[rb];
    if (g_e == 0 && row < S) lse[(int64_t)bh * S + row] = (m[rb] + __builtin_amdgcn_logf(l)) * kLn2;
    store_acc_rows_lds<D, SPLIT>(acc[rb], ot + rb * 32 * 2 * D, o + vw.o.at(bh, vw.heads), q0w + 32 * rb, S,
                                 1.0f / l, vw.o.r);
  }
  };  // segment

  if constexpr (!SPLIT) {
    segment(sched::query_tile(blk, n_qtiles, ZIG), 0, 0, -1);
  } else {
    sched::Segment seg[2];
    const int nseg = sched::split_segments(blk, n_qtiles, cut, seg);
    segment(seg[0].qt, seg[0].t0, seg[0].t1, seg[0].role);
    if (nseg > 1) {
      // Every wave has left the first segment's LDS (its O rows may have gone
      // out through the rings) before the second one's DMA writes them.
      lds_barrier();
      segment(seg[1].qt, seg[1].t0, seg[1].t1, seg[1].role);
    }
  }
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
// Wide head dims (D = 128 * nc, nc >= 2): the forward for D > 256, dQ and dK/dV
// for D >= 256 (the reference accepts any multiple of 128, flash_attention.py:
// 341-343). The products that contract over D (S = Q K^T, dP = dO V^T) run over
// the nc 128-column slabs of the operands, each staged through LDS in turn. The
// products that produce D columns (O, dQ, dK, dV) keep the accumulators of one
// 128-column output slab, chosen by the workgroup's place in the grid, so nc
// workgroups recompute a tile's scores and each writes its own slab. Register
// and LDS use therefore do not grow with D. Tile shapes, fragment layouts,
// masking and the exp2-domain softmax are those of the kernels above at D = 128.
// ===========================================================================
constexpr int kSlab = 128;

template <typename T>
struct Wide {
  static constexpr int BQ = 128;                  // queries per workgroup (forward, dQ)
  static constexpr int BKV = 128;                 // keys per workgroup (dK/dV)
  static constexpr int BS = AttnTiles<T>::kStep;  // streamed rows per step (64 bf16, 32 f32)
  static constexpr int NT = BS / 32;
  static constexpr int KS = kSlab / 16;  // 16-wide k chunks of one slab
  static constexpr int DT = kSlab / 32;  // 32-column output tiles of one slab
  static constexpr int kRowBytes = BS * RowTile<T, kSlab>::kPitch;
  static constexpr int kTrBytes = kSlab * 128;
  static constexpr int kFwdLds = kRowBytes + kTrBytes;
  static constexpr int kDqLds = 2 * kRowBytes + kTrBytes;
  static constexpr int kDkvLds = 2 * kRowBytes + 2 * kTrBytes + 2 * BS * 4;
};

// Workgroup -> (head, tile, output slab): sched::wide_coord.
struct WideCoord : sched::WideCoord {
  __device__ WideCoord(int bh_count, int n_tiles, bool heavy_last)
      : sched::WideCoord(sched::wide_coord((int)blockIdx.x, bh_count, n_tiles, heavy_last)) {}
};

template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads, ALIGNED ? 2 : 1) void attn_fwd_wide_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                                   const T* __restrict__ v, T* __restrict__ o,
                                                                   float* __restrict__ lse, int bh_count, int Sq,
                                                                   int Sk, int d, int causal, float scale_log2,
                                                                   int neg_q, int n_qtiles) {
  typedef Wide<T> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* kl = smem;                 // K rows of one slab
  char* vl = smem + F::kRowBytes;  // V^T of the output slab

  const int nc = d / kSlab;
  const WideCoord wc(bh_count, n_qtiles, true);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = wc.tile * F::BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + l32;

  const T* qb = q + (int64_t)wc.bh * Sq * d;
  const T* kb = k + (int64_t)wc.bh * Sk * d;
  const T* vb = v + (int64_t)wc.bh * Sk * d;

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const int n_tiles = causal ? min(q_last, Sk - 1) / F::BS + 1 : (Sk + F::BS - 1) / F::BS;
  const bool wave_active = q0w < Sq;
  const int wave_tiles = !wave_active ? 0 : causal ? min(q0w + 31, Sq - 1) / F::BS + 1 : n_tiles;

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  float m = -INFINITY;
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};
  Stager<T, kSlab, F::BS, ALIGNED> ks(kSlab, d), vs(kSlab, d);

  for (int j = 0; j < n_tiles; ++j) {
    const int kv0 = j * F::BS;
    const bool work = j < wave_tiles;
    // S^T = K Q^T over the slabs: s[t][r] is key kv0 + t*32 + g*16 + r, query qrow.
    f32x16 s[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
    for (int c = 0; c < nc; ++c) {
      ks.load(kb + c * kSlab, kv0, Sk, kSlab);
      __syncthreads();  // every wave is done with the previous slab
      ks.store_rows(kl);
      __syncthreads();
      if (work) {
        frag qf[F::KS];
        if (neg_q)
          load_row_frags<T, kSlab, ALIGNED, true>(qf, qb + c * kSlab, q0w, Sq, kSlab, d);
        else
          load_row_frags<T, kSlab, ALIGNED, false>(qf, qb + c * kSlab, q0w, Sq, kSlab, d);
        lds_mfma_pipeline<F::KS * F::NT>(
            [&](int i) { return RowTile<T, kSlab>::frag(kl, (i % F::NT) * 32 + l32, (i / F::NT) * 16 + g * 8); },
            [&](int i, const frag& a) { mma32(a, qf[i / F::NT], s[i % F::NT]); });
      }
    }
    // V^T of the output slab. Its previous readers finished before the slab
    // loop's barriers above.
    vs.load(vb + wc.slab * kSlab, kv0, Sk, kSlab);
    vs.store_transposed(vl);
    __syncthreads();
    if (!work) continue;

    if ((causal && kv0 + F::BS - 1 > q0w) || kv0 + F::BS > Sk) {
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
    // O^T (this slab) += V^T P^T
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
  store_acc_rows<T, kSlab, ALIGNED>(acc, o + (int64_t)wc.bh * Sq * d + wc.slab * kSlab, qrow, Sq, kSlab, inv, d);
  if (wc.slab == 0 && g == 0 && qrow < Sq) lse[(int64_t)wc.bh * Sq + qrow] = (m + __builtin_amdgcn_logf(l)) * kLn2;
}

template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads, ALIGNED ? 2 : 1) void attn_dq_wide_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                                  const T* __restrict__ v, const T* __restrict__ dout,
                                                                  const float* __restrict__ lse,
                                                                  const float* __restrict__ delta, T* __restrict__ dq,
                                                                  int bh_count, int Sq, int Sk, int d, int causal,
                                                                  float scale, float scale_log2, int n_qtiles) {
  typedef Wide<T> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* kl = smem;                     // K rows of one slab
  char* vl = smem + F::kRowBytes;      // V rows of the same slab
  char* ktl = smem + 2 * F::kRowBytes;  // K^T of the output slab

  const int nc = d / kSlab;
  const WideCoord wc(bh_count, n_qtiles, true);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = wc.tile * F::BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + l32;

  const T* qb = q + (int64_t)wc.bh * Sq * d;
  const T* dob = dout + (int64_t)wc.bh * Sq * d;
  const T* kb = k + (int64_t)wc.bh * Sk * d;
  const T* vb = v + (int64_t)wc.bh * Sk * d;

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const int n_tiles = causal ? min(q_last, Sk - 1) / F::BS + 1 : (Sk + F::BS - 1) / F::BS;
  const bool wave_active = q0w < Sq;
  const int wave_tiles = !wave_active ? 0 : causal ? min(q0w + 31, Sq - 1) / F::BS + 1 : n_tiles;
  const bool qok = qrow < Sq;
  const float lse2 = qok ? lse[(int64_t)wc.bh * Sq + qrow] * kLog2e : 0.f;
  const float dl = qok ? delta[(int64_t)wc.bh * Sq + qrow] : 0.f;

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  Stager<T, kSlab, F::BS, ALIGNED> ks(kSlab, d), vs(kSlab, d);

  for (int j = 0; j < n_tiles; ++j) {
    const int kv0 = j * F::BS;
    const bool work = j < wave_tiles;
    // S^T = K Q^T and dP^T = V dO^T over the slabs: [t][r] is key kv0 + t*32 + g*16 + r, query qrow.
    f32x16 s[F::NT], dp[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = 0.f;
        dp[t][r] = 0.f;
      }
    for (int c = 0; c < nc; ++c) {
      ks.load(kb + c * kSlab, kv0, Sk, kSlab);
      vs.load(vb + c * kSlab, kv0, Sk, kSlab);
      __syncthreads();
      ks.store_rows(kl);
      vs.store_rows(vl);
      __syncthreads();
      if (work) {
        frag qf[F::KS], dof[F::KS];
        load_row_frags<T, kSlab, ALIGNED>(qf, qb + c * kSlab, q0w, Sq, kSlab, d);
        load_row_frags<T, kSlab, ALIGNED>(dof, dob + c * kSlab, q0w, Sq, kSlab, d);
#pragma unroll
        for (int kk = 0; kk < F::KS; ++kk)
#pragma unroll
          for (int t = 0; t < F::NT; ++t) {
            mma32(RowTile<T, kSlab>::frag(kl, t * 32 + l32, kk * 16 + g * 8), qf[kk], s[t]);
            mma32(RowTile<T, kSlab>::frag(vl, t * 32 + l32, kk * 16 + g * 8), dof[kk], dp[t]);
          }
      }
    }
    ks.load(kb + wc.slab * kSlab, kv0, Sk, kSlab);
    ks.store_transposed(ktl);
    __syncthreads();
    if (!work) continue;

    const bool need_mask = (causal && kv0 + F::BS - 1 > q0w) || (kv0 + F::BS > Sk);
    frag dsf[F::NT][2];
#pragma unroll
    for (int t = 0; t < F::NT; ++t) {
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(s[t][r] * scale_log2 - lse2);
        if (need_mask) {
          const int kv = kv0 + t * 32 + g * 16 + r;
          if (kv >= Sk || (causal && kv > qrow)) p = 0.f;
        }
        ds[r] = p * (dp[t][r] - dl);
      }
      to_frag(ds, dsf[t][0]);
      to_frag(ds + 8, dsf[t][1]);
    }
    // dQ^T (this slab) += K^T dS^T
#pragma unroll
    for (int u = 0; u < F::DT; ++u)
#pragma unroll
      for (int t = 0; t < F::NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          mma32(TrTile<T>::frag(ktl, u * 32 + l32, t * 32 + g * 16 + h * 8), dsf[t][h], acc[u]);
  }
  if (!wave_active) return;
  store_acc_rows<T, kSlab, ALIGNED>(acc, dq + (int64_t)wc.bh * Sq * d + wc.slab * kSlab, qrow, Sq, kSlab, scale, d);
}

template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads, 1) void attn_dkv_wide_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                                   const T* __restrict__ v, const T* __restrict__ dout,
                                                                   const float* __restrict__ lse,
                                                                   const float* __restrict__ delta, T* __restrict__ dk,
                                                                   T* __restrict__ dv, int bh_count, int Sq, int Sk,
                                                                   int d, int causal, float scale, float scale_log2,
                                                                   int n_ktiles) {
  typedef Wide<T> F;
  typedef typename Elem<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* ql = smem;                          // Q rows of one slab
  char* dol = ql + F::kRowBytes;            // dO rows of the same slab
  char* qtl = dol + F::kRowBytes;           // Q^T of the output slab
  char* dotl = qtl + F::kTrBytes;           // dO^T of the output slab
  float* lsel = reinterpret_cast<float*>(dotl + F::kTrBytes);
  float* dll = lsel + F::BS;

  const int nc = d / kSlab;
  const WideCoord wc(bh_count, n_ktiles, false);  // heaviest (first) key tiles first
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int k0 = wc.tile * F::BKV;
  const int k0w = k0 + wave * 32;
  const int kvrow = k0w + l32;

  const T* qb = q + (int64_t)wc.bh * Sq * d;
  const T* dob = dout + (int64_t)wc.bh * Sq * d;
  const T* kb = k + (int64_t)wc.bh * Sk * d;
  const T* vb = v + (int64_t)wc.bh * Sk * d;
  const float* lseb = lse + (int64_t)wc.bh * Sq;
  const float* db = delta + (int64_t)wc.bh * Sq;

  const int first = causal ? k0 / F::BS : 0;
  const int n_qt = (Sq + F::BS - 1) / F::BS;
  const bool wave_active = k0w < Sk;

  f32x16 dka[F::DT], dva[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dka[u][r] = 0.f;
      dva[u][r] = 0.f;
    }
  Stager<T, kSlab, F::BS, ALIGNED> qs(kSlab, d), dos(kSlab, d);

  for (int it = first; it < n_qt; ++it) {
    const int qs0 = it * F::BS;
    // Causal: this wave's keys see queries >= k0w only.
    const bool work = wave_active && !(causal && qs0 + F::BS - 1 < k0w);
    // S = Q K^T and dP = dO V^T over the slabs: [t][r] is query qs0 + t*32 + g*16 + r, key kvrow.
    f32x16 s[F::NT], dp[F::NT];
#pragma unroll
    for (int t = 0; t < F::NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = 0.f;
        dp[t][r] = 0.f;
      }
    for (int c = 0; c < nc; ++c) {
      qs.load(qb + c * kSlab, qs0, Sq, kSlab);
      dos.load(dob + c * kSlab, qs0, Sq, kSlab);
      __syncthreads();
      qs.store_rows(ql);
      dos.store_rows(dol);
      __syncthreads();
      if (work) {
        frag kf[F::KS], vf[F::KS];
        load_row_frags<T, kSlab, ALIGNED>(kf, kb + c * kSlab, k0w, Sk, kSlab, d);
        load_row_frags<T, kSlab, ALIGNED>(vf, vb + c * kSlab, k0w, Sk, kSlab, d);
#pragma unroll
        for (int kk = 0; kk < F::KS; ++kk)
#pragma unroll
          for (int t = 0; t < F::NT; ++t) {
            mma32(RowTile<T, kSlab>::frag(ql, t * 32 + l32, kk * 16 + g * 8), kf[kk], s[t]);
            mma32(RowTile<T, kSlab>::frag(dol, t * 32 + l32, kk * 16 + g * 8), vf[kk], dp[t]);
          }
      }
    }
    // The output slab's Q^T and dO^T and the step's statistics; their
    // previous readers finished before the slab loop's barriers above.
    qs.load(qb + wc.slab * kSlab, qs0, Sq, kSlab);
    dos.load(dob + wc.slab * kSlab, qs0, Sq, kSlab);
    if (threadIdx.x < F::BS) {
      const int row = qs0 + threadIdx.x;
      // Rows past Sq get lse = +inf so that P = 0 there.
      lsel[threadIdx.x] = row < Sq ? lseb[row] * kLog2e : INFINITY;
      dll[threadIdx.x] = row < Sq ? db[row] : 0.f;
    }
    qs.store_transposed(qtl);
    dos.store_transposed(dotl);
    __syncthreads();
    if (!work) continue;

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
          if (need_mask && kvrow > qs0 + t * 32 + g * 16 + r) pv = 0.f;
          p[r] = pv;
          ds[r] = pv * (dp[t][r] - dd[e]);
        }
      }
      to_frag(p, pf[t][0]);
      to_frag(p + 8, pf[t][1]);
      to_frag(ds, dsf[t][0]);
      to_frag(ds + 8, dsf[t][1]);
    }
    // dV^T += dO^T P ; dK^T += Q^T dS (this slab)
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
  const int64_t off = (int64_t)wc.bh * Sk * d + wc.slab * kSlab;
  store_acc_rows<T, kSlab, ALIGNED>(dka, dk + off, kvrow, Sk, kSlab, scale, d);
  store_acc_rows<T, kSlab, ALIGNED>(dva, dv + off, kvrow, Sk, kSlab, 1.0f, d);
}

// ===========================================================================
// Backward, bf16 with D in {64, 128, 256}: streamed tiles read as rows and transposed
// ===========================================================================
// The backward kernels read each streamed 64-row tile twice: as row
// fragments (16-byte reads, A operand of S = Q K^T or S^T = K Q^T) and
// transposed (ds_read_b64_tr_b16, A operand of dK^T += Q^T dS or
// dQ^T += K^T dS^T). Row p sits in the 1 KB block of the rows congruent to p
// mod 16, at position p / 16, and block b is placed at index 4 (b % 4) + b / 4
// with a 1040-byte stride. Sixteen consecutive rows then lie in sixteen
// different 16-byte bank slots (row reads), four consecutive rows in four
// different 64-byte bank groups (transposed reads), and every fragment
// address is a per-lane base plus a constant. Rows are stored in the MFMA
// output order of perm_row, as in the forward K tile.
// D = 256 (512-byte rows): a 1 KB block holds two rows, so the tile is two
// such 16-block halves, rows 0-31 and 32-63, one after the other. Every
// offset inside a half differs from the D = 128 tile's only by multiples of
// 256 bytes (a row position times 512 instead of 256), so the lanes of a
// read meet the same banks as there. The DMA then moves 32 blocks of 1 KB
// (two rows each, every lane carrying data).
template <int D>
struct BwdTile {
  static_assert(D == 64 || D == 128 || D == 256, "128-, 256- or 512-byte rows");
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kChunks = kRowBytes / 16;
  static constexpr int kHalves = D == 256 ? 2 : 1;
  static constexpr int kBlocks = 16 * kHalves;  // 1 KB DMA blocks
  static constexpr int kStride = 1024 + 16;
  static constexpr int kHalfBytes = 16 * kStride;
  static constexpr int kBytes = kHalves * kHalfBytes;
  static __host__ __device__ constexpr int place(int b) { return 4 * (b & 3) + (b >> 2); }
  static __host__ __device__ constexpr int block_off(int b) { return (b >> 4) * kHalfBytes + place(b & 15) * kStride; }
  static __host__ __device__ constexpr int off(int p, int byte) {
    return D == 256 ? (p >> 5) * kHalfBytes + place(p & 15) * kStride + ((p >> 4) & 1) * kRowBytes + byte
                    : place(p & 15) * kStride + (p >> 4) * kRowBytes + byte;
  }
  // With 128-byte rows a block holds its four rows in its first 512 bytes;
  // lanes 32-63 of its DMA instruction are switched off (they write zeros
  // into the unused half). With 512-byte rows block b holds rows
  // 32 (b / 16) + b % 16 and that + 16.
  static __host__ __device__ constexpr int dma_row(int b, int L) {
    return D == 256 ? 32 * (b >> 4) + (b & 15) + 16 * (L / kChunks) : b + 16 * (L / kChunks);
  }
  static __host__ __device__ constexpr int dma_chunk(int L) { return L % kChunks; }
  static __device__ __forceinline__ bool dma_lane(int L) { return L / kChunks < 4; }
  // Row fragment (physical rows 32 half + l32, bytes 32 kk + 16 g): lane base
  // plus row_at(half, kk).
  static __device__ __forceinline__ int row_base(int lane) { return off(lane & 31, (lane >> 5) * 16); }
  static __host__ __device__ constexpr int row_at(int half, int kk) { return off(32 * half, 32 * kk); }
  // Transposed fragment of logical rows 32 half + 16 g + 8 h + e (e = 0..7),
  // column 32 u + l32: physical rows 32 half + 16 h + 4 g + (0..3), then + 8.
  static __device__ __forceinline__ int tr_base(int lane) {
    return off(4 * (lane >> 5) + ((lane & 15) >> 2), 2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));
  }
  static __host__ __device__ constexpr int tr_at(int half, int h, int u) { return off(32 * half + 16 * h, 64 * u); }
  static constexpr int kTrHi = off(8, 0);
  // A lane's fragment addresses: a base plus a constant.
  struct Bases {
    int r, t;
    __device__ __forceinline__ explicit Bases(int lane) : r(row_base(lane)), t(tr_base(lane)) {}
  };
  static __device__ __forceinline__ int row(const Bases& b, int half, int kk) { return b.r + row_at(half, kk); }
  static __device__ __forceinline__ int tr(const Bases& b, int half, int h, int u) { return b.t + tr_at(half, h, u); }
};

// Compile-time check of a BwdTile's DMA: lane L of block instruction b writes
// LDS bytes block_off(b) + 16 L, which must be where off() keeps the row and
// chunk the lane loads, every (row, chunk) of the 64 rows exactly once; and,
// for G waves sharing the instructions (PpDma), the source row of a wave's
// instruction i is its row for instruction 0 plus a delta independent of the
// wave and the lane.
template <int D, int G>
constexpr bool bwd_tile_dma_ok() {
  typedef BwdTile<D> T;
  bool seen[64 * T::kChunks] = {};
  for (int b = 0; b < T::kBlocks; ++b)
    for (int L = 0; L < 64; ++L) {
      if (L / T::kChunks >= 4) continue;
      const int p = T::dma_row(b, L), c = T::dma_chunk(L);
      if (p < 0 || p >= 64 || seen[p * T::kChunks + c]) return false;
      seen[p * T::kChunks + c] = true;
      if (T::block_off(b) + 16 * L != T::off(p, 16 * c)) return false;
    }
  for (bool x : seen)
    if (!x) return false;
  for (int gw = 0; gw < G; ++gw)
    for (int i = 0; i < T::kBlocks / G; ++i) {
      const int d0 = perm_src(T::dma_row(G * i, 0)) - perm_src(T::dma_row(0, 0));
      for (int L = 0; L < 64; ++L)
        if (L / T::kChunks < 4 && perm_src(T::dma_row(gw + G * i, L)) != perm_src(T::dma_row(gw, L)) + d0)
          return false;
    }
  return true;
}
static_assert(bwd_tile_dma_ok<64, 4>() && bwd_tile_dma_ok<64, 8>() && bwd_tile_dma_ok<128, 4>() &&
                  bwd_tile_dma_ok<128, 8>() && bwd_tile_dma_ok<256, 4>() && bwd_tile_dma_ok<256, 8>(),
              "BwdTile DMA blocks cover the tile once, where the reads expect them");

// Compact tile for D = 64 (128-byte rows): 8 KB of rows in 8 blocks of 8
// consecutive physical rows (row p in block p / 8 at position p % 8), the
// 16-byte chunks of each row XOR-swizzled by swz8(p % 8), and 128 bytes
// between blocks (a 1152-byte stride). A 16-lane pass of row reads (16
// consecutive rows, one chunk) then meets 16 different 16-byte bank slots,
// and a 32-lane pass of transposed reads (four consecutive rows, 64 bytes
// each) 32 different 8-byte bank pairs; a CPU model of the lane addresses
// confirms both patterns conflict-free. Every DMA lane carries data (BwdTile
// at D = 64 leaves half of each 1 KB block, and half of each DMA instruction,
// empty), so a tile takes 8 DMA instructions instead of 16, and a 4-slot ring
// of Q, dO and statistics takes 79 KB: two workgroups share a CU. Rows are in
// the permuted MFMA output order, as in BwdTile. The XOR makes the chunk
// offset lane-dependent, so a lane keeps one base per 32-byte column (row
// reads) and per 64-byte output tile (transposed reads).
struct BwdTileC64 {
  static constexpr int kRowBytes = 128;
  static constexpr int kChunks = 8;
  static constexpr int kBlocks = 8;
  static constexpr int kStride = 1024 + 128;
  static constexpr int kBytes = 7 * kStride + 1024;
  static __host__ __device__ constexpr int swz8(int t) { return (t & 1) | ((t & 2) << 1) | ((t & 4) >> 1); }
  static __host__ __device__ constexpr int off(int p, int byte) {
    return (p >> 3) * kStride + (p & 7) * kRowBytes + 16 * ((byte >> 4) ^ swz8(p & 7)) + (byte & 15);
  }
  static __host__ __device__ constexpr int block_off(int b) { return b * kStride; }
  // Lane L of the instruction filling block b writes LDS bytes 16 L .. 16 L + 15 of the block:
  // physical row 8 b + L / 8, physical chunk L % 8, which holds logical chunk (L % 8) ^ swz8(L / 8).
  static __host__ __device__ constexpr int dma_row(int b, int L) { return 8 * b + L / 8; }
  static __host__ __device__ constexpr int dma_chunk(int L) { return (L % 8) ^ swz8(L / 8); }
  static __device__ __forceinline__ bool dma_lane(int) { return true; }
  static constexpr int kTrHi = kStride;  // eight physical rows further: the next block
  struct Bases {
    int r[4], t[2];
    __device__ __forceinline__ explicit Bases(int lane) {
      const int l32 = lane & 31, g = lane >> 5;
      // Row fragment: physical row 32 half + l32, logical chunk 2 kk + g.
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) r[kk] = off(l32, 32 * kk + 16 * g);
      // Transposed fragment: physical row 32 half + 16 h + 4 g + (lane & 15) / 4,
      // logical byte 64 u + 32 ((lane >> 4) & 1) + 8 (lane & 3).
      const int tp = 4 * g + ((lane & 15) >> 2);
#pragma unroll
      for (int u = 0; u < 2; ++u) t[u] = off(tp, 64 * u + 32 * ((lane >> 4) & 1) + 8 * (lane & 3));
    }
  };
  static __device__ __forceinline__ int row(const Bases& b, int half, int kk) { return b.r[kk] + 4 * half * kStride; }
  static __device__ __forceinline__ int tr(const Bases& b, int half, int h, int u) {
    return b.t[u] + (4 * half + 2 * h) * kStride;
  }
};

template <int D>
struct DkvPp {
  static constexpr int kWaves = 4, kThreads = 64 * kWaves;
  static constexpr int BKV = 32 * kWaves, BQ = 64, KS = D / 16, DT = D / 32;
  typedef std::conditional_t<D == 64, BwdTileC64, BwdTile<D>> Tile;
  static constexpr int kSlots = 4;
  static constexpr int kMinBlocks = D == 64 ? 2 : 1;  // workgroups per CU the LDS admits
  static constexpr int kStatBytes = 2048;  // lse at +0, delta at +1024: one DMA instruction each
  static constexpr int kSlotBytes = 2 * Tile::kBytes + kStatBytes;
  static constexpr int kLds = kSlots * kSlotBytes;
  static constexpr int kDma = Tile::kBlocks / kWaves;  // per wave per tile, for Q and for dO
};

// DMA of 64 f32 row statistics (lse or delta) starting at row r0 into `lds`
// (lanes 0-15, 16 bytes each; the other lanes write zeros past them).
__device__ __forceinline__ void stat_dma(const float* base, int r0, int nrows, char* lds) {
  const int lane = threadIdx.x & 63;
  const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
  const uint64_t addr = reinterpret_cast<uint64_t>(base + r0);
  const u32x4 rsrc = {(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffffu)),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rows_left * 4), 0x00020000u};
  const uint32_t voff = lane < 16 ? (uint32_t)(lane * 16) : 0x80000000u;
  const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)reinterpret_cast<uintptr_t>(lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// One statistics row (64 floats from row r0 of base, zeros past nrows) into
// registers: lane L gets row r0 + L. A bounds-checked buffer load, counted in
// vmcnt like the DMA it replaces.
__device__ __forceinline__ float stat_load(const float* base, int r0, int nrows) {
  const int lane = threadIdx.x & 63;
  const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
  const uint64_t addr = reinterpret_cast<uint64_t>(base + r0);
  const uint64_t ua = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(ua), 0, __builtin_amdgcn_readfirstlane(rows_left * 4), 0x00020000);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 0));
}

// dK, dV, software-pipelined (the forward's scheme); D = 64 (D = 128 runs
// attn_dkv_rs_kernel below, which splits a key block over two waves). Half-step h of a wave
// (32 queries) first issues dV^T += dO^T P and dK^T += Q^T dS for half h - 1
// and turns the S and dP of half h into P and dS on the VALU between those
// products, then issues S = Q K^T and dP = dO V^T for half h + 1 into the same
// S / dP registers. The program order is the schedule: slot i holds one
// product, the LDS read of the product kAhead further on, a share of the VALU
// work and a share of the DMA, and a scheduling fence closes it. One
// workgroup barrier per 64-query tile (at odd half-steps); the DMA of tile
// t + 3 goes out during the two half-steps after the barrier that frees its
// slot.
// SAMEP: Q and dO share a row pitch (dense tensors), so one DMA descriptor serves both.
template <int D, bool SAMEP = true, bool SPLIT = false>
__global__ __launch_bounds__(256, DkvPp<D>::kMinBlocks) void attn_dkv_sw_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                            const bf16* __restrict__ v, const bf16* __restrict__ dout,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ delta, bf16* __restrict__ dk,
                                                            bf16* __restrict__ dv, int bh_count, int Sq, int Sk, int d,
                                                            int causal, float scale, float scale_log2, AttnViews vw,
                                                            int n_ktiles, int zig, char* __restrict__ ws,
                                                            int cut) {
  typedef DkvPp<D> F;
  typedef typename F::Tile Tile;
  constexpr int KS = F::KS, DT = F::DT;
  constexpr int kAhead = 3;
  // Per wave and tile: Q blocks, dO blocks, lse, delta (every wave loads the
  // two 256-byte statistics rows into the same place, so the count is uniform).
  constexpr int kTileDma = 2 * F::kDma + 2;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Heaviest (first) key blocks first. zig (a grid resident all at once, two
  // workgroups per CU): the second half of the grid takes the light blocks in
  // rising order, so block b and block b + grid / 2, which share a CU, pair a
  // long and a short causal sweep.
  const int bh = blockIdx.x % bh_count;
  const int blk = (int)(blockIdx.x / bh_count);
  static_assert(F::kSlots == sched::kDkvSwSlots, "the ring of the schedule");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;

  // Row pitches (elements; d for dense tensors).
  const int ldq = (int)vw.q.r, lddo = (int)vw.dout.r;
  const bf16* qb = q + vw.q.at(bh, vw.heads);
  const bf16* dob = dout + vw.dout.at(bh, vw.heads);
  const bf16* kb = k + vw.k.at(bh, vw.heads);
  const bf16* vb = v + vw.v.at(bh, vw.heads);
  const float* lseb = lse + (int64_t)bh * Sq;
  const float* db = delta + (int64_t)bh * Sq;

  // Query tiles first .. first + nt - 1 (tile t in ring slot t % kSlots),
  // halves 0 .. nh - 1 (half x: tile x / 2, queries 32 (x % 2) .. of it).
  // A sweep of fewer than three tiles is run as three: the tiles past the end
  // of the queries arrive as zeros (Q, dO, lse and delta all 0), so their
  // p = exp2(0) = 1 meets dO = 0 in dV and dS = p (0 - 0) = 0 in dK, and they
  // add exact zeros. One code path for every length keeps the register
  // allocation of the pipeline from splitting over short cases (38 spilled
  // registers at D = 128 with separate short paths; at D = 64 the single path
  // is what fits two waves per SIMD).
  // Key block kt over query tiles t0 .. t1 - 1 of its causal sweep (t1 =
  // sched::kWholeTile: to the end of the queries); role as in
  // sched::Segment. Without SPLIT every block is one whole sweep.
  auto segment = [&](int kt, int t0, int t1, int role) __attribute__((always_inline)) {
  const int k0 = kt * F::BKV;
  const int k0w = k0 + 32 * wave;
  const int kvrow = k0w + l32;
  int first, qlim;
  if constexpr (SPLIT) {
    // Causal self-attention with S % BKV == 0 (the host's conditions): rows
    // at or past qlim, the segment's end, arrive as zeros like rows past Sq.
    first = k0 / F::BQ + t0;
    qlim = t1 == sched::kWholeTile ? Sq : (k0 / F::BQ + t1) * F::BQ;
  } else {
    first = causal ? k0 / F::BQ : 0;
    qlim = Sq;
  }
  const int nt = max((qlim + F::BQ - 1) / F::BQ - first, 3);
  const int nh = 2 * nt;

  bf16x8 kf[KS], vf[KS];
  load_row_frags<bf16, D, true, false>(kf, kb, k0w, Sk, d, (int)vw.k.r);
  load_row_frags<bf16, D, true, false>(vf, vb, k0w, Sk, d, (int)vw.v.r);

  const PpDma<Tile, true> dma(wave, ldq);
  const PpDma<Tile, true> dma_do(wave, SAMEP ? ldq : lddo);
  auto slot = [&](int t) { return smem + (t % F::kSlots) * F::kSlotBytes; };
  // DMA instruction qd of tile t. Tiles (and rows) past the end of the queries
  // have an empty buffer range: the range check makes buffer_load ... lds write
  // zeros into their LDS bytes instead of reading memory. The padded sweeps of
  // D = 128 above read those slots, and their exactness rests on that zero
  // fill: Q, dO, lse and delta of every padded row (statistics lanes 16-63 of
  // stat_dma included) are 0 in LDS, never stale data of an earlier tile.
  auto dma_part = [&](int t, int qd) {
    char* sl = slot(t);
    const int r0 = (first + t) * F::BQ;
    if (qd < F::kDma)
      dma.issue_one(qb, r0, qlim, ldq, sl, qd);
    else if (qd < 2 * F::kDma)
      (SAMEP ? dma : dma_do).issue_one(dob, r0, qlim, SAMEP ? ldq : lddo, sl + Tile::kBytes, qd - F::kDma);
    else if (qd == 2 * F::kDma)
      stat_dma(lseb, r0, qlim, sl + 2 * Tile::kBytes);
    else
      stat_dma(db, r0, qlim, sl + 2 * Tile::kBytes + 1024);
  };
  // Tiles 0 and 1 first; the two half-steps after barrier t load tile t + 3.
#pragma unroll
  for (int qd = 0; qd < kTileDma; ++qd) dma_part(0, qd);
#pragma unroll
  for (int qd = 0; qd < kTileDma; ++qd) dma_part(1, qd);

  f32x16 dka[DT], dva[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dka[u][r] = 0.f;
      dva[u][r] = 0.f;
    }
  const typename Tile::Bases tb(lane);

  f32x16 sa, dpa;               // S and dP of one half (register r: query 16 g + r, key kvrow)
  bf16x8 pf[2][2], dsf[2][2];  // [half parity][8-query chunk]: P and dS fragments

  // Half-step h with parity P = h & 1.
  auto stage = [&](auto P_, auto SDP_, auto SG_, auto MASK_, auto GRAD_, int h) __attribute__((always_inline)) {
    constexpr int P = decltype(P_)::value;
    constexpr bool SDP = decltype(SDP_)::value, SG = decltype(SG_)::value;
    constexpr bool MASK = decltype(MASK_)::value, GRAD = decltype(GRAD_)::value;
    f32x16& sn = sa;
    f32x16& dpn = dpa;
    const f32x16& sc = sa;
    const f32x16& dpc = dpa;
    bf16x8(&pc)[2] = pf[P];
    bf16x8(&dsc)[2] = dsf[P];
    const bf16x8(&pp)[2] = pf[1 - P];
    const bf16x8(&dsp)[2] = dsf[1 - P];
    // Tiles and halves: SDP reads half h + 1, SG half h, GRAD half h - 1.
    const char* sl_n = slot((h + 1) >> 1);
    const int half_n = 1 - P;  // h & 1 == P
    const char* sl_c = slot(h >> 1);
    const int half_c = P;
    const char* sl_p = slot((h - 1) >> 1);
    const int half_p = 1 - P;
    constexpr int NS = SDP ? 2 * KS : 0;  // S (even) and dP (odd) products over the k-chunks
    constexpr int NG = GRAD ? 4 * DT : 0;  // per output tile: two key chunks, dV (even) and dK (odd)
    constexpr int NF = NS + NG;
    // Products 0 .. NG - 1 are GRAD, then NS SDP products (which overwrite S
    // and dP only after the softmax gradient has read them).
    auto which = [](int f, int& i) -> bool {  // true: SDP product i, false: GRAD product i
      if (f < NG) {
        i = f;
        return false;
      }
      i = f - NG;
      return true;
    };
    auto read = [&](int f) -> bf16x8 {
      int i;
      if (which(f, i))
        return *reinterpret_cast<const bf16x8*>(sl_n + ((i & 1) ? Tile::kBytes : 0) + Tile::row(tb, half_n, i >> 1));
      return tr_frag(sl_p + ((i & 1) ? 0 : Tile::kBytes) + Tile::tr(tb, half_p, (i >> 1) & 1, i >> 2), Tile::kTrHi);
    };
    auto prod = [&](int f, const bf16x8& a) {
      int i;
      if (which(f, i)) {
        if (i < 2) {
          if (i & 1)
            dpn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, vf[0], f32x16{}, 0, 0, 0);
          else
            sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kf[0], f32x16{}, 0, 0, 0);
        } else if (i & 1) {
          mma32(a, vf[i >> 1], dpn);
        } else {
          mma32(a, kf[i >> 1], sn);
        }
      } else {
        const int u = i >> 2, hh = (i >> 1) & 1;
        if (i & 1)
          mma32(a, dsp[hh], dka[u]);
        else
          mma32(a, pp[hh], dva[u]);
      }
    };
    // Softmax gradient of half h: element r (query 16 g + r of the half).
    const float* st = reinterpret_cast<const float*>(sl_c + 2 * Tile::kBytes) + 32 * half_c + 16 * g;
    // The lse row scaled by -log2(e), 512 bytes into the lse row's 1 KB of DMA space (which
    // holds zeros past the row): each wave writes the whole row at the tile's first softmax
    // half-step (P == 0) from the landed row and reads its part after its own write, so
    // every wave sees it without a barrier (the waves write the same values), and the
    // softmax spends no multiply on it per element.
    float* const lsc = reinterpret_cast<float*>(slot(h >> 1) + 2 * Tile::kBytes + 512);
    if constexpr (SG && P == 0) lsc[lane] = -reinterpret_cast<const float*>(sl_c + 2 * Tile::kBytes)[lane] * kLog2e;
    const float* const stl = lsc + 32 * half_c + 16 * g;
    const int qh = (first + (h >> 1)) * F::BQ + 32 * half_c + 16 * g;
    // -lse log2(e) and delta of queries 4 c .. 4 c + 3, read one group ahead of use.
    f32x4 ls[2], dl[2];
    auto read_stats = [&](int c) {
      ls[c & 1] = *reinterpret_cast<const f32x4*>(stl + 4 * c);
      dl[c & 1] = *reinterpret_cast<const f32x4*>(st + 256 + 4 * c);
    };
    float pv[8], dsv[8];
    auto sg_elem = [&](int r) {
      if ((r & 3) == 0 && (r >> 2) + 1 < 4) read_stats((r >> 2) + 1);
      const f32x4& l4 = ls[(r >> 2) & 1];
      const f32x4& d4 = dl[(r >> 2) & 1];
      float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, l4[r & 3]));
      if constexpr (MASK) p = (causal && kvrow > qh + r) ? 0.f : p;
      pv[r & 7] = p;
      dsv[r & 7] = p * (dpc[r] - d4[r & 3]);
      if ((r & 7) == 7) {
        to_frag(pv, pc[r >> 3]);
        to_frag(dsv, dsc[r >> 3]);
        pin(pc[r >> 3]);
        pin(dsc[r >> 3]);
      }
    };
    // DMA share: odd half-steps the first half of tile (h + 5) / 2's
    // instructions, even half-steps the rest.
    const int tdma = sched::dkv_sw_loaded(h);
    constexpr int QD0 = P ? 0 : kTileDma / 2;
    constexpr int NQ = P ? kTileDma / 2 : kTileDma - kTileDma / 2;

    if constexpr (SG) read_stats(0);
    if constexpr (SG && NG == 0) {
      // No GRAD products to hide it behind: the softmax gradient first.
#pragma unroll
      for (int r = 0; r < 16; ++r) sg_elem(r);
    }
    if constexpr (NF > 0) {
      bf16x8 buf[NF];
#pragma unroll
      for (int f = 0; f < kAhead && f < NF; ++f) buf[f] = read(f);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        if (f + kAhead < NF) buf[f + kAhead] = read(f + kAhead);
#pragma unroll
        for (int qd = 0; qd < NQ; ++qd)
          if (f == (2 * qd + 1) * NF / (2 * NQ)) dma_part(tdma, QD0 + qd);
        prod(f, buf[f]);
        if constexpr (SG && NG > 0) {
          // 16 elements over the NG GRAD products
          if (f < NG) {
            if constexpr (NG >= 16) {
              if (f % (NG / 16) == 0) sg_elem(f / (NG / 16));
            } else {
#pragma unroll
              for (int r = f * (16 / NG); r < (f + 1) * (16 / NG); ++r) sg_elem(r);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int qd = 0; qd < NQ; ++qd) dma_part(tdma, QD0 + qd);
    }
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // Barrier t opens half-step 2t + 1: this wave's part of tile t + 1 has
  // landed (tile t + 2 may be in flight) and every wave has finished half-step
  // 2t, the last to read tile t - 1, whose slot now takes tile t + 3.
  auto sync_tile = [&]() {
    wait_vmem<kTileDma>();
    lds_barrier();
  };
  // Half-step h: SDP for h + 1 < nh, SG for 0 <= h < nh, GRAD for 1 <= h <= nh
  // (nh is even and >= 6). The causal mask can only touch halves 0 .. 3 of
  // the sweep (the diagonal block): the first half-steps apply it on every
  // wave, where it is a no-op for halves below the wave's keys.
  sync_tile();
  stage(P1(), T_(), F_(), F_(), F_(), -1);
  stage(P0(), T_(), T_(), T_(), F_(), 0);
  sync_tile();
  stage(P1(), T_(), T_(), T_(), T_(), 1);
  stage(P0(), T_(), T_(), T_(), T_(), 2);
  sync_tile();
  stage(P1(), T_(), T_(), T_(), T_(), 3);
  stage(P0(), T_(), T_(), F_(), T_(), 4);
  // Full, unmasked half-steps in pairs, then the last two.
  for (int h = 5; h + 1 <= nh - 2; h += 2) {
    sync_tile();
    stage(P1(), T_(), T_(), F_(), T_(), h);
    stage(P0(), T_(), T_(), F_(), T_(), h + 1);
  }
  sync_tile();
  stage(P1(), F_(), T_(), F_(), T_(), nh - 1);
  stage(P0(), F_(), F_(), F_(), T_(), nh);
  wait_vmem<0>();

  if constexpr (SPLIT) {
    if (role >= 0) {
      // This share of the long block: every wave's dK and dV partial sums into
      // the pair's slot (counts first, then two shares per pair), then one
      // count per workgroup; the second to arrive adds the other share (a
      // sum, the same bits in either order) and stores.
      const int half = n_ktiles / 2, slot_id = bh * half + blk % half;
      constexpr int kShareFloats = F::kWaves * 2 * DT * 16 * 64;
      float* const part = reinterpret_cast<float*>(ws + split_counts_bytes(bh_count * half)) +
                          (int64_t)(2 * slot_id + role) * kShareFloats;
      float* const other = part + (role == 0 ? kShareFloats : -kShareFloats);
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r2 = 0; r2 < 8; ++r2) {
          xput2(part + xat((wave * 2 + 0) * DT + u, r2, lane), dka[u][2 * r2], dka[u][2 * r2 + 1]);
          xput2(part + xat((wave * 2 + 1) * DT + u, r2, lane), dva[u][2 * r2], dva[u][2 * r2 + 1]);
        }
      if (!pair_arrive_second(reinterpret_cast<int*>(ws) + slot_id)) return;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r2 = 0; r2 < 8; ++r2) {
          const f32x2 ok = xget2(other + xat((wave * 2 + 0) * DT + u, r2, lane));
          const f32x2 ov = xget2(other + xat((wave * 2 + 1) * DT + u, r2, lane));
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            dka[u][2 * r2 + e] += ok[e];
            dva[u][2 * r2 + e] += ov[e];
          }
        }
    }
  }

  if (d == D) {
    // Whole-row stores through LDS (store_acc_rows_lds); the barrier keeps the
    // other waves' last reads and DMA off this wave's region of the ring.
    static_assert(4 * 32 * 2 * D <= F::kLds, "every wave's rows fit the ring");
    lds_barrier();
    if (k0w >= Sk) return;
    char* const ot = smem + wave * (32 * 2 * D);
    store_acc_rows_lds<D>(dka, ot, dk + vw.dk.at(bh, vw.heads), k0w, Sk, scale, vw.dk.r);
    store_acc_rows_lds<D>(dva, ot, dv + vw.dv.at(bh, vw.heads), k0w, Sk, 1.0f, vw.dv.r);
    return;
  }
  if (k0w >= Sk) return;
  store_acc_rows<bf16, D, true>(dka, dk + vw.dk.at(bh, vw.heads), kvrow, Sk, d, scale, vw.dk.r);
  store_acc_rows<bf16, D, true>(dva, dv + vw.dv.at(bh, vw.heads), kvrow, Sk, d, 1.0f, vw.dv.r);
  };

  if constexpr (!SPLIT) {
    segment(sched::key_block(blk, n_ktiles, zig), 0, sched::kWholeTile, -1);
  } else {
    // The pair's sequence of query tiles (sched::split_segments, in the
    // forward's terms: its "long tile" n - 1 - p is key block p here, the
    // block with the longer causal sweep).
    sched::Segment seg[2];
    const int nseg = sched::split_segments(blk, n_ktiles, cut, seg);
    segment(n_ktiles - 1 - seg[0].qt, seg[0].t0, seg[0].t1, seg[0].role);
    if (nseg > 1) {
      // The first segment's stores went through LDS (a barrier before them,
      // none after): every wave is past them before the ring refills.
      lds_barrier();
      segment(n_ktiles - 1 - seg[1].qt, seg[1].t0, seg[1].t1, seg[1].role);
    }
  }
}

// dK, dV at D = 128 with the work of each 32-key block split over the two
// waves of a SIMD. Wave w < 4 (role A) computes S = Q K^T, P and
// dV^T += dO^T P for keys k0 + 32 w; wave w + 4 (role B, on the same SIMD)
// computes dP = dO V^T, dS = P (dP - delta) and dK^T += Q^T dS for the same
// keys. A hands P to B through LDS in f32, before any rounding, so dS is the
// reference's p * (dp - di) (flash_attention.py:191-193) exactly as in the
// one-wave kernel above. Each wave holds one accumulator set (64 registers)
// and one of K and V (32), so two waves fit on a SIMD and the VALU work of
// one overlaps the products of the other; the one-wave kernel, which holds
// both, takes 286 registers and runs one wave per SIMD.
// Half-step h (32 queries): A runs dV for half h - 1 with the softmax of half
// h between its products, then S for half h + 1; B runs dP for half h with dS
// of half h - 1 between its products (P from A, written in half-step h - 1),
// then dK for half h - 1. One workgroup barrier per half-step orders the P
// exchange (two buffers) and the three-slot Q / dO ring: tile t is read in
// half-steps 2t - 1 .. 2t + 2, and its DMA goes out in half-step 2t - 3 into
// the slot tile t - 3 left.
struct DkvRs {
  static constexpr int D = 128, kWaves = 8, kThreads = 64 * kWaves;
  static constexpr int BKV = 128, BQ = 64, KS = D / 16, DT = D / 32;
  typedef BwdTile<128> Tile;
  static constexpr int kSlots = 3;
  static constexpr int kStatBytes = 2048;  // lse at +0 (wave 0 loads it), delta at +1024 (wave 4)
  static constexpr int kSlotBytes = 2 * Tile::kBytes + kStatBytes;
  static constexpr int kXBytes = 4 * 4096;  // P of one half for the four SIMD pairs (f32)
  static constexpr int kLds = kSlots * kSlotBytes + 2 * kXBytes;
  static constexpr int kDma = Tile::kBlocks / kWaves;  // per wave per tile, for Q and for dO
};

template <bool SAMEP>
__global__ __launch_bounds__(512, 1) void attn_dkv_rs_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                            const bf16* __restrict__ v, const bf16* __restrict__ dout,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ delta, bf16* __restrict__ dk,
                                                            bf16* __restrict__ dv, int bh_count, int Sq, int Sk, int d,
                                                            int causal, float scale, float scale_log2, AttnViews vw,
                                                            int n_ktiles, int zig) {
  typedef DkvRs F;
  typedef F::Tile Tile;
  constexpr int KS = F::KS, DT = F::DT;
  constexpr int kAhead = 3;
  // Per wave and tile: Q blocks, dO blocks, and the statistics row (waves 0 and 4 only).
  constexpr int kTileDma = 2 * F::kDma + 1;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Heaviest (first) key blocks first; zig as in attn_dkv_sw_kernel.
  const int bh = blockIdx.x % bh_count;
  const int blk = (int)(blockIdx.x / bh_count);
  static_assert(F::kSlots == sched::kDkvRsSlots, "the ring of the schedule");
  const int kt = sched::key_block(blk, n_ktiles, zig);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = wave & 3, role = wave >> 2;
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int k0 = kt * F::BKV;
  const int k0w = k0 + 32 * pair;
  const int kvrow = k0w + l32;

  const int ldq = (int)vw.q.r, lddo = (int)vw.dout.r;
  const bf16* qb = q + vw.q.at(bh, vw.heads);
  const bf16* dob = dout + vw.dout.at(bh, vw.heads);
  const float* lseb = lse + (int64_t)bh * Sq;
  const float* db = delta + (int64_t)bh * Sq;

  // Sweeps of fewer than three tiles run as three (zero tiles add exact
  // zeros, as in attn_dkv_sw_kernel).
  const int first = causal ? k0 / F::BQ : 0;
  const int nt = max((Sq + F::BQ - 1) / F::BQ - first, 3);
  const int nh = 2 * nt;

  const PpDma<Tile, true, F::kWaves> dma(wave, ldq);
  const PpDma<Tile, true, F::kWaves> dma_do(wave, SAMEP ? ldq : lddo);
  auto slot = [&](int t) { return smem + (t % F::kSlots) * F::kSlotBytes; };
  char* const xring = smem + F::kSlots * F::kSlotBytes;
  // P of half h, pair p: chunk c (four queries) of lane L at xbuf(h) + p 4096 + c 1024 + 16 L.
  auto xbuf = [&](int h) { return xring + (h & 1) * F::kXBytes + pair * 4096; };
  // The lse row of a tile comes into wave 0's registers with the tile's DMA and goes to
  // the tile's slot scaled by -log2(e) at the next odd half-step (the first after the
  // barrier that waited for it), so that the softmax spends no multiply on it per element.
  float lse_next = 0.f;
  // DMA instruction qd of tile t; rows past the end of the queries arrive as
  // zeros (empty buffer range), which the padded sweeps rely on.
  auto dma_part = [&](int t, int qd) {
    char* sl = slot(t);
    const int r0 = (first + t) * F::BQ;
    if (qd < F::kDma)
      dma.issue_one(qb, r0, Sq, ldq, sl, qd);
    else if (qd < 2 * F::kDma)
      (SAMEP ? dma : dma_do).issue_one(dob, r0, Sq, SAMEP ? ldq : lddo, sl + Tile::kBytes, qd - F::kDma);
    else if (pair == 0 && role)
      stat_dma(db, r0, Sq, sl + 2 * Tile::kBytes + 1024);
    else if (pair == 0)
      lse_next = stat_load(lseb, r0, Sq);
  };
#pragma unroll
  for (int qd = 0; qd < kTileDma; ++qd) dma_part(0, qd);

  const typename Tile::Bases tb(lane);
  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;

  // Barrier opening half-step h. Tile t's DMA goes out in half-step 2t - 3 and
  // is first read in half-step 2t - 1: before an odd half-step every DMA of
  // this wave has landed; before an even one nothing new is needed.
  auto sync = [&](int h) {
    if (h & 1) wait_vmem<0>();
    lds_barrier();
  };
  // The DMA of tile (h + 3) / 2 in odd half-steps: instruction f of the
  // wave's share in the f-th product slot of the DMA's place in the stage.
  auto dma_at = [&](int h, int f) {
    if ((h & 1) && f < kTileDma) dma_part(sched::dkv_rs_loaded(h), f);
  };

  // Full-width K (role A) or V (role B) rows come by row-coalesced DMA
  // (dma_rows32) into tile slot 2 and the P exchange, which nothing writes
  // before stage 0 (P) and stage 1 (tile 2's DMA); each wave reads its rows
  // back in stage -1.
  static_assert(F::kSlots == 3 && F::kSlotBytes + 2 * F::kXBytes >= 8 * 32 * 256, "the K/V rows fit the idle LDS");
  const bool rows_lds = d == 128;
  char* const rst = smem + 2 * F::kSlotBytes + wave * (32 * 256);

  if (role == 0) {
    // ---- role A: S, P, dV ----
    const bf16* kb = k + vw.k.at(bh, vw.heads);
    bf16x8 kf[KS];
    if (rows_lds)
      dma_rows32<128>(kb, k0w, Sk, (int)vw.k.r, rst);
    else
      load_row_frags<bf16, 128, true, false>(kf, kb, k0w, Sk, d, (int)vw.k.r);
    f32x16 dva[DT];
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) dva[u][r] = 0.f;
    f32x16 sa[2];       // S of a half (register r: query 16 g + r, key kvrow), by parity
    bf16x8 pf[2][2];    // [parity][8-query chunk]: P fragments

    auto stage = [&](auto P_, auto GRAD_, auto SG_, auto MASK_, auto SDP_, int h) __attribute__((always_inline)) {
      constexpr int P = decltype(P_)::value;
      constexpr bool GRAD = decltype(GRAD_)::value, SG = decltype(SG_)::value;
      constexpr bool MASK = decltype(MASK_)::value, SDP = decltype(SDP_)::value;
      const f32x16& sc = sa[P];
      f32x16& sn = sa[1 - P];
      bf16x8(&pc)[2] = pf[P];
      const bf16x8(&pp)[2] = pf[1 - P];
      // Odd half-steps: wave 0 writes the lse row of tile (h + 1) / 2, loaded at h - 2 and
      // waited for at this half-step's barrier; read from half-step h + 1 on.
      if constexpr (P == 1)
        if (pair == 0) reinterpret_cast<float*>(slot((h + 1) >> 1) + 2 * Tile::kBytes)[lane] = -lse_next * kLog2e;
      const char* sl_n = slot((h + 1) >> 1);  // S of half h + 1: Q rows
      const int half_n = 1 - P;  // h & 1 == P
      const char* sl_p = slot((h - 1) >> 1);  // dV of half h - 1: dO^T
      const int half_p = 1 - P;
      const int half_c = P;
      // The S products come first and the dV products, with the softmax between
      // them, second: B's VALU work sits in the first half of its half-step, so
      // the two waves of a SIMD alternate between products and VALU work.
      constexpr int NS = SDP ? KS : 0;       // S: k-chunk i
      constexpr int NG = GRAD ? 2 * DT : 0;  // dV: output tile u = i / 2, query chunk i % 2
      constexpr int NF = NS + NG;
      // One lane address per read kind and half-step, opaque to the compiler: otherwise it
      // hoists a lane address per fragment out of the loop and adds the slot to each.
      int ro = (int)(sl_n - smem) + tb.r, to = (int)(sl_p - smem) + Tile::kBytes + tb.t;
      asm volatile("" : "+v"(ro), "+v"(to));
      auto read = [&](int f) -> bf16x8 {
        if (f < NS) return *reinterpret_cast<const bf16x8*>(smem + ro + Tile::row_at(half_n, f));
        const int i = f - NS;
        return tr_frag(smem + to + Tile::tr_at(half_p, i & 1, i >> 1), Tile::kTrHi);
      };
      auto prod = [&](int f, const bf16x8& a) {
        if (f < NS) {
          if (f == 0)
            sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kf[0], f32x16{}, 0, 0, 0);
          else
            mma32(a, kf[f], sn);
        } else {
          const int i = f - NS;
          mma32(a, pp[i & 1], dva[i >> 1]);
        }
      };
      // Softmax of half h: element r (query 16 g + r of the half).
      const float* st = reinterpret_cast<const float*>(slot(h >> 1) + 2 * Tile::kBytes) + 32 * half_c + 16 * g;
      const int qh = (first + (h >> 1)) * F::BQ + 32 * half_c + 16 * g;
      char* const xw = xbuf(h) + 16 * lane;
      f32x4 ls[2];
      float pv[8];
      f32x4 p4;
      auto sg_elem = [&](int r) {
        if ((r & 3) == 0 && (r >> 2) + 1 < 4) ls[((r >> 2) + 1) & 1] = *reinterpret_cast<const f32x4*>(st + 4 * ((r >> 2) + 1));
        const f32x4& l4 = ls[(r >> 2) & 1];
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, l4[r & 3]));  // l4: -lse log2(e)
        if constexpr (MASK) p = (causal && kvrow > qh + r) ? 0.f : p;
        pv[r & 7] = p;
        p4[r & 3] = p;
        if ((r & 3) == 3) *reinterpret_cast<f32x4*>(xw + (r >> 2) * 1024) = p4;
        if ((r & 7) == 7) {
          to_frag(pv, pc[r >> 3]);
          pin(pc[r >> 3]);
        }
      };
      if constexpr (SG) ls[0] = *reinterpret_cast<const f32x4*>(st);
      if constexpr (NF > 0) {
        bf16x8 buf[NF];
#pragma unroll
        for (int f = 0; f < kAhead && f < NF; ++f) buf[f] = read(f);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          if (f + kAhead < NF) buf[f + kAhead] = read(f + kAhead);
          dma_at(h, f);
          prod(f, buf[f]);
          if constexpr (SG && NG > 0) {
            if (f >= NS) {
#pragma unroll
              for (int r = (f - NS) * (16 / NG); r < (f - NS + 1) * (16 / NG); ++r) sg_elem(r);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int f = 0; f < kTileDma; ++f) dma_at(h, f);
      }
      if constexpr (SG && NG == 0) {
        // No dV products to hide it behind (the first half-step): the softmax last.
#pragma unroll
        for (int r = 0; r < 16; ++r) sg_elem(r);
      }
    };
    // Half-step h: GRAD (dV) for 1 <= h <= nh, SG for 0 <= h < nh, SDP (S) for
    // h + 1 < nh; the mask covers halves 0 .. 3 (the diagonal block).
    sync(-1);
    if (rows_lds) row_frags_lds<128>(kf, rst);
    stage(P1(), F_(), F_(), F_(), T_(), -1);
    sync(0);
    stage(P0(), F_(), T_(), T_(), T_(), 0);
    sync(1);
    stage(P1(), T_(), T_(), T_(), T_(), 1);
    sync(2);
    stage(P0(), T_(), T_(), T_(), T_(), 2);
    sync(3);
    stage(P1(), T_(), T_(), T_(), T_(), 3);
    sync(4);
    stage(P0(), T_(), T_(), F_(), T_(), 4);
    for (int h = 5; h + 1 <= nh - 2; h += 2) {
      sync(h);
      stage(P1(), T_(), T_(), F_(), T_(), h);
      sync(h + 1);
      stage(P0(), T_(), T_(), F_(), T_(), h + 1);
    }
    sync(nh - 1);
    stage(P1(), T_(), T_(), F_(), F_(), nh - 1);
    sync(nh);
    stage(P0(), T_(), F_(), F_(), F_(), nh);
    wait_vmem<0>();
    if (d == 128) {
      lds_barrier();  // as role B's: whole-row stores through LDS
      if (k0w >= Sk) return;
      store_acc_rows_lds<128>(dva, smem + wave * (32 * 256), dv + vw.dv.at(bh, vw.heads), k0w, Sk, 1.0f, vw.dv.r);
      return;
    }
    if (k0w >= Sk) return;
    store_acc_rows<bf16, 128, true>(dva, dv + vw.dv.at(bh, vw.heads), kvrow, Sk, d, 1.0f, vw.dv.r);
  } else {
    // ---- role B: dP, dS, dK ----
    const bf16* vb = v + vw.v.at(bh, vw.heads);
    bf16x8 vf[KS];
    if (rows_lds)
      dma_rows32<128>(vb, k0w, Sk, (int)vw.v.r, rst);
    else
      load_row_frags<bf16, 128, true, false>(vf, vb, k0w, Sk, d, (int)vw.v.r);
    f32x16 dka[DT];
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) dka[u][r] = 0.f;
    f32x16 dpa[2];   // dP of a half, by parity
    bf16x8 dsf[2];   // dS fragments of the half the stage's dK products use

    auto stage = [&](auto P_, auto SDP_, auto SG_, auto GRAD_, int h) __attribute__((always_inline)) {
      constexpr int P = decltype(P_)::value;
      constexpr bool SDP = decltype(SDP_)::value, SG = decltype(SG_)::value, GRAD = decltype(GRAD_)::value;
      f32x16& dpn = dpa[P];             // dP of half h
      const f32x16& dpc = dpa[1 - P];   // dP of half h - 1
      const char* sl_c = slot(h >> 1);  // dP of half h: dO rows
      const int half_c = P;
      const char* sl_p = slot((h - 1) >> 1);  // dS and dK of half h - 1: Q^T, delta
      const int half_p = 1 - P;
      constexpr int NS = SDP ? KS : 0;       // dP: k-chunk i
      constexpr int NG = GRAD ? 2 * DT : 0;  // dK: output tile u = i / 2, query chunk i % 2
      constexpr int NF = NS + NG;
      // One lane address per read kind and half-step (as role A's).
      int ro = (int)(sl_c - smem) + Tile::kBytes + tb.r, to = (int)(sl_p - smem) + tb.t;
      asm volatile("" : "+v"(ro), "+v"(to));
      auto read = [&](int f) -> bf16x8 {
        if (f < NS) return *reinterpret_cast<const bf16x8*>(smem + ro + Tile::row_at(half_c, f));
        const int i = f - NS;
        return tr_frag(smem + to + Tile::tr_at(half_p, i & 1, i >> 1), Tile::kTrHi);
      };
      auto prod = [&](int f, const bf16x8& a) {
        if (f < NS) {
          if (f == 0)
            dpn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, vf[0], f32x16{}, 0, 0, 0);
          else
            mma32(a, vf[f], dpn);
        } else {
          const int i = f - NS;
          mma32(a, dsf[i & 1], dka[i >> 1]);
        }
      };
      // dS of half h - 1: element r (query 16 g + r), P from A's half-step h - 1.
      const float* st = reinterpret_cast<const float*>(sl_p + 2 * Tile::kBytes) + 256 + 32 * half_p + 16 * g;
      const char* xr = xbuf(h - 1) + 16 * lane;
      f32x4 dl[2], px[2];
      float dsv[8];
      auto sg_elem = [&](int r) {
        if ((r & 3) == 0 && (r >> 2) + 1 < 4) {
          const int c = (r >> 2) + 1;
          dl[c & 1] = *reinterpret_cast<const f32x4*>(st + 4 * c);
          px[c & 1] = *reinterpret_cast<const f32x4*>(xr + c * 1024);
        }
        const float p = px[(r >> 2) & 1][r & 3];
        dsv[r & 7] = p * (dpc[r] - dl[(r >> 2) & 1][r & 3]);
        if ((r & 7) == 7) {
          to_frag(dsv, dsf[r >> 3]);
          pin(dsf[r >> 3]);
        }
      };
      if constexpr (SG) {
        dl[0] = *reinterpret_cast<const f32x4*>(st);
        px[0] = *reinterpret_cast<const f32x4*>(xr);
      }
      if constexpr (SG && NS == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sg_elem(r);
      }
      if constexpr (NF > 0) {
        bf16x8 buf[NF];
#pragma unroll
        for (int f = 0; f < kAhead && f < NF; ++f) buf[f] = read(f);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          if (f + kAhead < NF) buf[f + kAhead] = read(f + kAhead);
          // This wave's share of the DMA goes out between its dK products, where
          // the VALU is idle (A issues its share among its S products).
          if (NG == 0 || f >= NS) dma_at(h, NG > 0 ? f - NS : f);
          prod(f, buf[f]);
          if constexpr (SG && NS > 0) {
            if (f < NS) {
#pragma unroll
              for (int r = f * (16 / NS); r < (f + 1) * (16 / NS); ++r) sg_elem(r);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int f = 0; f < kTileDma; ++f) dma_at(h, f);
      }
    };
    // Half-step h: SDP (dP) for 0 <= h < nh, SG (dS) and GRAD (dK) for 1 <= h <= nh.
    sync(-1);
    if (rows_lds) row_frags_lds<128>(vf, rst);
    stage(P1(), F_(), F_(), F_(), -1);
    sync(0);
    stage(P0(), T_(), F_(), F_(), 0);
    for (int h = 1; h + 1 <= nh - 1; h += 2) {
      sync(h);
      stage(P1(), T_(), T_(), T_(), h);
      sync(h + 1);
      stage(P0(), T_(), T_(), T_(), h + 1);
    }
    sync(nh - 1);
    stage(P1(), T_(), T_(), T_(), nh - 1);
    sync(nh);
    stage(P0(), F_(), T_(), T_(), nh);
    wait_vmem<0>();
    if (d == 128) {
      // Whole-row stores through LDS (store_acc_rows_lds), each wave in its own
      // 8 KB of the ring; the barrier (role A passes one too) keeps the other
      // waves' last reads and DMA off it.
      static_assert(8 * 32 * 256 <= DkvRs::kLds, "every wave's rows fit the ring");
      lds_barrier();
      if (k0w >= Sk) return;
      store_acc_rows_lds<128>(dka, smem + wave * (32 * 256), dk + vw.dk.at(bh, vw.heads), k0w, Sk, scale, vw.dk.r);
      return;
    }
    if (k0w >= Sk) return;
    store_acc_rows<bf16, 128, true>(dka, dk + vw.dk.at(bh, vw.heads), kvrow, Sk, d, scale, vw.dk.r);
  }
}

// ---- dK/dV at D = 256 -------------------------------------------------------
// A 32-row granule of a 256-column bf16 tile: the first half of BwdTile<256>
// (rows 0-31, 16 DMA blocks of 1 KB holding two rows each), so that its row
// and transposed fragment reads are BwdTile<256>'s at half 0.
struct BwdHalf256 {
  typedef BwdTile<256> Full;
  static constexpr int kRowBytes = Full::kRowBytes, kChunks = Full::kChunks;
  static constexpr int kBlocks = 16;
  static constexpr int kBytes = Full::kHalfBytes;
  static __host__ __device__ constexpr int off(int p, int byte) { return Full::off(p, byte); }
  static __host__ __device__ constexpr int block_off(int b) { return Full::block_off(b); }
  static __host__ __device__ constexpr int dma_row(int b, int L) { return Full::dma_row(b, L); }
  static __host__ __device__ constexpr int dma_chunk(int L) { return Full::dma_chunk(L); }
  static __device__ __forceinline__ bool dma_lane(int L) { return Full::dma_lane(L); }
};

// Compile-time check of the granule's DMA, as bwd_tile_dma_ok: lane L of block
// instruction b (every lane carries data) writes LDS bytes block_off(b) + 16 L
// inside the granule, where off() keeps the row and chunk it loads, each of
// the 32 rows x 32 chunks once; for G waves sharing the instructions, a
// wave's instruction i loads its rows of instruction 0 moved by a delta that
// depends on i alone.
template <int G>
constexpr bool half256_dma_ok() {
  typedef BwdHalf256 T;
  bool seen[32 * T::kChunks] = {};
  for (int b = 0; b < T::kBlocks; ++b)
    for (int L = 0; L < 64; ++L) {
      const int p = T::dma_row(b, L), c = T::dma_chunk(L);
      if (p < 0 || p >= 32 || seen[p * T::kChunks + c]) return false;
      seen[p * T::kChunks + c] = true;
      if (T::block_off(b) + 16 * L != T::off(p, 16 * c) || T::block_off(b) + 16 * L + 16 > T::kBytes) return false;
    }
  for (bool x : seen)
    if (!x) return false;
  for (int gw = 0; gw < G; ++gw)
    for (int i = 0; i < T::kBlocks / G; ++i) {
      const int d0 = perm_src(T::dma_row(G * i, 0)) - perm_src(T::dma_row(0, 0));
      for (int L = 0; L < 64; ++L)
        if (perm_src(T::dma_row(gw + G * i, L)) != perm_src(T::dma_row(gw, L)) + d0) return false;
    }
  return true;
}
static_assert(half256_dma_ok<8>() && half256_dma_ok<4>(),
              "the 256-column granule's DMA blocks cover it once, where the reads expect them");

// DMA of 64 f32 row statistics (lse or delta) starting at row r0 into `lds`, 4
// bytes a lane: 256 bytes of LDS (rows past nrows arrive as zeros).
__device__ __forceinline__ void stat_dma4(const float* base, int r0, int nrows, char* lds) {
  const int lane = threadIdx.x & 63;
  const int rows_left = nrows - r0 > 0 ? nrows - r0 : 0;
  const uint64_t addr = reinterpret_cast<uint64_t>(base + r0);
  const u32x4 rsrc = {(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffffu)),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rows_left * 4), 0x00020000u};
  const uint32_t voff = (uint32_t)(lane * 4);
  const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)reinterpret_cast<uintptr_t>(lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// dK, dV at D = 256 in one pass: four roles per 32-key block, two blocks (64
// keys) per workgroup. A 32-key block's K and V rows and its dK and dV
// accumulators (512 registers in all) do not fit one SIMD's two waves; spread
// over four waves (two SIMDs), S and dP are still computed once:
//   role A (waves 0, 2): S = Q K^T over 256 columns, P, dV^T[0:128] += dO^T P;
//   role B (waves 1, 3): dP = dO V^T, dS = P (dP - delta), dK^T[0:128] += Q^T dS;
//   role A' (waves 4, 6): dV^T[128:256] += dO^T P, P from role A;
//   role B' (waves 5, 7): dK^T[128:256] += Q^T dS, dS from role B.
// Waves w and w + 4 share a SIMD: each SIMD pairs a role A or B wave (24
// products a step) with an A' or B' wave (8 products, and the workgroup's DMA).
// P crosses from A to B and A' in f32 through LDS (A' rounds it to the same
// fragments A uses), dS from B to B' as fragments. B' runs one step behind B,
// so a Q granule is read in steps x - 1 (S), x + 1 (dK, B) and x + 2 (dK, B'):
// a ring of five Q granules and three dO granules (sched::dkv256q_*), the P and
// dS buffers: 156 KB.
struct Dkv256Q {
  static constexpr int D = 256, kWaves = 8, kThreads = 64 * kWaves;
  static constexpr int BKV = 64, BG = 32;  // keys per workgroup, queries per granule
  static constexpr int KS = D / 16, SDT = 4;
  typedef BwdHalf256 G;
  typedef BwdTile<256> Tile;
  static constexpr int kQSlots = sched::kDkv256qQSlots, kDoSlots = sched::kDkv256qDoSlots;
  static constexpr int kStatBytes = 256;  // 64 rows of lse (Q ring) or delta (dO ring): stat_dma4
  static constexpr int kSlotBytes = G::kBytes + kStatBytes;
  static constexpr int kDoRing = kQSlots * kSlotBytes;
  static constexpr int kXP = kDoRing + kDoSlots * kSlotBytes;  // P (f32) by parity and block: 4 KB each
  static constexpr int kXDS = kXP + 2 * 2 * 4096;              // dS fragments by parity and block: 2 KB each
  static constexpr int kLds = kXDS + 2 * 2 * 2048;
  static constexpr int kLight = 4;                   // waves 4 .. 7 issue the ring's DMA
  static constexpr int kDma = G::kBlocks / kLight;   // per light wave per granule, for Q and for dO
  static constexpr int kStage = kSlotBytes;          // roles A and B: K / V rows from Q slot 1 on, 16 KB a wave
  static_assert(kLds <= 160 * 1024, "one workgroup per CU");
  static_assert(kStage + 4 * 32 * 2 * D <= kDoRing, "the K / V rows stage inside Q slots 1 ..");
};

template <bool SAMEP>
__global__ __launch_bounds__(512, 1) void attn_dkv_q256_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                              const bf16* __restrict__ v,
                                                              const bf16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta, bf16* __restrict__ dk,
                                                              bf16* __restrict__ dv, int bh_count, int Sq, int Sk,
                                                              int causal, float scale, float scale_log2, AttnViews vw) {
  typedef Dkv256Q F;
  typedef F::G G;
  typedef F::Tile Tile;
  constexpr int KS = F::KS, SDT = F::SDT;
  constexpr int kAhead = 3;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Blocks: heads fastest, then 64-key blocks from the heaviest causal sweep on.
  const int bh = blockIdx.x % bh_count;
  const int kt = (int)(blockIdx.x / bh_count);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool light = wave >= 4;
  const int blk = (wave >> 1) & 1, role = wave & 1;  // role 0: A / A', 1: B / B'
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;
  const int k0 = kt * F::BKV;
  const int kb0 = k0 + 32 * blk;  // the wave's 32 keys
  const int kvrow = kb0 + (lane & 31);

  const int ldq = (int)vw.q.r, lddo = (int)vw.dout.r;
  const bf16* qb = q + vw.q.at(bh, vw.heads);
  const bf16* dob = dout + vw.dout.at(bh, vw.heads);
  const float* lseb = lse + (int64_t)bh * Sq;
  const float* db = delta + (int64_t)bh * Sq;

  // Granules first .. first + nh - 1 of the queries; nh even and at least 4
  // (granules past the end of the queries arrive as zeros and add exact zeros).
  const int first = causal ? k0 / F::BG : 0;
  int nh = max((Sq + F::BG - 1) / F::BG - first, 4);
  nh += nh & 1;

  auto qslot = [&](int x) { return smem + ((x + F::kQSlots) % F::kQSlots) * F::kSlotBytes; };
  auto doslot = [&](int x) { return smem + F::kDoRing + ((x + F::kDoSlots) % F::kDoSlots) * F::kSlotBytes; };
  // P of granule x (f32, chunk c of four queries of lane L at + c 1024 + 16 L), dS fragments of granule x.
  auto xp = [&](int x) { return smem + F::kXP + ((x & 1) * 2 + blk) * 4096 + 16 * lane; };
  auto xds = [&](int x) { return smem + F::kXDS + ((x & 1) * 2 + blk) * 2048 + 16 * lane; };

  // The light waves' DMA of step h: Q and lse of granule h + 2, dO and delta of
  // granule h + 1 (none past the sweep; rows past the queries arrive as zeros).
  const PpDma<G, true, F::kLight> dma(light ? wave - 4 : 0, ldq);
  const PpDma<G, true, F::kLight> dma_do(light ? wave - 4 : 0, SAMEP ? ldq : lddo);
  auto step_dma = [&](int h) {
    const int xq = sched::dkv256q_q_loaded(h), xd = sched::dkv256q_do_loaded(h);
    if (xq < nh) {
#pragma unroll
      for (int i = 0; i < F::kDma; ++i) dma.issue_one(qb, (first + xq) * F::BG, Sq, ldq, qslot(xq), i);
      if (wave == 4) stat_dma4(lseb, (first + xq) * F::BG, Sq, qslot(xq) + G::kBytes);
    }
    if (xd < nh) {
#pragma unroll
      for (int i = 0; i < F::kDma; ++i)
        (SAMEP ? dma : dma_do).issue_one(dob, (first + xd) * F::BG, Sq, SAMEP ? ldq : lddo, doslot(xd), i);
      if (wave == 5) stat_dma4(db, (first + xd) * F::BG, Sq, doslot(xd) + G::kBytes);
    }
  };

  // Prologue: roles A and B stage their K or V rows; the light waves load Q and lse of granule 0.
  char* const rst = smem + F::kStage + (wave & 3) * (32 * 2 * F::D);
  if (!light) {
    const bf16* kvb = role == 0 ? k + vw.k.at(bh, vw.heads) : v + vw.v.at(bh, vw.heads);
    dma_rows32<256>(kvb, kb0, Sk, role == 0 ? (int)vw.k.r : (int)vw.v.r, rst);
  } else {
#pragma unroll
    for (int i = 0; i < F::kDma; ++i) dma.issue_one(qb, first * F::BG, Sq, ldq, qslot(0), i);
    if (wave == 4) stat_dma4(lseb, first * F::BG, Sq, qslot(0) + G::kBytes);
  }

  const Tile::Bases tb(lane);
  const int trs0 = tb.t, trs1 = tb.t + 256;  // transposed reads of the two slabs
  auto tr_slab = [&](const char* sl, int trs, int hh, int uu) -> bf16x8 {
    return tr_frag(sl + trs + Tile::tr_at(0, hh, uu), Tile::kTrHi);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  auto sync = [&]() {
    wait_vmem<0>();
    lds_barrier();
  };
  bf16x8 kvf[KS];  // roles A and B: K or V rows, all 256 columns
  sync();
  if (!light) row_frags_lds<256>(kvf, rst);
  lds_barrier();  // every staging read is done before step -1's loads

  f32x16 acc[SDT];
#pragma unroll
  for (int u = 0; u < SDT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;

  if (light) {
    // ---- roles A' and B': the second slab's products from the partner role's P or dS ----
    const int lag = role == 0 ? 1 : 2;  // A': dV for granule h - 1; B': dK for granule h - 2
    for (int h = -1; h <= nh + 1; ++h) {
      if (h >= 0) sync();
      step_dma(h);
      const int x = h - lag;
      if (x < 0 || x >= nh) continue;
      bf16x8 fr[2];
      if (role == 0) {
        // P of granule x in f32 from role A, rounded to the fragments A uses.
        const char* src = xp(x);
        float pv[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 p4 = *reinterpret_cast<const f32x4*>(src + c * 1024);
#pragma unroll
          for (int e = 0; e < 4; ++e) pv[4 * c + e] = p4[e];
        }
        to_frag(pv, fr[0]);
        to_frag(pv + 8, fr[1]);
      } else {
        fr[0] = *reinterpret_cast<const bf16x8*>(xds(x));
        fr[1] = *reinterpret_cast<const bf16x8*>(xds(x) + 1024);
      }
      const char* sl = role == 0 ? doslot(x) : qslot(x);  // dO^T or Q^T of granule x
      bf16x8 buf[2 * SDT];
#pragma unroll
      for (int i = 0; i < 2 * SDT; ++i) buf[i] = tr_slab(sl, trs1, i & 1, i >> 1);
#pragma unroll
      for (int i = 0; i < 2 * SDT; ++i) mma32(buf[i], fr[i & 1], acc[i >> 1]);
    }
    wait_vmem<0>();
    lds_barrier();
    if (kb0 >= Sk) return;
    if (role == 0)
      store_acc_rows_lds<128>(acc, smem + wave * (32 * 256), dv + vw.dv.at(bh, vw.heads) + 128, kb0, Sk, 1.0f,
                              vw.dv.r);
    else
      store_acc_rows_lds<128>(acc, smem + wave * (32 * 256), dk + vw.dk.at(bh, vw.heads) + 128, kb0, Sk, scale,
                              vw.dk.r);
    return;
  }

  if (role == 0) {
    // ---- role A: S, P, dV^T[0:128] ----
    f32x16 sa[2];     // S of a granule (register r: query 16 g + r, key kvrow), by parity
    bf16x8 pf[2][2];  // [parity][8-query chunk]: P fragments

    auto stage = [&](auto P_, auto GRAD_, auto SG_, auto MASK_, auto SDP_, int h) __attribute__((always_inline)) {
      constexpr int P = decltype(P_)::value;
      constexpr bool GRAD = decltype(GRAD_)::value, SG = decltype(SG_)::value;
      constexpr bool MASK = decltype(MASK_)::value, SDP = decltype(SDP_)::value;
      const f32x16& sc = sa[P];
      f32x16& sn = sa[1 - P];
      bf16x8(&pc)[2] = pf[P];
      const bf16x8(&pp)[2] = pf[1 - P];
      const char* qn = qslot(h + 1);
      const char* dop = doslot(h - 1);
      constexpr int NS = SDP ? KS : 0;
      constexpr int NG = GRAD ? 2 * SDT : 0;
      constexpr int NF = NS + NG;
      auto read = [&](int f) -> bf16x8 {
        if (f < NS) return *reinterpret_cast<const bf16x8*>(qn + Tile::row(tb, 0, f));
        const int i = f - NS;
        return tr_slab(dop, trs0, i & 1, i >> 1);
      };
      auto prod = [&](int f, const bf16x8& a) {
        if (f < NS) {
          if (f == 0)
            sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kvf[0], f32x16{}, 0, 0, 0);
          else
            mma32(a, kvf[f], sn);
        } else {
          const int i = f - NS;
          mma32(a, pp[i & 1], acc[i >> 1]);
        }
      };
      const float* st = reinterpret_cast<const float*>(qslot(h) + G::kBytes) + 16 * g;
      const int qh = (first + h) * F::BG + 16 * g;
      char* const xw = xp(h);
      f32x4 ls[2];
      float pv[8];
      f32x4 p4;
      auto sg_elem = [&](int r) {
        if ((r & 3) == 0 && (r >> 2) + 1 < 4) ls[((r >> 2) + 1) & 1] = *reinterpret_cast<const f32x4*>(st + 4 * ((r >> 2) + 1));
        const f32x4& l4 = ls[(r >> 2) & 1];
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, -l4[r & 3] * kLog2e));
        if constexpr (MASK) p = (causal && kvrow > qh + r) ? 0.f : p;
        pv[r & 7] = p;
        p4[r & 3] = p;
        if ((r & 3) == 3) *reinterpret_cast<f32x4*>(xw + (r >> 2) * 1024) = p4;
        if ((r & 7) == 7) {
          to_frag(pv, pc[r >> 3]);
          pin(pc[r >> 3]);
        }
      };
      if constexpr (SG) ls[0] = *reinterpret_cast<const f32x4*>(st);
      if constexpr (NF > 0) {
        bf16x8 buf[NF];
#pragma unroll
        for (int f = 0; f < kAhead && f < NF; ++f) buf[f] = read(f);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          if (f + kAhead < NF) buf[f + kAhead] = read(f + kAhead);
          prod(f, buf[f]);
          if constexpr (SG && NG > 0) {
            if (f >= NS) {
#pragma unroll
              for (int r = (f - NS) * (16 / NG); r < (f - NS + 1) * (16 / NG); ++r) sg_elem(r);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if constexpr (SG && NG == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sg_elem(r);
      }
    };
    // Step h: GRAD (dV) for 1 <= h <= nh, SG for 0 <= h < nh, SDP (S) for
    // h + 1 < nh; the mask covers granules 0 and 1 (the diagonal block).
    stage(P1(), F_(), F_(), F_(), T_(), -1);
    sync();
    stage(P0(), F_(), T_(), T_(), T_(), 0);
    sync();
    stage(P1(), T_(), T_(), T_(), T_(), 1);
    int h = 2;
    for (; h + 1 < nh - 2; h += 2) {
      sync();
      stage(P0(), T_(), T_(), F_(), T_(), h);
      sync();
      stage(P1(), T_(), T_(), F_(), T_(), h + 1);
    }
    sync();
    stage(P0(), T_(), T_(), F_(), T_(), nh - 2);
    sync();
    stage(P1(), T_(), T_(), F_(), F_(), nh - 1);
    sync();
    stage(P0(), T_(), F_(), F_(), F_(), nh);
    sync();  // step nh + 1: role B' only
    wait_vmem<0>();
    lds_barrier();
    if (kb0 >= Sk) return;
    store_acc_rows_lds<128>(acc, smem + wave * (32 * 256), dv + vw.dv.at(bh, vw.heads), kb0, Sk, 1.0f, vw.dv.r);
  } else {
    // ---- role B: dP, dS, dK^T[0:128] ----
    f32x16 dpa[2];  // dP of a granule, by parity
    bf16x8 dsf[2];  // dS fragments of the granule the step's dK products use

    auto stage = [&](auto P_, auto SDP_, auto SG_, auto GRAD_, int h) __attribute__((always_inline)) {
      constexpr int P = decltype(P_)::value;
      constexpr bool SDP = decltype(SDP_)::value, SG = decltype(SG_)::value, GRAD = decltype(GRAD_)::value;
      f32x16& dpn = dpa[P];
      const f32x16& dpc = dpa[1 - P];
      const char* doc = doslot(h);
      const char* qp = qslot(h - 1);
      constexpr int NS = SDP ? KS : 0;
      constexpr int NG = GRAD ? 2 * SDT : 0;
      constexpr int NF = NS + NG;
      auto read = [&](int f) -> bf16x8 {
        if (f < NS) return *reinterpret_cast<const bf16x8*>(doc + Tile::row(tb, 0, f));
        const int i = f - NS;
        return tr_slab(qp, trs0, i & 1, i >> 1);
      };
      auto prod = [&](int f, const bf16x8& a) {
        if (f < NS) {
          if (f == 0)
            dpn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kvf[0], f32x16{}, 0, 0, 0);
          else
            mma32(a, kvf[f], dpn);
        } else {
          const int i = f - NS;
          mma32(a, dsf[i & 1], acc[i >> 1]);
        }
      };
      // dS of granule h - 1: element r (query 16 g + r), P from A's step h - 1;
      // its fragments also go to role B' for the second slab.
      const float* st = reinterpret_cast<const float*>(doslot(h - 1) + G::kBytes) + 16 * g;
      const char* xr = xp(h - 1);
      char* const xw = xds(h - 1);
      f32x4 dl[2], px[2];
      float dsv[8];
      auto sg_elem = [&](int r) {
        if ((r & 3) == 0 && (r >> 2) + 1 < 4) {
          const int c = (r >> 2) + 1;
          dl[c & 1] = *reinterpret_cast<const f32x4*>(st + 4 * c);
          px[c & 1] = *reinterpret_cast<const f32x4*>(xr + c * 1024);
        }
        const float p = px[(r >> 2) & 1][r & 3];
        dsv[r & 7] = p * (dpc[r] - dl[(r >> 2) & 1][r & 3]);
        if ((r & 7) == 7) {
          to_frag(dsv, dsf[r >> 3]);
          pin(dsf[r >> 3]);
          *reinterpret_cast<bf16x8*>(xw + (r >> 3) * 1024) = dsf[r >> 3];
        }
      };
      if constexpr (SG) {
        dl[0] = *reinterpret_cast<const f32x4*>(st);
        px[0] = *reinterpret_cast<const f32x4*>(xr);
      }
      if constexpr (SG && NS == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sg_elem(r);
      }
      if constexpr (NF > 0) {
        bf16x8 buf[NF];
#pragma unroll
        for (int f = 0; f < kAhead && f < NF; ++f) buf[f] = read(f);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          if (f + kAhead < NF) buf[f + kAhead] = read(f + kAhead);
          prod(f, buf[f]);
          if constexpr (SG && NS > 0) {
            if (f < NS) {
#pragma unroll
              for (int r = f * (16 / NS); r < (f + 1) * (16 / NS); ++r) sg_elem(r);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    // Step h: SDP (dP) for 0 <= h < nh, SG (dS) and GRAD (dK) for 1 <= h <= nh.
    sync();
    stage(P0(), T_(), F_(), F_(), 0);
    for (int h = 1; h + 1 <= nh - 1; h += 2) {
      sync();
      stage(P1(), T_(), T_(), T_(), h);
      sync();
      stage(P0(), T_(), T_(), T_(), h + 1);
    }
    sync();
    stage(P1(), T_(), T_(), T_(), nh - 1);
    sync();
    stage(P0(), F_(), T_(), T_(), nh);
    sync();  // step nh + 1: role B' only
    wait_vmem<0>();
    lds_barrier();
    if (kb0 >= Sk) return;
    store_acc_rows_lds<128>(acc, smem + wave * (32 * 256), dk + vw.dk.at(bh, vw.heads), kb0, Sk, scale, vw.dk.r);
  }
}

// W waves of 32 queries; SLOTS K/V tile slots in LDS (3: tiles t + 1 and t + 2
// load while tile t is used; 2: only t + 1, which halves the LDS so that two
// workgroups share a CU).
// KSPLIT = 2: waves w and w + W / 2 (one SIMD) take the same queries and
// split every 64-key tile, keys 0-31 and 32-63; their dQ partials add up at
// the end.
template <int D, int W = 8, int SLOTS = 3, int KSPLIT = 1>
struct DqPp {
  static constexpr int kWaves = W, kThreads = 64 * kWaves;
  static constexpr int BQ = 32 * kWaves / KSPLIT, BK = 64, KS = D / 16, DT = D / 32;
  typedef BwdTile<D> Tile;
  static constexpr int kSlots = SLOTS;
  static constexpr int kSlotBytes = 2 * Tile::kBytes;  // K then V
  static constexpr int kLds = kSlots * kSlotBytes;
  static constexpr int kDma = Tile::kBlocks / kWaves;  // per wave per tile, for K and for V
  static_assert(SLOTS == 2 || SLOTS == 3, "two or three slots");
  static_assert(Tile::kBlocks % kWaves == 0, "tile blocks split evenly over the waves");
};

// dQ for 32 W queries (32 per wave, Q and dO fragments in registers),
// sweeping 64-key tiles up to the diagonal. With 8 waves, waves w and w + 4
// share a SIMD. ZIG (a grid resident all at once, two workgroups per CU):
// the second half of the grid takes the light query tiles in rising order,
// so that block b and block b + grid / 2 pair a long and a short sweep.
// Per 32-key half: S^T = K Q^T and dP^T = V dO^T from row reads of the K and
// V tiles, dS^T = P^T (dP^T - delta) on the VALU (one query per lane, so lse
// and delta are per-lane scalars), then dQ^T += K^T dS^T from transposed
// reads of the K tile.
// FUSED: delta is not read but computed here from O and dO (the rows' dO
// fragments are loaded anyway) and written out for the dK/dV kernel, which
// then runs after this one: the separate delta pass over O and dO goes away.
template <int D, int W, int SLOTS, bool ZIG, bool FUSED = false, int KSPLIT = 1, bool SPLIT = false>
__global__ __launch_bounds__((64 * W), (KSPLIT > 1 ? 4 : D > 128 ? 1 : 2)) void attn_dq_pp_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                                const bf16* __restrict__ v,
                                                                const bf16* __restrict__ dout,
                                                                const float* __restrict__ lse,
                                                                float* __restrict__ delta,
                                                                bf16* __restrict__ dq, int bh_count, int Sq, int Sk,
                                                                int d, int causal, float scale, float scale_log2,
                                                                int n_qtiles, const bf16* __restrict__ o,
                                                                AttnViews vw, char* __restrict__ ws, int cut) {
  typedef DqPp<D, W, SLOTS, KSPLIT> F;
  typedef typename F::Tile Tile;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // Heaviest (last) query tiles first.
  const int bh = blockIdx.x % bh_count;
  const int blk = (int)(blockIdx.x / bh_count);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  static_assert(!SPLIT || (KSPLIT == 2 && D == 64), "the split runs the key-split kernel at D = 64");
  // Query tile qt over key tiles t0 .. t1 - 1 of its causal sweep (t1 =
  // sched::kWholeTile: to the diagonal); role as in sched::Segment. Without
  // SPLIT every block is one whole sweep.
  auto segment = [&](int qt, int t0, int t1, int role) __attribute__((always_inline)) {
  // 8 waves: SIMD w % 4 holds row blocks 2 (w % 4) and 2 (w % 4) + 1.
  const int q0 = qt * F::BQ;
  // With KSPLIT = 2, kh is the wave's half of every key tile.
  const int kh = KSPLIT == 1 ? 0 : wave / (W / KSPLIT);
  const int q0w =
      q0 + 32 * (KSPLIT > 1 ? wave % (W / KSPLIT) : W == 8 ? 2 * (wave & 3) + (wave >> 2) : wave);
  const int qrow = q0w + l32;

  // Row pitches (elements; d for dense tensors). K and V share one (the host checks).
  const int ldk = (int)vw.k.r;
  const bf16* qb = q + vw.q.at(bh, vw.heads);
  const bf16* dob = dout + vw.dout.at(bh, vw.heads);
  const bf16* kb = k + vw.k.at(bh, vw.heads);
  const bf16* vb = v + vw.v.at(bh, vw.heads);

  const int q_last = min(q0 + F::BQ, Sq) - 1;
  const bool wave_active = q0w < Sq;
  // n tiles in this sweep (or segment), the wave's first n_w of them up to
  // its rows' diagonal; tile t of the sweep is key tile t0 + t.
  int n, n_w;
  if constexpr (SPLIT) {
    // Causal self-attention with S % 128 == 0 (the host's conditions).
    const int n_all = q_last / F::BK + 1;
    n = (t1 == sched::kWholeTile ? n_all : t1) - t0;
    n_w = min(max(min(q0w + 31, Sq - 1) / F::BK + 1 - t0, 0), n);
  } else {
    n = causal ? min(q_last, Sk - 1) / F::BK + 1 : (Sk + F::BK - 1) / F::BK;
    n_w = !wave_active ? 0 : causal ? min(min(q0w + 31, Sq - 1), Sk - 1) / F::BK + 1 : n;
  }

  const PpDma<Tile, true, W> dma(wave, ldk);
  auto slot = [&](int t) { return smem + (t % F::kSlots) * F::kSlotBytes; };
  auto issue_tile = [&](int t) {
    char* sl = slot(t);
    dma.issue(kb, (t0 + t) * F::BK, Sk, ldk, sl);
    dma.issue(vb, (t0 + t) * F::BK, Sk, ldk, sl + Tile::kBytes);
  };

  bf16x8 qf[F::KS], dof[F::KS];
  load_row_frags<bf16, D, true, false>(qf, qb, q0w, Sq, d, (int)vw.q.r);
  load_row_frags<bf16, D, true, false>(dof, dob, q0w, Sq, d, (int)vw.dout.r);
  const bool qok = qrow < Sq;
  const float nlse2 = qok ? -lse[(int64_t)bh * Sq + qrow] * kLog2e : 0.f;
  float dl;
  if constexpr (FUSED) {
    // delta = sum_d f32(dO) f32(O) (flash_attention.py:328-329): this lane
    // holds half of its row's elements, lane ^ 32 the other half.
    bf16x8 of[F::KS];
    load_row_frags<bf16, D, true, false>(of, o + vw.o.at(bh, vw.heads), q0w, Sq, d, (int)vw.o.r);
    float part = 0.f;
#pragma unroll
    for (int kk = 0; kk < F::KS; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) part = __builtin_fmaf((float)dof[kk][e], (float)of[kk][e], part);
    dl = lane32_sum(part);
    // (Of a split tile, block A's share writes it; both compute the same.)
    if (qok && g == 0 && kh == 0 && role != 1) delta[(int64_t)bh * Sq + qrow] = dl;
  } else {
    dl = qok ? delta[(int64_t)bh * Sq + qrow] : 0.f;
  }

  // Tiles 0 .. SLOTS - 2 go out first; tile t + SLOTS - 1 is issued after
  // tile t's barrier, into the slot tile t - 1 left.
  issue_tile(0);
  if (SLOTS == 3 && n > 1) issue_tile(1);

  f32x16 acc[F::DT];
#pragma unroll
  for (int u = 0; u < F::DT; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;

  const int rb = Tile::row_base(lane);
  const int tb = Tile::tr_base(lane);

  // S^T and dP^T of half `half` of the tile at sl: s[r] / dp[r] is key
  // 32 half + 16 g + r of the tile, query qrow. `valu` runs between products.
  constexpr int kAheadQ = 4;
  auto sdp = [&](const char* sl, int half, f32x16& s, f32x16& dp, auto&& valu) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = 0.f;
      dp[r] = 0.f;
    }
    const char* kp = sl + rb;
    const char* vp = sl + Tile::kBytes + rb;
    auto read = [&](int i) {
      return *reinterpret_cast<const bf16x8*>(((i & 1) ? vp : kp) + Tile::row_at(half, i >> 1));
    };
    constexpr int N = 2 * F::KS;  // S^T and dP^T products alternate over the k-chunks
    bf16x8 buf[N];
#pragma unroll
    for (int i = 0; i < kAheadQ; ++i) buf[i] = read(i);
    valu();
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i + kAheadQ < N) buf[i + kAheadQ] = read(i + kAheadQ);
      if (i & 1)
        mma32(buf[i], dof[i >> 1], dp);
      else
        mma32(buf[i], qf[i >> 1], s);
    }
#pragma unroll
    for (int i = 0; i < kAheadQ; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kAheadQ < N) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
    }
  };

  // dS^T of a half (MASK: keys past the query are zero).
  auto grad_s = [&](int kv0, const f32x16& s, const f32x16& dp, bf16x8 (&dsf)[2], auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], scale_log2, nlse2));
      if constexpr (MASK) p = kv0 + 16 * g + r > qrow ? 0.f : p;
      ds[r] = p * (dp[r] - dl);
    }
    to_frag(ds, dsf[0]);
    to_frag(ds + 8, dsf[1]);
  };

  // dQ^T += K^T dS^T for half `half` of the tile at sl.
  constexpr int kAheadTr = 4;
  auto grad_q = [&](const char* sl, int half, const bf16x8 (&dsf)[2]) {
    const char* kp = sl + tb;
    // Product i: output tile u = i / 2, key chunk h = i % 2.
    auto read = [&](int i) { return tr_frag(kp + Tile::tr_at(half, i & 1, i >> 1), Tile::kTrHi); };
    constexpr int N = 2 * F::DT;  // per output tile: two key chunks
    bf16x8 buf[N];
#pragma unroll
    for (int i = 0; i < kAheadTr; ++i) buf[i] = read(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i + kAheadTr < N) buf[i + kAheadTr] = read(i + kAheadTr);
      mma32(buf[i], dsf[i & 1], acc[i >> 1]);
    }
#pragma unroll
    for (int i = 0; i < kAheadTr; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kAheadTr < N) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };

  f32x16 s0, dp0, s1, dp1;
  bf16x8 dsf[2];
  auto nop = [] {};
  if constexpr (KSPLIT > 1) {
    static_assert(D == 64, "the split path ends in the direct stores");
    // This wave's half of every tile: S and dP, dS, then its dQ products.
    for (int t = 0; t < n; ++t) {
      if (sched::dq_in_flight(t, n, SLOTS, 1))
        wait_vmem<2 * F::kDma>();
      else
        wait_vmem<0>();
      lds_barrier();
      if (sched::dq_loaded(t, SLOTS) < n) issue_tile(sched::dq_loaded(t, SLOTS));
      if (t >= n_w) continue;
      const char* sl = slot(t);
      const int kv0 = (t0 + t) * F::BK + 32 * kh;
      sdp(sl, kh, s0, dp0, nop);
      if (causal && kv0 + 31 > q0w)
        grad_s(kv0, s0, dp0, dsf, std::true_type{});
      else
        grad_s(kv0, s0, dp0, dsf, std::false_type{});
      grad_q(sl, kh, dsf);
    }
    // The upper half adds its dQ partial to the lower half's through the idle
    // ring (every DMA has landed: the last tile's wait was vmcnt(0)).
    static_assert(W / KSPLIT * 16 * F::DT * 64 * 4 <= F::kLds, "the partials fit the ring");
    float* const xs = reinterpret_cast<float*>(smem) + (wave % (W / KSPLIT)) * (16 * F::DT * 64);
    lds_barrier();
    if (kh == 1) {
#pragma unroll
      for (int u = 0; u < F::DT; ++u)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<f32x4*>(xs + ((u * 4 + r4) * 64 + lane) * 4) =
              f32x4{acc[u][4 * r4], acc[u][4 * r4 + 1], acc[u][4 * r4 + 2], acc[u][4 * r4 + 3]};
    }
    lds_barrier();
    if constexpr (!SPLIT) {
      if (kh == 1) return;
    }
    if (kh == 0) {
#pragma unroll
      for (int u = 0; u < F::DT; ++u)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 o1 = *reinterpret_cast<const f32x4*>(xs + ((u * 4 + r4) * 64 + lane) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[u][4 * r4 + e] += o1[e];
        }
    }
    if constexpr (SPLIT) {
      if (role >= 0) {
        // This share of the long tile: the lower waves' dQ partial sums into
        // the pair's slot (counts first, then two shares per pair), then one
        // count per workgroup (every wave takes part); the second to arrive
        // adds the other share (a sum, the same bits in either order).
        const int half = n_qtiles / 2, slot_id = bh * half + blk % half;
        constexpr int kShareFloats = (W / KSPLIT) * F::DT * 16 * 64;
        float* const part = reinterpret_cast<float*>(ws + split_counts_bytes(bh_count * half)) +
                            (int64_t)(2 * slot_id + role) * kShareFloats;
        float* const other = part + (role == 0 ? kShareFloats : -kShareFloats);
        const int wr = wave % (W / KSPLIT);
        if (kh == 0) {
#pragma unroll
          for (int u = 0; u < F::DT; ++u)
#pragma unroll
            for (int r2 = 0; r2 < 8; ++r2) xput2(part + xat(wr * F::DT + u, r2, lane), acc[u][2 * r2], acc[u][2 * r2 + 1]);
        }
        if (!pair_arrive_second(reinterpret_cast<int*>(ws) + slot_id)) return;
        if (kh == 0) {
#pragma unroll
          for (int u = 0; u < F::DT; ++u)
#pragma unroll
            for (int r2 = 0; r2 < 8; ++r2) {
              const f32x2 oo = xget2(other + xat(wr * F::DT + u, r2, lane));
              acc[u][2 * r2] += oo[0];
              acc[u][2 * r2 + 1] += oo[1];
            }
        }
      }
      if (kh == 1) return;
    }
  } else {
    for (int t = 0; t < n; ++t) {
      // Tile t complete for this wave (with three slots tile t + 1 may be in
      // flight); after the barrier every wave has left tile t - 1's slot, which
      // tile t + SLOTS - 1 takes.
      if (sched::dq_in_flight(t, n, SLOTS, 1))
        wait_vmem<2 * F::kDma>();
      else
        wait_vmem<0>();
      lds_barrier();
      if (sched::dq_loaded(t, SLOTS) < n) issue_tile(sched::dq_loaded(t, SLOTS));
      if (t >= n_w) continue;
      const char* sl = slot(t);
      const int kv0 = (t0 + t) * F::BK;
      const bool mask0 = causal && kv0 + 31 > q0w;
      const bool mask1 = causal && kv0 + 63 > q0w;
      sdp(sl, 0, s0, dp0, nop);
      if (mask0)
        sdp(sl, 1, s1, dp1, [&] { grad_s(kv0, s0, dp0, dsf, std::true_type{}); });
      else
        sdp(sl, 1, s1, dp1, [&] { grad_s(kv0, s0, dp0, dsf, std::false_type{}); });
      grad_q(sl, 0, dsf);
      if (mask1)
        grad_s(kv0 + 32, s1, dp1, dsf, std::true_type{});
      else
        grad_s(kv0 + 32, s1, dp1, dsf, std::false_type{});
      grad_q(sl, 1, dsf);
    }
  }

  if (D >= 128 && d == D) {
    // Whole-row stores through LDS (store_acc_rows_lds); the barrier keeps the
    // other waves' last reads off this wave's region (every DMA has landed: the
    // last tile's wait was vmcnt(0)). At D = 64 (two workgroups per CU, 128-byte
    // rows) the direct stores measured as fast.
    static_assert(W * 32 * 2 * D <= F::kLds, "every wave's rows fit the ring");
    lds_barrier();
    if (!wave_active) return;
    store_acc_rows_lds<D>(acc, smem + wave * (32 * 2 * D), dq + vw.dq.at(bh, vw.heads), q0w, Sq, scale, vw.dq.r);
    return;
  }
  if (!wave_active) return;
  store_acc_rows<bf16, D, true>(acc, dq + vw.dq.at(bh, vw.heads), qrow, Sq, d, scale, vw.dq.r);
  };

  if constexpr (!SPLIT) {
    segment(sched::query_tile(blk, n_qtiles, ZIG), 0, sched::kWholeTile, -1);
  } else {
    sched::Segment seg[2];
    const int nseg = sched::split_segments(blk, n_qtiles, cut, seg);
    segment(seg[0].qt, seg[0].t0, seg[0].t1, seg[0].role);
    if (nseg > 1) {
      // The first segment's last LDS reads (the partials' merge through the
      // ring) are done on every wave before the ring refills.
      lds_barrier();
      segment(seg[1].qt, seg[1].t0, seg[1].t1, seg[1].role);
    }
  }
}

// ===========================================================================
// Host side
// ===========================================================================
// The kernel's dynamic-LDS limit on the stream's device, raised once per device.
template <typename K>
int set_lds(K kernel, int bytes, hipStream_t stream) {
  return allow_lds(reinterpret_cast<const void*>(kernel), bytes, stream, "ferrite_hip_attn");
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
  (void)bwd;
  if (s.d > 128 && s.d % kSlab != 0)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": head_dim " + std::to_string(s.d) +
                                                  " not supported (head_dim <= 128 or a multiple of 128)");
  if (s.b * s.h > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": b*h too large");
  // In-kernel offsets within one (b, h) head are 32-bit byte offsets.
  const int64_t head_bytes = (s.sq > s.sk ? s.sq : s.sk) * s.d * (dtype == FERRITE_BF16 ? 2 : 4);
  if (head_bytes > 0x7fff0000)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": one (b, h) head must be under 2 GiB");
  return FERRITE_OK;
}

int pad_dim(int64_t d) { return d <= 64 ? 64 : d <= 128 ? 128 : 256; }

// Strides of dense [B, H, Sq, d] (q, o, dO, dQ) and [B, H, Sk, d] (k, v, dK, dV) tensors.
AttnViews dense_views(const Shape& s) {
  const View vq{s.h * s.sq * s.d, s.sq * s.d, s.d}, vk{s.h * s.sk * s.d, s.sk * s.d, s.d};
  return AttnViews{vq, vk, vk, vq, vq, vq, vk, vk, (int)s.h};
}

// The split long-context forward (attn_fwd_sw_kernel with SPLIT): where it
// applies and where the cut falls are sched::fwd_split_applies and
// sched::fwd_split_cut, for bf16 causal self-attention with head dims <= 64
// (the key-split kernel).
bool fwd_split_applies(const Shape& s, int dtype, int causal, int cus) {
  if (dtype != FERRITE_BF16 || !causal || s.sq != s.sk || s.d > 64 || s.d % 8 != 0) return false;
  return sched::fwd_split_applies(s.b * s.h, s.sq, cus);
}
int fwd_split_cut(const Shape& s, int cus) { return sched::fwd_split_cut(s.b * s.h, s.sq, cus); }
// Workspace bytes of the split forward, 0 where it does not apply: two partial
// states per pair of tiles (128 x 64 f32 O, row max and row sum) and one count
// per pair.
int64_t fwd_split_bytes(const Shape& s, int dtype, int causal, int cus) {
  typedef FwdW<64, 1, 8, 2> F;
  if (!fwd_split_applies(s, dtype, causal, cus)) return 0;
  const int64_t pairs = s.b * s.h * (s.sq / F::BQ / 2);
  constexpr int64_t kPart = (4 * 2 * 16 * 64 + 2 * F::BQ) * 4;
  return pairs * (2 * kPart + 4);
}

// Where the split dK/dV and dQ apply (sched::kDkvSplit, sched::kDqSplit): bf16
// causal self-attention with head dims <= 64, the shapes of the key-split
// long-context kernels.
bool bwd_split_shape(const Shape& s, int dtype, int causal) {
  return dtype == FERRITE_BF16 && causal && s.sq == s.sk && s.d <= 64 && s.d % 8 == 0;
}
bool dkv_split_applies(const Shape& s, int dtype, int causal, int cus) {
  return bwd_split_shape(s, dtype, causal) && sched::split_applies(s.b * s.h, s.sq, cus, sched::kDkvSplit);
}
bool dq_split_applies(const Shape& s, int dtype, int causal, int cus) {
  return bwd_split_shape(s, dtype, causal) && sched::split_applies(s.b * s.h, s.sq, cus, sched::kDqSplit);
}
// Workspace bytes of the split backward, 0 where neither kernel splits: one
// count per pair of tiles (split_counts_bytes), then two shares per pair, each
// a 128 x 64 f32 dK and dV (dK/dV) or a 128 x 64 f32 dQ (dQ). The two kernels
// run one after the other on a stream and take turns with one workspace.
int64_t bwd_split_bytes(const Shape& s, int dtype, int causal, int cus) {
  const int64_t share = dkv_split_applies(s, dtype, causal, cus)  ? 2 * 128 * 64 * 4
                        : dq_split_applies(s, dtype, causal, cus) ? 128 * 64 * 4
                                                                  : 0;
  if (share == 0) return 0;
  const int64_t pairs = s.b * s.h * (s.sq / sched::kSplitRows / 2);
  return split_counts_bytes(pairs) + 2 * pairs * share;
}
// A caller's workspace that holds `need` > 0 bytes at a 256-byte boundary.
bool split_ws_ok(const void* ws, int64_t ws_bytes, int64_t need) {
  return need > 0 && ws && ws_bytes >= need && (reinterpret_cast<uintptr_t>(ws) & 255) == 0;
}

template <int D, int RB = 1, int W = 8, bool ZIG = false, int KSPLIT = 1, bool SPLIT = false>
int fwd_sw_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, float c, int neg_q,
                  hipStream_t stream, const AttnViews* views = nullptr, void* ws = nullptr) {
  typedef FwdW<D, RB, W, KSPLIT> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  auto kern = attn_fwd_sw_kernel<D, RB, W, ZIG, KSPLIT, SPLIT>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(F::kThreads), F::kLds, stream, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<bf16*>(o), lse, (int)bh,
                     (int)s.sq, (int)s.d, c, neg_q, (int)nq, views ? *views : dense_views(s), static_cast<char*>(ws),
                     fwd_split_cut(s, cu_count(stream)));
  return check_launch("ferrite_flash_attention_fwd");
}

template <int D>
int fwd_pp_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, int causal,
                  float c, int neg_q, hipStream_t stream) {
  typedef FwdPp<D> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  auto kern = attn_fwd_pp_kernel<D>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(F::kThreads), F::kLds, stream, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<bf16*>(o), lse, (int)bh,
                     (int)s.sq, (int)s.sk, (int)s.d, causal, c, neg_q, (int)nq);
  return check_launch("ferrite_flash_attention_fwd");
}

// ws / ws_bytes: the caller's workspace for the split long-context forward
// (fwd_split_bytes), or nullptr.
template <typename T, int D, bool AL>
int fwd_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, int causal,
               float scale, hipStream_t stream, void* ws = nullptr, int64_t ws_bytes = 0) {
  typedef Fwd<T, D, AL> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  auto kern = attn_fwd_kernel<T, D, AL>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  // The kernel takes the row max on raw scores, which needs a positive
  // multiplier: a negative scale negates q instead, and a zero scale becomes a
  // tiny positive one (uniform weights either way).
  float c = scale * kLog2e;
  const int neg_q = c < 0.f;
  c = fmaxf(fabsf(c), 1e-30f);
  if constexpr (sizeof(T) == 2 && AL && D <= 128) {
    if (causal && s.sq == s.sk && s.sq % 64 == 0) {
      if constexpr (D == 64) {
        // 128-row workgroups, two per CU (51 KB of LDS each): the two
        // workgroups on a CU hide each other's barriers and tails. When the
        // whole grid is resident at once, the second half of the grid takes
        // the light tiles in rising order so that each CU pairs a long and a
        // short tile (1x8x8192x64: 120 -> 91 us on MI355X). Each workgroup is
        // 8 waves that split every key tile between the two waves of a SIMD
        // (128 VGPRs, four waves per SIMD): the long tile that outlasts its
        // partner still runs two waves per SIMD (93.7 -> 84.7 us; 8x12x1024x64
        // 24.4 -> 23.5 us).
        // With a workspace, a resident grid of an even number of 128-row tiles
        // splits its long tiles between the two workgroups of a CU (the SPLIT
        // kernel above): every workgroup then sweeps the same number of key tiles.
        typedef FwdW<64, 1, 8, 2> F4;
        const int cus = cu_count(stream);
        const int64_t split = fwd_split_bytes(s, FERRITE_BF16, causal, cus);
        if (split > 0 && ws && ws_bytes >= split && (reinterpret_cast<uintptr_t>(ws) & 255) == 0)
          return fwd_sw_launch<D, 1, 8, true, 2, true>(q, k, v, o, lse, s, c, neg_q, stream, nullptr, ws);
        const bool one_round = sched::resident(cdiv(s.sq, F4::BQ) * s.b * s.h, 2, cus);
        return one_round ? fwd_sw_launch<D, 1, 8, true, 2>(q, k, v, o, lse, s, c, neg_q, stream)
                         : fwd_sw_launch<D, 1, 8, false, 2>(q, k, v, o, lse, s, c, neg_q, stream);
      } else {
        return fwd_sw_launch<D>(q, k, v, o, lse, s, c, neg_q, stream);
      }
    }
    return fwd_pp_launch<D>(q, k, v, o, lse, s, causal, c, neg_q, stream);
  }
  if constexpr (sizeof(T) == 2 && AL && D == 256) {
    // 128-row workgroups of four waves, one per SIMD (an O accumulator of 256
    // columns and the Q fragments of 32 rows take ~300 VGPRs), over a two-slot
    // K/V ring (136 KB of LDS): one workgroup per CU.
    if (causal && s.sq == s.sk && s.sq % 64 == 0) return fwd_sw_launch<256, 1, 4>(q, k, v, o, lse, s, c, neg_q, stream);
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o), lse, (int)bh, (int)s.sq,
                     (int)s.sk, (int)s.d, causal, c, neg_q, (int)nq);
  return check_launch("ferrite_flash_attention_fwd");
}

// o == nullptr: read delta; otherwise compute it from o and dout and write it.
// SPLIT: the split kernel, with the workspace ws and the pairs' cut.
template <int D, int W, int SLOTS, bool ZIG, int KSPLIT = 1, bool SPLIT = false>
int dq_pp_launch_t(const void* q, const void* k, const void* v, const void* dout, const float* lse, float* delta,
                   void* dq, const Shape& s, int causal, float scale, hipStream_t stream, const void* o,
                   const AttnViews& vw, void* ws = nullptr, int cut = 0) {
  typedef DqPp<D, W, SLOTS, KSPLIT> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: grid too large");
  auto kern = o ? attn_dq_pp_kernel<D, W, SLOTS, ZIG, true, KSPLIT, SPLIT>
                : attn_dq_pp_kernel<D, W, SLOTS, ZIG, false, KSPLIT, SPLIT>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(F::kThreads), F::kLds, stream, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<const bf16*>(dout), lse,
                     delta, static_cast<bf16*>(dq), (int)bh, (int)s.sq, (int)s.sk, (int)s.d, causal, scale,
                     scale * kLog2e, (int)nq, static_cast<const bf16*>(o), vw, static_cast<char*>(ws), cut);
  return check_launch("ferrite_flash_attention_bwd_dq");
}

// ws / ws_bytes: the caller's workspace for the split long-context dQ
// (bwd_split_bytes), or nullptr.
template <int D>
int dq_pp_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, float* delta,
                 void* dq, const Shape& s, int causal, float scale, hipStream_t stream, const void* o = nullptr,
                 const AttnViews* views = nullptr, void* ws = nullptr, int64_t ws_bytes = 0) {
  const AttnViews vw = views ? *views : dense_views(s);
  if constexpr (D == 64) {
    // 128-query workgroups with two LDS slots (67 KB): two share a CU. A grid
    // resident all at once (the long-context case) pairs long and short causal
    // sweeps on each CU, and its workgroups are 8 waves that split every key
    // tile between the two waves of a SIMD, so that the long sweep that
    // outlasts its partner still runs two waves per SIMD (1x8x8192x64:
    // 136 -> 122 us). Otherwise 4 waves each take whole tiles (the split
    // measured 10% slower at 8x12x1024x64).
    // With a workspace, a resident grid of an even number of 128-row tiles
    // splits its long tiles between the two workgroups of a CU, as the forward.
    typedef DqPp<64, 8, 2, 2> F4;
    const int cus = cu_count(stream);
    if (dq_split_applies(s, FERRITE_BF16, causal, cus) &&
        split_ws_ok(ws, ws_bytes, bwd_split_bytes(s, FERRITE_BF16, causal, cus)))
      return dq_pp_launch_t<D, 8, 2, true, 2, true>(q, k, v, dout, lse, delta, dq, s, causal, scale, stream, o, vw, ws,
                                                    sched::split_cut(s.b * s.h, s.sq, cus, sched::kDqSplit));
    const bool one_round = causal && sched::resident(cdiv(s.sq, F4::BQ) * s.b * s.h, 2, cus);
    return one_round ? dq_pp_launch_t<D, 8, 2, true, 2>(q, k, v, dout, lse, delta, dq, s, causal, scale, stream, o, vw)
                     : dq_pp_launch_t<D, 4, 2, false>(q, k, v, dout, lse, delta, dq, s, causal, scale, stream, o, vw);
  } else if constexpr (D == 128) {
    // 4-wave 128-query workgroups over a two-slot K/V ring (64 KB of LDS):
    // two share a CU, so one's prologue (Q, dO and O loads, the first tiles)
    // and its dQ store overlap the other's sweep. Against 8-wave 256-query
    // workgroups over three slots, one per CU (MI355X, one process, outputs
    // bitwise equal): 4x16x2048x128 113 -> 106 us, 2x8x4096x128 143 -> 117,
    // 16x16x512x128 58 -> 52, 8x12x1024x128 56.8 -> 54.6; 1x16x8192x128
    // 362 -> 368.
    return dq_pp_launch_t<D, 4, 2, false>(q, k, v, dout, lse, delta, dq, s, causal, scale, stream, o, vw);
  } else {
    // D = 256: the Q and dO fragments of 32 rows (128 VGPRs) and a dQ
    // accumulator of 256 columns (128) take one SIMD's registers for one wave:
    // four waves, one per SIMD, over a two-slot K/V ring (130 KB of LDS).
    return dq_pp_launch_t<D, 4, 2, false>(q, k, v, dout, lse, delta, dq, s, causal, scale, stream, o, vw);
  }
}

template <typename T, int D, bool AL>
int dq_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
              void* dq, const Shape& s, int causal, float scale, hipStream_t stream, void* ws = nullptr,
              int64_t ws_bytes = 0) {
  if constexpr (sizeof(T) == 2 && AL && D <= 128)
    return dq_pp_launch<D>(q, k, v, dout, lse, const_cast<float*>(delta), dq, s, causal, scale, stream, nullptr,
                           nullptr, ws, ws_bytes);
  typedef Dq<T, D, AL> F;
  const int64_t nq = cdiv(s.sq, F::BQ);
  const int64_t bh = s.b * s.h;
  if (nq * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: grid too large");
  auto kern = attn_dq_kernel<T, D, AL>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<const T*>(dout), lse, delta,
                     static_cast<T*>(dq), (int)bh, s.sq, s.sk, (int)s.d, causal, scale, scale * kLog2e, (int)nq);
  return check_launch("ferrite_flash_attention_bwd_dq");
}

template <int D>
int dkv_pp_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
                  void* dk, void* dv, const Shape& s, int causal, float scale, hipStream_t stream,
                  const AttnViews* views = nullptr, void* ws = nullptr, int64_t ws_bytes = 0) {
  typedef DkvPp<D> F;
  const int64_t nk = cdiv(s.sk, F::BKV);
  const int64_t bh = s.b * s.h;
  if (nk * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: grid too large");
  const AttnViews vw = views ? *views : dense_views(s);
  if constexpr (D == 128) {
    // Two waves per SIMD with the work of a key block split between them.
    typedef DkvRs R;
    auto kern = vw.q.r == vw.dout.r ? attn_dkv_rs_kernel<true> : attn_dkv_rs_kernel<false>;
    if (int rc = set_lds(kern, R::kLds, stream)) return rc;
    hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh)), dim3(R::kThreads), R::kLds, stream, static_cast<const bf16*>(q),
                       static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<const bf16*>(dout), lse,
                       delta, static_cast<bf16*>(dk), static_cast<bf16*>(dv), (int)bh, (int)s.sq, (int)s.sk, (int)s.d,
                       causal, scale, scale * kLog2e, vw, (int)nk, 0);
    return check_launch("ferrite_flash_attention_bwd_dkv");
  } else {
    // With a workspace, a resident grid of an even number of 128-key blocks
    // splits the long causal sweeps between the two workgroups of a CU, as the
    // forward splits its long query tiles.
    const int cus = cu_count(stream);
    const bool split = dkv_split_applies(s, FERRITE_BF16, causal, cus) &&
                       split_ws_ok(ws, ws_bytes, bwd_split_bytes(s, FERRITE_BF16, causal, cus));
    auto kern = split ? (vw.q.r == vw.dout.r ? attn_dkv_sw_kernel<D, true, true> : attn_dkv_sw_kernel<D, false, true>)
                      : (vw.q.r == vw.dout.r ? attn_dkv_sw_kernel<D, true> : attn_dkv_sw_kernel<D, false>);
    if (int rc = set_lds(kern, F::kLds, stream)) return rc;
    const int zig = causal && F::kMinBlocks == 2 && sched::resident(nk * bh, 2, cus);
    const int cut = split ? sched::split_cut(bh, s.sq, cus, sched::kDkvSplit) : 0;
    hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh)), dim3(F::kThreads), F::kLds, stream, static_cast<const bf16*>(q),
                       static_cast<const bf16*>(k), static_cast<const bf16*>(v), static_cast<const bf16*>(dout), lse,
                       delta, static_cast<bf16*>(dk), static_cast<bf16*>(dv), (int)bh, (int)s.sq, (int)s.sk, (int)s.d,
                       causal, scale, scale * kLog2e, vw, (int)nk, zig, split ? static_cast<char*>(ws) : nullptr, cut);
    return check_launch("ferrite_flash_attention_bwd_dkv");
  }
}

// bf16 dK/dV at head dim 256 (d == 256, 16-byte aligned rows) in one pass
// (attn_dkv_q256_kernel): four roles per 32-key block, 64 keys per workgroup.
int dkv256q_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
                   void* dk, void* dv, const Shape& s, int causal, float scale, hipStream_t stream) {
  typedef Dkv256Q F;
  const int64_t nk = cdiv(s.sk, F::BKV);
  const int64_t bh = s.b * s.h;
  if (nk * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: grid too large");
  const AttnViews vw = dense_views(s);
  auto kern = attn_dkv_q256_kernel<true>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh)), dim3(F::kThreads), F::kLds, stream,
                     static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                     static_cast<const bf16*>(dout), lse, delta, static_cast<bf16*>(dk), static_cast<bf16*>(dv),
                     (int)bh, (int)s.sq, (int)s.sk, causal, scale, scale * kLog2e, vw);
  return check_launch("ferrite_flash_attention_bwd_dkv");
}

template <typename T, int D, bool AL>
int dkv_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
               void* dk, void* dv, const Shape& s, int causal, float scale, hipStream_t stream, void* ws = nullptr,
               int64_t ws_bytes = 0) {
  if constexpr (sizeof(T) == 2 && AL && D <= 128)
    return dkv_pp_launch<D>(q, k, v, dout, lse, delta, dk, dv, s, causal, scale, stream, nullptr, ws, ws_bytes);
  typedef Dkv<T, D, AL> F;
  const int64_t nk = cdiv(s.sk, F::BKV);
  const int64_t bh = s.b * s.h;
  if (nk * bh > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: grid too large");
  auto kern = attn_dkv_kernel<T, D, AL>;
  if (int rc = set_lds(kern, F::kLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh)), dim3(kThreads), F::kLds, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<const T*>(dout), lse, delta,
                     static_cast<T*>(dk), static_cast<T*>(dv), (int)bh, s.sq, s.sk, (int)s.d, causal, scale,
                     scale * kLog2e);
  return check_launch("ferrite_flash_attention_bwd_dkv");
}

// Wide head dims: grid = heads x tiles x 128-column output slabs.
template <typename T, bool AL>
int fwd_wide_launch(const void* q, const void* k, const void* v, void* o, float* lse, const Shape& s, int causal,
                    float scale, hipStream_t stream) {
  typedef Wide<T> F;
  const int64_t nq = cdiv(s.sq, F::BQ), bh = s.b * s.h, nc = s.d / kSlab;
  if (nq * bh * nc > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: grid too large");
  float c = scale * kLog2e;  // see fwd_launch: a positive multiplier, the sign moved onto q
  const int neg_q = c < 0.f;
  c = fmaxf(fabsf(c), 1e-30f);
  auto kern = attn_fwd_wide_kernel<T, AL>;
  if (int rc = set_lds(kern, F::kFwdLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh * nc)), dim3(kThreads), F::kFwdLds, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o),
                     lse, (int)bh, (int)s.sq, (int)s.sk, (int)s.d, causal, c, neg_q, (int)nq);
  return check_launch("ferrite_flash_attention_fwd");
}

template <typename T, bool AL>
int dq_wide_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse, const float* delta,
                   void* dq, const Shape& s, int causal, float scale, hipStream_t stream) {
  typedef Wide<T> F;
  const int64_t nq = cdiv(s.sq, F::BQ), bh = s.b * s.h, nc = s.d / kSlab;
  if (nq * bh * nc > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: grid too large");
  auto kern = attn_dq_wide_kernel<T, AL>;
  if (int rc = set_lds(kern, F::kDqLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nq * bh * nc)), dim3(kThreads), F::kDqLds, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<const T*>(dout), lse, delta, static_cast<T*>(dq), (int)bh, (int)s.sq, (int)s.sk,
                     (int)s.d, causal, scale, scale * kLog2e, (int)nq);
  return check_launch("ferrite_flash_attention_bwd_dq");
}

template <typename T, bool AL>
int dkv_wide_launch(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                    const float* delta, void* dk, void* dv, const Shape& s, int causal, float scale,
                    hipStream_t stream) {
  typedef Wide<T> F;
  const int64_t nk = cdiv(s.sk, F::BKV), bh = s.b * s.h, nc = s.d / kSlab;
  if (nk * bh * nc > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: grid too large");
  auto kern = attn_dkv_wide_kernel<T, AL>;
  if (int rc = set_lds(kern, F::kDkvLds, stream)) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nk * bh * nc)), dim3(kThreads), F::kDkvLds, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<const T*>(dout), lse, delta, static_cast<T*>(dk), static_cast<T*>(dv), (int)bh,
                     (int)s.sq, (int)s.sk, (int)s.d, causal, scale, scale * kLog2e, (int)nk);
  return check_launch("ferrite_flash_attention_bwd_dkv");
}

// (dtype, aligned) dispatch of a wide launcher.
#define FERRITE_WIDE(LAUNCH, dtype, aligned, ...)                                                       \
  return (dtype) == FERRITE_BF16                                                                        \
             ? ((aligned) ? LAUNCH<bf16, true>(__VA_ARGS__) : LAUNCH<bf16, false>(__VA_ARGS__))         \
             : ((aligned) ? LAUNCH<float, true>(__VA_ARGS__) : LAUNCH<float, false>(__VA_ARGS__))

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

extern "C" int64_t ferrite_hip_attn_fwd_workspace(int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype,
                                                  int causal) {
  if (b < 1 || h < 1 || sq < 1 || sk < 1 || d < 1) return -1;
  // No stream here: sized for the current device's CU count.
  return fwd_split_bytes(Shape{b, h, sq, sk, d}, dtype, causal, cu_count_of(-1));
}

extern "C" int ferrite_hip_attn_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse, int64_t b,
                                       int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                       float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_fwd", s, dtype, causal, false)) return rc;
  if (!q || !k || !v || !o || !lse) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: null pointer");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_fwd: workspace_bytes > 0 needs a workspace");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(o);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d > 256) FERRITE_WIDE(fwd_wide_launch, dtype, al, q, k, v, o, lse, s, causal, scale, st);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return (aligned) ? LAUNCH<T, 256, true>(__VA_ARGS__) : LAUNCH<T, 256, false>(__VA_ARGS__)
  FERRITE_DISPATCH(fwd_launch, s, dtype, al, q, k, v, o, lse, s, causal, scale, st, workspace, workspace_bytes);
#undef FERRITE_DISPATCH_256
}

extern "C" int ferrite_hip_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t b,
                                    int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                    void* stream) {
  return ferrite_hip_attn_fwd_ex(q, k, v, o, lse, b, h, sq, sk, d, dtype, causal, scale, nullptr, 0, stream);
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

extern "C" int64_t ferrite_hip_attn_bwd_workspace(int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype,
                                                  int causal) {
  if (b < 1 || h < 1 || sq < 1 || sk < 1 || d < 1) return -1;
  // No stream here: sized for the current device's CU count.
  return bwd_split_bytes(Shape{b, h, sq, sk, d}, dtype, causal, cu_count_of(-1));
}

extern "C" int ferrite_hip_attn_bwd_dkv_ex(const void* q, const void* k, const void* v, const void* dout,
                                           const float* lse, const float* delta, void* dk, void* dv, int64_t b,
                                           int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                           float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_bwd_dkv", s, dtype, causal, true)) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: null pointer");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dkv: workspace_bytes > 0 needs a workspace");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(dout) && aligned16(dk) && aligned16(dv);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d == 256 && dtype == FERRITE_BF16 && al)
    return dkv256q_launch(q, k, v, dout, lse, delta, dk, dv, s, causal, scale, st);
  if (d > 128) FERRITE_WIDE(dkv_wide_launch, dtype, al, q, k, v, dout, lse, delta, dk, dv, s, causal, scale, st);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return fail(FERRITE_ERR_INVALID_ARGUMENT, "unreachable head_dim")
  FERRITE_DISPATCH(dkv_launch, s, dtype, al, q, k, v, dout, lse, delta, dk, dv, s, causal, scale, st, workspace,
                   workspace_bytes);
#undef FERRITE_DISPATCH_256
}

extern "C" int ferrite_hip_attn_bwd_dkv(const void* q, const void* k, const void* v, const void* dout,
                                        const float* lse, const float* delta, void* dk, void* dv, int64_t b,
                                        int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                        float scale, void* stream) {
  return ferrite_hip_attn_bwd_dkv_ex(q, k, v, dout, lse, delta, dk, dv, b, h, sq, sk, d, dtype, causal, scale, nullptr,
                                     0, stream);
}

namespace ferrite {
namespace {

// q, k, v heads inside a token-major [B, S, 3, H, d] projection, and O / dO as
// token-major [B, S, H, d] (the layouts either side of model/gpt.py:137-138).
AttnViews packed_views(int64_t b, int64_t s, int64_t h, int64_t d) {
  const View vqkv{s * 3 * h * d, d, 3 * h * d}, vo{s * h * d, d, h * d};
  return AttnViews{vqkv, vqkv, vqkv, vo, vo, vqkv, vqkv, vqkv, (int)h};
}

int check_packed(const char* name, int64_t b, int64_t s, int64_t h, int64_t d) {
  if (b < 1 || s < 1 || h < 1 || (d != 64 && d != 128))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need b, s, h >= 1 and head_dim 64 or 128");
  if (s % 64 != 0) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need seq % 64 == 0");
  if (s * 3 * h * d * 2 >= 0x7fffffff || b * h > 0x7fffffff)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": a sequence spans over 2 GiB");
  return FERRITE_OK;
}

}  // namespace
}  // namespace ferrite

extern "C" int ferrite_hip_attn_fwd_qkv(const void* qkv, void* o, float* lse, int64_t b, int64_t s, int64_t h,
                                        int64_t d, float scale, void* stream) {
  const char* name = "ferrite_hip_attn_fwd_qkv";
  if (int rc = check_packed(name, b, s, h, d)) return rc;
  if (!qkv || !o || !lse) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  if (!aligned16(qkv) || !aligned16(o))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": qkv and o must be 16-byte aligned");
  const Shape sh{b, h, s, s, d};
  const AttnViews vw = packed_views(b, s, h, d);
  const bf16* base = static_cast<const bf16*>(qkv);
  const bf16 *q = base, *k = base + h * d, *v = base + 2 * h * d;
  float c = scale * kLog2e;
  const int neg_q = c < 0.f;
  c = fmaxf(fabsf(c), 1e-30f);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d == 64) {
    typedef FwdW<64, 1, 8, 2> F4;
    const bool one_round = sched::resident(cdiv(s, F4::BQ) * b * h, 2, cu_count(st));
    return one_round ? fwd_sw_launch<64, 1, 8, true, 2>(q, k, v, o, lse, sh, c, neg_q, st, &vw)
                     : fwd_sw_launch<64, 1, 8, false, 2>(q, k, v, o, lse, sh, c, neg_q, st, &vw);
  }
  return fwd_sw_launch<128>(q, k, v, o, lse, sh, c, neg_q, st, &vw);
}

extern "C" int ferrite_hip_attn_bwd_qkv(const void* qkv, const void* o, const void* dout, const float* lse,
                                        float* delta, void* dqkv, int64_t b, int64_t s, int64_t h, int64_t d,
                                        float scale, void* stream) {
  const char* name = "ferrite_hip_attn_bwd_qkv";
  if (int rc = check_packed(name, b, s, h, d)) return rc;
  if (!qkv || !o || !dout || !lse || !delta || !dqkv)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  if (!aligned16(qkv) || !aligned16(o) || !aligned16(dout) || !aligned16(dqkv))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": tensors must be 16-byte aligned");
  const Shape sh{b, h, s, s, d};
  const AttnViews vw = packed_views(b, s, h, d);
  const bf16* base = static_cast<const bf16*>(qkv);
  const bf16 *q = base, *k = base + h * d, *v = base + 2 * h * d;
  bf16* gbase = static_cast<bf16*>(dqkv);
  bf16 *dq = gbase, *dk = gbase + h * d, *dv = gbase + 2 * h * d;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // dQ computes delta from O and dO and writes it; dK/dV then reads it.
  int rc = d == 64 ? dq_pp_launch<64>(q, k, v, dout, lse, delta, dq, sh, 1, scale, st, o, &vw)
                   : dq_pp_launch<128>(q, k, v, dout, lse, delta, dq, sh, 1, scale, st, o, &vw);
  if (rc) return rc;
  return d == 64 ? dkv_pp_launch<64>(q, k, v, dout, lse, delta, dk, dv, sh, 1, scale, st, &vw)
                 : dkv_pp_launch<128>(q, k, v, dout, lse, delta, dk, dv, sh, 1, scale, st, &vw);
}

extern "C" int ferrite_hip_attn_bwd_dq_ex(const void* q, const void* k, const void* v, const void* dout,
                                          const float* lse, const float* delta, void* dq, int64_t b, int64_t h,
                                          int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                          void* workspace, int64_t workspace_bytes, void* stream);

extern "C" int ferrite_hip_attn_bwd_dq_delta_ex(const void* q, const void* k, const void* v, const void* o,
                                                const void* dout, const float* lse, float* delta, void* dq, int64_t b,
                                                int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                                float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_bwd_dq_delta", s, dtype, causal, true)) return rc;
  if (!q || !k || !v || !o || !dout || !lse || !delta || !dq)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq_delta: null pointer");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq_delta: workspace_bytes > 0 needs a workspace");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(o) && aligned16(dout) && aligned16(dq);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int dp = pad_dim(d);
  if (dtype == FERRITE_BF16 && al && dp <= 128) {
    if (dp == 64)
      return dq_pp_launch<64>(q, k, v, dout, lse, delta, dq, s, causal, scale, st, o, nullptr, workspace,
                              workspace_bytes);
    return dq_pp_launch<128>(q, k, v, dout, lse, delta, dq, s, causal, scale, st, o);
  }
  if (dtype == FERRITE_BF16 && al && d == 256)
    return dq_pp_launch<256>(q, k, v, dout, lse, delta, dq, s, causal, scale, st, o);
  // Other dtypes and head dims: the delta kernel, then dQ reading it.
  if (int rc = ferrite_hip_attn_bwd_delta(o, dout, delta, b, h, sq, d, dtype, stream)) return rc;
  return ferrite_hip_attn_bwd_dq_ex(q, k, v, dout, lse, delta, dq, b, h, sq, sk, d, dtype, causal, scale, workspace,
                                    workspace_bytes, stream);
}

extern "C" int ferrite_hip_attn_bwd_dq_delta(const void* q, const void* k, const void* v, const void* o,
                                             const void* dout, const float* lse, float* delta, void* dq, int64_t b,
                                             int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype, int causal,
                                             float scale, void* stream) {
  return ferrite_hip_attn_bwd_dq_delta_ex(q, k, v, o, dout, lse, delta, dq, b, h, sq, sk, d, dtype, causal, scale,
                                          nullptr, 0, stream);
}

extern "C" int ferrite_hip_attn_bwd_dq_ex(const void* q, const void* k, const void* v, const void* dout,
                                          const float* lse, const float* delta, void* dq, int64_t b, int64_t h,
                                          int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                          void* workspace, int64_t workspace_bytes, void* stream) {
  const Shape s{b, h, sq, sk, d};
  if (int rc = check_shape("ferrite_hip_attn_bwd_dq", s, dtype, causal, true)) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dq)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: null pointer");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_attn_bwd_dq: workspace_bytes > 0 needs a workspace");
  const bool al = d % (dtype == FERRITE_BF16 ? 8 : 4) == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(dout) && aligned16(dq);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d == 256 && dtype == FERRITE_BF16 && al)
    return dq_pp_launch<256>(q, k, v, dout, lse, const_cast<float*>(delta), dq, s, causal, scale, st);
  if (d > 128) FERRITE_WIDE(dq_wide_launch, dtype, al, q, k, v, dout, lse, delta, dq, s, causal, scale, st);
#define FERRITE_DISPATCH_256(LAUNCH, T, aligned, ...) \
  return fail(FERRITE_ERR_INVALID_ARGUMENT, "unreachable head_dim")
  FERRITE_DISPATCH(dq_launch, s, dtype, al, q, k, v, dout, lse, delta, dq, s, causal, scale, st, workspace,
                   workspace_bytes);
#undef FERRITE_DISPATCH_256
}

extern "C" int ferrite_hip_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                                       const float* lse, const float* delta, void* dq, int64_t b, int64_t h,
                                       int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale,
                                       void* stream) {
  return ferrite_hip_attn_bwd_dq_ex(q, k, v, dout, lse, delta, dq, b, h, sq, sk, d, dtype, causal, scale, nullptr, 0,
                                    stream);
}
