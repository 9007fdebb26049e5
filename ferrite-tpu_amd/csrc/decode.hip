// Decode attention over a static KV cache, for gfx950.
//
// Reference: src/ferrite/serving/engine.py:89-104 (_cache_attention and
// _write_cache): one query row per (batch, head) attends over the cached keys
// 0..pos[b] (later positions are masked), in f32, and the new key/value row is
// written into the cache at pos[b]. The reference leaves this step to XLA and
// names a decode-attention kernel as its next step (README.md:283-285).
//
// HBM-bound: a step reads (pos + 1) keys and values per head once. Keys are
// split into chunks per workgroup (flash-decoding), so short batches still
// spread over the CUs; each chunk keeps an online (max, sum, acc) softmax and
// writes f32 partials, and a second kernel merges the chunks of a head. A row
// of LPR = D / (16 / sizeof(T)) lanes holds one key: each lane loads 16 bytes
// of K and V and the row's score is a shuffle reduction within those lanes.
// The new key/value are read from k_new / v_new, not from the cache row this
// launch writes, so no workgroup reads a row another writes.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace ferrite {
namespace {

constexpr int kDecThreads = 256;  // 4 waves
constexpr int kUnroll = 4;        // row steps whose loads are issued together
// Keys per workgroup: the smallest power of two from kChunkMin up that keeps
// the grid (B H chunks) within kGridTarget workgroups, two per CU of MI355X, so
// that each wave streams one long contiguous stretch of the cache with kUnroll
// row steps of non-temporal loads in flight. Measured on MI355X against the
// previous fixed choice (1024-key chunks for grids of >= 512 such workgroups,
// else 256; two row steps per batch of loads), one of the B sequences at a
// third of the cache: 8x32x8192x128 bf16 186.7 -> 162.4 us (4096-key chunks),
// 32x32x2048x128 bf16 190.9 -> 160.2 us, 8x16x8192x128 f32 168.8 -> 155.3 us,
// 1x32x8192x128 bf16 28.6 -> 20 us.
constexpr int kChunkMin = 256;
constexpr int64_t kGridTarget = 512;

template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  const u32x4 raw = *reinterpret_cast<const u32x4*>(p);
  if constexpr (sizeof(T) == 2) {
    const bf16x8 v = __builtin_bit_cast(bf16x8, raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
  } else {
    const f32x4 v = __builtin_bit_cast(f32x4, raw);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = v[e];
  }
}

// Element e of 16 raw bytes as f32 (rows stay raw in registers until used:
// half the registers of rows widened to f32 for bf16).
template <typename T>
__device__ __forceinline__ float elem_f32(const u32x4& raw, int e) {
  if constexpr (sizeof(T) == 2)
    return (float)__builtin_bit_cast(bf16x8, raw)[e];
  else
    return __builtin_bit_cast(f32x4, raw)[e];
}

// Merge (m2, l2, acc2) into (m, l, acc); m = -inf marks an empty state.
template <int N>
__device__ __forceinline__ void merge_state(float& m, float& l, float* acc, float m2, float l2, const float* acc2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float a = exp2f(m - mn), b = exp2f(m2 - mn);
  l = l * a + l2 * b;
#pragma unroll
  for (int e = 0; e < N; ++e) acc[e] = acc[e] * a + acc2[e] * b;
  m = mn;
}

// grid (chunks, H, B), `chunk` keys per workgroup (a power of two >= kChunkMin).
// Partials: [B, H, chunks, D + 2] = (acc[D], m, l) in the log2 domain.
template <typename T, int D, bool DIRECT>
__global__ __launch_bounds__(kDecThreads) void decode_attn_kernel(const T* __restrict__ q, const T* __restrict__ k_new,
                                                                  const T* __restrict__ v_new, T* __restrict__ k_cache,
                                                                  T* __restrict__ v_cache, const int32_t* __restrict__ pos,
                                                                  T* __restrict__ out, float* __restrict__ part,
                                                                  int max_len, float c, int chunk) {
  constexpr int V = Vec16<T>::N;
  constexpr int LPR = D / V;          // lanes per key row
  constexpr int RPW = 64 / LPR;       // rows per wave step
  static_assert(D % V == 0 && LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "head dim");
  // A wave's rows (chunk / 4, a power of two >= kChunkMin / 4) in whole unrolled steps.
  static_assert((kChunkMin / (kDecThreads / 64)) % (RPW * kUnroll) == 0, "a wave's rows in whole unrolled steps");
  const int wave_rows = chunk / (kDecThreads / 64);
  __shared__ float red[kDecThreads / 64][D + 2];

  const int h = blockIdx.y, b = blockIdx.z;
  const int H = gridDim.y, nchunks = gridDim.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;  // row group within the wave, lane within the row
  const int64_t bh = (int64_t)b * H + h;
  const int p = pos[b];
  const bool valid = p >= 0 && p < max_len;

  // The new row goes into the cache at pos (one workgroup per head does it).
  if (valid && blockIdx.x == 0 && wave == 0) {
    for (int e = lane * V; e < D; e += 64 * V) {
      *reinterpret_cast<u32x4*>(k_cache + (bh * max_len + p) * D + e) =
          *reinterpret_cast<const u32x4*>(k_new + bh * D + e);
      *reinterpret_cast<u32x4*>(v_cache + (bh * max_len + p) * D + e) =
          *reinterpret_cast<const u32x4*>(v_new + bh * D + e);
    }
  }

  float qv[V];
  load_vec(q + bh * D + sub * V, qv);
  float m = -INFINITY, l = 0.f, acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;

  const int last = valid ? p : -1;  // keys 0..last
  const int r0 = blockIdx.x * chunk + wave * wave_rows;
  // Rows 0 .. last - 1 of the head's cache through descriptors whose range ends
  // at row `last`: an offset past it reads zeros without touching memory, so
  // the loads need no branch and go out together. Row `last` comes from
  // k_new / v_new. A head's cache is under 4 GiB (max_len < 2^22, D sizeof(T)
  // <= 1024 bytes a row), so 32-bit offsets reach all of it.
  constexpr uint32_t kRowBytes = D * sizeof(T);
  // readfirstlane: the descriptors must be provably uniform, or every load
  // becomes a loop over the lanes' distinct descriptors.
  auto uniform = [](const T* ptr) {
    const uint64_t a = reinterpret_cast<uint64_t>(ptr);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return reinterpret_cast<T*>(lo | (hi << 32));
  };
  const uint32_t cached_bytes = (uint32_t)__builtin_amdgcn_readfirstlane(last > 0 ? last : 0) * kRowBytes;
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(uniform(k_cache + bh * max_len * D), (short)0, (int)cached_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(uniform(v_cache + bh * max_len * D), (short)0, (int)cached_bytes, 0x00020000);
  const u32x4 knr = *reinterpret_cast<const u32x4*>(k_new + bh * D + sub * V);
  const u32x4 vnr = *reinterpret_cast<const u32x4*>(v_new + bh * D + sub * V);
  for (int rs = 0; rs < wave_rows; rs += RPW * kUnroll) {
    if (r0 + rs > last) break;
    // Raw rows; aux 2 makes the loads non-temporal (the cache is read once a step).
    u32x4 kr[kUnroll], vr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = r0 + rs + u * RPW + grp;
      const uint32_t off = r < last ? (uint32_t)r * kRowBytes + (uint32_t)(sub * 16) : 0xfffffff0u;
      kr[u] = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)off, 0, 2);
      vr[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)off, 0, 2);
    }
    // Past the last key the rows are zeros, weighted 0 below.
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (r0 + rs + u * RPW + grp == last) {
        kr[u] = knr;
        vr[u] = vnr;
      }
    }
    // The kUnroll scores of a row group first, then one rescale to their max.
    float sc[kUnroll];
    float mb = -INFINITY;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = r0 + rs + u * RPW + grp;
      float s = 0.f;
      if (r <= last) {
#pragma unroll
        for (int e = 0; e < V; ++e) s += qv[e] * elem_f32<T>(kr[u], e);
      }
#pragma unroll
      for (int off = 1; off < LPR; off <<= 1) s += __shfl_xor(s, off, 64);
      sc[u] = r <= last ? s * c : -INFINITY;
      mb = fmaxf(mb, sc[u]);
    }
    if (mb > -INFINITY) {
      const float mn = fmaxf(m, mb);
      const float a = exp2f(m - mn);
      l *= a;
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] *= a;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float pr = exp2f(sc[u] - mn);
        l += pr;
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] = __builtin_fmaf(pr, elem_f32<T>(vr[u], e), acc[e]);
      }
      m = mn;
    }
  }

  // Merge the RPW row groups of the wave (lanes with the same sub), then the waves.
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
    float acc2[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc2[e] = __shfl_xor(acc[e], off, 64);
    merge_state<V>(m, l, acc, m2, l2, acc2);
  }
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < V; ++e) red[wave][sub * V + e] = acc[e];
    if (sub == 0) {
      red[wave][D] = m;
      red[wave][D + 1] = l;
    }
  }
  __syncthreads();
  if (wave != 0 || grp != 0) return;
  for (int w = 1; w < kDecThreads / 64; ++w) {
    float a2[V];
#pragma unroll
    for (int e = 0; e < V; ++e) a2[e] = red[w][sub * V + e];
    merge_state<V>(m, l, acc, red[w][D], red[w][D + 1], a2);
  }
  if constexpr (DIRECT) {
    const float inv = valid ? 1.f / l : NAN;
#pragma unroll
    for (int e = 0; e < V; ++e) out[bh * D + sub * V + e] = Elem<T>::from_f32(acc[e] * inv);
  } else {
    float* dst = part + (bh * nchunks + blockIdx.x) * (D + 2);
#pragma unroll
    for (int e = 0; e < V; ++e) dst[sub * V + e] = acc[e];
    if (sub == 0) {
      dst[D] = m;
      dst[D + 1] = l;
    }
  }
}

// One block per head: merge the chunks that hold keys (0..pos) and normalise.
// Loads go out eight chunks at a time, so a thread waits on a few batches of
// independent loads rather than on one chain of dependent ones. An empty chunk
// (m = -inf, l = acc = 0) gets weight exp2(-inf) = 0.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(const float* __restrict__ part, const int32_t* __restrict__ pos,
                                                             T* __restrict__ out, int nchunks, int max_len, int chunk) {
  constexpr int G = 8;
  constexpr int S = D + 2;  // floats per chunk partial
  const int h = blockIdx.x, b = blockIdx.y, H = gridDim.x;
  const int64_t bh = (int64_t)b * H + h;
  const int p = pos[b];
  const bool valid = p >= 0 && p < max_len;
  const int used = valid ? min(nchunks, p / chunk + 1) : 0;
  const float* src = part + bh * nchunks * S;
  float mx = -INFINITY;
  int s0 = 0;
  for (; s0 + G <= used; s0 += G) {
    float m[G];
#pragma unroll
    for (int j = 0; j < G; ++j) m[j] = src[(s0 + j) * S + D];
#pragma unroll
    for (int j = 0; j < G; ++j) mx = fmaxf(mx, m[j]);
  }
  for (; s0 < used; ++s0) mx = fmaxf(mx, src[s0 * S + D]);
  for (int e = threadIdx.x; e < D; e += blockDim.x) {
    float l = 0.f, a = 0.f;
    int s = 0;
    for (; s + G <= used; s += G) {
      float m[G], lv[G], av[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        m[j] = src[(s + j) * S + D];
        lv[j] = src[(s + j) * S + D + 1];
        av[j] = src[(s + j) * S + e];
      }
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const float w = exp2f(m[j] - mx);
        l += lv[j] * w;
        a += av[j] * w;
      }
    }
    for (; s < used; ++s) {
      const float w = exp2f(src[s * S + D] - mx);
      l += src[s * S + D + 1] * w;
      a += src[s * S + e] * w;
    }
    out[bh * D + e] = Elem<T>::from_f32(valid ? a / l : NAN);
  }
}

int64_t chunk_for(int64_t b, int64_t h, int64_t max_len) {
  int64_t c = kChunkMin;
  while (c < max_len && b * h * cdiv(max_len, c) > kGridTarget) c *= 2;
  return c;
}
int64_t chunks_for(int64_t b, int64_t h, int64_t max_len) { return cdiv(max_len, chunk_for(b, h, max_len)); }

template <typename T, int D>
int decode_launch(const void* q, const void* kn, const void* vn, void* kc, void* vc, const int32_t* pos, void* out,
                  int64_t B, int64_t H, int64_t L, float scale, void* ws, int64_t ws_bytes, hipStream_t st) {
  const int64_t chunk = chunk_for(B, H, L), nch = cdiv(L, chunk);
  const float c = scale * kLog2e;
  const dim3 grid((unsigned)nch, (unsigned)H, (unsigned)B);
  auto tq = static_cast<const T*>(q);
  auto tk = static_cast<const T*>(kn);
  auto tv = static_cast<const T*>(vn);
  auto ck = static_cast<T*>(kc);
  auto cv = static_cast<T*>(vc);
  auto to = static_cast<T*>(out);
  if (nch == 1) {
    hipLaunchKernelGGL((decode_attn_kernel<T, D, true>), grid, dim3(kDecThreads), 0, st, tq, tk, tv, ck, cv, pos, to,
                       nullptr, (int)L, c, (int)chunk);
  } else {
    if (!ws || ws_bytes < B * H * nch * (D + 2) * (int64_t)sizeof(float))
      return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_decode_attention: workspace too small");
    hipLaunchKernelGGL((decode_attn_kernel<T, D, false>), grid, dim3(kDecThreads), 0, st, tq, tk, tv, ck, cv, pos, to,
                       static_cast<float*>(ws), (int)L, c, (int)chunk);
    hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3((unsigned)H, (unsigned)B), dim3(std::min(D, 256)), 0, st,
                       static_cast<const float*>(ws), pos, to, (int)nch, (int)L, (int)chunk);
  }
  return check_launch("ferrite_decode_attention");
}

}  // namespace
}  // namespace ferrite

extern "C" int64_t ferrite_hip_decode_attention_workspace(int64_t b, int64_t h, int64_t max_len, int64_t d) {
  if (b < 0 || h < 1 || max_len < 1 || d < 1) return -1;
  const int64_t nch = ferrite::chunks_for(b, h, max_len);
  return nch > 1 ? b * h * nch * (d + 2) * (int64_t)sizeof(float) : 0;
}

extern "C" int ferrite_hip_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_cache,
                                            void* v_cache, const int32_t* pos, void* out, int64_t b, int64_t h,
                                            int64_t max_len, int64_t d, int dtype, float scale, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  using namespace ferrite;
  const char* name = "ferrite_hip_decode_attention";
  if (!valid_dtype(dtype)) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (b < 0 || h < 1 || max_len < 1 || b > 65535 || h > 65535 || max_len > 0x7fffffff / 512)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need 0 <= b, h <= 65535 and 1 <= max_len < 2^22");
  if (b == 0) return FERRITE_OK;
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !pos || !out)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a16(q) || !a16(k_new) || !a16(v_new) || !a16(k_cache) || !a16(v_cache) || !a16(out))
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
#define FERRITE_DEC_CASE(T, DD)                                                                          \
  if (d == DD) return decode_launch<T, DD>(q, k_new, v_new, k_cache, v_cache, pos, out, b, h, max_len, scale, \
                                           workspace, workspace_bytes, s)
  if (dtype == FERRITE_BF16) {
    FERRITE_DEC_CASE(bf16, 64);
    FERRITE_DEC_CASE(bf16, 128);
    FERRITE_DEC_CASE(bf16, 256);
  } else {
    FERRITE_DEC_CASE(float, 64);
    FERRITE_DEC_CASE(float, 128);
    FERRITE_DEC_CASE(float, 256);
  }
#undef FERRITE_DEC_CASE
  return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": head dim must be 64, 128 or 256");
}
