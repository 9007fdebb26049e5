// Head layout changes around the attention kernels, for gfx950.
//
// The QKV projection produces rows [G, H, D] per token ([B, S, G, H, D], G = 3
// for q, k, v), and the attention kernels read and write head-major
// [B, H, S, D] tensors; the attention output goes back to token-major rows
// ([B, S, H, D], G = 1) for the output projection. Reference: the transposes of
// src/ferrite/model/gpt.py:137-138, which XLA turns into copy fusions.
//
// HBM-bound permutes: every thread moves one 16-byte vector; the token-major
// side is read or written in whole contiguous rows and the head-major side in
// D-element runs, so both sides are coalesced.
#include "common.h"

namespace ferrite {
namespace {

constexpr int kMaxGroups = 4;

struct HeadPtrs {
  void* p[kMaxGroups];
};

// Element (b, s, g, h, e) of the token-major tensor <-> element (b, h, s, e) of
// head-major tensor g. V elements per thread (V = 16 bytes / sizeof(T), or 1).
template <typename T, int V, bool SPLIT>
__global__ __launch_bounds__(256) void heads_kernel(T* __restrict__ tok, HeadPtrs heads, int64_t S, int G, int H,
                                                    int D, int64_t total_vecs) {
  typedef __attribute__((ext_vector_type(4))) uint32_t vec_t;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total_vecs) return;
  const int dv = D / V;
  const int64_t row_vecs = (int64_t)G * H * dv;
  const int64_t bs = i / row_vecs;
  const int64_t c = i - bs * row_vecs;
  const int g = (int)(c / ((int64_t)H * dv));
  const int rem = (int)(c - (int64_t)g * H * dv);
  const int h = rem / dv, e = (rem - h * dv) * V;
  const int64_t b = bs / S, s = bs - b * S;
  T* head = static_cast<T*>(heads.p[g]) + ((b * H + h) * S + s) * D + e;
  T* t = tok + i * V;
  if constexpr (V * sizeof(T) == 16) {
    if constexpr (SPLIT)
      *reinterpret_cast<vec_t*>(head) = *reinterpret_cast<const vec_t*>(t);
    else
      *reinterpret_cast<vec_t*>(t) = *reinterpret_cast<const vec_t*>(head);
  } else {
    if constexpr (SPLIT)
      *head = *t;
    else
      *t = *head;
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T, bool SPLIT>
int heads_launch(void* tok, void* const* heads, int64_t B, int64_t S, int64_t G, int64_t H, int64_t D,
                 hipStream_t stream) {
  constexpr int kVec = 16 / sizeof(T);
  HeadPtrs hp{};
  bool vec = D % kVec == 0 && al16(tok);
  for (int g = 0; g < G; ++g) {
    hp.p[g] = heads[g];
    vec = vec && al16(heads[g]);
  }
  const int64_t elems = B * S * G * H * D;
  const int64_t total = vec ? elems / kVec : elems;
  const int64_t blocks = cdiv(total, 256);
  if (blocks > 0x7fffffff) return fail(FERRITE_ERR_INVALID_ARGUMENT, "ferrite_hip_heads: tensor too large");
  T* tp = static_cast<T*>(tok);
  if (vec)
    hipLaunchKernelGGL((heads_kernel<T, kVec, SPLIT>), dim3((unsigned)blocks), dim3(256), 0, stream, tp, hp, S, (int)G,
                       (int)H, (int)D, total);
  else
    hipLaunchKernelGGL((heads_kernel<T, 1, SPLIT>), dim3((unsigned)blocks), dim3(256), 0, stream, tp, hp, S, (int)G,
                       (int)H, (int)D, total);
  return check_launch(SPLIT ? "ferrite_heads_split" : "ferrite_heads_merge");
}

template <bool SPLIT>
int heads_dispatch(const char* name, void* tok, void* const* heads, int64_t b, int64_t s, int64_t g, int64_t h,
                   int64_t d, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": dtype must be FERRITE_F32 or FERRITE_BF16");
  if (b < 0 || s < 0 || g < 1 || g > kMaxGroups || h < 1 || d < 1 || g * h * d > 0x7fffffff)
    return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": need b, s >= 0, 1 <= groups <= 4, heads, dim >= 1");
  if (b * s == 0) return FERRITE_OK;
  if (!tok || !heads) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  for (int i = 0; i < g; ++i)
    if (!heads[i]) return fail(FERRITE_ERR_INVALID_ARGUMENT, std::string(name) + ": null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FERRITE_BF16) return heads_launch<bf16, SPLIT>(tok, heads, b, s, g, h, d, st);
  return heads_launch<float, SPLIT>(tok, heads, b, s, g, h, d, st);
}

}  // namespace
}  // namespace ferrite

extern "C" int ferrite_hip_heads_split(const void* tokens, void* const* heads, int64_t b, int64_t s, int64_t groups,
                                       int64_t h, int64_t d, int dtype, void* stream) {
  return ferrite::heads_dispatch<true>("ferrite_hip_heads_split", const_cast<void*>(tokens), heads, b, s, groups, h,
                                       d, dtype, stream);
}

extern "C" int ferrite_hip_heads_merge(void* const* heads, void* tokens, int64_t b, int64_t s, int64_t groups,
                                       int64_t h, int64_t d, int dtype, void* stream) {
  return ferrite::heads_dispatch<false>("ferrite_hip_heads_merge", tokens, heads, b, s, groups, h, d, dtype, stream);
}
