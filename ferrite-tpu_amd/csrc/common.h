// Shared device helpers for the gfx950 (CDNA4) kernels: element traits, bf16
// conversion, 16-byte vector I/O, the 32x32 MFMA fragment abstraction and the
// per-thread error slot of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/ferrite_hip.h"

namespace ferrite {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Element traits. A "vector" is 16 bytes of elements (one global/LDS b128
// access). A "fragment" is the 8 elements one lane contributes to one K=16
// chunk of a 32x32 MFMA tile (lane group g = lane/32 holds k = 8g .. 8g+7).
// ---------------------------------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16 bytes
  typedef f32x4 vec;
  typedef f32x8 frag;
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
};

template <>
struct Elem<bf16> {
  static constexpr int kVec = 8;
  typedef bf16x8 vec;
  typedef bf16x8 frag;
  static __device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
  // Round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
  static __device__ __forceinline__ bf16 from_f32(float x) { return (bf16)x; }
};

// acc(32x32, f32) += A(32x16) * B(16x32). For bf16 this is one
// v_mfma_f32_32x32x16_bf16. For f32 it is eight v_mfma_f32_32x32x2_f32 (true
// fp32 products): instruction e takes element e of every lane, so lane group g
// of A and B both contribute k = 8g + e, and the eight instructions together
// cover the same 16 k values as the bf16 form.
__device__ __forceinline__ void mma32(const bf16x8& a, const bf16x8& b, f32x16& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(const f32x8& a, const f32x8& b, f32x16& acc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], acc, 0, 0, 0);
}

// Convert 8 f32 values to a fragment of T.
// Two floats rounded to bf16 (round to nearest even) and packed, a in the
// low half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ void to_frag(const float* v, bf16x8& out) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (bf16)v[e];
}
__device__ __forceinline__ void to_frag(const float* v, f32x8& out) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = v[e];
}

// Swap with the lane 32 away (gfx950 v_permlane32_swap) and combine: returns
// op(x[lane % 32], x[lane % 32 + 32]) in every lane.
__device__ __forceinline__ float lane32_max(float x) {
  uint32_t b = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane32_sum(float x) {
  uint32_t b = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Full-wave sum (64 lanes) with cross-lane butterflies.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) x += __shfl_xor(x, off, kWave);
  return lane32_sum(x);
}

// ---------------------------------------------------------------------------
// Host-side error slot.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline bool valid_dtype(int dt) { return dt == FERRITE_F32 || dt == FERRITE_BF16; }
inline const char* dtype_name(int dt) { return dt == FERRITE_F32 ? "f32" : dt == FERRITE_BF16 ? "bf16" : "?"; }

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ferrite
