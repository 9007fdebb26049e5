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

// ---- LDS DMA and transposed LDS reads (gfx950) ------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));

// Two transposed 8-byte reads at `p` and `p + hi_off`, joined into one
// 8-element A fragment. Within each 16-lane group the instruction hands lane
// 4a + b element b of the 4-element pieces addressed by lanes a, a+4, a+8, a+12.
__device__ __forceinline__ bf16x8 tr_frag(const char* p, int hi_off) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  lds_i16x4* p0 = reinterpret_cast<lds_i16x4*>(reinterpret_cast<uintptr_t>(p));
  lds_i16x4* p1 = reinterpret_cast<lds_i16x4*>(reinterpret_cast<uintptr_t>(p + hi_off));
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1);
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that leaves outstanding global loads (DMA rings) alone
// and that the scheduler may not move any instruction across.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Buffer descriptor (raw, unswizzled, bounds-checked) of `bytes` bytes at p.
// The operands must be wave-uniform; readfirstlane keeps them in SGPRs.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* p, uint32_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffffu)),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000u};
}

// One buffer_load_dwordx4 ... lds: lane L copies the 16 bytes at voff into
// LDS at `lds` + 16 L; lanes whose voff is past the range write zeros. Inline
// assembly, so that the compiler's wait insertion does not tie later LDS
// reads to it: callers order it with wait_vmem and barriers.
__device__ __forceinline__ void dma16(const u32x4& rsrc, char* lds, uint32_t voff) {
  const uint32_t m0 =
      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)reinterpret_cast<uintptr_t>(lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// The lane (0-63), formed where it is called: two mbcnt instructions in a
// volatile asm, which the compiler neither merges with another call nor hoists.
// Code after a kernel's main loop (or in a later work segment) that takes its
// lane terms from here keeps nothing lane-derived live (or spilled) across the
// loop; the thread index would be one value for the whole kernel.
__device__ __forceinline__ int lane_id() {
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return lane;
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
// The device a stream's launches run on (the current device for the null and
// per-thread streams), or -1. Every per-device lookup of an entry point goes
// through the stream it was given, not through the thread's current device.
int stream_device(hipStream_t s);
// Compute units of device `dev` (the current device when dev < 0; 256 on an MI355X).
int cu_count_of(int dev);
// Compute units of the stream's device.
int cu_count(hipStream_t s);
// Makes `dev` current for its lifetime (no-op when it already is or dev < 0).
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev);
  ~DeviceGuard();
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int prev_;
};
// Raises `kernel`'s dynamic-LDS limit to `bytes` on the stream's device, once per
// (kernel, device); FERRITE_OK, or an error code with the message set (`what`
// names the entry point).
int allow_lds(const void* kernel, int bytes, hipStream_t s, const char* what);

inline bool valid_dtype(int dt) { return dt == FERRITE_F32 || dt == FERRITE_BF16; }
inline const char* dtype_name(int dt) { return dt == FERRITE_F32 ? "f32" : dt == FERRITE_BF16 ? "bf16" : "?"; }

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ferrite
