// Shared host/device definitions for libanima_hip (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#include "anima_hip.h"
#include "status.hpp"

namespace anima {

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Validation failures throw Error (status.hpp) with the status code the C ABI
// returns; messages follow the reference's AnimapkError.validation strings where
// one exists (AttentionExecutor.swift:778-847, LinearExecutor.swift:412-459).
inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(ANIMA_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define ANIMA_HIP(call) ::anima::hip_check((call), #call)

// Overflow-checked products / ends (checkedProduct / checkedEnd of the reference).
inline int64_t checked_mul(int64_t a, int64_t b, const char* what) {
  int64_t r;
  if (__builtin_mul_overflow(a, b, &r)) fail(ANIMA_E_OVERFLOW, std::string(what) + " byte size overflow");
  return r;
}
inline int64_t checked_product(std::initializer_list<int64_t> v, const char* what) {
  int64_t r = 1;
  for (int64_t x : v) r = checked_mul(r, x, what);
  return r;
}
inline int64_t checked_end(int64_t off, int64_t bytes, const char* what) {
  int64_t r;
  if (__builtin_add_overflow(off, bytes, &r)) fail(ANIMA_E_OVERFLOW, std::string(what) + " buffer range overflow");
  return r;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

inline const char* byte_ptr(const anima_buffer& b, int64_t off) {
  return static_cast<const char*>(b.ptr) + off;
}
inline char* byte_ptr_mut(const anima_buffer& b, int64_t off) { return static_cast<char*>(b.ptr) + off; }

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ floatx16 mfma32(half8v a, half8v b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16(half8v a, half8v b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// fp32 -> fp16 with the reference's double rounding: the fp32 result is
// materialised first (an empty asm register barrier), then converted with RNE.
// Without the barrier the compiler folds the producing FMA and the conversion
// into v_fma_mix{lo,hi}_f16, a single rounding that differs from
// Float16(Float(x)) at fp16 ties.
__device__ __forceinline__ half_t f32_to_f16(float v) {
  asm volatile("" : "+v"(v));
  return (half_t)v;
}

// erf by the Chebyshev fit of erfc in Numerical Recipes (erfcc: for z = |x|,
// t = 1 / (1 + z/2), erfc(z) = t exp(-z^2 + P(t)) with a degree-9 P, fractional
// error below 1.2e-7), the form of the reference's erf_f32
// (AnimaKernels.metal:252-272); the coefficients are the published table.  The
// reciprocal and the exponential are the hardware's v_rcp_f32 and v_exp_f32
// (1 ulp each): branch-free, about 20 VALU operations.
__device__ __forceinline__ float erf_nr(float x) {
  const float z = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  const float erfc = t * __builtin_amdgcn_exp2f(fmaf(-z, z, p) * 1.4426950408889634f);
  return copysignf(1.0f - erfc, x);
}

// Exact-erf GELU of an fp16 value, rounded once more to fp16
// (dit_gelu_half_inplace, AnimaKernels.metal:312-322).
__device__ __forceinline__ half_t gelu_erf_half(half_t h) {
  const float x = (float)h;
  return f32_to_f16(0.5f * x * (1.0f + erf_nr(x * 0.7071067811865475f)));
}

// SiLU in fp32 (silu, AnimaKernels.metal:388-397).
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// s_waitcnt vmcnt(n) alone (expcnt / lgkmcnt unconstrained), n in [0, 15].
template <int N>
__device__ __forceinline__ void wait_vmcnt_imm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8));
}

// 16-byte load through a raw buffer descriptor of n bytes at base: offsets at or
// past n read zeros without touching memory.  (The descriptor type exists in the
// device pass only.)
// soff is a wave-uniform byte offset added to every lane's voff.
__device__ __forceinline__ u32x4 load16_bounded(const void* base, int n, uint32_t voff, int soff = 0) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
#else
  return u32x4{};
#endif
}

// 16-byte store through a raw buffer descriptor of n bytes at base: stores at offsets
// at or past n are dropped.  No branch guards it, so the compiler's count of vector
// memory operations in flight does not fork at each store.
__device__ __forceinline__ void store16_bounded(void* base, int n, uint32_t voff, u32x4 v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, (short)0, n, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, 0);
#endif
}

// 2-byte variant of load16_bounded (zero-extended).
__device__ __forceinline__ uint32_t load2_bounded(const void* base, int n, uint32_t voff, int soff = 0) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
#else
  return 0u;
#endif
}

// Workgroup id remapped so that consecutive logical ids share an XCD: the
// dispatcher places workgroup i on XCD i % 8, so logical id L is given to
// physical id (L % per) * 8 + L / per when the grid is a multiple of 8.
__device__ __forceinline__ int xcd_logical_block(int bid, int nblk) {
  if ((nblk & 7) != 0) return bid;
  int per = nblk >> 3;
  return (bid & 7) * per + (bid >> 3);
}

}  // namespace anima
