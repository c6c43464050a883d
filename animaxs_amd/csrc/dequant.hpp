// Device-side dequantisation of packed W4/W8 weights into MFMA operand
// fragments, shared by the tiled GEMM kernels.  Every path reproduces the
// reference decoder's half(fl32(q*scale + zero)) bit for bit (see
// one_rounding_exact in linear.hpp for when one fp16 rounding gives the same
// bits).
#pragma once

#include "linear.hpp"

namespace anima {

// 8 W4 codes of one 32-bit word (k = 0..7, even k in the low nibble) -> fp16 in
// the order k = 0,4,1,5,2,6,3,7, one rounding (caller checked exactness), in two
// halves: part 0 gives k = 0,4,1,5 from the low nibbles of bytes 0 and 2 and the
// high nibbles; part 1 the same from the word shifted right by 8 (k = 2,6,3,7).
// The masks and the 0x6400 pattern come in registers (k = {0x000F000F,
// 0x00F000F0, 0x64006400}) so that each mask-and-set is one v_and_or_b32.
__device__ __forceinline__ half4v w4_half_one_rounding(uint32_t x, half2v s2, half2v z2, const uint32_t (&k)[3]) {
  const half2v c1024 = {(half_t)1024.f, (half_t)1024.f};
  const half2v sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
  const half2v m64 = {(half_t)-64.f, (half_t)-64.f};
  // 0x6400 | q is the fp16 value 1024 + q; (1024 + 16q)/16 - 64 = q exactly.
  const half2v qa = __builtin_bit_cast(half2v, (x & k[0]) | k[2]) - c1024;
  const half2v qb = __builtin_elementwise_fma(__builtin_bit_cast(half2v, (x & k[1]) | k[2]), sixteenth, m64);
  const half2v wa = __builtin_elementwise_fma(qa, s2, z2);
  const half2v wb = __builtin_elementwise_fma(qb, s2, z2);
  return half4v{wa[0], wa[1], wb[0], wb[1]};
}

// Same codes and order, reference rounding: half(fl32(q*s + z)).
__device__ __forceinline__ half8v w4_frag_exact(uint32_t x, float s, float z) {
  const uint32_t lo = x & 0x0F0F0F0Fu;          // bytes: k = 0, 2, 4, 6
  const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;   // bytes: k = 1, 3, 5, 7
  auto d = [&](uint32_t v, int b) __attribute__((always_inline)) {
    return f32_to_f16(fmaf((float)((v >> (8 * b)) & 0xFFu), s, z));
  };
  return half8v{d(lo, 0), d(lo, 2), d(hi, 0), d(hi, 2), d(lo, 1), d(lo, 3), d(hi, 1), d(hi, 3)};
}

// 4 W8 codes of one word (k = 0..3) -> fp16 in k order, one rounding.
__device__ __forceinline__ half4v w8_half_one_rounding(uint32_t x, half2v s2, half2v z2) {
  const half2v c1024 = {(half_t)1024.f, (half_t)1024.f};
  // v_perm: (byte b, 0x64, byte b+1, 0x64) = fp16 pair (1024 + q_b, 1024 + q_{b+1}).
  auto pair = [&](uint32_t sel) __attribute__((always_inline)) {
    const half2v q = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, sel)) - c1024;
    return __builtin_elementwise_fma(q, s2, z2);
  };
  const half2v a = pair(0x04010400u), b = pair(0x04030402u);
  return half4v{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ half8v w8_frag_exact(uint32_t x0, uint32_t x1, float s, float z) {
  auto d = [&](uint32_t v, int b) __attribute__((always_inline)) {
    return f32_to_f16(fmaf((float)((v >> (8 * b)) & 0xFFu), s, z));
  };
  return half8v{d(x0, 0), d(x0, 1), d(x0, 2), d(x0, 3), d(x1, 0), d(x1, 1), d(x1, 2), d(x1, 3)};
}

// 8 consecutive fp16 X values (x0..x7) -> the order x0,x4,x1,x5,x2,x6,x3,x7.
__device__ __forceinline__ u32x4 interleave_w4_order(u32x4 d) {
  return u32x4{__builtin_amdgcn_perm(d[2], d[0], 0x05040100u), __builtin_amdgcn_perm(d[2], d[0], 0x07060302u),
               __builtin_amdgcn_perm(d[3], d[1], 0x05040100u), __builtin_amdgcn_perm(d[3], d[1], 0x07060302u)};
}

}  // namespace anima
