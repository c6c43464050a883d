// Device helpers shared by the flash attention kernels (attention_v2.hip,
// attention_wide.hip): cross-half reductions of the S^T layout and the Q fragment load
// with the fused per-head RMSNorm and split-half RoPE.
#pragma once

#include "attention.hpp"

namespace anima {

typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float xlane32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xlane32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Q fragment of one 32-row block (B operand of S^T): lane holds
// Q[row][16s + 8h + 0..7] with the per-head RMSNorm and split-half RoPE fused.
// issue_q_loads starts the loads of the raw row and of the norm weight (so a caller
// can put other loads in flight beside them); finish_q_fragment waits for them and
// applies the norm and the RoPE (whose table rows it loads itself).
template <int D>
__device__ __forceinline__ void issue_q_loads(const FlashParams& p, int b, int head, int qi, int hh,
                                              half8v (&qf)[D / 16], half8v (&wn)[D / 16]) {
  constexpr int QS = D / 16;
  const int qrow = qi < p.Sq ? qi : p.Sq - 1;
  const half_t* qp = p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + (int64_t)qrow * p.q_tok;
#pragma unroll
  for (int s = 0; s < QS; ++s) qf[s] = *reinterpret_cast<const half8v*>(qp + 16 * s + 8 * hh);
  if (p.q_norm_w) {
#pragma unroll
    for (int s = 0; s < QS; ++s) wn[s] = *reinterpret_cast<const half8v*>(p.q_norm_w + 16 * s + 8 * hh);
  }
}

template <int D>
__device__ __forceinline__ void finish_q_fragment(const FlashParams& p, int qi, int hh, half8v (&qf)[D / 16],
                                                  const half8v (&wn)[D / 16]) {
  constexpr int QS = D / 16;
  if (p.q_norm_w || p.rope) {
    const int qrow = qi < p.Sq ? qi : p.Sq - 1;
    float x[QS][8];
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) x[s][i] = (float)qf[s][i];
    if (p.q_norm_w) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(x[s][i], x[s][i], ss);
      ss = xlane32_sum(ss);
      const float inv = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[s][i] = x[s][i] * inv * (float)wn[s][i];
    }
    if (p.rope) {
      const float* rr = p.rope + (int64_t)qrow * (D / 2) * 4;
#pragma unroll
      for (int s = 0; s < QS / 2; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const floatx4 blk = *reinterpret_cast<const floatx4*>(rr + (16 * s + 8 * hh + i) * 4);
          const float a = x[s][i], bb = x[s + QS / 2][i];
          x[s][i] = blk[0] * a + blk[1] * bb;
          x[s + QS / 2][i] = blk[2] * a + blk[0] * bb;
        }
    }
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[s][i] = f32_to_f16(x[s][i]);
  }
}

template <int D>
__device__ __forceinline__ void load_q_fragment(const FlashParams& p, int b, int head, int qi, int hh,
                                                half8v (&qf)[D / 16]) {
  half8v wn[D / 16];
  issue_q_loads<D>(p, b, head, qi, hh, qf, wn);
  finish_q_fragment<D>(p, qi, hh, qf, wn);
}

}  // namespace anima
