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

// Q fragment of one 32-row block (B operand of S^T): lane (c32, hh) holds
// Q[row][16s + 8hh + 0..7] with the per-head RMSNorm and split-half RoPE fused.
// issue_q_loads starts the loads of the raw rows, of the norm weight and of the RoPE
// table rows (so a caller can put other loads in flight behind them); finish_q_fragment
// waits for them, applies the norm and the RoPE, then multiplies by qmul before the
// one fp16 rounding (a kernel that folds the softmax scale into Q passes it here).
//
// All workgroups of a launch run this at once, and the vector memory path (about 32
// bytes per cycle per CU for 16-byte loads) is what limits it, so the loads move as
// few bytes as they can and the data that lanes share goes through LDS:
//  * the Q rows: a fragment load would have the 64 lanes of an instruction touch 32
//    rows with 32 bytes each (about 16 bytes per cycle per CU for that pattern), so
//    each instruction loads whole row pieces (D/8 lanes per row) into a register,
//    which goes to LDS rows of QPITCH bytes and back as the lane's fragment;
//  * the norm weight ([D] fp16, the same for every lane) is one 4-byte piece per lane,
//    written to LDS and read back as the 16-byte pieces each lane needs;
//  * of each [cos, -sin, sin, cos] table block only (cos, -sin) is loaded (8 bytes);
//    lane (c32, hh) needs blocks 16s + 8hh + i (s < D/32, i < 8) of the table row of
//    its query row, which per-lane loads would fetch as 64 different 128-byte lines
//    per instruction.  Instead the wave loads its 32 rows coalesced (one row piece of
//    D/2 blocks per D/2 lanes), writes them to LDS rows of PITCH bytes (the 16-byte
//    pad puts 16 consecutive rows on distinct banks) and each lane reads its blocks
//    two at a time.
// The wave's LDS region (QStage<D>::BYTES) is private to it; the caller must not reuse
// it for other data before every wave of the workgroup is past finish_q_fragment.
//
// STAGED = false is for a caller that has loaded qf in the fragment layout itself (at a
// time when the vector memory path is not the limit) and keeps the norm weight in LDS:
// region is then the wave's copy of the weight (D halfs), and only the norm runs.
template <int D>
struct QStage {
  static constexpr int E = D / 2;                 // table blocks per row
  static constexpr int PITCH = E * 8 + 16;        // LDS row pitch (bytes)
  static constexpr int LOADS = E / 2;             // 8-byte loads per lane (64 / E rows per load)
  static constexpr int WN = 32 * PITCH;           // offset of the norm weight copy
  static constexpr int BYTES = WN + D * 2;        // LDS bytes per wave
  static constexpr int QPITCH = D * 2 + 16;       // LDS row pitch of the Q rows (reuses offset 0)
  static constexpr int QLPR = D / 8;              // lanes per Q row in one load
  static_assert(E <= 64 && 64 % E == 0 && E % 16 == 0, "whole rows per load");
  static_assert(32 * QPITCH <= WN && 64 % QLPR == 0, "Q rows fit before the norm weight");
};

// ROPE = false compiles the RoPE table out (for kernels that never take one).
template <int D, bool ROPE = true>
__device__ __forceinline__ void issue_q_loads(const FlashParams& p, int b, int head, int hh, int wq0,
                                              int lane, half8v (&qf)[D / 16], uint32_t& wn,
                                              uint64_t (&rp)[QStage<D>::LOADS]) {
  using R = QStage<D>;
  constexpr int QS = D / 16;
  // Q rows: load t moves rows t * 64/QLPR + lane/QLPR, chunk lane % QLPR (rows past the
  // sequence repeat the last row); finish_q_fragment turns them into the fragment.
  const half_t* qp = p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + 8 * (lane % R::QLPR);
#pragma unroll
  for (int t = 0; t < QS; ++t) {
    const int row = wq0 + t * (64 / R::QLPR) + lane / R::QLPR;
    qf[t] = *reinterpret_cast<const half8v*>(qp + (int64_t)(row < p.Sq ? row : p.Sq - 1) * p.q_tok);
  }
  if (p.q_norm_w && lane < D / 2) wn = *reinterpret_cast<const uint32_t*>(p.q_norm_w + 2 * lane);
  if (ROPE && p.rope) {
    const char* tab = reinterpret_cast<const char*>(p.rope);
#pragma unroll
    for (int t = 0; t < R::LOADS; ++t) {
      const int row = t * (64 / R::E) + lane / R::E;
      const int rrow = wq0 + row < p.Sq ? wq0 + row : p.Sq - 1;
      rp[t] = *reinterpret_cast<const uint64_t*>(tab + (int64_t)rrow * (8 * D) + (lane % R::E) * 16);
    }
  }
}

template <int D, bool ROPE = true, bool STAGED = true>
__device__ __forceinline__ void finish_q_fragment(const FlashParams& p, int hh, int lane, half8v (&qf)[D / 16],
                                                  uint32_t wn, const uint64_t (&rp)[QStage<D>::LOADS],
                                                  __attribute__((address_space(3))) char* region,
                                                  float qmul = 1.f) {
  constexpr int QS = D / 16;
  using R = QStage<D>;
  typedef __attribute__((address_space(3))) uint64_t lds_u64;
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  typedef __attribute__((address_space(3))) half8v lds_half8v;
  typedef __attribute__((address_space(3))) floatx4 lds_floatx4;
  static_assert(STAGED || !ROPE, "the RoPE table is staged with the Q rows");
  constexpr int WOFF = STAGED ? R::WN : 0;   // offset of the norm weight copy in region
  if constexpr (STAGED) {
    // Q rows to LDS and back as the fragment (lane (c32, hh): row c32, columns 16s + 8hh ..).
#pragma unroll
    for (int t = 0; t < QS; ++t)
      *(lds_half8v*)(region + (t * (64 / R::QLPR) + lane / R::QLPR) * R::QPITCH + (lane % R::QLPR) * 16) = qf[t];
    const int c32 = lane & 31;
#pragma unroll
    for (int s = 0; s < QS; ++s) qf[s] = *(const lds_half8v*)(region + c32 * R::QPITCH + (16 * s + 8 * hh) * 2);
    if (p.q_norm_w && lane < D / 2) *(lds_u32*)(region + R::WN + 4 * lane) = wn;
  }
  if (ROPE && p.rope) {
#pragma unroll
    for (int t = 0; t < R::LOADS; ++t)
      *(lds_u64*)(region + (t * (64 / R::E) + lane / R::E) * R::PITCH + (lane % R::E) * 8) = rp[t];
  }
  if (p.q_norm_w || (ROPE && p.rope) || qmul != 1.f) {
    // x = q * w (v_fma_mix: the fp16 operands enter the fp32 FMA unconverted, and the
    // product of two fp16 values is exact in fp32), or q itself without a norm; the
    // norm factor and qmul join into one fp32 factor g applied once per element (to
    // the rotation coefficients with RoPE).  Each result is rounded to fp32 and then to
    // fp16 (f32_to_f16 keeps the compiler from fusing the last product and the
    // conversion into one v_fma_mix*_f16 rounding, which it does or not depending on
    // the surrounding kernel), so every kernel gets the same bits.
    float g = qmul;
    float x[QS][8];
    if (p.q_norm_w) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf((float)qf[s][i], (float)qf[s][i], ss);
      ss = xlane32_sum(ss);
      g *= rsqrtf(ss / (float)D + p.eps);
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        const half8v w = *(const lds_half8v*)(region + WOFF + (16 * s + 8 * hh) * 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[s][i] = fmaf((float)qf[s][i], (float)w[i], 0.f);
      }
    } else {
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[s][i] = (float)qf[s][i];
    }
    if (ROPE && p.rope) {
      const int c32 = lane & 31;
#pragma unroll
      for (int s = 0; s < QS / 2; ++s)
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          // blocks 16s + 8hh + i and + i + 1: (cos, -sin) each
          const floatx4 cs = *(const lds_floatx4*)(region + c32 * R::PITCH + (16 * s + 8 * hh + i) * 8);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const float c = cs[2 * u] * g, ns = cs[2 * u + 1] * g;
            const float a = x[s][i + u], bb = x[s + QS / 2][i + u];
            qf[s][i + u] = f32_to_f16(c * a + ns * bb);
            qf[s + QS / 2][i + u] = f32_to_f16(c * bb - ns * a);
          }
        }
    } else if (p.q_norm_w) {
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[s][i] = f32_to_f16(x[s][i] * g);
    } else {
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[s][i] = f32_to_f16(fmaf((float)qf[s][i], g, 0.f));
    }
  }
}

}  // namespace anima
