// Attention for gfx950: MFMA flash kernel (head_dim 64/128), generic fp32 kernel
// (any head_dim <= 512) and the per-head RMSNorm + split-half RoPE prologue.
//
// Replaces the reference's AttentionExecutor backends
// (AnimaXS/Runtime/Metal/AttentionExecutor.swift:122-733) and the Metal kernels
// attention_softmax_rows, attention_*_f32, streaming_*, dit_flash_attention_h128_*,
// rms_rope_split_half and rmsnorm_heads_half (AnimaXS/Shaders/AnimaKernels.metal:
// 660-729, 1051-1185, 2069-2427).  Maths: O = softmax(scale * Q K^T + mask) V per
// head, kv head = h / (heads / kv_heads) (AttentionExecutor.swift:222).
#include <algorithm>
#include <cmath>
#include <vector>

#include "attention.hpp"

namespace anima {

// ===========================================================================
// Flash kernel.
//
// One workgroup = 4 waves = 128 query rows of one (batch, head); each wave owns
// 32 rows.  Per 64-key tile a wave computes S^T = K Q^T with two 32x32 tiles of
// v_mfma_f32_32x32x16_f16 (keys on M, queries on N), so every lane holds 32
// scores of ONE query row (lane%32) and the row max needs a single exchange with
// lane^32.  P^T stays in registers and is the B operand of O^T += V^T P^T: the
// C-operand layout of S^T maps register j of lane (n, h) to key
// 32t + 8(j/4) + 4h + j%4, which is a valid K-slot order for the next MFMA as
// long as the A operand (V^T, read from a transposed LDS tile) uses the same key
// permutation.  Online softmax in base 2 with the scale folded into one FMA; the
// running max is only raised when it grows by more than 2^8 (P stays <= 256,
// exact maths, far fewer O rescales).  K/V tiles are double-buffered in LDS with
// XOR swizzles, the next tile's global loads are issued before the current
// tile's MFMAs.
// ===========================================================================
constexpr int FA_BM = 128;
constexpr int FA_BN = 64;
constexpr int FA_NT = 256;
constexpr float FA_RESCALE_THRESHOLD = 8.0f;

__device__ __forceinline__ int vt_swz(int d) { return ((d & 15) + (d >> 4)) & 15; }

template <int D>
__global__ __launch_bounds__(FA_NT, 2) void flash_attention_kernel(FlashParams p) {
  constexpr int DCH = D / 8;                       // 16-byte chunks per K row
  constexpr int QS = D / 16;                       // k-steps of S^T = K Q^T
  constexpr int OB = D / 32;                       // 32-row blocks of O^T
  constexpr int KQ = FA_BN / 4;                    // key quads per tile
  constexpr int KLOADS = (FA_BN * DCH) / FA_NT;    // 16-byte K loads per thread
  constexpr int VBLOCKS = KQ * DCH;                // 4x8 V blocks per tile
  static_assert(KLOADS >= 1 && VBLOCKS <= FA_NT, "tile shape");

  __shared__ __attribute__((aligned(16))) half_t Ks[2][FA_BN * D];
  __shared__ __attribute__((aligned(16))) half_t Vt[2][D * FA_BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c32 = lane & 31, hh = lane >> 5;

  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  // Heads vary slowest (as in the 256-row kernel): each XCD's range of logical blocks
  // is whole heads over every batch entry.
  const int qt = lb % p.q_tiles;
  lb /= p.q_tiles;
  const int b = lb % p.nbatch;
  const int head = lb / p.nbatch;
  const int kvh = head / p.group;
  const int q0 = qt * FA_BM;
  const int qi = q0 + wave * 32 + c32;
  const int wave_row0 = q0 + wave * 32;

  int kv_len = p.Sk;
  if (p.key_lengths_dev) {
    int L = p.key_lengths_dev[b];
    kv_len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
  } else if (p.use_host_lengths) {
    kv_len = p.host_lengths[b];
  }
  int kend = kv_len;
  if (p.causal) kend = min(kend, q0 + FA_BM);
  const int ntiles = (kend + FA_BN - 1) / FA_BN;

  const half_t* kbase = p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head;
  const half_t* vbase = p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head;

  // ---- Q fragment (B operand of S^T): lane holds Q[qi][16s + 8h + 0..7] ----
  half8v qf[QS];
  {
    const int qrow = qi < p.Sq ? qi : p.Sq - 1;
    const half_t* qp = p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + (int64_t)qrow * p.q_tok;
#pragma unroll
    for (int s = 0; s < QS; ++s) qf[s] = *reinterpret_cast<const half8v*>(qp + 16 * s + 8 * hh);
    if (p.q_norm_w || p.rope) {
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
        ss += __shfl_xor(ss, 32);
        const float inv = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
        for (int s = 0; s < QS; ++s) {
          const half8v w = *reinterpret_cast<const half8v*>(p.q_norm_w + 16 * s + 8 * hh);
#pragma unroll
          for (int i = 0; i < 8; ++i) x[s][i] = x[s][i] * inv * (float)w[i];
        }
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

  // ---- K/V tile staging ----
  half8v kreg[KLOADS];
  half8v vreg[4];
  const half8v zero8 = {};
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int r = 0; r < KLOADS; ++r) {
      const int c = tid + FA_NT * r;
      const int key = c / DCH, ch = c % DCH;
      const int kg = k0 + key;
      kreg[r] = kg < p.Sk ? *reinterpret_cast<const half8v*>(kbase + (int64_t)kg * p.k_tok + ch * 8) : zero8;
    }
    if (tid < VBLOCKS) {
      const int dch = tid % DCH, kq = tid / DCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kg = k0 + 4 * kq + r;
        vreg[r] = kg < p.Sk ? *reinterpret_cast<const half8v*>(vbase + (int64_t)kg * p.v_tok + dch * 8) : zero8;
      }
    }
  };
  auto store_tile = [&](int st) {
#pragma unroll
    for (int r = 0; r < KLOADS; ++r) {
      const int c = tid + FA_NT * r;
      const int key = c / DCH, ch = c % DCH;
      *reinterpret_cast<half8v*>(&Ks[st][key * D + ((ch ^ (key & (DCH - 1))) * 8)]) = kreg[r];
    }
    if (tid < VBLOCKS) {
      const int dch = tid % DCH, kq = tid / DCH;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = dch * 8 + e;
        half4v val = {vreg[0][e], vreg[1][e], vreg[2][e], vreg[3][e]};
        *reinterpret_cast<half4v*>(&Vt[st][d * FA_BN + ((kq ^ vt_swz(d)) * 4)]) = val;
      }
    }
  };

  floatx16 accO[OB];
#pragma unroll
  for (int c = 0; c < OB; ++c) accO[c] = floatx16{};
  float m_run = -INFINITY, l_run = 0.f;

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int st = it & 1;
    const int k0 = it * FA_BN;
    if (it + 1 < ntiles) load_tile(k0 + FA_BN);

    const bool skip = p.causal && (k0 > wave_row0 + 31);
    if (!skip) {
      floatx16 sacc[2] = {floatx16{}, floatx16{}};
#pragma unroll
      for (int s = 0; s < QS; ++s) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int key = 32 * t + c32;
          const half8v a = *reinterpret_cast<const half8v*>(&Ks[st][key * D + (((2 * s + hh) ^ (key & (DCH - 1))) * 8)]);
          sacc[t] = mfma32(a, qf[s], sacc[t]);
        }
      }
      const bool need_mask = (k0 + FA_BN > kv_len) || (p.causal && k0 + FA_BN - 1 > wave_row0);
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int kidx = k0 + 32 * t + (j >> 2) * 8 + 4 * hh + (j & 3);
            if (kidx >= kv_len || (p.causal && kidx > qi)) sacc[t][j] = -INFINITY;
          }
      }
      float mloc = sacc[0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, sacc[t][j]);
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float cand = mloc * p.scale_log2;
      if (__any(cand > m_run + FA_RESCALE_THRESHOLD)) {
        const float mnew = fmaxf(m_run, cand);
        const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m_run - mnew);
        l_run *= alpha;
#pragma unroll
        for (int c = 0; c < OB; ++c) accO[c] *= alpha;
        m_run = mnew;
      }
      const float msub = (m_run == -INFINITY) ? 0.f : m_run;
      half8v pb[4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float pv = fast_exp2(fmaf(sacc[t][j], p.scale_log2, -msub));
          l_run += pv;
          pb[2 * t + (j >> 3)][j & 7] = (half_t)pv;
        }
#pragma unroll
      for (int c = 0; c < OB; ++c) {
        const int d = 32 * c + c32;
        const int f = vt_swz(d);
        const half_t* vrow = &Vt[st][d * FA_BN];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const half4v lo = *reinterpret_cast<const half4v*>(vrow + (((4 * u + hh) ^ f) * 4));
          const half4v hi = *reinterpret_cast<const half4v*>(vrow + (((4 * u + 2 + hh) ^ f) * 4));
          const half8v a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          accO[c] = mfma32(a, pb[u], accO[c]);
        }
      }
    }
    if (it + 1 < ntiles) store_tile(st ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qi < p.Sq) {
    half_t* op = p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head + (int64_t)qi * p.o_tok;
#pragma unroll
    for (int c = 0; c < OB; ++c)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        half4v val = {(half_t)(accO[c][4 * jj + 0] * inv), (half_t)(accO[c][4 * jj + 1] * inv),
                      (half_t)(accO[c][4 * jj + 2] * inv), (half_t)(accO[c][4 * jj + 3] * inv)};
        *reinterpret_cast<half4v*>(op + 32 * c + 8 * jj + 4 * hh) = val;
      }
  }
}

// ===========================================================================
// Generic kernel: one 64-lane workgroup per (batch, head, query row), fp32
// scores / online softmax / accumulation, any head_dim <= 512 and any
// alignment.  The diagnostic fp32 path (encodeFP32, AttentionExecutor.swift:
// 325-405) re-cut as a single fused kernel.
// ===========================================================================
constexpr int GEN_MAX_D = 512;

__global__ __launch_bounds__(64) void generic_attention_kernel(FlashParams p, int D) {
  __shared__ float qs[GEN_MAX_D];
  __shared__ float ps[64];
  const int lane = threadIdx.x;
  const int qi = blockIdx.x;
  const int head = blockIdx.y % p.H;
  const int b = blockIdx.y / p.H;
  const int kvh = head / p.group;

  int kv_len = p.Sk;
  if (p.key_lengths_dev) {
    int L = p.key_lengths_dev[b];
    kv_len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
  } else if (p.use_host_lengths) {
    kv_len = p.host_lengths[b];
  }
  int kend = kv_len;
  if (p.causal) kend = min(kend, qi + 1);

  const half_t* qp = p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + (int64_t)qi * p.q_tok;
  for (int d = lane; d < D; d += 64) qs[d] = (float)qp[d];
  __syncthreads();

  const half_t* kb = p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head;
  const half_t* vb = p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head;
  constexpr int EMAX = GEN_MAX_D / 64;
  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) acc[e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int j = k0 + lane;
    float s = -INFINITY;
    if (j < kend) {
      const half_t* kr = kb + (int64_t)j * p.k_tok;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(qs[d], (float)kr[d], dot);
      s = dot * p.scale_log2;
    }
    float mc = s;
    for (int off = 32; off > 0; off >>= 1) mc = fmaxf(mc, __shfl_xor(mc, off));
    const float mnew = fmaxf(m_run, mc);
    const float alpha = (m_run == -INFINITY) ? 0.f : exp2f(m_run - mnew);
    const float pj = (s == -INFINITY) ? 0.f : exp2f(s - mnew);
    float psum = pj;
    for (int off = 32; off > 0; off >>= 1) psum += __shfl_xor(psum, off);
    l_run = l_run * alpha + psum;
    m_run = mnew;
    ps[lane] = pj;
    __syncthreads();
    const int cnt = min(64, kend - k0);
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      const int d = lane + 64 * e;
      if (d < D) {
        float a = acc[e] * alpha;
        for (int jj = 0; jj < cnt; ++jj) a = fmaf(ps[jj], (float)vb[(int64_t)(k0 + jj) * p.v_tok + d], a);
        acc[e] = a;
      }
    }
    __syncthreads();
  }
  half_t* op = p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head + (int64_t)qi * p.o_tok;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int d = lane + 64 * e;
    if (d < D) op[d] = f32_to_f16(acc[e] * inv);
  }
}

// ===========================================================================
// MPS-rounding kernel: the reference's score-tile backends (legacyHeadMajorMPS,
// stridedTokenMajorMPS; AttentionExecutor.swift:221-301, 412-496) under legacy
// numerics store the scaled scores as fp16 (MPSMatrixMultiplication with
// alpha = scale into an fp16 matrix), take the row max, exp and sum in fp32, store
// the normalised probabilities as fp16 (attention_softmax_rows,
// AnimaKernels.metal:1051-1100), then multiply them with V in fp32 into an fp16
// output.  This kernel keeps exactly those rounding points: one 64-lane workgroup
// per (batch, head, query row), lane j of a pass owning key k0 + j; the three
// passes (max, sum, probabilities and PV) recompute the same fp16 scores instead
// of storing a score tile.
// ===========================================================================
__device__ __forceinline__ float legacy_score(const float* qs, const half_t* kr, int D, float scale) {
  float dot = 0.f;
  for (int d = 0; d < D; ++d) dot = fmaf(qs[d], (float)kr[d], dot);
  return (float)f32_to_f16(dot * scale);
}

__global__ __launch_bounds__(64) void legacy_mps_attention_kernel(FlashParams p, int D) {
  __shared__ float qs[GEN_MAX_D];
  __shared__ float ps[64];
  const int lane = threadIdx.x;
  const int qi = blockIdx.x;
  const int head = blockIdx.y % p.H;
  const int b = blockIdx.y / p.H;
  const int kvh = head / p.group;

  int kv_len = p.Sk;
  if (p.key_lengths_dev) {
    int L = p.key_lengths_dev[b];
    kv_len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
  } else if (p.use_host_lengths) {
    kv_len = p.host_lengths[b];
  }
  int kend = kv_len;
  if (p.causal) kend = min(kend, qi + 1);

  const half_t* qp = p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + (int64_t)qi * p.q_tok;
  for (int d = lane; d < D; d += 64) qs[d] = (float)qp[d];
  __syncthreads();
  const half_t* kb = p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head;
  const half_t* vb = p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head;

  // pass 1: row max of the fp16 scores
  float m = -INFINITY;
  for (int j = lane; j < kend; j += 64) m = fmaxf(m, legacy_score(qs, kb + (int64_t)j * p.k_tok, D, p.scale));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  // pass 2: fp32 sum of exp(s - max)
  float l = 0.f;
  for (int j = lane; j < kend; j += 64) l += expf(legacy_score(qs, kb + (int64_t)j * p.k_tok, D, p.scale) - m);
  for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
  const float inv = 1.f / l;
  // pass 3: fp16 probabilities, fp32 PV
  constexpr int EMAX = GEN_MAX_D / 64;
  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) acc[e] = 0.f;
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int j = k0 + lane;
    float pj = 0.f;
    if (j < kend)
      pj = (float)f32_to_f16(expf(legacy_score(qs, kb + (int64_t)j * p.k_tok, D, p.scale) - m) * inv);
    ps[lane] = pj;
    __syncthreads();
    const int cnt = min(64, kend - k0);
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      const int d = lane + 64 * e;
      if (d < D) {
        float a = acc[e];
        for (int jj = 0; jj < cnt; ++jj) a = fmaf(ps[jj], (float)vb[(int64_t)(k0 + jj) * p.v_tok + d], a);
        acc[e] = a;
      }
    }
    __syncthreads();
  }
  half_t* op = p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head + (int64_t)qi * p.o_tok;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int d = lane + 64 * e;
    if (d < D) op[d] = f32_to_f16(acc[e]);
  }
}

// ===========================================================================
// Q/K prologue: per-(batch, token, head) RMSNorm with a shared [D] weight and
// optional split-half RoPE, fp32 maths, fp16 dense head-major output
// [batch][heads][rows][D].  One wave per row; lane p owns the pairs
// (p + 64e, p + 64e + D/2) (the pairing of rms_rope_split_half,
// AnimaKernels.metal:696-729; without RoPE rmsnorm_heads_half, :660-689).
// ===========================================================================
__global__ __launch_bounds__(256) void qk_prologue_kernel(PrologueParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t total = (int64_t)p.batch * p.rows * p.heads;
  if (row >= total) return;
  const int h = (int)(row % p.heads);
  const int64_t t = (row / p.heads) % p.rows;
  const int b = (int)(row / ((int64_t)p.heads * p.rows));
  const half_t* x = p.in + (int64_t)b * p.in_batch + t * p.in_tok + (int64_t)h * p.in_head;
  half_t* y = p.out + (int64_t)b * p.out_batch + t * p.out_tok + (int64_t)h * p.out_head;
  const int half = p.D / 2;
  constexpr int EMAX = GEN_MAX_D / 128;  // pairs per lane
  float a[EMAX], c[EMAX];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int i = lane + 64 * e;
    a[e] = 0.f;
    c[e] = 0.f;
    if (i < half) {
      a[e] = (float)x[i];
      c[e] = (float)x[i + half];
      ss = fmaf(a[e], a[e], fmaf(c[e], c[e], ss));
    }
  }
  // odd head_dim: the middle element has no RoPE partner
  float mid = 0.f;
  const bool odd = (p.D & 1) != 0;
  if (odd && lane == 0) {
    mid = (float)x[p.D - 1];
    ss = fmaf(mid, mid, ss);
  }
  float inv = 1.f;
  if (p.norm_w) {
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    inv = rsqrtf(ss / (float)p.D + p.eps);
  }
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int i = lane + 64 * e;
    if (i < half) {
      float va = a[e], vc = c[e];
      if (p.norm_w) {
        va = va * inv * (float)p.norm_w[i];
        vc = vc * inv * (float)p.norm_w[i + half];
      }
      if (p.rope) {
        const float* blk = p.rope + (t * half + i) * 4;
        const float cs = blk[0], ns = blk[1], sn = blk[2];
        const float ra = cs * va + ns * vc;
        const float rc = sn * va + cs * vc;
        va = ra;
        vc = rc;
      }
      y[i] = f32_to_f16(va);
      y[i + half] = f32_to_f16(vc);
    }
  }
  if (odd && lane == 0) {
    float v = mid;
    if (p.norm_w) v = v * inv * (float)p.norm_w[p.D - 1];
    y[p.D - 1] = f32_to_f16(v);
  }
}

// head_dim 128 fast path: a group of 8 lanes takes HPT heads of one token; lane
// sub holds the pairs (8sub+i, 64+8sub+i), i < 8, of each head as two 16-byte
// loads, so the token's RoPE blocks (eight float4 loads per lane) and the norm
// weights are read once per HPT heads.  The per-head sum of squares needs three
// lane exchanges.  Same arithmetic as the generic kernel (and as the fused Q path
// of the flash kernels).  Every byte is touched once, so the loads and stores are
// nontemporal, and small (128-thread) workgroups spread the one-pass grid evenly:
// 6.5-7 us against 8 us with cached accesses in 256-thread groups at S=4096, H=16.
constexpr int PRO_D128_THREADS = 128;

template <int HPT>
__global__ __launch_bounds__(PRO_D128_THREADS) void qk_prologue_d128_kernel(PrologueParams p) {
  const int sub = threadIdx.x & 7;
  const int groups = p.heads / HPT;
  const int64_t unit = (int64_t)blockIdx.x * (PRO_D128_THREADS / 8) + (threadIdx.x >> 3);
  const int64_t total = (int64_t)p.batch * p.rows * groups;
  const bool live = unit < total;
  const int64_t uu = live ? unit : total - 1;   // tail lanes recompute the last unit, never store
  const int hg = (int)(uu % groups);
  const int64_t t = (uu / groups) % p.rows;
  const int b = (int)(uu / ((int64_t)groups * p.rows));
  float a[HPT][8], c[HPT][8];
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const half_t* x = p.in + (int64_t)b * p.in_batch + t * p.in_tok + (int64_t)(hg * HPT + j) * p.in_head;
    const half8v xa = __builtin_nontemporal_load(reinterpret_cast<const half8v*>(x + 8 * sub));
    const half8v xc = __builtin_nontemporal_load(reinterpret_cast<const half8v*>(x + 64 + 8 * sub));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[j][i] = (float)xa[i];
      c[j][i] = (float)xc[i];
    }
  }
  // The norm weight and the table row go out with the rows (one memory round trip for
  // the thread, not one for the rows and another for the table after the norm).
  half8v wa{}, wc{};
  if (p.norm_w) {
    wa = *reinterpret_cast<const half8v*>(p.norm_w + 8 * sub);
    wc = *reinterpret_cast<const half8v*>(p.norm_w + 64 + 8 * sub);
  }
  floatx4 rrow[8];
  if (p.rope) {
    const floatx4* blk = reinterpret_cast<const floatx4*>(p.rope + (t * 64 + 8 * sub) * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) rrow[i] = blk[i];
  }
  if (p.norm_w) {
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(a[j][i], a[j][i], fmaf(c[j][i], c[j][i], ss));
      ss += __shfl_xor(ss, 1, 8);
      ss += __shfl_xor(ss, 2, 8);
      ss += __shfl_xor(ss, 4, 8);
      const float inv = rsqrtf(ss / 128.f + p.eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        a[j][i] = a[j][i] * inv * (float)wa[i];
        c[j][i] = c[j][i] * inv * (float)wc[i];
      }
    }
  }
  if (p.rope) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const floatx4 r = rrow[i];
#pragma unroll
      for (int j = 0; j < HPT; ++j) {
        const float ra = r[0] * a[j][i] + r[1] * c[j][i];
        const float rc = r[2] * a[j][i] + r[0] * c[j][i];
        a[j][i] = ra;
        c[j][i] = rc;
      }
    }
  }
  if (live) {
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      half8v oa, oc;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        oa[i] = f32_to_f16(a[j][i]);
        oc[i] = f32_to_f16(c[j][i]);
      }
      half_t* y = p.out + (int64_t)b * p.out_batch + t * p.out_tok + (int64_t)(hg * HPT + j) * p.out_head;
      __builtin_nontemporal_store(oa, reinterpret_cast<half8v*>(y + 8 * sub));
      __builtin_nontemporal_store(oc, reinterpret_cast<half8v*>(y + 64 + 8 * sub));
    }
  }
}

// ===========================================================================
// Host launchers.
// ===========================================================================
// Workgroups the key splits aim for: one per compute unit.
constexpr int64_t F2_MIN_BLOCKS = 256;

// Key splits for the 256-row kernel when its query tiles alone cannot cover the chip
// (non-causal, no per-sequence key lengths, automatic row choice): enough splits to
// reach F2_MIN_BLOCKS workgroups, each of at least F2_MIN_SPLIT_KEYS keys.
// 512 rather than 256: at S=1024 (16 heads) two splits of 512 keys run 24.7 us against
// 26.1 us for four of 256 (each split pays a workgroup prologue, partial rows and merge).
constexpr int F2_MIN_SPLIT_KEYS = 512;

int flash_kv_splits(const FlashParams& p, int D, int batch, int flash_rows) {
  if (p.causal || p.key_lengths_dev || p.use_host_lengths) return 1;
  if (D != 128 && D != 64 && D != 384) return 1;
  if (D != 384 && flash_rows != 0) return 1;
  // Query tiles of the kernel that will run: 256 rows (head_dim 64 / 128) or the wide
  // kernel's 128 rows (head_dim 384, which has no other flash kernel).
  const int rows = D == 384 ? FLASH_WIDE_ROWS : FLASH_V2_ROWS;
  const int64_t t256 = (int64_t)((p.Sq + rows - 1) / rows) * p.H * batch;
  if (t256 >= F2_MIN_BLOCKS || t256 <= 0) return 1;
  if (64 * std::max(p.k_tok, p.v_tok) * (int64_t)sizeof(half_t) >= ((int64_t)1 << 31)) return 1;
  int splits = (int)((F2_MIN_BLOCKS + t256 - 1) / t256);
  splits = std::min<int>(splits, FLASH_MAX_SPLITS);
  splits = std::min<int>(splits, p.Sk / F2_MIN_SPLIT_KEYS);
  return splits >= 2 ? splits : 1;
}

// Key-split workspace: the partial rows (rows x D fp16 normalised rows), padded to 256
// bytes, then the fp32 (max, sum) pair of each row.
int64_t flash_split_o_bytes(const FlashParams& p, int D, int batch, int splits) {
  const int64_t rows = checked_product({(int64_t)splits, (int64_t)batch, (int64_t)p.H, (int64_t)p.Sq}, "attention");
  return (checked_product({rows, (int64_t)D, 2}, "attention") + 255) / 256 * 256;
}

int64_t flash_split_bytes(const FlashParams& p, int D, int batch, int splits) {
  const int64_t rows = checked_product({(int64_t)splits, (int64_t)batch, (int64_t)p.H, (int64_t)p.Sq}, "attention");
  return flash_split_o_bytes(p, D, batch, splits) + checked_product({rows, 8}, "attention");
}

// Head dim 384: the wide kernel, 128 query rows per workgroup, keys split when the query
// tiles alone cannot cover the chip.
static void launch_flash_wide_plan(FlashParams p, int D, int batch, hipStream_t stream) {
  p.nbatch = batch;
  if (32 * std::max(p.k_tok, p.v_tok) * (int64_t)sizeof(half_t) >= ((int64_t)1 << 31))
    fail(ANIMA_E_INVALID_SHAPE, "wide flash attention requires 32 key rows to span < 2 GiB");
  p.q_tiles = (p.Sq + FLASH_WIDE_ROWS - 1) / FLASH_WIDE_ROWS;
  const int64_t tiles = (int64_t)p.q_tiles * p.H * batch;
  if (tiles <= 0) return;
  if (p.kv_splits > 1) {
    if (p.kv_splits != flash_kv_splits(p, D, batch, 0) || !p.part_o || !p.part_ml)
      fail(ANIMA_E_INVALID_ARGUMENT, "flash key splits do not match the shape");
    p.nbatch = batch;
    p.kv_chunk = ((p.Sk + p.kv_splits - 1) / p.kv_splits + 63) / 64 * 64;
  } else {
    p.kv_splits = 0;
  }
  const int64_t blocks = tiles * (p.kv_splits > 1 ? p.kv_splits : 1);
  if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "attention grid too large");
  launch_flash_wide(p, D, dim3((unsigned)blocks), stream);
  if (p.kv_splits > 1) launch_flash_combine(p, D, batch, stream);
}

void launch_flash(FlashParams p, int D, int batch, int flash_rows, hipStream_t stream) {
  p.nbatch = batch;   // the kernels map block -> (query tile, batch, head) through it
  if (D == 384) {
    launch_flash_wide_plan(p, D, batch, stream);
    return;
  }
  if (D != 128 && D != 64) fail(ANIMA_E_UNSUPPORTED, "flash attention requires head_dim 64, 128 or 384");
  const int64_t t256 = (int64_t)((p.Sq + FLASH_V2_ROWS - 1) / FLASH_V2_ROWS) * p.H * batch;
  // The 256-row kernel addresses one 64-key tile with 32-bit byte offsets.
  const bool v2_fits = 64 * std::max(p.k_tok, p.v_tok) * (int64_t)sizeof(half_t) < ((int64_t)1 << 31);
  if (flash_rows == 256 && !v2_fits)
    fail(ANIMA_E_INVALID_SHAPE, "256-row flash attention requires 64 key rows to span < 2 GiB");
  if (p.kv_splits > 1) {
    if (p.kv_splits != flash_kv_splits(p, D, batch, flash_rows) || !p.part_o || !p.part_ml)
      fail(ANIMA_E_INVALID_ARGUMENT, "flash key splits do not match the shape");
    p.nbatch = batch;
    p.kv_chunk = ((p.Sk + p.kv_splits - 1) / p.kv_splits + 63) / 64 * 64;
    p.q_tiles = (p.Sq + FLASH_V2_ROWS - 1) / FLASH_V2_ROWS;
    const int64_t blocks = t256 * p.kv_splits;
    if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "attention grid too large");
    launch_flash_v2(p, D, dim3((unsigned)blocks), stream);
    launch_flash_combine(p, D, batch, stream);
    return;
  }
  p.kv_splits = 0;
  // The 256-row kernel is chosen whenever it can address the keys: measured against the
  // 128-row kernel on grids of 32-128 of its workgroups (causal, key-length-masked and
  // GQA shapes, head_dim 128) it ran 1.3-2x faster even with most CUs idle, and tied at
  // head_dim 64.  The 128-row kernel stays selectable (flash_rows = 128).
  const bool v2 = flash_rows == 256 || (flash_rows == 0 && v2_fits);
  p.q_tiles = v2 ? (p.Sq + FLASH_V2_ROWS - 1) / FLASH_V2_ROWS : (p.Sq + FA_BM - 1) / FA_BM;
  const int64_t blocks = (int64_t)p.q_tiles * p.H * batch;
  if (blocks <= 0) return;
  if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "attention grid too large");
  const dim3 grid((unsigned)blocks);
  if (v2) {
    // Batched non-causal calls without Q RoPE whose query tiles x heads fill whole
    // rounds of the chip run persistent: one workgroup per (query tile, head) walks the
    // batch entries, so an entry's Q rows and first tiles load behind the previous
    // entry's key loop and epilogue (the same number of rounds as one workgroup per
    // entry, balanced because every workgroup takes the same entries in order).
    const int64_t qh = (int64_t)p.q_tiles * p.H;
    const bool persist = batch >= 2 && !p.causal && !p.rope && qh % F2_MIN_BLOCKS == 0 &&
                         flash_v2_persist_fits(p, D);
    if (persist)
      launch_flash_v2(p, D, dim3((unsigned)qh), stream, true);
    else
      launch_flash_v2(p, D, grid, stream);
  } else {
    if (p.nbatch < 1 || p.H < 1 || blocks != (int64_t)p.q_tiles * p.H * p.nbatch)
      fail(ANIMA_E_INVALID_ARGUMENT, "flash attention grid does not match its tiles, heads and batch");
    if (D == 128)
      hipLaunchKernelGGL(flash_attention_kernel<128>, grid, dim3(FA_NT), 0, stream, p);
    else
      hipLaunchKernelGGL(flash_attention_kernel<64>, grid, dim3(FA_NT), 0, stream, p);
  }
  ANIMA_HIP(hipGetLastError());
}

void launch_generic(const FlashParams& p, int D, int batch, hipStream_t stream) {
  if (D > GEN_MAX_D) fail(ANIMA_E_UNSUPPORTED, "generic attention supports head_dim <= 512");
  if ((int64_t)p.H * batch > 65535) fail(ANIMA_E_INVALID_SHAPE, "attention heads * batch too large");
  dim3 grid((unsigned)p.Sq, (unsigned)(p.H * batch)), block(64);
  hipLaunchKernelGGL(generic_attention_kernel, grid, block, 0, stream, p, D);
  ANIMA_HIP(hipGetLastError());
}

void launch_legacy_mps(const FlashParams& p, int D, int batch, hipStream_t stream) {
  if (D > GEN_MAX_D) fail(ANIMA_E_UNSUPPORTED, "MPS-rounding attention supports head_dim <= 512");
  if ((int64_t)p.H * batch > 65535) fail(ANIMA_E_INVALID_SHAPE, "attention heads * batch too large");
  dim3 grid((unsigned)p.Sq, (unsigned)(p.H * batch)), block(64);
  hipLaunchKernelGGL(legacy_mps_attention_kernel, grid, block, 0, stream, p, D);
  ANIMA_HIP(hipGetLastError());
}

void launch_prologue(const PrologueParams& p, hipStream_t stream) {
  if (p.D > GEN_MAX_D) fail(ANIMA_E_UNSUPPORTED, "Q/K prologue supports head_dim <= 512");
  const int64_t rows = (int64_t)p.batch * p.rows * p.heads;
  if (rows <= 0) return;
  const bool fast = p.D == 128 && aligned16(p.in) && p.in_tok % 8 == 0 && p.in_head % 8 == 0 &&
                    p.in_batch % 8 == 0 && aligned16(p.out) && p.out_tok % 8 == 0 && p.out_head % 8 == 0 &&
                    p.out_batch % 8 == 0 && (!p.norm_w || aligned16(p.norm_w)) && (!p.rope || aligned16(p.rope));
  if (fast) {
    const int hpt = p.heads % 4 == 0 ? 4 : (p.heads % 2 == 0 ? 2 : 1);
    constexpr int units = PRO_D128_THREADS / 8;
    const int64_t blocks = (rows / hpt + units - 1) / units;
    if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "prologue grid too large");
    const dim3 block(PRO_D128_THREADS);
    if (hpt == 4)
      hipLaunchKernelGGL(qk_prologue_d128_kernel<4>, dim3((unsigned)blocks), block, 0, stream, p);
    else if (hpt == 2)
      hipLaunchKernelGGL(qk_prologue_d128_kernel<2>, dim3((unsigned)blocks), block, 0, stream, p);
    else
      hipLaunchKernelGGL(qk_prologue_d128_kernel<1>, dim3((unsigned)blocks), block, 0, stream, p);
    ANIMA_HIP(hipGetLastError());
    return;
  }
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "prologue grid too large");
  hipLaunchKernelGGL(qk_prologue_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
