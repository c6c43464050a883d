// Flash attention, 256-query-row variant for long sequences (gfx950).
//
// Same maths and numerics as the 128-row kernel in attention.hip (S^T = K Q^T on
// v_mfma_f32_32x32x16_f16, fp32 online softmax in base 2, fp16 P, O^T += V^T P^T,
// Q RMSNorm + split-half RoPE fused into the Q fragment load), re-organised for
// MFMA throughput:
//   * 8 waves x 32 query rows share one K/V tile stream (1 workgroup per CU,
//     2 waves per SIMD so the hardware interleaves two instruction streams).
//   * K and V tiles (64 keys) go global -> LDS with global_load_lds_dwordx4 (no
//     staging registers).  Rows are padded (K: +16 B, V: +64 B) so the fragment
//     reads below hit distinct LDS banks (64 banks x 4 B); lanes whose linear slot
//     falls in a pad load a harmless duplicate chunk.  Padding instead of an XOR
//     swizzle keeps every fragment address "per-lane base + immediate".
//   * V^T fragments come straight from the row-major V tile with
//     ds_read_b64_tr_b16: within each 16-lane group, lane i receives column i of
//     the 4 rows the group's lanes point at (4 consecutive keys for one d).
//   * The pipeline steps over 32-key halves.  Each half-step reads the K
//     fragments of the next half, runs the next half's QK MFMAs interleaved with
//     this half's softmax VALU, then reads this half's V^T fragments and runs the
//     PV MFMAs.  Exps use the running max; if any row's max grew by more than 2^8
//     a side path rescales O and redoes the exps.  Three LDS stages: tile j+2
//     loads while tiles j and j+1 are read.
//   * Everything (Q, O accumulators, scores) lives in the 256 VGPRs a wave gets
//     at 2 waves/SIMD; row sums use v_dot2_f32_f16 on the fp16 P that feeds the
//     PV MFMA.
#include <type_traits>

#include "attention.hpp"

namespace anima {

constexpr int F2_WAVES = 8;
constexpr int F2_NT = 64 * F2_WAVES;
constexpr int F2_BN = 64;
constexpr int F2_STAGES = 3;
constexpr float F2_RESCALE_THRESHOLD = 8.0f;
static_assert(FLASH_V2_ROWS == 32 * F2_WAVES, "one 32-row block per wave");

typedef short short4v __attribute__((ext_vector_type(4)));
#define F2_LDS(p) ((__attribute__((address_space(3))) void*)(p))
#define F2_LDS4(p) ((__attribute__((address_space(3))) short4v*)(p))

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
template <int D>
__device__ __forceinline__ void load_q_fragment(const FlashParams& p, int b, int head, int qi, int hh,
                                                half8v (&qf)[D / 16]) {
  constexpr int QS = D / 16;
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
      ss = xlane32_sum(ss);
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

template <int D>
__global__ __launch_bounds__(F2_NT, 1) void flash_attention_v2_kernel(FlashParams p) {
  constexpr int DCH = D / 8;             // 16-byte data chunks per row
  constexpr int QS = D / 16;
  constexpr int OB = D / 32;
  constexpr int KROW = D + 8;            // padded K row (halfs)
  constexpr int VROW = D + 32;           // padded V row (halfs)
  constexpr int KRCH = KROW / 8, VRCH = VROW / 8;
  constexpr int KTILE = F2_BN * KROW, VTILE = F2_BN * VROW;   // halfs; whole 1 KiB segments
  static_assert(KTILE % 512 == 0 && VTILE % 512 == 0, "tile must be whole 1 KiB segments");

  __shared__ __attribute__((aligned(1024))) half_t Ks[F2_STAGES][KTILE];
  __shared__ __attribute__((aligned(1024))) half_t Vs[F2_STAGES][VTILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c32 = lane & 31, hh = lane >> 5;
  const int jj = lane & 15, gg = lane >> 4;

  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qt = lb % p.q_tiles;
  lb /= p.q_tiles;
  const int head = lb % p.H;
  const int b = lb / p.H;
  const int kvh = head / p.group;
  const int q0 = qt * FLASH_V2_ROWS;
  const int wq0 = q0 + wave * 32;
  const int qi = wq0 + c32;

  int kv_len = p.Sk;
  if (p.key_lengths_dev) {
    int L = p.key_lengths_dev[b];
    kv_len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
  } else if (p.use_host_lengths) {
    kv_len = p.host_lengths[b];
  }
  int kend = kv_len;
  if (p.causal) kend = min(kend, q0 + FLASH_V2_ROWS);
  const int ntiles = (kend + F2_BN - 1) / F2_BN;

  const half_t* kbase = p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head;
  const half_t* vbase = p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head;

  // Direct global -> LDS copy of tile j: segment sg of a padded tile holds linear
  // 16-byte slots sg*64 .. sg*64+63; slot -> (row, chunk) of the padded layout.
  // Wave w copies segments w, w+8, w+16.  Offsets are 32-bit byte offsets from
  // the tile's first key row (the host checks that 64 key rows fit in 2^31 bytes),
  // so the copies use the scalar-base + vector-offset address form; they are
  // recomputed per tile (a few VALU) instead of being held in registers.  Rows
  // past the last key re-read the last key row (masked in the softmax).
  constexpr int KR = (KRCH + F2_WAVES - 1) / F2_WAVES;
  constexpr int VR = (VRCH + F2_WAVES - 1) / F2_WAVES;
  auto seg_offset = [&](int sg, int rch, int64_t tok, int rmax, int ln) -> uint32_t {
    const int pos = sg * 64 + ln;
    const int ch = pos % rch;
    const int row = min(pos / rch, rmax);
    return ((uint32_t)(row * tok) + (uint32_t)((ch < DCH ? ch : 0) * 8)) * 2u;
  };
  auto issue_tile = [&](int j) {
    const int k0 = j * F2_BN;
    half_t* kd = Ks[j % F2_STAGES];
    half_t* vd = Vs[j % F2_STAGES];
    const half_t* kt = kbase + (int64_t)k0 * p.k_tok;
    const half_t* vt = vbase + (int64_t)k0 * p.v_tok;
    const int rmax = min(p.Sk - 1 - k0, F2_BN - 1);
    int ln = lane;
    asm volatile("" : "+v"(ln));   // recompute the offsets per tile rather than keep them live
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int sg = wave + F2_WAVES * r;
      if (sg < KRCH) {
        const uint32_t o = seg_offset(sg, KRCH, p.k_tok, rmax, ln);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(kt) + o, F2_LDS(kd + sg * 512), 16, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < VR; ++r) {
      const int sg = wave + F2_WAVES * r;
      if (sg < VRCH) {
        const uint32_t o = seg_offset(sg, VRCH, p.v_tok, rmax, ln);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(vt) + o, F2_LDS(vd + sg * 512), 16, 0, 0);
      }
    }
  };

  half8v qf[QS];
  load_q_fragment<D>(p, b, head, qi, hh, qf);

  floatx16 acc[OB];
#pragma unroll
  for (int c = 0; c < OB; ++c) acc[c] = floatx16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c2 = p.scale_log2;

  // Per-lane fragment bases (halfs); everything else is an immediate offset.
  const int kfrag = c32 * KROW + hh * 8;
  const int vfrag = (4 * hh + (jj >> 2)) * VROW + 16 * (gg & 1) + 4 * (jj & 3);

  // K fragment s of half hf: lane holds K[32hf + c32][16s + 8h .. +7].
  auto load_kfrags = [&](int j, int hf, half8v (&kf)[QS]) {
    const half_t* ks = Ks[j % F2_STAGES] + kfrag + hf * 32 * KROW;
#pragma unroll
    for (int s = 0; s < QS; ++s) kf[s] = *reinterpret_cast<const half8v*>(ks + 16 * s);
  };
  // V^T fragment (c, uu) of half hf: lane (d, h) holds V[key(u, h, 0..7)][32c + d]
  // with key(u, h, i) = 16u + 8(i/4) + 4h + i%4, the key order of the S^T C layout.
  auto load_vfrags = [&](int j, int hf, half8v (&vf)[OB][2]) {
    const half_t* vs = Vs[j % F2_STAGES] + vfrag;
#pragma unroll
    for (int c = 0; c < OB; ++c)
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) {
        const int u = 2 * hf + uu;
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(F2_LDS4(vs + 16 * u * VROW + 32 * c));
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(F2_LDS4(vs + (16 * u + 8) * VROW + 32 * c));
        const half4v lo_h = __builtin_bit_cast(half4v, lo);
        const half4v hi_h = __builtin_bit_cast(half4v, hi);
        vf[c][uu] = half8v{lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
      }
  };

  auto qk_mfma = [&](const half8v (&kf)[QS], floatx16& S) {
    S = floatx16{};
#pragma unroll
    for (int s = 0; s < QS; ++s) S = mfma32(kf[s], qf[s], S);
  };

  auto pv_mfma = [&](const half8v (&vf)[OB][2], const half8v (&P)[2]) {
#pragma unroll
    for (int uu = 0; uu < 2; ++uu)
#pragma unroll
      for (int c = 0; c < OB; ++c) acc[c] = mfma32(vf[c][uu], P[uu], acc[c]);
  };

  // P = fp16(exp2(S*c - m)) with the running max; returns whether any row of the
  // wave must raise its max (S is kept intact for that path).
  auto softmax = [&](int j, int hf, floatx16& S, half8v (&P)[2], bool masked) -> bool {
    if (masked) {
      const int k0 = j * F2_BN + 32 * hf;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kidx = k0 + (e >> 2) * 8 + 4 * hh + (e & 3);
        if (kidx >= kv_len || (p.causal && kidx > qi)) S[e] = -INFINITY;
      }
    }
    float mloc = S[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, S[e]);
    mloc = xlane32_max(mloc);
    const bool need = mloc * c2 > m_run + F2_RESCALE_THRESHOLD;
    const float msub = (m_run == -INFINITY) ? 0.f : m_run;
#pragma unroll
    for (int e = 0; e < 16; ++e) P[e >> 3][e & 7] = (half_t)fast_exp2(fmaf(S[e], c2, -msub));
    return need;
  };

  auto rescale = [&](floatx16& S, half8v (&P)[2]) {
    float mloc = S[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, S[e]);
    mloc = xlane32_max(mloc);
    const float mnew = fmaxf(m_run, mloc * c2);
    const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m_run - mnew);
    l_run *= alpha;
#pragma unroll
    for (int c = 0; c < OB; ++c) acc[c] *= alpha;
    m_run = mnew;
    const float msub = (mnew == -INFINITY) ? 0.f : mnew;
#pragma unroll
    for (int e = 0; e < 16; ++e) P[e >> 3][e & 7] = (half_t)fast_exp2(fmaf(S[e], c2, -msub));
  };

  auto rowsum = [&](const half8v (&P)[2]) {
    const half2v one = {(half_t)1.f, (half_t)1.f};
    float s = l_run;
#pragma unroll
    for (int uu = 0; uu < 2; ++uu)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half2v pr = {P[uu][2 * e], P[uu][2 * e + 1]};
        s = __builtin_amdgcn_fdot2(pr, one, s, false);
      }
    l_run = s;
  };

  auto half_masked = [&](int j, int hf) {
    const int k0 = j * F2_BN + 32 * hf;
    return (k0 + 32 > kv_len) || (p.causal && k0 + 31 > wq0);
  };

  floatx16 SA, SB;
  half8v P[2];

  // One half-step, in phases separated by scheduling fences:
  //   A  K fragment reads for the next QK;
  //   B  QK(next) MFMAs interleaved with this half's softmax VALU;
  //   C  V^T fragment reads, the rare rescale, the row sum and the PV MFMAs.
  auto half_step = [&](int j, int hf, floatx16& Scur, floatx16& Snext, auto has_next_c, auto masked_c) {
    constexpr bool HAS_NEXT = decltype(has_next_c)::value;
    constexpr bool MASKED = decltype(masked_c)::value;
    const int nj = hf ? j + 1 : j;
    const int nhf = hf ^ 1;
    half8v kf[QS];
    half8v vf[OB][2];
    if (HAS_NEXT) load_kfrags(nj, nhf, kf);
    __builtin_amdgcn_sched_barrier(0);
    if (HAS_NEXT) qk_mfma(kf, Snext);
    const bool need = softmax(j, hf, Scur, P, MASKED);
    if (HAS_NEXT) {
#pragma unroll
      for (int i = 0; i < QS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // six VALU
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_vfrags(j, hf, vf);
    if (__any(need)) rescale(Scur, P);
    rowsum(P);
    pv_mfma(vf, P);
  };

  auto run_half = [&](int j, int hf, floatx16& Scur, floatx16& Snext) {
    using T = std::integral_constant<bool, true>;
    using F = std::integral_constant<bool, false>;
    const bool has_next = (hf ? j + 1 : j) < ntiles;
    const bool masked = half_masked(j, hf);
    if (has_next) {
      if (masked) half_step(j, hf, Scur, Snext, T{}, T{});
      else half_step(j, hf, Scur, Snext, T{}, F{});
    } else {
      if (masked) half_step(j, hf, Scur, Snext, F{}, T{});
      else half_step(j, hf, Scur, Snext, F{}, F{});
    }
  };

  if (ntiles > 0) {
    issue_tile(0);
    if (ntiles > 1) issue_tile(1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    half8v kf[QS];
    load_kfrags(0, 0, kf);
    qk_mfma(kf, SA);
  }
  for (int j = 0; j < ntiles; ++j) {
    // Tile j (and j+1) are resident once every wave's copies have landed; the
    // barrier also retires all reads of stage (j+2)%3 = (j-1)%3 from step j-1.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (j + 2 < ntiles) issue_tile(j + 2);
    run_half(j, 0, SA, SB);
    run_half(j, 1, SB, SA);
  }

  const float l_tot = xlane32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qi < p.Sq) {
    half_t* op = p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head + (int64_t)qi * p.o_tok;
#pragma unroll
    for (int c = 0; c < OB; ++c)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        half4v val = {(half_t)(acc[c][4 * e4 + 0] * inv), (half_t)(acc[c][4 * e4 + 1] * inv),
                      (half_t)(acc[c][4 * e4 + 2] * inv), (half_t)(acc[c][4 * e4 + 3] * inv)};
        *reinterpret_cast<half4v*>(op + 32 * c + 8 * e4 + 4 * hh) = val;
      }
  }
}

void launch_flash_v2(const FlashParams& p, int D, dim3 grid, hipStream_t stream) {
  if (D == 128)
    hipLaunchKernelGGL(flash_attention_v2_kernel<128>, grid, dim3(F2_NT), 0, stream, p);
  else if (D == 64)
    hipLaunchKernelGGL(flash_attention_v2_kernel<64>, grid, dim3(F2_NT), 0, stream, p);
  else
    fail(ANIMA_E_UNSUPPORTED, "flash attention requires head_dim 64 or 128");
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
