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
//     a side path rescales O and redoes the exps.  Four LDS stages: tiles j+2
//     and j+3 load while tiles j and j+1 are read.
//   * Everything (Q, O accumulators, scores) lives in the 256 VGPRs a wave gets
//     at 2 waves/SIMD; row sums use v_dot2_f32_f16 on the fp16 P that feeds the
//     PV MFMA.
#include <type_traits>

#include "attention.hpp"

namespace anima {

constexpr int F2_WAVES = 8;
constexpr int F2_NT = 64 * F2_WAVES;
constexpr int F2_BN = 64;
constexpr int F2_STAGES = 4;
constexpr float F2_RESCALE_THRESHOLD = 8.0f;
static_assert(FLASH_V2_ROWS == 32 * F2_WAVES, "one 32-row block per wave");

typedef short short4v __attribute__((ext_vector_type(4)));
#define F2_LDS(p) ((__attribute__((address_space(3))) void*)(p))
#define F2_LDS4(p) ((__attribute__((address_space(3))) short4v*)(p))

// s_waitcnt vmcnt(n) alone (expcnt / lgkmcnt unconstrained), n wave-uniform in [0, 15].
template <int N>
__device__ __forceinline__ void wait_vmcnt_imm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
    case 0: wait_vmcnt_imm<0>(); break;
    case 1: wait_vmcnt_imm<1>(); break;
    case 2: wait_vmcnt_imm<2>(); break;
    case 3: wait_vmcnt_imm<3>(); break;
    case 4: wait_vmcnt_imm<4>(); break;
    case 5: wait_vmcnt_imm<5>(); break;
    case 6: wait_vmcnt_imm<6>(); break;
    case 7: wait_vmcnt_imm<7>(); break;
    case 8: wait_vmcnt_imm<8>(); break;
    case 9: wait_vmcnt_imm<9>(); break;
    case 10: wait_vmcnt_imm<10>(); break;
    case 11: wait_vmcnt_imm<11>(); break;
    default: wait_vmcnt_imm<12>(); break;
  }
}

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

  // One LDS object per stage: every access names its stage at compile time, so the
  // compiler can tell an in-flight global->LDS copy into one stage from reads of
  // another and does not make the reads wait for the copy.
  __shared__ __attribute__((aligned(1024))) half_t K0[KTILE], K1[KTILE], K2[KTILE], K3[KTILE];
  __shared__ __attribute__((aligned(1024))) half_t V0[VTILE], V1[VTILE], V2[VTILE], V3[VTILE];
  static_assert(F2_STAGES == 4, "four stage objects");
  auto kstage = [&](auto st) __attribute__((always_inline)) -> half_t* {
    constexpr int S = decltype(st)::value % F2_STAGES;
    if constexpr (S == 0) return K0;
    else if constexpr (S == 1) return K1;
    else if constexpr (S == 2) return K2;
    else return K3;
  };
  auto vstage = [&](auto st) __attribute__((always_inline)) -> half_t* {
    constexpr int S = decltype(st)::value % F2_STAGES;
    if constexpr (S == 0) return V0;
    else if constexpr (S == 1) return V1;
    else if constexpr (S == 2) return V2;
    else return V3;
  };

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
  // The K segments (0 .. KRCH-1) and V segments (KRCH .. NSEG-1) of a tile are
  // dealt round-robin: wave w copies combined segments w, w+8, w+16, ...  Every
  // wave issues exactly SPW copies per tile (slots past NSEG, and every slot of a
  // tile past the last one, copy a harmless 1 KiB into a scratch LDS object), so
  // "all but the newest tile landed" is always the single wait vmcnt(SPW).
  // Offsets are 32-bit byte offsets from the tile's first key row (the host checks
  // that 64 key rows fit in 2^31 bytes), so the copies use the scalar-base +
  // vector-offset address form; they are the same for every full tile (computed
  // once); a tile running past the last key clamps its rows to the last key row
  // (masked in the softmax).
  constexpr int NSEG = KRCH + VRCH;
  constexpr int SPW = (NSEG + F2_WAVES - 1) / F2_WAVES;
  __shared__ __attribute__((aligned(1024))) half_t Dummy[512];
  auto seg_offset = [&](int sg, int rmax, int ln) __attribute__((always_inline)) -> uint32_t {
    const bool isk = sg < KRCH;
    const int rch = isk ? KRCH : VRCH;
    const int64_t tok = isk ? p.k_tok : p.v_tok;
    const int pos = (isk ? sg : sg - KRCH) * 64 + ln;
    const int ch = pos % rch;
    const int row = min(pos / rch, rmax);
    return ((uint32_t)(row * tok) + (uint32_t)((ch < DCH ? ch : 0) * 8)) * 2u;
  };
  uint32_t soff[SPW];
#pragma unroll
  for (int r = 0; r < SPW; ++r) soff[r] = seg_offset(min(wave + F2_WAVES * r, NSEG - 1), F2_BN - 1, lane);

  auto issue_tile = [&](int j, auto st) __attribute__((always_inline)) {
    const int k0 = j * F2_BN;
    half_t* kd = kstage(st);
    half_t* vd = vstage(st);
    const bool live = j < ntiles;
    const char* kt = reinterpret_cast<const char*>(kbase + (int64_t)k0 * p.k_tok);
    const char* vt = reinterpret_cast<const char*>(vbase + (int64_t)k0 * p.v_tok);
    const int rmax = min(p.Sk - 1 - k0, F2_BN - 1);
    const bool full = rmax == F2_BN - 1;
#pragma unroll
    for (int r = 0; r < SPW; ++r) {
      const int sg = wave + F2_WAVES * r;
      if (live && sg < KRCH) {
        const uint32_t o = full ? soff[r] : seg_offset(sg, rmax, lane);
        __builtin_amdgcn_global_load_lds(kt + o, F2_LDS(kd + sg * 512), 16, 0, 0);
      } else if (live && sg < NSEG) {
        const uint32_t o = full ? soff[r] : seg_offset(sg, rmax, lane);
        __builtin_amdgcn_global_load_lds(vt + o, F2_LDS(vd + (sg - KRCH) * 512), 16, 0, 0);
      } else {
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(kbase) + 16 * lane, F2_LDS(Dummy), 16, 0, 0);
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

  typedef __attribute__((address_space(3))) short4v lds_short4v;

  // Per-lane fragment bases (halfs); everything else is an immediate offset.
  const int kfrag = c32 * KROW + hh * 8;
  const int vfrag = (4 * hh + (jj >> 2)) * VROW + 16 * (gg & 1) + 4 * (jj & 3);

  // K fragment s of half hf: lane holds K[32hf + c32][16s + 8h .. +7].
  auto load_kfrags = [&](auto st, int hf, half8v (&kf)[QS]) {
    const half_t* ks = kstage(st) + kfrag + hf * 32 * KROW;
#pragma unroll
    for (int s = 0; s < QS; ++s) kf[s] = *reinterpret_cast<const half8v*>(ks + 16 * s);
  };
  // V^T fragment (c, uu) of half hf: lane (d, h) holds V[key(u, h, 0..7)][32c + d]
  // with key(u, h, i) = 16u + 8(i/4) + 4h + i%4, the key order of the S^T C layout.
  // Reads through an LDS-space pointer formed from the shared array itself, so
  // every read is "lane base + immediate" (no per-read address arithmetic).
  auto load_vfrags = [&](auto st, int hf, half8v (&vf)[OB][2]) {
    lds_short4v* vs = (lds_short4v*)vstage(st) + (vfrag + 32 * hf * VROW) / 4;
#pragma unroll
    for (int c = 0; c < OB; ++c)
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) {
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + (16 * uu * VROW + 32 * c) / 4);
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + ((16 * uu + 8) * VROW + 32 * c) / 4);
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

  auto half_masked = [&](int j, int hf) __attribute__((always_inline)) {
    const int k0 = j * F2_BN + 32 * hf;
    return (k0 + 32 > kv_len) || (p.causal && k0 + 31 > wq0);
  };

  floatx16 SA, SB;
  half8v P[2];

  // Scores of keys past the sequence (or above the diagonal) -> -inf, in place.
  auto mask_scores = [&](int j, int hf, floatx16& S) __attribute__((always_inline)) {
    const int k0 = j * F2_BN + 32 * hf;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kidx = k0 + (e >> 2) * 8 + 4 * hh + (e & 3);
      if (kidx >= kv_len || (p.causal && kidx > qi)) S[e] = -INFINITY;
    }
  };

  // One half-step (32 keys), a single code path for every half-step so the O
  // accumulators never move between registers:
  //   A  K fragment reads for the next half's QK (past the last tile they re-read
  //      the current stage and the scores are discarded);
  //   B  QK(next) MFMAs interleaved with this half's softmax VALU and the V^T
  //      fragment reads;
  //   C  the rare rescale, the row sum and the PV MFMAs.
  // Masking is a wave-uniform in-place fix-up of the current scores.
  // st: stage of tile j; the next half's K comes from the same stage (hf = 0) or
  // the next one (hf = 1; past the last tile that stage holds stale keys and the
  // scores are discarded).
  auto half_step = [&](int j, int hf, floatx16& Scur, floatx16& Snext, auto st) __attribute__((always_inline)) {
    constexpr int ST = decltype(st)::value;
    half8v kf[QS];
    if (hf == 0)
      load_kfrags(st, 1, kf);
    else
      load_kfrags(std::integral_constant<int, (ST + 1) % F2_STAGES>{}, 0, kf);
    if (half_masked(j, hf)) mask_scores(j, hf, Scur);
    __builtin_amdgcn_sched_barrier(0);
    qk_mfma(kf, Snext);
    const bool need = softmax(j, hf, Scur, P, false);
    // P is used here, above the rescale branch: otherwise the compiler sinks the
    // exponentials below it (into both paths) and they no longer overlap the MFMAs.
    asm volatile("" ::"v"(P[0]), "v"(P[1]));
    half8v vf[OB][2];
    load_vfrags(st, hf, vf);
#pragma unroll
    for (int i = 0; i < QS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // two V^T fragment reads
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // six VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    if (__any(need)) rescale(Scur, P);
    rowsum(P);
    pv_mfma(vf, P);
  };

  // Four stages, two tiles of prefetch: iteration j reads tiles j and j+1 (the
  // second half-step starts the next tile's QK), tile j+2 is in flight and tile
  // j+3 is issued into the stage tile j-1 used.  Loads retire in order and every
  // tile is SPW copies per wave, so "tiles <= j+1 landed" is vmcnt(SPW).  The
  // barrier is written out (s_barrier after lgkmcnt(0)) so that the compiler does
  // not turn it into a wait for every copy in flight.
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  if (ntiles > 0) {
    issue_tile(0, S0{});
    issue_tile(1, S1{});
    issue_tile(2, S2{});
    wait_vmcnt_imm<2 * SPW>();   // tile 0 landed
    lds_barrier();
    half8v kf[QS];
    load_kfrags(S0{}, 0, kf);
    qk_mfma(kf, SA);
  }
  // Tile j uses stage j % 4; the loop is unrolled by four so every stage is static.
  auto tile_iter = [&](int j, auto st) __attribute__((always_inline)) {
    constexpr int ST = decltype(st)::value;
    // Tiles j, j+1 resident for every wave; the barrier also retires all reads of
    // stage (j+3)%4 = (j-1)%4 from iteration j-1 before it is overwritten.
    wait_vmcnt_imm<SPW>();
    lds_barrier();
    issue_tile(j + 3, std::integral_constant<int, (ST + 3) % F2_STAGES>{});
    half_step(j, 0, SA, SB, st);
    half_step(j, 1, SB, SA, st);
  };
  for (int j = 0; j < ntiles; j += F2_STAGES) {
    tile_iter(j, S0{});
    if (j + 1 < ntiles) tile_iter(j + 1, S1{});
    if (j + 2 < ntiles) tile_iter(j + 2, S2{});
    if (j + 3 < ntiles) tile_iter(j + 3, S3{});
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
