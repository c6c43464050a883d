// Flash attention for wide heads (head_dim 384: the VAE decoder's single-head mid-block
// attention, VAEDecoder.swift:396-404, through AttentionExecutor.execute) on gfx950.
//
// Same maths and numerics as the other flash kernels (S^T = K Q^T on
// v_mfma_f32_32x32x16_f16, fp32 online softmax in base 2 with the lazy running max,
// fp16 P, O^T += V^T P^T; a Q RMSNorm / RoPE runs in the prologue kernel), organised so
// that a 384-wide O fits the registers:
//   * 8 waves, 2 per SIMD, 128 query rows per workgroup.  Waves 2p and 2p+1 are a pair
//     over query rows 32p .. 32p+31; wave 2p owns O columns 0-191 and wave 2p+1 columns
//     192-383 (6 accumulator tiles each), and each holds the Q fragments of its half.
//   * Per 32-key tile each wave of a pair computes the partial S^T over its 192 columns
//     (12 MFMAs) and writes it to LDS; after the next barrier both waves add the
//     partner's half (a + b equals b + a, so both hold the same scores and take the same
//     softmax steps), then each accumulates its half of O^T += V^T P^T (12 MFMAs).
//   * Waves 0-3 (group 0) and 4-7 (group 1) put one wave of each group on every SIMD and
//     run a phase apart: while one group issues its MFMAs (M phase: PV of tile j-1, then
//     the partial QK^T of tile j) the other runs the softmax of its previous tile and the
//     tile copies (X phase), and the two swap at every barrier.  A pair lives in one
//     group, so its score exchange needs no extra synchronisation.
//   * K and V tiles have two LDS stages each.  Group 1 copies K tiles and group 0 V
//     tiles, each at the start of its X phase: registers take a tile's loads in the
//     group's previous X phase, two phases before they are written to LDS (8 threads
//     move one key row's 768 bytes, 128 contiguous bytes per instruction), and each
//     tile is read through one buffer descriptor sized to the last key row in use, so
//     rows past it read as zeros without touching memory.  K
//     rows are padded to D+8 halfs and V rows to D+32 (the bank-conflict-free pitches of
//     the 128-wide kernel); V^T fragments come straight from the row-major V tile with
//     ds_read_b64_tr_b16.
//   * One query head has only ceil(Sq/128) workgroups, so the keys are split across
//     workgroups (flash_kv_splits) and flash_combine_kernel merges the partial rows.
//     Query tiles are the fastest grid index, so the workgroups of one XCD share one key
//     split in their L2.
#include "flash_common.hpp"

namespace anima {

constexpr int FW_WAVES = 8;
constexpr int FW_NT = 64 * FW_WAVES;
constexpr int FW_BN = 32;                 // keys per tile
constexpr float FW_LAZY_LIMIT = 32768.f;  // largest row-sum share the lazy exponentials accept
static_assert(FLASH_WIDE_ROWS == 32 * (FW_WAVES / 2), "one 32-row block per wave pair");

template <int D>
__global__ __launch_bounds__(FW_NT, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_attention_wide_kernel(FlashParams p) {
  constexpr int DH = D / 2;              // columns per wave
  constexpr int QS = DH / 16;            // d-steps of the partial QK^T
  constexpr int OB = DH / 32;            // 32-wide O blocks per wave
  constexpr int KROW = D + 8, VROW = D + 32;
  constexpr int KTILE = FW_BN * KROW, VTILE = FW_BN * VROW;   // halfs
  constexpr int VBASE = 2 * KTILE;       // K stages 0-1, then V stages 0-1
  constexpr int GT = FW_NT / 2;          // threads per wave group
  constexpr int TPR = GT / FW_BN;        // copy threads per key row (8)
  constexpr int CPR = D / 8 / TPR;       // 16-byte chunks per copy thread (6)
  constexpr int XBUF = 64 * 16;          // floats of one wave's partial scores
  static_assert(D % (8 * TPR) == 0 && DH % 32 == 0, "tile splits evenly");
  __shared__ __attribute__((aligned(1024))) half_t smem[2 * KTILE + 2 * VTILE];
  __shared__ __attribute__((aligned(16))) float xbuf[FW_WAVES * XBUF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave >> 2;
  const int pr = wave >> 1, dh = wave & 1;       // query block, column half
  const int c32 = lane & 31, hh = lane >> 5;
  const int jj = lane & 15, gg = lane >> 4;

  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qt = lb % p.q_tiles;
  lb /= p.q_tiles;
  int split = 0;
  if (p.kv_splits > 1) {
    split = lb % p.kv_splits;
    lb /= p.kv_splits;
  }
  const int head = lb % p.H;
  const int b = lb / p.H;
  const int kvh = head / p.group;
  const int q0 = qt * FLASH_WIDE_ROWS;
  const int wq0 = q0 + pr * 32;
  const int qi = wq0 + c32;

  int kv_len = p.Sk;
  if (p.key_lengths_dev) {
    const int L = p.key_lengths_dev[b];
    kv_len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
  } else if (p.use_host_lengths) {
    kv_len = p.host_lengths[b];
  }
  const int kofs = p.kv_splits > 1 ? split * p.kv_chunk : 0;
  if (p.kv_splits > 1) kv_len = max(0, min(kv_len, kofs + p.kv_chunk) - kofs);
  int kend = kv_len;
  if (p.causal) kend = min(kend, q0 + FLASH_WIDE_ROWS);
  const int ntiles = (kend + FW_BN - 1) / FW_BN;

  // Tile copies: group 1 moves K tiles, group 0 V tiles.  Thread t of the group moves
  // row t/8 of the tile, 16-byte chunks (t%8) + 8r for r < CPR.
  const int gt = tid & (GT - 1);
  const int crow = gt / TPR, cc = gt % TPR;
  const half_t* const cbase =
      group ? p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head + (int64_t)kofs * p.k_tok
            : p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head + (int64_t)kofs * p.v_tok;
  const uint32_t ctok2 = (uint32_t)(group ? p.k_tok : p.v_tok) * 2u;
  const uint32_t goff = (uint32_t)crow * ctok2 + (uint32_t)cc * 16u;
  const int64_t cstep = (int64_t)FW_BN * ctok2;
  const int64_t cbytes = kend > 0 ? (int64_t)(kend - 1) * ctok2 + D * 2 : 0;
  const int crowp = group ? KROW : VROW;
  const int loff = (group ? 0 : VBASE) + crow * crowp + cc * 8;   // halfs within stage 0
  const int cstage = group ? KTILE : VTILE;                      // halfs between stages
  u32x4 stg[CPR];
  auto load_copy = [&](int j) __attribute__((always_inline)) {
    // Chunk r goes through its own descriptor, based 16 * TPR * r bytes further on, so
    // that every load shares the one lane offset goff.
    const char* t = reinterpret_cast<const char*>(cbase) + j * cstep;
    const int64_t rem = cbytes - j * cstep;
    const int n = rem <= 0 ? 0 : (rem >= 0x7fffffff ? 0x7fffffff : (int)rem);
#pragma unroll
    for (int r = 0; r < CPR; ++r) stg[r] = load16_bounded(t + 16 * TPR * r, max(n - 16 * TPR * r, 0), goff);
  };
  auto store_copy = [&](int s) __attribute__((always_inline)) {
    half_t* st = smem + loff + s * cstage;
#pragma unroll
    for (int r = 0; r < CPR; ++r) *reinterpret_cast<u32x4*>(st + 8 * TPR * r) = stg[r];
  };

  // Q fragments of this wave's column half (B operand of S^T): lane holds
  // Q[row][DH*dh + 16s + 8hh .. +7].
  half8v qf[QS];
  {
    const int qrow = qi < p.Sq ? qi : p.Sq - 1;
    const half_t* qp =
        p.q + (int64_t)b * p.q_batch + (int64_t)head * p.q_head + (int64_t)qrow * p.q_tok + DH * dh + 8 * hh;
#pragma unroll
    for (int s = 0; s < QS; ++s) qf[s] = *reinterpret_cast<const half8v*>(qp + 16 * s);
  }

  floatx16 acc[OB];
#pragma unroll
  for (int c = 0; c < OB; ++c) acc[c] = floatx16{};
  float m_run = -INFINITY;
  float lrow = 0.f;    // this lane's share of the row sum (the other half is in lane c32 + 32)
  const float c2 = p.scale_log2;

  typedef __attribute__((address_space(3))) half8v lds_half8v;
  typedef __attribute__((address_space(3))) short4v lds_short4v;
  const int kfrag = c32 * KROW + DH * dh + hh * 8;
  const int vfrag = VBASE + (4 * hh + (jj >> 2)) * VROW + DH * dh + 16 * (gg & 1) + 4 * (jj & 3);
  float* const xmine = xbuf + wave * XBUF + lane * 16;
  const float* const xpeer = xbuf + (wave ^ 1) * XBUF + lane * 16;

  // V^T fragment (c, u) of V stage vs: lane (d, hh) holds
  // V[16u + 8(i/4) + 4hh + i%4][DH*dh + 32c + d].
  auto vfrag_read = [&](int vs, int u, int c) __attribute__((always_inline)) -> half8v {
    lds_short4v* vp = (lds_short4v*)(smem + vs * VTILE + vfrag);
    const int off = 16 * u * VROW + 32 * c;
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vp + off / 4);
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vp + (off + 8 * VROW) / 4);
    const half4v lo_h = __builtin_bit_cast(half4v, lo), hi_h = __builtin_bit_cast(half4v, hi);
    return half8v{lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
  };

  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  // Score element e of a lane (column c32 = query) is key 8(e/4) + 4hh + e%4 of the
  // tile; P[u][i] = p(S[8u + i]) is the B operand of k-step u of PV.
  floatx16 S;
  half8v P[2];
  auto exps = [&](float msub) __attribute__((always_inline)) -> float {
    float ls[4];   // started from the first four terms, not from 0.f (same bits)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = fast_exp2(fmaf(S[e], c2, -msub));
      P[e >> 3][e & 7] = (half_t)pe;
      if (e < 4)
        ls[e] = pe;
      else
        ls[e & 3] += pe;
    }
    return (ls[0] + ls[1]) + (ls[2] + ls[3]);
  };

  // M phase of tile j: O^T += V^T P^T of tile j-1 (P is free after it), then this wave's
  // partial S^T of tile j into its exchange buffer.  (Interleaving the two products'
  // MFMAs with a deeper fragment read-ahead shortened this phase but lengthened the other
  // group's X phase by more: the two phases share the LDS, and it is the limit here.)
  auto m_phase = [&](int j) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
    if (j > 0) {
      const int vs = (j - 1) & 1;
      half8v vr[2];
      vr[0] = vfrag_read(vs, 0, 0);
#pragma unroll
      for (int i = 0; i < 2 * OB; ++i) {
        if (i + 1 < 2 * OB) vr[(i + 1) & 1] = vfrag_read(vs, (i + 1) / OB, (i + 1) % OB);
        acc[i % OB] = mfma32(vr[i & 1], P[i / OB], acc[i % OB]);
      }
    }
    if (j < ntiles) {
      const lds_half8v* ks = (const lds_half8v*)(smem + (j & 1) * KTILE + kfrag);
      half8v kr[2];
      kr[0] = ks[0];
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        if (s + 1 < QS) kr[(s + 1) & 1] = ks[2 * (s + 1)];
        S = mfma32(kr[s & 1], qf[s], s == 0 ? floatx16{} : S);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<floatx4*>(xmine + 4 * q) = floatx4{S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]};
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // X phase of tile j: first this group's tile copy (the tile loaded in its previous X
  // phase goes to LDS and the next one is loaded), then the full scores (own partial +
  // the partner's), masking and the exponentials against the running max (the exact
  // path, with the row max and the O / row-sum rescale, when a lane's share exceeds the
  // lazy bound).  Group 0 stores V tile j and loads V tile j+1; group 1 (one phase later
  // in the schedule) stores K tile j+2 and loads K tile j+3.
  auto x_phase = [&](int j) __attribute__((always_inline)) {
    const int cj = group ? j + 2 : j;
    if (cj < ntiles) {
      store_copy(cj & 1);
      load_copy(cj + 1);
    }
    if (j >= 0 && j < ntiles) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 o = *reinterpret_cast<const floatx4*>(xpeer + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[4 * q + e] += o[e];
      }
      const int k0 = j * FW_BN;
      if ((k0 + FW_BN > kv_len) || (p.causal && k0 + FW_BN - 1 > wq0)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kidx = k0 + 8 * (e >> 2) + 4 * hh + (e & 3);
          if (kidx >= kv_len || (p.causal && kofs + kidx > qi)) S[e] = -INFINITY;
        }
      }
      float tsum = exps(m_run);
      if (__any(!(tsum <= FW_LAZY_LIMIT))) {
        auto mx = [](float a, float bb) __attribute__((always_inline)) { return __builtin_elementwise_maximum(a, bb); };
        float part[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) part[i] = mx(mx(S[4 * i], S[4 * i + 1]), mx(S[4 * i + 2], S[4 * i + 3]));
        const float mloc = xlane32_max(mx(mx(part[0], part[1]), mx(part[2], part[3]))) * c2;
        const float mnew = fmaxf(m_run, mloc);
        if (mnew > m_run) {
          const float alpha = (m_run == -INFINITY) ? 1.f : fast_exp2(m_run - mnew);
          lrow *= alpha;
#pragma unroll
          for (int c = 0; c < OB; ++c) acc[c] *= alpha;
          m_run = mnew;
        }
        tsum = exps((m_run == -INFINITY) ? 0.f : m_run);
      }
      lrow += tsum;
    }
  };

  // Prologue: group 1 brings K tile 0 to LDS and loads K tile 1, group 0 loads V tile 0.
  if (group) {
    load_copy(0);
    store_copy(0);
    load_copy(1);
  } else {
    load_copy(0);
  }
  barrier();
  // Group 1 runs one phase behind group 0: it starts with the copy step of X(-1), so in
  // every later phase one group issues MFMAs while the other runs its X phase.  Both
  // groups then run the same loop, and every wave passes 2 (ntiles + 1) barriers.
  if (group) {
    x_phase(-1);
    barrier();
  }
  for (int t = 0; t < ntiles; ++t) {
    m_phase(t);
    barrier();
    x_phase(t);
    barrier();
  }
  m_phase(ntiles);   // PV of the last tile
  barrier();
  if (!group) barrier();
  wait_vmcnt_imm<0>();   // tile loads past the end (no memory traffic)

  const float l_tot = xlane32_sum(lrow);
  // A key split stores its normalised rows O_s / l_s in fp16 (the same whole-row path as
  // O, below) beside the fp32 (max, sum) pair of each row; the merge weighs them by l_s.
  if (p.kv_splits > 1 && qi < p.Sq && hh == 0 && dh == 0) {
    const int64_t row = (((int64_t)split * p.nbatch + b) * p.H + head) * p.Sq + qi;
    *reinterpret_cast<float2*>(p.part_ml + row * 2) = make_float2(m_run, l_tot);
  }
  // The fp16 rows go through LDS so that every global store is a 16-byte piece of a
  // 384-byte half row (24 lanes per row); the register layout would scatter each store
  // instruction over 32 rows.  Wave w stages its 32 rows x 192 columns in its own slice
  // of the K/V stages, which every wave finished reading before the loop's last barrier.
  constexpr int OPITCH = DH + 8;           // halfs per staged row
  constexpr int OCH = DH / 8;              // 16-byte chunks per staged row
  static_assert(FW_WAVES * 32 * OPITCH <= 2 * KTILE + 2 * VTILE, "staged rows fit the K/V stages");
  static_assert((32 * OCH) % 64 == 0, "whole store instructions");
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  half_t* const ost = smem + wave * 32 * OPITCH;
#pragma unroll
  for (int c = 0; c < OB; ++c)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const half4v val = {(half_t)(acc[c][4 * e4 + 0] * inv), (half_t)(acc[c][4 * e4 + 1] * inv),
                          (half_t)(acc[c][4 * e4 + 2] * inv), (half_t)(acc[c][4 * e4 + 3] * inv)};
      *reinterpret_cast<half4v*>(ost + c32 * OPITCH + 32 * c + 8 * e4 + 4 * hh) = val;
    }
  half_t* const obase = p.kv_splits > 1
                            ? static_cast<half_t*>(p.part_o) + (((int64_t)split * p.nbatch + b) * p.H + head) * p.Sq * D
                            : p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head;
  const int64_t otok = p.kv_splits > 1 ? D : p.o_tok;
#pragma unroll
  for (int i = 0; i < 32 * OCH / 64; ++i) {
    const int n = i * 64 + lane, r = n / OCH, ch = n % OCH;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ost + r * OPITCH + ch * 8);
    if (wq0 + r < p.Sq) *reinterpret_cast<u32x4*>(obase + (int64_t)(wq0 + r) * otok + DH * dh + ch * 8) = v;
  }
}

void launch_flash_wide(const FlashParams& p, int D, dim3 grid, hipStream_t stream) {
  if (D != 384) fail(ANIMA_E_UNSUPPORTED, "wide flash attention requires head_dim 384");
  const int64_t want = (int64_t)p.q_tiles * p.H * p.nbatch * (p.kv_splits > 1 ? p.kv_splits : 1);
  if (want != (int64_t)grid.x) fail(ANIMA_E_INVALID_SHAPE, "wide flash attention grid does not match its tiles");
  hipLaunchKernelGGL(flash_attention_wide_kernel<384>, grid, dim3(FW_NT), 0, stream, p);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
