// Flash attention for wide heads (head_dim 384: the VAE decoder's single-head mid-block
// attention, VAEDecoder.swift:396-404, through AttentionExecutor.execute) on gfx950.
//
// Same maths and numerics as the other flash kernels (S^T = K Q^T on
// v_mfma_f32_32x32x16_f16, fp32 online softmax in base 2 with the lazy running max,
// fp16 P, O^T += V^T P^T; a Q RMSNorm / RoPE runs in the prologue kernel), organised so
// that a 384-wide O fits the registers:
//   * 8 waves, 2 per SIMD, 128 query rows per workgroup.  Waves w and w+4 (one SIMD) are
//     a pair over the same 32 query rows; wave w owns O columns 0-191 and wave w+4 columns
//     192-383 (6 accumulator tiles each), and each holds the Q fragments of its half.
//   * Per 32-key tile each wave of a pair computes the partial S^T over its 192 columns
//     (12 MFMAs), the pair swaps partial sums through LDS and both add them (a + b equals
//     b + a, so both waves hold the same scores and take the same softmax steps), then
//     each wave accumulates its half of O^T += V^T P^T (12 MFMAs).
//   * K and V tiles are register-staged copies into two LDS stages (16 threads move one
//     key row's 768 bytes, 256 contiguous bytes per instruction); each tile is read through
//     one buffer descriptor sized to the last key row in use, so rows past it read as
//     zeros without touching memory.  K rows are padded to D+8 halfs and V rows to D+32
//     (the bank-conflict-free pitches of the 128-wide kernel), and V^T fragments come
//     straight from the row-major V tile with ds_read_b64_tr_b16.
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
  constexpr int STAGE = KTILE + VTILE;
  constexpr int TPR = FW_NT / FW_BN;     // copy threads per key row (16)
  constexpr int CPR = D / 8 / TPR;       // 16-byte chunks per copy thread and row (3)
  constexpr int XBUF = 64 * 16;          // floats of one wave's partial scores
  static_assert(D % (8 * TPR) == 0 && DH % 32 == 0, "tile splits evenly");
  __shared__ __attribute__((aligned(1024))) half_t smem[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float xbuf[FW_WAVES * XBUF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int pr = wave & 3, dh = wave >> 2;       // query block, column half
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

  const half_t* kbase = p.k + (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head + (int64_t)kofs * p.k_tok;
  const half_t* vbase = p.v + (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head + (int64_t)kofs * p.v_tok;

  // Tile copies: thread t moves row t/16 of the tile, 16-byte chunks (t%16) + 16r for
  // r < CPR, of K and of V.
  const int crow = tid / TPR, cc = tid % TPR;
  const uint32_t ktok2 = (uint32_t)p.k_tok * 2u, vtok2 = (uint32_t)p.v_tok * 2u;
  const uint32_t goff_k = (uint32_t)crow * ktok2 + (uint32_t)cc * 16u;
  const uint32_t goff_v = (uint32_t)crow * vtok2 + (uint32_t)cc * 16u;
  const int loff_k = crow * KROW + cc * 8, loff_v = KTILE + crow * VROW + cc * 8;   // halfs within a stage
  const int64_t kstep = (int64_t)FW_BN * ktok2, vstep = (int64_t)FW_BN * vtok2;
  const int64_t kbytes = kend > 0 ? (int64_t)(kend - 1) * ktok2 + D * 2 : 0;
  const int64_t vbytes = kend > 0 ? (int64_t)(kend - 1) * vtok2 + D * 2 : 0;
  auto clamp_bytes = [](int64_t rem) __attribute__((always_inline)) -> int {
    return rem <= 0 ? 0 : (rem >= 0x7fffffff ? 0x7fffffff : (int)rem);
  };
  u32x4 stg[2 * CPR];
  auto load_tile = [&](int j) __attribute__((always_inline)) {
    const char* kt = reinterpret_cast<const char*>(kbase) + j * kstep;
    const char* vt = reinterpret_cast<const char*>(vbase) + j * vstep;
    const int nk = clamp_bytes(kbytes - j * kstep), nv = clamp_bytes(vbytes - j * vstep);
#pragma unroll
    for (int r = 0; r < CPR; ++r) stg[r] = load16_bounded(kt, nk, goff_k + 16u * TPR * r);
#pragma unroll
    for (int r = 0; r < CPR; ++r) stg[CPR + r] = load16_bounded(vt, nv, goff_v + 16u * TPR * r);
  };
  auto store_tile = [&](int s) __attribute__((always_inline)) {
    half_t* st = smem + s * STAGE;
#pragma unroll
    for (int r = 0; r < CPR; ++r) *reinterpret_cast<u32x4*>(st + loff_k + 8 * TPR * r) = stg[r];
#pragma unroll
    for (int r = 0; r < CPR; ++r) *reinterpret_cast<u32x4*>(st + loff_v + 8 * TPR * r) = stg[CPR + r];
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
  const int vfrag = KTILE + (4 * hh + (jj >> 2)) * VROW + DH * dh + 16 * (gg & 1) + 4 * (jj & 3);
  float* const xmine = xbuf + wave * XBUF + lane * 16;
  const float* const xpeer = xbuf + (wave ^ 4) * XBUF + lane * 16;

  // V^T fragment (c, u): lane (d, hh) holds V[16u + 8(i/4) + 4hh + i%4][DH*dh + 32c + d].
  auto vfrag_read = [&](int sbase, int u, int c) __attribute__((always_inline)) -> half8v {
    lds_short4v* vs = (lds_short4v*)(smem + sbase + vfrag);
    const int off = 16 * u * VROW + 32 * c;
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + off / 4);
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + (off + 8 * VROW) / 4);
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

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
    load_tile(1);
    for (int j = 0; j < ntiles; ++j) {
      const int st = (j & 1) * STAGE;
      // Tile j is resident and every wave has finished tile j-1: its stage takes tile
      // j+1, the staging registers the loads of tile j+2, and xbuf is free again.
      barrier();
      store_tile((j + 1) & 1);
      load_tile(j + 2);
      // Partial S^T over this wave's columns.
      const lds_half8v* ks = (const lds_half8v*)(smem + st + kfrag);
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
      barrier();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 o = *reinterpret_cast<const floatx4*>(xpeer + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[4 * q + e] += o[e];
      }
      // Masking, then the exponentials against the running max; the exact path (row
      // max, O / row-sum rescale) when a lane's share exceeds the lazy bound.
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
      // O^T += V^T P^T over this wave's columns.
      half8v vr[2];
      vr[0] = vfrag_read(st, 0, 0);
#pragma unroll
      for (int i = 0; i < 2 * OB; ++i) {
        if (i + 1 < 2 * OB) vr[(i + 1) & 1] = vfrag_read(st, (i + 1) / OB, (i + 1) % OB);
        acc[i % OB] = mfma32(vr[i & 1], P[i / OB], acc[i % OB]);
      }
    }
    wait_vmcnt_imm<0>();   // staged loads past the end (no memory traffic)
  }

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
  // of the K/V stages, which every wave has finished reading after this barrier.
  constexpr int OPITCH = DH + 8;           // halfs per staged row
  constexpr int OCH = DH / 8;              // 16-byte chunks per staged row
  static_assert(FW_WAVES * 32 * OPITCH <= 2 * STAGE, "staged rows fit the K/V stages");
  static_assert((32 * OCH) % 64 == 0, "whole store instructions");
  barrier();
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
  hipLaunchKernelGGL(flash_attention_wide_kernel<384>, grid, dim3(FW_NT), 0, stream, p);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
