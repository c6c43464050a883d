// Quantized GEMM for M > 64 on gfx950: Y[M,N] = X[M,K] deq(W)[N,K]^T for W4/W8
// weights, computed as C^T = W X^T on v_mfma_f32_32x32x16_f16.
//
// Replaces the qgemm_w4/w8 path of LinearExecutor.encodeQGEMM
// (AnimaXS/Runtime/Metal/LinearExecutor.swift:304-361; kernels at
// AnimaXS/Shaders/AnimaKernels.metal:955-1047).  Organisation:
//   * Workgroup tile 128 (M) x 256 (N), 8 waves in two groups of 4.  Wave w of a
//     group owns output columns 64w .. 64w+63 and all 128 rows (2 x 4 MFMA
//     tiles); waves w and w+4 share a SIMD and the same output tile.  Group 0
//     takes the first half of the K blocks (64 = one quantisation group), group 1
//     the second; the two partial sums meet in LDS at the end (fp32, fixed order).
//   * Each K block j of a group is two phases per wave, separated by workgroup
//     barriers:
//       M  the 32 MFMAs of block j, X fragments read from LDS a few MFMAs ahead,
//          with the dequantisation of block j+1 interleaved (half a fragment per
//          MFMA pair, into the registers the MFMAs have finished with);
//       V  scale/zero of block j+2 from the LDS window, the X tile of block j+1 to
//          LDS, and the loads of X(j+2) and of the weights of block j+3.
//     Group 1 runs one phase behind group 0, so in every barrier interval one
//     wave of each SIMD issues MFMAs while the other issues the memory work.
//   * Weights never touch LDS: each lane loads its own rows' packed bytes (16 B
//     per row per block for W4, two blocks in flight) and dequantises them in
//     registers.  X is shared through LDS (one stage per group); scale/zero pairs
//     are read 8 groups at a time per row into an LDS window when the rows allow.
//   * Dequantisation is bit-identical to the reference decoder's
//     half(fl32(q*scale + zero)).  When q*scale + zero is exact in fp32 for every
//     code (one_rounding_exact), packed fp16 arithmetic gives the same bits with
//     one rounding: q is rebuilt exactly from the fp16 pattern 0x6400|q
//     (= 1024 + q) and v_pk_fma_f16(q, s, z) rounds once.  The MFMA phase always
//     runs that form, branch-free; a wave whose block fails the test redoes it
//     with the fp32 FMA and separate RNE conversion (a rare, wave-uniform branch
//     after the MFMAs).
//   * W4 pairs come out as (k, k+4) from the nibble layout, so the A fragment
//     holds k in the order 0,4,1,5,2,6,3,7 of each 8; the X tile is written to LDS
//     in the same order (v_perm) and the MFMA's sum over k is unchanged.
//   * Buffer descriptors bound X, W and the scales by the tile's first row: rows
//     past M or N read as zeros without touching memory.  Every global load in the
//     loop is unconditional, so the compiler's in-order wait counts stay exact.
#include <type_traits>

#include "dequant.hpp"

namespace anima {

constexpr int PG_BM = 128;                  // output rows (M) per workgroup
constexpr int PG_BN = 256;                  // output columns (N) per workgroup: 4 waves x 64
constexpr int PG_BK = 64;                   // K per block: one quantisation group
constexpr int PG_GM = 4;                    // M blocks per tile group (tile order)
constexpr int PG_NT = 512;                  // two groups of 4 waves
constexpr int PG_XROW = PG_BK + 8;          // padded X row in LDS (halfs)
constexpr int PG_XSTAGE = PG_BM * PG_XROW * 2;   // bytes per X stage (one per group)
constexpr int PG_RED = 16384;               // bytes per wave for the final K-split sum
constexpr int PG_SMEM = 8 * PG_RED;         // reduction area, overlaying the two X stages
constexpr int PG_WIN = 8;                   // K blocks per scale/zero window
constexpr int PG_WINBUF = PG_BN * PG_WIN * 2 * 2;    // one window: scale and zero of 256 rows (8 KiB)
constexpr int PG_WINOFF = 2 * PG_XSTAGE;    // windows: [group][buffer] after the X stages
static_assert(PG_WINOFF + 4 * PG_WINBUF <= PG_SMEM, "X stages and windows fit in the reduction area");
constexpr int PG_OROW = PG_BN + 8;          // padded output-tile row in LDS (halfs)
static_assert(PG_BM * PG_OROW * 2 <= PG_SMEM, "output tile fits in the reduction area");
// M-split form (MSPLIT): 256-row tiles, the two groups on rows 0-127 and 128-255 over the
// whole K range; its 256-row output tile needs more LDS than the reduction area.
constexpr int PG_SMEM_M = 2 * PG_BM * PG_OROW * 2;
static_assert(PG_SMEM_M >= PG_SMEM, "the M-split LDS area also holds the X stages and windows");
constexpr int PG_GM_M = 4;                  // 256-row M blocks per tile group (M-split form)

typedef __attribute__((address_space(3))) half8v lds_half8v;

// ---------------------------------------------------------------------------
// Dequantisation of one lane's packed weights into A fragments.
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// SWIN: the scale/zero rows are 16-byte aligned runs of 8 groups (groups % 8 == 0),
// read 8 groups at a time per row into an LDS window instead of one 2-byte load per
// row and block.
// MSPLIT: the workgroup tile is 256 (M) x 256 (N) and the two wave groups split the rows
// instead of the K range: group g computes rows 128g .. 128g+127 over every K block, so
// there is no partial-sum exchange, and a launch has half the workgroups, each with the
// first loads and output stage of one tile.  Every wave still owns 64 columns x 128 rows
// and dequantises the same weights per MFMA as in the K-split form.  Only single plain
// or fused-output launches without split K take it (pingpong_msplit); its sums run over
// K in one order, so its bits differ from the K-split form's in the last place.
template <int STORAGE, bool SWIN, bool MSPLIT>
__global__ __launch_bounds__(PG_NT, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void pingpong_gemm_kernel(GemmGroup gp) {
  constexpr bool W4 = STORAGE == ANIMA_STORAGE_W4;
  constexpr int QBITS = W4 ? 4 : 8;
  constexpr int WCH = W4 ? 1 : 2;           // 16-byte weight chunks per lane per row per block
  constexpr int XCH = PG_BM * PG_BK / 8 / 256;   // X chunks per thread of a group (4)
  // X fragments read ahead of their MFMAs (W8's two weight blocks in flight leave
  // fewer registers).
  constexpr int PG_READ_AHEAD = W4 ? 3 : 2;
  __shared__ __attribute__((aligned(1024))) char smem[MSPLIT ? PG_SMEM_M : PG_SMEM];
  constexpr int BM = MSPLIT ? 2 * PG_BM : PG_BM;     // output rows per workgroup
  constexpr int GM = MSPLIT ? PG_GM_M : PG_GM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave >> 2, wg = wave & 3;
  const int c32 = lane & 31, hh = lane >> 5;
  // Problem of this workgroup: logical tiles [first_tile[i], first_tile[i+1]) belong
  // to problem i (every problem of a group shares K and storage).
  const int lbg = xcd_logical_block(blockIdx.x, gridDim.x);
  int pi = 0;
#pragma unroll
  for (int i = 1; i < PG_GROUP; ++i)
    if (i < gp.count && lbg >= gp.first_tile[i]) pi = i;
  const GemmParams& p = gp.p[pi];
  const int vec_store = gp.vec[pi];
  const int ntn = (p.N + PG_BN - 1) / PG_BN;
  const int lb = lbg - gp.first_tile[pi];
  // Split K: workgroup lb takes K-block range `split` of tile lb / ksplit.
  const int ks = p.ksplit > 1 ? p.ksplit : 1;
  const int split = lb % ks;
  const int lt = lb / ks;
  // Tiles go in groups of PG_GM M blocks x all N tiles, M varying fastest: the 32
  // consecutive tiles an XCD runs in one round are 4 M blocks x 8 N tiles, so each weight
  // tile it loads serves four workgroups from its L2 (N varying fastest, a round of a wide
  // GEMM took one M block x 32 N tiles and streamed the whole weight into every XCD).
  const int ntm = (p.M + BM - 1) / BM;
  const int gfirst = (lt / (GM * ntn)) * GM;
  const int gm = ntm - gfirst < GM ? ntm - gfirst : GM;
  const int gr = lt % (GM * ntn);
  const int tm = gfirst + gr % gm, tn = gr / gm;
  const int m0 = tm * BM, n0 = tn * PG_BN;
  const int nk = p.K / PG_BK / ks;
  const int kbeg = split * nk;
  // Group 0 takes K blocks [0, half), group 1 [half, nk); with windows, half is a
  // multiple of the window so every window is aligned.
  int half = SWIN ? PG_WIN * ((nk + 2 * PG_WIN - 1) / (2 * PG_WIN)) : (nk + 1) / 2;
  half = half < nk ? half : nk;
  const int kb0 = MSPLIT || group == 0 ? 0 : half;
  const int nown = MSPLIT ? nk : (group == 0 ? half : nk - half);

  // Tile-relative buffers (sizes fit in 31 bits; checked on the host).
  // With split K they start at the split's first K block; the sizes end where they did.
  // The group's X rows start at xr0 (M-split: its 128-row half of the tile, which can
  // lie past M on the last tile row: then the descriptor is empty and reads zeros).
  const int xr0 = m0 + (MSPLIT ? PG_BM * group : 0);
  const half_t* xb = p.x + (int64_t)xr0 * p.K + kbeg * PG_BK;
  const int xrem = (p.M - xr0) * p.K * 2 - kbeg * PG_BK * 2;
  const int xbytes = xrem > 0 ? xrem : 0;
  const uint8_t* wb = p.w + (int64_t)n0 * p.row_stride + kbeg * 32 * WCH;
  const int wbytes = (int)((int64_t)(p.N - n0) * p.row_stride) - kbeg * 32 * WCH;
  const half_t* sb = p.scale + (int64_t)n0 * p.groups + kbeg;
  const half_t* zb = p.zero + (int64_t)n0 * p.groups + kbeg;
  const int sbytes = (p.N - n0) * p.groups * 2 - kbeg * 2;

  // X copies: thread t of a group moves chunks t + 256r (r < 4) of its group's
  // block: row t/8 + 32r, 16-byte column t%8 (8 lanes read one 128-byte row).
  const int tg = tid & 255;
  const int xrow = tg >> 3, xch = tg & 7;
  uint32_t goff_x[XCH];
#pragma unroll
  for (int r = 0; r < XCH; ++r) goff_x[r] = (uint32_t)(xrow + 32 * r) * (uint32_t)p.K * 2u + (uint32_t)xch * 16u;
  char* const xstage = smem + group * PG_XSTAGE;
  const int loff_x = (xrow * PG_XROW + xch * 8) * 2;

  // Weights: lane (c32, hh) of wave wg holds rows 64wg + 32t + c32 (t = 0, 1),
  // k = 32hh .. 32hh+31 of each block.
  uint32_t goff_w[2], goff_s[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t row = (uint32_t)(64 * wg + 32 * t + c32);
    goff_w[t] = row * (uint32_t)p.row_stride + (uint32_t)hh * 16u * WCH;
    goff_s[t] = row * (uint32_t)p.groups * 2u;
  }

  u32x4 xs[XCH];           // staged X chunks of the group's next block
  u32x4 wr[2][2][WCH];     // packed weights, two blocks in flight: [buffer][row tile][chunk]
  uint32_t sr[2], zr[2];   // scale / zero bits of the block after next (without windows)
  u32x4 swin[2];           // staged scale / zero window chunk of row tg (with windows)
  char* const winbase = smem + PG_WINOFF + group * 2 * PG_WINBUF;
  half8v wf[2][4];         // dequantised A fragments (row tile, k step) of the current block
  floatx16 acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[t][m] = floatx16{};

  auto load_x = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < XCH; ++r) xs[r] = load16_bounded(xb, xbytes, goff_x[r], kb * PG_BK * 2);
  };
  auto load_w = [&](int kb, auto buf_c) __attribute__((always_inline)) {
    constexpr int B = decltype(buf_c)::value;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < WCH; ++c) wr[B][t][c] = load16_bounded(wb, wbytes, goff_w[t] + 16u * c, kb * 32 * WCH);
  };
  // Scale / zero of one block, without windows: one 2-byte load per row.
  auto load_sz = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sr[t] = load2_bounded(sb, sbytes, goff_s[t], kb * 2);
      zr[t] = load2_bounded(zb, sbytes, goff_s[t], kb * 2);
    }
  };
  // Window of K blocks kw .. kw+7: thread tg of the group fetches row tg's 16-byte
  // scale and zero runs; the window lands in LDS buffer (kw - kb0) / 8 % 2 as
  // [scale | zero][row][8 groups].
  const uint32_t goff_win = (uint32_t)tg * (uint32_t)p.groups * 2u;
  // A window load with real == false reads nothing (an empty descriptor) and
  // returns zeros.
  auto load_win = [&](int kw, bool real) __attribute__((always_inline)) {
    const int n = real ? sbytes : 0;
    swin[0] = load16_bounded(sb, n, goff_win, kw * 2);
    swin[1] = load16_bounded(zb, n, goff_win, kw * 2);
  };
  auto store_win = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<u32x4*>(winbase + buf * PG_WINBUF + tg * 16) = swin[0];
    *reinterpret_cast<u32x4*>(winbase + buf * PG_WINBUF + PG_WINBUF / 2 + tg * 16) = swin[1];
  };

  auto store_x = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < XCH; ++r) {
      const u32x4 v = W4 ? interleave_w4_order(xs[r]) : xs[r];
      *reinterpret_cast<u32x4*>(xstage + loff_x + r * 32 * PG_XROW * 2) = v;
    }
  };

  uint32_t w4k[3] = {0x000F000Fu, 0x00F000F0u, 0x64006400u};
#pragma unroll
  for (int i = 0; i < 3; ++i) asm volatile("" : "+v"(w4k[i]));

  // Scale and zero of the block the next M phase dequantises (local block j), and
  // whether every lane of the wave may take the one-rounding dequantisation.
  half_t sh[2], zh[2];
  auto fetch_sz = [&](int j) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if constexpr (SWIN) {
        const half_t* w = reinterpret_cast<const half_t*>(winbase + ((j / PG_WIN) & 1) * PG_WINBUF);
        const int e = (64 * wg + 32 * t + c32) * PG_WIN + j % PG_WIN;
        sh[t] = w[e];
        zh[t] = w[PG_WINBUF / 4 + e];
      } else {
        sh[t] = __builtin_bit_cast(half_t, (uint16_t)sr[t]);
        zh[t] = __builtin_bit_cast(half_t, (uint16_t)zr[t]);
      }
    }
    return (bool)__all(one_rounding_exact<QBITS>(sh[0], zh[0]) & one_rounding_exact<QBITS>(sh[1], zh[1]));
  };
  // Step s of row tile t of the block in weight buffer B -> wf[t][s].
  // Half (part 0: elements 0-3, part 1: elements 4-7) of step s of row tile t,
  // one rounding.
  auto dq_half = [&](auto buf_c, int t, int s, int part) __attribute__((always_inline)) {
    constexpr int B = decltype(buf_c)::value;
    const half2v s2 = {sh[t], sh[t]}, z2 = {zh[t], zh[t]};
    half4v h;
    if constexpr (W4) {
      const uint32_t x = wr[B][t][0][s];
      h = w4_half_one_rounding(part ? x >> 8 : x, s2, z2, w4k);
    } else {
      h = w8_half_one_rounding(wr[B][t][s >> 1][2 * (s & 1) + part], s2, z2);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) wf[t][s][4 * part + e] = h[e];
    // Pin the result here: the exact redo after the MFMAs overwrites wf, so without
    // this the compiler sinks the whole one-rounding dequantisation out of the MFMA
    // sequence into the branch where it survives, after the last MFMA.
    asm volatile("" : "+v"(wf[t][s]));
  };
  auto dq_step = [&](auto fast_c, auto buf_c, int t, int s) __attribute__((always_inline)) {
    constexpr bool F = decltype(fast_c)::value;
    constexpr int B = decltype(buf_c)::value;
    if constexpr (F) {
      dq_half(buf_c, t, s, 0);
      dq_half(buf_c, t, s, 1);
    } else {
      const float sf = (float)sh[t], zf = (float)zh[t];
      if constexpr (W4)
        wf[t][s] = w4_frag_exact(wr[B][t][0][s], sf, zf);
      else
        wf[t][s] = w8_frag_exact(wr[B][t][s >> 1][2 * (s & 1)], wr[B][t][s >> 1][2 * (s & 1) + 1], sf, zf);
    }
  };

  // M phase: op i reads X fragment (k step i/4, row tile i%4) -- lane (c32, hh)
  // reads row 32(i%4) + c32, k = 32hh + 8(i/4) .. +7 -- and issues the MFMAs of
  // both weight row tiles with it.  Fragments come PG_READ_AHEAD ops ahead through
  // a register ring; the sched_barriers pin that order.  The wave also dequantises
  // the next block (weight buffer B) into the fragments the MFMAs have finished
  // with, spread over the ops of the following steps (step 3 after the last op),
  // so the vector work of the next block runs under this block's MFMAs.
  const lds_half8v* xfrag = (const lds_half8v*)(xstage + (c32 * PG_XROW + 32 * hh) * 2);
  // The M phase always runs the one-rounding dequantisation of the next block,
  // branch-free (a branch costs about as much as a whole word's dequantisation, and
  // two copies of the MFMA sequence would not keep one register assignment for
  // the accumulators).  When a lane's scale/zero pair is not exact in one rounding
  // the wave redoes the block with the fp32 FMA after the MFMAs (next_exact).
  auto m_phase = [&](auto buf_c) __attribute__((always_inline)) {
    constexpr int NOPS = 16, RING = PG_READ_AHEAD + 1;
    // The MFMA phase's wave issues ahead of its SIMD partner's memory phase.
    __builtin_amdgcn_s_setprio(1);
    half8v ring[RING];
    auto read_op = [&](int i) __attribute__((always_inline)) -> half8v {
      return xfrag[((i & 3) * 32 * PG_XROW + (i >> 2) * 8) / 8];
    };
#pragma unroll
    for (int i = 0; i < PG_READ_AHEAD; ++i) ring[i] = read_op(i);
#pragma unroll
    for (int i = 0; i < NOPS; ++i) {
      if (i + PG_READ_AHEAD < NOPS) ring[(i + PG_READ_AHEAD) % RING] = read_op(i + PG_READ_AHEAD);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[t][i & 3] = mfma32(wf[t][i >> 2], ring[i % RING], acc[t][i & 3]);
      // Steps 0-2 of the next block, half a (row tile, step) per op from op 4 on:
      // step s is last read by op 4s+3.
      if (i >= 4) dq_half(buf_c, ((i - 4) >> 1) & 1, (i - 4) >> 2, (i - 4) & 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    dq_step(std::true_type{}, buf_c, 0, 3);
    dq_step(std::true_type{}, buf_c, 1, 3);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int m = 0; m < 4; ++m) asm volatile("" ::"v"(acc[t][m]));
    __builtin_amdgcn_s_setprio(0);
  };

  // The barrier is written out (s_barrier after lgkmcnt(0)) so that the compiler
  // does not turn it into a wait for the loads in flight.
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using YES = std::true_type;
  using NO = std::false_type;

  // Every global load below is issued unconditionally, so that each iteration
  // issues the same loads in the same order and the compiler's in-order wait
  // counts stay exact (a conditional load makes it wait for everything in
  // flight).  Loads past a group's last block read other blocks or, past the
  // buffers, zeros from the bounded descriptors; their results are never used.
  // Prologue: stage block 0 (X, weights, first scale window), dequantise it, and
  // start the loads of blocks 1 and 2.
  if constexpr (SWIN)
    load_win(kb0, true);
  else
    load_sz(kb0);
  load_w(kb0, B0{});
  load_w(kb0 + 1, B1{});
  load_x(kb0);
  if constexpr (SWIN) store_win(0);
  store_x();
  barrier();
  {
    const bool fast0 = fetch_sz(0);
    if (fast0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) { dq_step(YES{}, B0{}, 0, s); dq_step(YES{}, B0{}, 1, s); }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) { dq_step(NO{}, B0{}, 0, s); dq_step(NO{}, B0{}, 1, s); }
    }
  }
  if constexpr (!SWIN) load_sz(kb0 + 1);
  load_x(kb0 + 1);
  load_w(kb0 + 2, B0{});
  barrier();
  if (group == 1) barrier();   // group 1 runs one phase behind
  bool fast = fetch_sz(1);
  if constexpr (!SWIN) load_sz(kb0 + 2);
  // Local block j: the M phase multiplies block j and dequantises block j+1 (weight
  // buffer (j+1)%2); the V phase writes the X tile of block j+1 to LDS, fetches
  // the scale/zero of block j+2 and starts the loads of X(j+2) and of the weights
  // of block j+3 (into the buffer the M phase just emptied).  Scale windows: the
  // next window is loaded in the V phase of its predecessor's fifth block, written
  // to LDS in that of the sixth and first read two V phases later (every phase
  // ends in a barrier).  Unrolled by two so the weight buffers are static.
  auto step = [&](int j, auto buf_c) __attribute__((always_inline)) {
    using BN = decltype(buf_c);   // buffer of block j+1 (and of block j+3)
    m_phase(BN{});
    if (!fast && j + 1 < nown) {
#pragma unroll
      for (int s = 0; s < 4; ++s) { dq_step(NO{}, BN{}, 0, s); dq_step(NO{}, BN{}, 1, s); }
    }
    barrier();
    const int jn = j + 1;
    const bool next_win = SWIN && (jn / PG_WIN + 1) * PG_WIN < nown;
    if (jn < nown) {
      // The scale/zero reads go first: LDS operations of a wave complete in order,
      // and behind the X tile writes they would wait for all of them.
      if (j + 2 < nown) fast = fetch_sz(j + 2);
      store_x();
      if constexpr (SWIN) {
        if (jn % PG_WIN == 5 && next_win) store_win((jn / PG_WIN + 1) & 1);
      }
    }
    load_x(kb0 + j + 2);
    if constexpr (SWIN)
      load_win(kb0 + (jn / PG_WIN + 1) * PG_WIN, jn % PG_WIN == 4 && next_win);
    else
      load_sz(kb0 + j + 3);
    load_w(kb0 + j + 3, BN{});
    barrier();
  };
  int j = 0;
  for (; j + 1 < nown; j += 2) {
    step(j, B1{});
    step(j + 1, B0{});
  }
  if (j < nown) step(j, B1{});
  wait_vmcnt_imm<0>();   // loads past the end
  // Same barrier count for both groups: group g passes 2 + g + 2*nown(g).
  {
    const int bars0 = 2 + 2 * (MSPLIT ? nk : half), bars1 = 3 + 2 * (MSPLIT ? nk : nk - half);
    const int mine = group == 0 ? bars0 : bars1;
    const int target = bars0 > bars1 ? bars0 : bars1;
    for (int i = mine; i < target; ++i) barrier();
  }

  // K-split sum: group 0 finishes row tiles 0-1, group 1 row tiles 2-3; each hands
  // the other half to its partner wave (same SIMD, same columns) through LDS.  The
  // rounded fp16 sums then go to an output tile in LDS (rows padded to PG_OROW) so
  // that the output stage reads whole 16-byte row chunks: every global access of
  // the output (and of the residual for the gate-add stage) is a full-row burst.
  auto finish = [&](auto mine_c) __attribute__((always_inline)) {
    constexpr int MINE = decltype(mine_c)::value, GIVE = 2 - MINE;
    char* own = smem + (group * 4 + wg) * PG_RED;
    const char* partner = smem + ((1 - group) * 4 + wg) * PG_RED;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 v = {acc[t][GIVE + j][4 * q], acc[t][GIVE + j][4 * q + 1], acc[t][GIVE + j][4 * q + 2],
                             acc[t][GIVE + j][4 * q + 3]};
          *reinterpret_cast<floatx4*>(own + (((t * 2 + j) * 4 + q) * 64 + lane) * 16) = v;
        }
    barrier();
    if (p.ksplit > 1) {
      // Split K: the fp32 sums of this K range go to the split's partial rows.
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = m0 + 32 * (MINE + j) + c32;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const floatx4 o = *reinterpret_cast<const floatx4*>(partner + (((t * 2 + j) * 4 + q) * 64 + lane) * 16);
            const floatx4 sv = {acc[t][MINE + j][4 * q] + o[0], acc[t][MINE + j][4 * q + 1] + o[1],
                                acc[t][MINE + j][4 * q + 2] + o[2], acc[t][MINE + j][4 * q + 3] + o[3]};
            const int n = n0 + 64 * wg + 32 * t + 8 * q + 4 * hh;
            if (m < p.M) {
              float* prow = p.part + ((int64_t)split * p.M + m) * p.N;
              if ((p.N & 3) == 0 && n + 3 < p.N) {
                *reinterpret_cast<floatx4*>(prow + n) = sv;
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  if (n + e < p.N) prow[n + e] = sv[e];
              }
            }
          }
        }
      return;
    }
    half4v out[2][2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 o = *reinterpret_cast<const floatx4*>(partner + (((t * 2 + j) * 4 + q) * 64 + lane) * 16);
          out[t][j][q] = half4v{(half_t)(acc[t][MINE + j][4 * q] + o[0]), (half_t)(acc[t][MINE + j][4 * q + 1] + o[1]),
                                (half_t)(acc[t][MINE + j][4 * q + 2] + o[2]),
                                (half_t)(acc[t][MINE + j][4 * q + 3] + o[3])};
        }
    barrier();  // every partner read done: the tile may overwrite the exchange area
    half_t* tile = reinterpret_cast<half_t*>(smem);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<half4v*>(tile + (32 * (MINE + j) + c32) * PG_OROW + 64 * wg + 32 * t + 8 * q + 4 * hh) =
              out[t][j][q];
  };
  if constexpr (MSPLIT) {
    // Both groups are past their last K block (the barrier counts above match), so the
    // X stages are free: each wave writes its rounded 64 x 128 sums straight into the
    // group's half of the output tile.
    half_t* tile = reinterpret_cast<half_t*>(smem);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<half4v*>(tile + (PG_BM * group + 32 * m + c32) * PG_OROW + 64 * wg + 32 * t + 8 * q +
                                     4 * hh) =
              half4v{(half_t)acc[t][m][4 * q], (half_t)acc[t][m][4 * q + 1], (half_t)acc[t][m][4 * q + 2],
                     (half_t)acc[t][m][4 * q + 3]};
  } else {
    if (group == 0)
      finish(std::integral_constant<int, 0>{});
    else
      finish(std::integral_constant<int, 2>{});
    if (p.ksplit > 1) return;   // partial rows written; splitk_reduce_kernel finishes
  }
  barrier();

  // Output stage: thread tid takes 16-byte chunk tid % 32 of tile rows tid / 32 + 16i.
  const half_t* tile = reinterpret_cast<const half_t*>(smem);
  const int ochunk = tid & 31, orow = tid >> 5;
  const int n = n0 + 8 * ochunk;
  auto store_tile = [&](auto epi_c) __attribute__((always_inline)) {
    constexpr int EPI = decltype(epi_c)::value;
#pragma unroll 2
    for (int i = 0; i < BM / 16; ++i) {
      const int r = orow + 16 * i, m = m0 + r;
      half8v v = *reinterpret_cast<const half8v*>(tile + r * PG_OROW + 8 * ochunk);
      if (m >= p.M) continue;
      if (EPI == GEMM_QK_NORM) {
        // Per-head RMSNorm: 16 lanes hold one 128-column head row.
        float x[8];
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] = (float)v[e];
          ss = fmaf(x[e], x[e], ss);
        }
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        const float inv = rsqrtf(ss / 128.f + p.eps);
        const int dh = 8 * (ochunk & 15);
        const half8v w = *reinterpret_cast<const half8v*>(p.norm_w + dh);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = f32_to_f16(x[e] * inv * (float)w[e]);
      }
      if (EPI == GEMM_GELU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = gelu_erf_half(v[e]);
      }
      if (EPI == GEMM_RESIDUAL_ADD) {
        float* rrow = p.residual + (int64_t)m * p.N;
        if (vec_store && n + 8 <= p.N) {
          floatx4 r0 = *reinterpret_cast<const floatx4*>(rrow + n);
          floatx4 r1 = *reinterpret_cast<const floatx4*>(rrow + n + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            r0[e] += (float)v[e];
            r1[e] += (float)v[4 + e];
          }
          *reinterpret_cast<floatx4*>(rrow + n) = r0;
          *reinterpret_cast<floatx4*>(rrow + n + 4) = r1;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < p.N) rrow[n + e] += (float)v[e];
        }
      } else if (EPI == GEMM_GATE_ADD) {
        float* rrow = p.residual + (int64_t)m * p.N;
        if (vec_store && n + 8 <= p.N) {
          floatx4 r0 = *reinterpret_cast<const floatx4*>(rrow + n);
          floatx4 r1 = *reinterpret_cast<const floatx4*>(rrow + n + 4);
          const floatx4 g0 = *reinterpret_cast<const floatx4*>(p.gate + n);
          const floatx4 g1 = *reinterpret_cast<const floatx4*>(p.gate + n + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            r0[e] = fmaf((float)v[e], g0[e], r0[e]);
            r1[e] = fmaf((float)v[4 + e], g1[e], r1[e]);
          }
          *reinterpret_cast<floatx4*>(rrow + n) = r0;
          *reinterpret_cast<floatx4*>(rrow + n + 4) = r1;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < p.N) rrow[n + e] = fmaf((float)v[e], p.gate[n + e], rrow[n + e]);
        }
      } else {
        half_t* yrow = p.y + (int64_t)m * p.N;
        if (vec_store && n + 8 <= p.N) {
          *reinterpret_cast<half8v*>(yrow + n) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < p.N) yrow[n + e] = v[e];
        }
      }
    }
  };
  if (p.epilogue == GEMM_GELU)
    store_tile(std::integral_constant<int, GEMM_GELU>{});
  else if (p.epilogue == GEMM_GATE_ADD)
    store_tile(std::integral_constant<int, GEMM_GATE_ADD>{});
  else if (p.epilogue == GEMM_RESIDUAL_ADD)
    store_tile(std::integral_constant<int, GEMM_RESIDUAL_ADD>{});
  else if (p.epilogue == GEMM_QK_NORM)
    store_tile(std::integral_constant<int, GEMM_QK_NORM>{});
  else
    store_tile(std::integral_constant<int, GEMM_STORE>{});
}

bool pingpong_supported(const GemmParams& p, int storage) {
  if (storage != ANIMA_STORAGE_W4 && storage != ANIMA_STORAGE_W8) return false;
  if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % PG_BK != 0 || p.groups != p.K / PG_BK) return false;
  if (!aligned16(p.x) || !aligned16(p.w) || p.row_stride % 16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.scale) & 1u) || (reinterpret_cast<uintptr_t>(p.zero) & 1u)) return false;
  const int64_t lim = 0x7fffffff;
  return (int64_t)p.M * p.K * 2 <= lim && (int64_t)p.N * p.row_stride <= lim && (int64_t)p.N * p.groups * 2 <= lim;
}

// Sum of the K splits in a fixed order, rounded once to fp16: y = half(sum_s part[s]),
// or residual += float(half(sum_s part[s])) when residual is given.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, half_t* __restrict__ y,
                                                            float* __restrict__ residual, int64_t count, int ksplit,
                                                            int vec) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= count) return;
  if (vec && i0 + 4 <= count) {
    // Eight splits' loads go out together (indices past the last split re-read it and
    // add -0, the identity of fp32 addition even for a -0 sum), then the adds run in
    // split order: one memory round trip per eight splits instead of one per split.
    floatx4 acc = floatx4{-0.f, -0.f, -0.f, -0.f};
    for (int s0 = 0; s0 < ksplit; s0 += 8) {
      floatx4 b[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const floatx4*>(part + min(s0 + j, ksplit - 1) * count + i0);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += s0 + j < ksplit ? b[j] : floatx4{-0.f, -0.f, -0.f, -0.f};
    }
    const half4v h = {(half_t)acc[0], (half_t)acc[1], (half_t)acc[2], (half_t)acc[3]};
    if (residual) {
      floatx4 r = *reinterpret_cast<const floatx4*>(residual + i0);
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += (float)h[e];
      *reinterpret_cast<floatx4*>(residual + i0) = r;
    } else {
      *reinterpret_cast<half4v*>(y + i0) = h;
    }
  } else {
    for (int64_t i = i0; i < count && i < i0 + 4; ++i) {
      float acc = part[i];
      for (int s = 1; s < ksplit; ++s) acc += part[s * count + i];
      if (residual)
        residual[i] += (float)(half_t)acc;
      else
        y[i] = (half_t)acc;
    }
  }
}

int pingpong_ksplit(const GemmParams& p, int storage) {
  if (!pingpong_supported(p, storage) || (p.epilogue != GEMM_STORE && p.epilogue != GEMM_RESIDUAL_ADD)) return 1;
  const int64_t tiles = (int64_t)((p.M + PG_BM - 1) / PG_BM) * ((p.N + PG_BN - 1) / PG_BN);
  if (tiles >= 128) return 1;
  const int nk = p.K / PG_BK;
  const bool swin = p.groups % PG_WIN == 0 && aligned16(p.scale) && aligned16(p.zero);
  int best = 1;
  for (int k = 2; k <= 8; ++k) {
    if (nk % k != 0 || nk / k < 16 || (swin && (nk / k) % PG_WIN != 0) || tiles * k > 256) continue;
    best = k;
  }
  return best;
}

// A single launch of p takes the M-split form when its 256-row tiles still fill at least
// two whole rounds of the chip (512 workgroups): it then pays half as many first loads
// and output stages per output, and no partial-sum exchange.  Fewer tiles would leave
// CUs idle that the 128-row form fills.  Split-K launches keep the K-split form.
bool pingpong_msplit(const GemmParams& p, int storage) {
  if (!pingpong_supported(p, storage) || pingpong_ksplit(p, storage) > 1) return false;
  const int64_t wide = (int64_t)((p.M + 2 * PG_BM - 1) / (2 * PG_BM)) * ((p.N + PG_BN - 1) / PG_BN);
  return wide >= 512;
}

template <int STORAGE, bool SWIN>
static void launch_pingpong_t(const GemmGroup& g, int64_t tiles, bool msplit, hipStream_t stream) {
  if (msplit)
    hipLaunchKernelGGL((pingpong_gemm_kernel<STORAGE, SWIN, true>), dim3((unsigned)tiles), dim3(PG_NT), 0, stream, g);
  else
    hipLaunchKernelGGL((pingpong_gemm_kernel<STORAGE, SWIN, false>), dim3((unsigned)tiles), dim3(PG_NT), 0, stream, g);
}

void launch_pingpong_group(const GemmParams* ps, int count, int storage, hipStream_t stream) {
  if (count < 1 || count > PG_GROUP) fail(ANIMA_E_INVALID_ARGUMENT, "ping-pong GEMM group holds 1 to 3 problems");
  GemmGroup g{};
  bool swin = true;
  int64_t tiles = 0;
  const bool msplit = count == 1 && pingpong_msplit(ps[0], storage);
  const int bm = msplit ? 2 * PG_BM : PG_BM;
  for (int i = 0; i < count; ++i) {
    const GemmParams& p = ps[i];
    if (!pingpong_supported(p, storage)) fail(ANIMA_E_INVALID_SHAPE, "ping-pong GEMM: unsupported shape or alignment");
    if (p.K != ps[0].K) fail(ANIMA_E_INVALID_SHAPE, "ping-pong GEMM group: problems must share K");
    if (p.epilogue == GEMM_GATE_ADD && (!p.residual || !p.gate))
      fail(ANIMA_E_INVALID_ARGUMENT, "GEMM gate-add epilogue needs residual and gate");
    if (p.epilogue == GEMM_RESIDUAL_ADD && !p.residual)
      fail(ANIMA_E_INVALID_ARGUMENT, "GEMM residual-add epilogue needs the residual");
    if (p.epilogue == GEMM_QK_NORM && (!p.norm_w || p.N % 128 != 0 || !aligned16(p.norm_w)))
      fail(ANIMA_E_INVALID_ARGUMENT, "GEMM Q/K-norm epilogue needs 128-column heads and the norm weight");
    swin = swin && p.groups % PG_WIN == 0 && aligned16(p.scale) && aligned16(p.zero);
    if (p.ksplit > 1) {
      if (count != 1 || !p.part || p.ksplit != pingpong_ksplit(p, storage))
        fail(ANIMA_E_INVALID_ARGUMENT, "ping-pong GEMM: split K needs a single plain GEMM and its partial buffer");
    }
    g.p[i] = p;
    g.first_tile[i] = (int)tiles;
    // 16-byte output accesses: every row start 16-byte aligned.
    g.vec[i] = p.epilogue == GEMM_GATE_ADD       ? (aligned16(p.residual) && aligned16(p.gate) && p.N % 8 == 0 ? 1 : 0)
               : p.epilogue == GEMM_RESIDUAL_ADD ? (aligned16(p.residual) && p.N % 8 == 0 ? 1 : 0)
                                                 : (aligned16(p.y) && p.N % 8 == 0 ? 1 : 0);
    tiles += (int64_t)((p.M + bm - 1) / bm) * ((p.N + PG_BN - 1) / PG_BN) * (p.ksplit > 1 ? p.ksplit : 1);
    if (tiles > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "GEMM grid too large");
  }
  for (int i = count; i < PG_GROUP; ++i) g.first_tile[i] = (int)tiles;
  g.count = count;
  if (tiles <= 0) return;
  if (storage == ANIMA_STORAGE_W4) {
    if (swin)
      launch_pingpong_t<ANIMA_STORAGE_W4, true>(g, tiles, msplit, stream);
    else
      launch_pingpong_t<ANIMA_STORAGE_W4, false>(g, tiles, msplit, stream);
  } else {
    if (swin)
      launch_pingpong_t<ANIMA_STORAGE_W8, true>(g, tiles, msplit, stream);
    else
      launch_pingpong_t<ANIMA_STORAGE_W8, false>(g, tiles, msplit, stream);
  }
  ANIMA_HIP(hipGetLastError());
  if (count == 1 && ps[0].ksplit > 1) {
    const GemmParams& p = ps[0];
    const int64_t n = (int64_t)p.M * p.N;
    float* res = p.epilogue == GEMM_RESIDUAL_ADD ? p.residual : nullptr;
    // The vector form reads split s at part + s*n + i0 as 16 bytes: aligned for every
    // split only when n is a multiple of 4.
    const int vec = (n % 4 == 0 && aligned16(p.part) && (res ? aligned16(res) : aligned8(p.y))) ? 1 : 0;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, stream, p.part, p.y, res,
                       n, p.ksplit, vec);
    ANIMA_HIP(hipGetLastError());
  }
}

void launch_pingpong(const GemmParams& p, int storage, hipStream_t stream) {
  launch_pingpong_group(&p, 1, storage, stream);
}

void launch_splitk_reduce(const float* part, half_t* y, int64_t count, int ksplit, hipStream_t stream) {
  const int vec = (count % 4 == 0 && aligned16(part) && aligned8(y)) ? 1 : 0;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((count + 1023) / 1024)), dim3(256), 0, stream, part, y,
                     static_cast<float*>(nullptr), count, ksplit, vec);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
