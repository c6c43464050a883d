// Flash attention, 256-query-row variant for long sequences (gfx950).
//
// Same maths and numerics as the 128-row kernel in attention.hip (S^T = K Q^T on
// v_mfma_f32_32x32x16_f16, fp32 online softmax in base 2, fp16 P, O^T += V^T P^T,
// Q RMSNorm + split-half RoPE fused into the Q fragment load), organised so that
// the matrix cores and the vector ALUs of every SIMD stay busy at the same time:
//   * 8 waves x 32 query rows share one K/V tile stream (1 workgroup per CU,
//     2 waves per SIMD).  The waves form two groups, one wave of each group per
//     SIMD (waves w and w+4 share a SIMD).  Work per key tile j is split into two
//     phases:
//       G(j)  MFMA phase: QK^T of tile j and PV of tile j-1 on the matrix cores,
//             as one fixed sequence of MFMAs whose LDS fragment reads run a few
//             MFMAs ahead;
//       X(j)  VALU phase: the tile copies (below), masking, exp2, fp16 P and the
//             fp32 row sums of tile j (row max and O rescale only when needed).
//     Phases are separated by workgroup barriers, and group 1 runs one phase
//     behind group 0 (one extra barrier at the start, group 0 one at the end), so
//     in every barrier interval one wave of each SIMD issues MFMAs while the
//     other issues VALU work ("ping-pong").  A single wave issues VALU work at
//     about half the SIMD's VALU rate, so the two streams overlap instead of both
//     waves waiting on the same unit.
//   * K and V tiles (64 keys) are copied global -> VGPR -> LDS: during X(j) a wave
//     stores its staged segments of tile j+2 (ds_write_b128) and issues the
//     buffer loads of tile j+4 into the staging registers those leave (two
//     buffers), so two tile periods hide the load latency, and the LDS writes
//     never queue ahead of the same wave's fragment reads.  Buffer
//     descriptors bound every tile by the last key row in use: rows past it read
//     as zeros without touching memory.
//   * Rows are padded in LDS (K: +16 B, V: +64 B) so the fragment reads hit
//     distinct banks (64 banks x 4 B); padding instead of an XOR swizzle keeps
//     every fragment address "per-lane base + immediate".  V^T fragments come
//     straight from the row-major V tile with ds_read_b64_tr_b16.
//   * Q carries scale * log2(e) and the QK MFMAs start from C = -m, so the scores
//     come out as exp2 arguments.  Exps use the running max without computing the
//     tile's row max: a lane's share of the tile's row sum above 2^15 (or not
//     finite), or a row with no max yet, sends the wave to the exact path (row max,
//     O / row-sum rescale, exps again), which the first tile always takes.  Four LDS
//     stages: tile j is read by QK while tile j-1 is read by PV and tile j+2 is
//     written.
//   * Everything (Q, O accumulators, scores, row sums) lives in the 256 VGPRs a
//     wave gets at 2 waves/SIMD.
#include <type_traits>

#include "flash_common.hpp"

namespace anima {

constexpr int F2_WAVES = 8;
constexpr int F2_NT = 64 * F2_WAVES;
constexpr int F2_BN = 64;
constexpr int F2_STAGES = 4;
constexpr float F2_LAZY_LIMIT = 32768.f;   // largest tile row-sum share the fast path accepts
constexpr int F2_READ_AHEAD = 4;    // MFMA operand fragments read from LDS ahead of their MFMA
// PERSIST: the next batch entry's Q rows load in the key loop's last two tile periods
// (true) or after the key loop, behind the epilogue (false; 1.2 us slower on a B4 cross
// attention of 4096 queries over 418/506/86/149 keys).
constexpr bool F2_Q_PREFETCH = true;
static_assert(FLASH_V2_ROWS == 32 * F2_WAVES, "one 32-row block per wave");

// PERSIST: the grid covers query tiles x heads and every workgroup walks all batch entries
// of its (tile, head), so the work per workgroup is the same.  The workgroups of head h
// start at entry h % nbatch: at any moment the heads are spread over entries of different
// key lengths, so their Q-row loads and O-row stores do not all fall at the same time.
// Across entries the next entry's Q rows load into the tile-staging registers in this
// entry's last two tile periods, and its first two K/V tiles load before this entry's
// epilogue, so neither the Q rows' HBM round trip nor the first tiles' wait is paid again
// per entry (measured on a B4 cross attention, 4096 queries over 418/506/86/149 keys: the
// Q wait went from 4.9 us to the 2.7 us of the fragment's own norm and barriers).
// Requires no fused Q RoPE, no key splits and the per-(batch, head) Q rows within 2 GiB
// (launch_flash_v2 checks).
template <int D, bool PERSIST = false>
__global__ __launch_bounds__(F2_NT, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_attention_v2_kernel(FlashParams p) {
  constexpr int DCH = D / 8;             // 16-byte data chunks per row
  constexpr int QS = D / 16;
  constexpr int OB = D / 32;
  constexpr int KROW = D + 8;            // padded K row (halfs)
  constexpr int VROW = D + 32;           // padded V row (halfs)
  constexpr int KTILE = F2_BN * KROW, VTILE = F2_BN * VROW;   // halfs

  // One LDS object per stage: every access names its stage at compile time, so the
  // compiler can tell an in-flight global->LDS copy into one stage from reads of
  // another and does not make the reads wait for the copy.
  __shared__ __attribute__((aligned(1024))) half_t K0[KTILE], K1[KTILE], K2[KTILE], K3[KTILE];
  __shared__ __attribute__((aligned(1024))) half_t V0[VTILE], V1[VTILE], V2[VTILE], V3[VTILE];
  // PERSIST: each wave's copy of the Q norm weight, written in the first entry.
  __shared__ __attribute__((aligned(16))) half_t QW[PERSIST ? F2_NT / 64 * D : 8];
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

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  // Waves w and w+4 share a SIMD; one of them is in each group.
  const int group = wave >> 2;

  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  int split = 0;
  if (p.kv_splits > 1) {
    split = lb % p.kv_splits;
    lb /= p.kv_splits;
  }
  // Consecutive logical blocks share an XCD (and its L2).  They take p.head_group heads of
  // one query tile, then the next query tile, and the remaining heads vary slowest.  With
  // head_group 1 an XCD gets whole heads (their K/V stay in its L2) over every batch entry,
  // so batches of different key lengths spread evenly over the XCDs; with 8 (single-image
  // launches that fill the chip) an XCD's reads spread over 8 heads' pieces of each token
  // row and it needs fewer of the RoPE table rows.
  const int hgp = PERSIST ? 1 : p.head_group;   // the persistent form keeps whole heads per XCD
  const int hl = lb % hgp;
  lb /= hgp;
  const int qt = lb % p.q_tiles;
  lb /= p.q_tiles;
  const int head = (PERSIST ? lb : lb / p.nbatch) * hgp + hl;
  // PERSIST: the workgroups of head h start at entry h % nbatch and wrap around, so at any
  // time the heads are spread over the entries (of different key lengths) and their Q-row
  // loads and O-row stores do not all fall at the same moment.
  int b = PERSIST ? head % p.nbatch : lb % p.nbatch;
  const int kvh = head / p.group;
  const int q0 = qt * FLASH_V2_ROWS;
  const int wq0 = q0 + wave * 32;
  // With key splits (non-causal, no key lengths) this workgroup's keys start at kofs;
  // kv_len and kend count keys from there.
  const int kofs = p.kv_splits > 1 ? split * p.kv_chunk : 0;
  // Valid keys of batch entry bb, and the keys this workgroup uses of them.
  auto entry_kv_len = [&](int bb) __attribute__((always_inline)) -> int {
    int len = p.Sk;
    if (p.key_lengths_dev) {
      // A scalar load (constant address space: the kernel never writes the lengths).  A
      // vector load here would have to wait for every vector memory operation in flight,
      // in a later batch entry (PERSIST) the previous entry's O stores among them.
      int L = *reinterpret_cast<const __attribute__((address_space(4))) int*>(
          reinterpret_cast<uintptr_t>(p.key_lengths_dev + bb));
      len = L < 1 ? 1 : (L > p.Sk ? p.Sk : L);
    } else if (p.use_host_lengths) {
      len = p.host_lengths[bb];
    }
    if (p.kv_splits > 1) len = max(0, min(len, kofs + p.kv_chunk) - kofs);
    return len;
  };
  auto entry_kend = [&](int len) __attribute__((always_inline)) -> int {
    return p.causal ? min(len, q0 + FLASH_V2_ROWS) : len;
  };
  auto entry_k = [&](int bb) __attribute__((always_inline)) -> const char* {
    return reinterpret_cast<const char*>(p.k + (int64_t)bb * p.k_batch + (int64_t)kvh * p.k_head + (int64_t)kofs * p.k_tok);
  };
  auto entry_v = [&](int bb) __attribute__((always_inline)) -> const char* {
    return reinterpret_cast<const char*>(p.v + (int64_t)bb * p.v_batch + (int64_t)kvh * p.v_head + (int64_t)kofs * p.v_tok);
  };

  constexpr int CPT = F2_BN * DCH / F2_NT;   // chunks per thread per tensor per tile
  constexpr int RSTEP = F2_NT / DCH;
  constexpr int NCP = 2 * CPT;               // copies per thread per tile: K chunks, then V chunks
  static_assert(CPT * F2_NT == F2_BN * DCH && F2_NT % DCH == 0, "tile splits evenly over the threads");
  // Carried from one batch entry to the next (PERSIST): the tile-staging registers (the
  // next entry's tiles 0 and 1 in flight) and its Q fragment.
  u32x4 stg2[2][NCP];
  half8v qf[QS];

  for (int entry = 0;; ++entry) {   // batch entries (one pass unless PERSIST)
  // PERSIST: the lane index is re-derived per entry (v_mbcnt in an asm the compiler
  // cannot hoist) so that per-lane values are computed in the entry that uses them
  // instead of living across all entries.
  int tid = threadIdx.x;
  if constexpr (PERSIST) {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    tid = wave * 64 + l;
  }
  const int lane = tid & 63;
  const int c32 = lane & 31, hh = lane >> 5;
  const int jj = lane & 15, gg = lane >> 4;
  const int qi = wq0 + c32;
  const int kv_len = entry_kv_len(b);
  const int kend = entry_kend(kv_len);
  const int ntiles = (kend + F2_BN - 1) / F2_BN;
  const char* const kbase = entry_k(b);
  const char* const vbase = entry_v(b);
  uint64_t rp[QStage<D>::LOADS];   // RoPE table pieces (never with PERSIST)
  uint32_t wn = 0;                 // Q norm weight piece

  // Tile copies: thread t moves the 16-byte chunks t + F2_NT*r (r < CPT) of the K
  // tile and of the V tile (chunk -> row, column: 16-lane coalesced rows in
  // memory, padded rows in LDS), so only the tile's own bytes move.  Chunk r sits
  // RSTEP*r rows below chunk 0.  A tile is read through one buffer descriptor per
  // tensor whose size ends at the last key row this workgroup uses (kend): rows
  // past it, and every row of a tile past the last one, read as zeros without
  // touching memory.  64 key rows fit in 2^31 bytes (checked on the host), so the
  // per-lane offsets and sizes are 32-bit.
  const int crow = tid / DCH, cch = tid % DCH;
  const uint32_t ktok2 = (uint32_t)p.k_tok * 2u, vtok2 = (uint32_t)p.v_tok * 2u;
  uint32_t goff_k[CPT], goff_v[CPT];
#pragma unroll
  for (int r = 0; r < CPT; ++r) {
    goff_k[r] = (uint32_t)(crow + RSTEP * r) * ktok2 + (uint32_t)cch * 16u;
    goff_v[r] = (uint32_t)(crow + RSTEP * r) * vtok2 + (uint32_t)cch * 16u;
  }
  const uint32_t loff_k = (uint32_t)(crow * KROW + cch * 8) * 2u;
  const uint32_t loff_v = (uint32_t)(crow * VROW + cch * 8) * 2u;
  // Valid bytes of a tile from its first row: the descriptor of tile j spans from the
  // tile's first row to the end (column D) of the last key row in use, so rows past
  // kend read as zeros.  The loop loads tiles 4, 5, 6, ... in order, so it keeps one
  // running base pointer and one remaining-byte count per tensor and advances them by
  // a tile per load (scalar adds) instead of recomputing base + j * 64 * row_stride.
  const int64_t kstep = (int64_t)F2_BN * ktok2, vstep = (int64_t)F2_BN * vtok2;
  const int64_t kbytes = kend > 0 ? (int64_t)(kend - 1) * ktok2 + D * 2 : 0;
  const int64_t vbytes = kend > 0 ? (int64_t)(kend - 1) * vtok2 + D * 2 : 0;
  auto clamp_bytes = [](int64_t rem) __attribute__((always_inline)) -> int {
    return rem <= 0 ? 0 : (rem >= 0x7fffffff ? 0x7fffffff : (int)rem);
  };

  // Copies go global -> VGPR -> LDS: load_tile fetches this thread's chunks of a tile
  // into staging buffer j % 2, store_seg writes copy r into a stage two tile
  // periods later (two buffers keep two tiles in flight).
  auto load_at = [&](const char* kt, int nk, const char* vt, int nv, auto bufc) __attribute__((always_inline)) {
    u32x4 (&stg)[NCP] = stg2[decltype(bufc)::value];
#pragma unroll
    for (int r = 0; r < CPT; ++r) stg[r] = load16_bounded(kt, nk, goff_k[r]);
#pragma unroll
    for (int r = 0; r < CPT; ++r) stg[CPT + r] = load16_bounded(vt, nv, goff_v[r]);
  };
  auto load_tile = [&](int j, auto bufc) __attribute__((always_inline)) {
    load_at(kbase + j * kstep, clamp_bytes(kbytes - j * kstep), vbase + j * vstep, clamp_bytes(vbytes - j * vstep), bufc);
  };
  const char* k_next = kbase + 4 * kstep;
  const char* v_next = vbase + 4 * vstep;
  int64_t k_rem = kbytes - 4 * kstep, v_rem = vbytes - 4 * vstep;
  auto load_next = [&](auto bufc) __attribute__((always_inline)) {
    load_at(k_next, clamp_bytes(k_rem), v_next, clamp_bytes(v_rem), bufc);
    k_next += kstep; v_next += vstep;
    k_rem -= kstep; v_rem -= vstep;
  };
  // PERSIST: this entry's load stream is its tiles 0 .. ntiles-1 (positions 0 .. ntiles-1,
  // zero-size loads at ntiles and ntiles+1), then the next entry's Q rows in two parts of
  // NCP loads at positions qa = ntiles+2 and qa+1: the last two loads of the stream, so
  // nothing overwrites their staging buffers (position pos lands in buffer pos % 2) before
  // the key loop ends.  The Q rows load in the fragment layout (lane (c32, hh): row c32,
  // columns 16s + 8hh .. +7; rows past the sequence repeat the last row) through one
  // descriptor over the (batch, head) rows: part P holds s = NCP*P .. NCP*P + NCP-1.
  // These loads touch 32 rows with 32 bytes each per instruction, half the vector memory
  // rate of whole-row loads, but they run beside a key loop that leaves that path idle
  // most of the time, and the fragment then needs no pass through LDS.
  static_assert(QS == 2 * NCP, "one Q part fills one staging buffer");
  const uint32_t qtok2 = (uint32_t)p.q_tok * 2u;
  const int qnbytes = (int)((uint32_t)(p.Sq - 1) * qtok2 + D * 2);
  auto next_entry = [&]() __attribute__((always_inline)) { return PERSIST && entry + 1 < p.nbatch; };
  const int bn = b + 1 == p.nbatch ? 0 : b + 1;   // next entry (PERSIST)
  auto q_frag_load = [&](int bb, int s) __attribute__((always_inline)) -> u32x4 {
    const char* qb = reinterpret_cast<const char*>(p.q + (int64_t)bb * p.q_batch + (int64_t)head * p.q_head);
    const uint32_t row = (uint32_t)min(qi, p.Sq - 1);
    return load16_bounded(qb, qnbytes, row * qtok2 + (uint32_t)(32 * s + 16 * hh));
  };
  auto load_q_part = [&](int part, auto bufc) __attribute__((always_inline)) {
    u32x4 (&stg)[NCP] = stg2[decltype(bufc)::value];
#pragma unroll
    for (int r = 0; r < NCP; ++r) stg[r] = q_frag_load(bn, NCP * part + r);
  };
  // Load of stream position pos into buffer pos % 2; FIRST: one of positions 0..3 (by
  // tile index), else the next tile of the running pointers.
  auto load_slot = [&](int pos, auto bufc, auto first) __attribute__((always_inline)) {
    if constexpr (PERSIST) {
      if (F2_Q_PREFETCH && next_entry() && pos >= ntiles + 2) {
        load_q_part(pos - ntiles - 2, bufc);
        return;
      }
    }
    if constexpr (decltype(first)::value)
      load_tile(pos, bufc);
    else
      load_next(bufc);
  };
  auto store_seg = [&](int r, auto st, auto bufc) __attribute__((always_inline)) {
    u32x4 (&stg)[NCP] = stg2[decltype(bufc)::value];
    if (r < CPT)
      *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(kstage(st)) + loff_k + RSTEP * r * KROW * 2) = stg[r];
    else
      *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(vstage(st)) + loff_v + RSTEP * (r - CPT) * VROW * 2) = stg[r];
  };
  auto store_tile = [&](auto st, auto bufc) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < NCP; ++r) store_seg(r, st, bufc);
  };

  floatx16 acc[OB];
#pragma unroll
  for (int c = 0; c < OB; ++c) acc[c] = floatx16{};
  float m_run = -INFINITY;
  // Row sum of the fp32 probabilities over this lane's 32 keys of each tile (the
  // other 32 are in lane c32 + 32(1-hh)); the two halves meet at the end.  Summing
  // on the VALU costs 32 adds per tile in the VALU phase; the four MFMAs of an
  // ones x P^T product cost more (they lengthen every MFMA phase by 1/8).
  float lrow = 0.f;
  const float c2 = p.scale_log2;
  // Q carries the factor c2 = scale * log2(e) (folded in before its fp16 rounding), and
  // the first QK MFMA of each key half starts from C = MB = -mbase: all 16 entries of a
  // lane's S^T column belong to its query row, so S comes out as the exp2 argument
  // s * c2 - mbase with no per-score VALU work.  mbase is m_run once a row max exists
  // (0 before); it changes only on the exact path below.
  float mbase = 0.f;
  floatx16 MB = floatx16{};

  typedef __attribute__((address_space(3))) half8v lds_half8v;
  typedef __attribute__((address_space(3))) short4v lds_short4v;

  // Per-lane fragment bases (halfs); everything else is an immediate offset.
  const int kfrag = c32 * KROW + hh * 8;
  const int vfrag = (4 * hh + (jj >> 2)) * VROW + 16 * (gg & 1) + 4 * (jj & 3);

  floatx16 S[2];     // scores of the current tile: keys 0..31, 32..63
  half8v P[2][2];    // fp16 probabilities of the previous tile (keys 32h + 16u + ...)
  // G(0) runs the PV step of a tile "-1" in stage 3: P = 0 and V = 0 make it add
  // exact zeros (stage 3 is zeroed after the prologue's RoPE staging and first filled
  // in G(1), after two barriers).
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int u = 0; u < 2; ++u) P[h][u] = half8v{};

  // V^T fragment (c, u) of key half h: lane (d, hh) holds V[key(u, hh, 0..7)][32c + d]
  // with key(u, hh, i) = 32h + 16u + 8(i/4) + 4hh + i%4, the key order of the
  // S^T C layout, read through an LDS-space pointer ("lane base + immediate").
  auto vfrag_read = [&](auto st, int h, int u, int c) __attribute__((always_inline)) -> half8v {
    lds_short4v* vs = (lds_short4v*)vstage(st) + vfrag / 4;
    const int off = (32 * h + 16 * u) * VROW + 32 * c;
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + off / 4);
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vs + (off + 8 * VROW) / 4);
    const half4v lo_h = __builtin_bit_cast(half4v, lo);
    const half4v hi_h = __builtin_bit_cast(half4v, hi);
    return half8v{lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
  };

  // G(j): S = K_j Q^T - m (each key half's first MFMA starts from C = MB),
  // O += V_{j-1}^T P_{j-1}.
  auto g_phase = [&](int j, auto st) __attribute__((always_inline)) {
    constexpr int ST = decltype(st)::value;
    // The MFMA phase's wave issues ahead of its SIMD partner's VALU phase (the
    // partner fills the gaps): -1 % at S=4096 against equal priorities.
    __builtin_amdgcn_s_setprio(1);
    using SPREV = std::integral_constant<int, (ST + 3) % F2_STAGES>;
    const lds_half8v* ks = (const lds_half8v*)(kstage(st) + kfrag);
    // Anchor the keys-32..63 exponentials in this phase (the compiler would hoist
    // them above the barrier into the VALU phase).
    // The phase is a fixed sequence of NOPS MFMAs: QK (op i < 2*QS: key half i/QS,
    // d-step i%QS) and PV (op 2*QS + k: key half k/(4*OB), 16-key block k/OB % 2,
    // d block k%OB).  Operand fragments come from LDS
    // F2_READ_AHEAD ops ahead of their MFMA through a small register ring; the
    // sched_barriers pin that order (the scheduler would otherwise trade the
    // read-ahead for registers).
    constexpr int NQK = 2 * QS, NPV = 4 * OB, NOPS = NQK + NPV;
    constexpr int RING = F2_READ_AHEAD + 1;
    half8v ring[RING];
    auto read_op = [&](int i) __attribute__((always_inline)) -> half8v {
      if (i < NQK) return ks[(i / QS) * (32 * KROW / 8) + 2 * (i % QS)];
      const int k = i - NQK;
      return vfrag_read(SPREV{}, k / (2 * OB), (k / OB) & 1, k % OB);
    };
#pragma unroll
    for (int i = 0; i < F2_READ_AHEAD; ++i) ring[i % RING] = read_op(i);
#pragma unroll
    for (int i = 0; i < NOPS; ++i) {
      if (i + F2_READ_AHEAD < NOPS) ring[(i + F2_READ_AHEAD) % RING] = read_op(i + F2_READ_AHEAD);
      if (i < NQK) {
        const int h = i / QS;
        S[h] = mfma32(ring[i % RING], qf[i % QS], i % QS == 0 ? MB : S[h]);
      } else {
        const int k = i - NQK;
        acc[k % OB] = mfma32(ring[i % RING], P[k / (2 * OB)][(k / OB) & 1], acc[k % OB]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::"v"(S[0]), "v"(S[1]));
    __builtin_amdgcn_s_setprio(0);
  };

  // Final PV of the last tile (stage st).
  auto pv_last = [&](auto st) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int c = 0; c < OB; ++c) acc[c] = mfma32(vfrag_read(st, h, u, c), P[h][u], acc[c]);
  };

  // X(j): the tile copies (tile j+2, staged in registers during X(j-2), goes to
  // LDS; the loads of tile j+4 start into the buffer it leaves), then P = fp16(exp2(S))
  // (S already holds s * c2 - mbase; the running max m and mbase are updated, with the
  // O rescale, only on the exact path below).  The
  // copies sit in the VALU phase so that their LDS writes never queue ahead of
  // the fragment reads of this wave's MFMA phase.
  auto x_phase = [&](int j, auto st) __attribute__((always_inline)) {
    using SW = std::integral_constant<int, (decltype(st)::value + 2) % F2_STAGES>;
    using BUF = std::integral_constant<int, decltype(st)::value % 2>;
    store_tile(SW{}, BUF{});   // tile j+2 (never one of the next entry's Q parts)
    load_slot(j + 4, BUF{}, std::false_type{});   // tile j+4 (all zeros past the last tile)
    const int k0 = j * F2_BN;
    if ((k0 + F2_BN > kv_len) || (p.causal && k0 + F2_BN - 1 > wq0)) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kidx = k0 + 32 * h + (e >> 2) * 8 + 4 * hh + (e & 3);
          if (kidx >= kv_len || (p.causal && kidx > qi)) S[h][e] = -INFINITY;
        }
    }
    // Exponentials against the running max m_run (log2 units), fp16 P and this lane's
    // fp32 row-sum share of the tile.  The row max is not computed on this path: a
    // tile sum <= 2^15 bounds every p by 2^15, well inside fp16, and the sum is
    // needed anyway.  Only when a lane's sum exceeds that (the first tile, where m_run
    // is -inf, or a row max that grew by about 15) or is not finite does the wave take
    // the exact path: the row max, the O / row-sum rescale, then the exponentials again.
    // exps(sub, d): exponentials of S - d (the fast path has d = 0 and no subtraction).
    auto exps = [&](auto sub, float d) __attribute__((always_inline)) -> float {
      constexpr bool SUB = decltype(sub)::value;
      // The four partial sums start from the first four terms (not from 0.f, whose
      // addition the compiler must keep): same bits, four adds fewer.
      float ls[4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pe = fast_exp2(SUB ? S[h][e] - d : S[h][e]);
          P[h][e >> 3][e & 7] = (half_t)pe;
          if (h == 0 && e < 4)
            ls[e] = pe;
          else
            ls[e & 3] += pe;
        }
      return (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    float tsum = exps(std::false_type{}, 0.f);
    // A row with no maximum yet (m_run = -inf: the first tile) always takes the exact
    // path, so m_run ends up the true running max and mbase = m_run from then on.
    if (__any(!(tsum <= F2_LAZY_LIMIT) || m_run == -INFINITY)) {
      // NaN-propagating maximum (v_maximum3_f32, no operand canonicalisation) as a
      // shallow tree: 32 scores -> 8 partial maxima -> 1.
      auto mx = [](float a, float b) __attribute__((always_inline)) { return __builtin_elementwise_maximum(a, b); };
      float part[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) part[i] = mx(mx(S[i >> 2][4 * (i & 3)], S[i >> 2][4 * (i & 3) + 1]),
                                              mx(S[i >> 2][4 * (i & 3) + 2], S[i >> 2][4 * (i & 3) + 3]));
      float mloc = mx(mx(mx(part[0], part[1]), mx(part[2], part[3])), mx(mx(part[4], part[5]), mx(part[6], part[7])));
      mloc = xlane32_max(mloc) + mbase;
      const float mnew = fmaxf(m_run, mloc);
      if (mnew > m_run) {
        const float alpha = (m_run == -INFINITY) ? 1.f : fast_exp2(m_run - mnew);
        lrow *= alpha;
#pragma unroll
        for (int c = 0; c < OB; ++c) acc[c] *= alpha;
        m_run = mnew;
      }
      tsum = exps(std::true_type{}, (m_run == -INFINITY) ? 0.f : m_run - mbase);
      mbase = (m_run == -INFINITY) ? 0.f : m_run;
#pragma unroll
      for (int e = 0; e < 16; ++e) MB[e] = -mbase;
    }
    lrow += tsum;
    asm volatile("" ::"v"(P[0][0]), "v"(P[0][1]), "v"(P[1][0]), "v"(P[1][1]));
  };

  // The barrier is written out (s_barrier after lgkmcnt(0)) so that the compiler
  // does not turn it into a wait for every copy in flight.
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Prologue: the loads of the Q rows, of the Q norm weight, of the RoPE table rows and
  // of tiles 0 and 1 are all in flight together, so the workgroup pays one memory round
  // trip before its first MFMA instead of three.  A later batch entry (PERSIST) finds its
  // Q rows in qf and its tiles 0 and 1 in flight, loaded during the previous entry.
  if constexpr (!PERSIST) {
    half_t* const rreg = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? K2 : wave == 3 ? K3
                       : wave == 4 ? V0 : wave == 5 ? V1 : wave == 6 ? V2 : V3;
    // The Q loads go first (they are on the critical path), then tiles 0 and 1.  The Q
    // rows, the Q norm weight and the RoPE table rows are staged through LDS
    // (finish_q_fragment): waves 0-3 use K stages 0-3, waves 4-7 V stages 0-3, all free
    // until the tile stores below, which wait behind one barrier for every wave's
    // staged reads.
    static_assert(QStage<D>::BYTES <= KTILE * 2 && QStage<D>::BYTES <= VTILE * 2, "Q staging fits a stage");
    issue_q_loads<D, true>(p, b, head, hh, wq0, lane, qf, wn, rp);
    load_tile(0, B0{});
    load_tile(1, B1{});
    finish_q_fragment<D, true>(p, hh, lane, qf, wn, rp, (__attribute__((address_space(3))) char*)rreg, c2);
    barrier();
  } else {
    // The first entry loads its Q fragment, the norm weight (into the wave's LDS copy)
    // and tiles 0 and 1; a later entry finds its fragment in qf and its tiles in flight.
    // Only the norm runs here, on registers and the wave's own weight copy, so the one
    // barrier left is the one that keeps the tile stores below behind every wave's reads
    // of the previous entry's O rows (K stages).
    auto* const wcopy = (__attribute__((address_space(3))) char*)(QW + wave * D);
    if (entry == 0) {
#pragma unroll
      for (int s = 0; s < QS; ++s) qf[s] = __builtin_bit_cast(half8v, q_frag_load(b, s));
      if (p.q_norm_w && lane < D / 2) wn = *reinterpret_cast<const uint32_t*>(p.q_norm_w + 2 * lane);
      load_tile(0, B0{});
      load_tile(1, B1{});
      if (p.q_norm_w && lane < D / 2) *(__attribute__((address_space(3))) uint32_t*)(wcopy + 4 * lane) = wn;
      finish_q_fragment<D, false, false>(p, hh, lane, qf, wn, rp, wcopy, c2);
      // Nothing this path loaded is left pending where it meets the path of a later entry.
      // There the previous entry's O stores were issued after tiles 0 and 1, and the
      // compiler's wait counts take the worse of the two paths: with tile loads pending
      // here, the tile stores below would also wait for every O store to complete.
      wait_vmcnt_imm<0>();
    } else {
      finish_q_fragment<D, false, false>(p, hh, lane, qf, wn, rp, wcopy, c2);
      barrier();
    }
  }
  {
    // The zero quad is made here (not hoisted out of the batch-entry loop, where the
    // register allocator would keep it in scratch memory across the key loop).
    u32x4 z;
    asm volatile("v_mov_b32 %0, 0\n\tv_mov_b32 %1, 0\n\tv_mov_b32 %2, 0\n\tv_mov_b32 %3, 0"
                 : "=v"(z[0]), "=v"(z[1]), "=v"(z[2]), "=v"(z[3]));
    for (int i = tid; i < VTILE / 8; i += F2_NT) reinterpret_cast<u32x4*>(V3)[i] = z;
  }
  store_tile(S0{}, B0{});
  store_tile(S1{}, B1{});
  load_slot(2, B0{}, std::true_type{});
  load_slot(3, B1{}, std::true_type{});
  barrier();                      // tiles 0 and 1 resident
  if (group == 1) barrier();      // group 1 runs one phase behind
  // Tile j uses stage j % 4; the loop is unrolled by four so every stage is static.
  // Stage (j+2)%4, written in X(j), last held tile j-2, whose V was read by
  // G(j-1) of both groups (at least one barrier back for either group); tile j+2
  // is first read by G(j+2), two or more barriers later.
  auto step = [&](int j, auto st) __attribute__((always_inline)) {
    g_phase(j, st);
    barrier();
    x_phase(j, st);
    barrier();
    if (j == ntiles - 1) pv_last(st);
  };
  for (int j = 0; j < ntiles; j += F2_STAGES) {
    step(j, S0{});
    if (j + 1 < ntiles) step(j + 1, S1{});
    if (j + 2 < ntiles) step(j + 2, S2{});
    if (j + 3 < ntiles) step(j + 3, S3{});
  }
  if (group == 0) barrier();      // same barrier count for both groups
  wait_vmcnt_imm<0>();            // loads of tiles past the end (no memory traffic)
  const bool more = next_entry();
  if constexpr (PERSIST) {
    if (more) {
      // The next entry's Q rows (stream positions ntiles+2 and ntiles+3) move to qf, and
      // its tiles 0 and 1 load into the staging buffers they leave: that latency hides
      // behind this entry's epilogue.
      if constexpr (F2_Q_PREFETCH) {
        const bool odd = (ntiles & 1) != 0;
#pragma unroll
        for (int r = 0; r < NCP; ++r) {
          qf[r] = __builtin_bit_cast(half8v, odd ? stg2[1][r] : stg2[0][r]);
          qf[NCP + r] = __builtin_bit_cast(half8v, odd ? stg2[0][r] : stg2[1][r]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < QS; ++s) qf[s] = __builtin_bit_cast(half8v, q_frag_load(bn, s));
      }
      const int nkend = entry_kend(entry_kv_len(bn));
      const int64_t nkb = nkend > 0 ? (int64_t)(nkend - 1) * ktok2 + D * 2 : 0;
      const int64_t nvb = nkend > 0 ? (int64_t)(nkend - 1) * vtok2 + D * 2 : 0;
      const char* const nk = entry_k(bn);
      const char* const nv = entry_v(bn);
      load_at(nk, clamp_bytes(nkb), nv, clamp_bytes(nvb), B0{});
      load_at(nk + kstep, clamp_bytes(nkb - kstep), nv + vstep, clamp_bytes(nvb - vstep), B1{});
    }
  }

  const float l_tot = xlane32_sum(lrow);
  // A key split stores its normalised rows O_s / l_s in fp16 (below, through the same
  // whole-row path as O) beside the fp32 (max, sum) pair of each row; the merge weighs
  // them by l_s.
  if (!PERSIST && p.kv_splits > 1 && qi < p.Sq && hh == 0) {
    const int64_t row = (((int64_t)split * p.nbatch + b) * p.H + head) * p.Sq + qi;
    *reinterpret_cast<float2*>(p.part_ml + row * 2) = make_float2(m_run, l_tot);
  }
  // The fp16 O rows go through LDS so that every global store is a 16-byte piece of a
  // whole row (D/8 lanes per row).  In registers a lane holds 4-column pieces of one
  // row, and storing those directly scatters each instruction over 32 rows.  Wave w
  // uses half of K stage w/2 (32 rows of D+8 halfs), free once both groups are past
  // their last PV: group 1 finishes its last PV after group 0's final barrier above, so
  // one more barrier for all waves comes first.
  barrier();
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  half_t* const ost = ((wave >> 1) == 0 ? K0 : (wave >> 1) == 1 ? K1 : (wave >> 1) == 2 ? K2 : K3) +
                      (wave & 1) * 32 * KROW;
#pragma unroll
  for (int c = 0; c < OB; ++c)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const half4v val = {(half_t)(acc[c][4 * e4 + 0] * inv), (half_t)(acc[c][4 * e4 + 1] * inv),
                          (half_t)(acc[c][4 * e4 + 2] * inv), (half_t)(acc[c][4 * e4 + 3] * inv)};
      *reinterpret_cast<half4v*>(ost + c32 * KROW + 32 * c + 8 * e4 + 4 * hh) = val;
    }
  constexpr int CPR = D / 8, RPI = 64 / CPR;   // 16-byte chunks per row, rows per store
  half_t* const obase = !PERSIST && p.kv_splits > 1
                            ? static_cast<half_t*>(p.part_o) + (((int64_t)split * p.nbatch + b) * p.H + head) * p.Sq * D
                            : p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head;
  const int64_t otok = !PERSIST && p.kv_splits > 1 ? D : p.o_tok;
  if constexpr (PERSIST) {
    // Through one descriptor over the (batch, head) rows (within 2 GiB, checked on the
    // host), which drops the rows past the sequence: with a branch per store instead, the
    // compiler's wait counts in the next entry would take the path that skips every store
    // and make the tile stores wait for these stores to complete.
    const uint32_t otok2 = (uint32_t)p.o_tok * 2u;
    const int onbytes = (int)((uint32_t)(p.Sq - 1) * otok2 + D * 2);
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + lane / CPR, ch = lane % CPR;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ost + r * KROW + ch * 8);
      const uint32_t off = wq0 + r < p.Sq ? (uint32_t)(wq0 + r) * otok2 + (uint32_t)ch * 16u : 0x80000000u;
      store16_bounded(obase, onbytes, off, v);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + lane / CPR, ch = lane % CPR;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ost + r * KROW + ch * 8);
      if (wq0 + r < p.Sq) *reinterpret_cast<u32x4*>(obase + (int64_t)(wq0 + r) * otok + ch * 8) = v;
    }
  }
  if (!more) break;
  b = bn;
  }   // batch entries
}

// Merge of the key splits: O = sum_s w_s O_s / sum_s w_s l_s with w_s = 2^(m_s - max m).
// The kernels store O_s as l_s * Ohat_s with Ohat_s its fp16 normalised row.  Thread t
// of a row handles columns 8t .. 8t+7; it issues every split's loads before the first
// use, so all of them are in flight at once.
template <int D>
__global__ __launch_bounds__(256) void flash_combine_kernel(FlashParams p, int64_t rows) {
  constexpr int TPR = D / 8;
  constexpr int RPB = 256 / TPR;   // rows per block (threads past RPB * TPR idle)
  if ((int)threadIdx.x >= RPB * TPR) return;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  if (row >= rows) return;
  const int qi = (int)(row % p.Sq);
  const int head = (int)((row / p.Sq) % p.H);
  const int b = (int)(row / ((int64_t)p.Sq * p.H));
  const int ns = p.kv_splits;
  float2 ml[FLASH_MAX_SPLITS];
  half8v a[FLASH_MAX_SPLITS];
#pragma unroll
  for (int s = 0; s < FLASH_MAX_SPLITS; ++s)
    if (s < ns) {
      ml[s] = *reinterpret_cast<const float2*>(p.part_ml + (s * rows + row) * 2);
      a[s] = *reinterpret_cast<const half8v*>(static_cast<const half_t*>(p.part_o) + (s * rows + row) * D + 8 * t);
    }
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < FLASH_MAX_SPLITS; ++s)
    if (s < ns) mmax = fmaxf(mmax, ml[s].x);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
#pragma unroll
  for (int s = 0; s < FLASH_MAX_SPLITS; ++s)
    if (s < ns) {
      const float w = ml[s].x == -INFINITY ? 0.f : fast_exp2(ml[s].x - mmax);
      const float wl = w * ml[s].y;
      l += wl;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(wl, (float)a[s][e], acc[e]);
    }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  half8v o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (half_t)(acc[e] * inv);
  half_t* op = p.o + (int64_t)b * p.o_batch + (int64_t)head * p.o_head + (int64_t)qi * p.o_tok + 8 * t;
  *reinterpret_cast<half8v*>(op) = o;
}

void launch_flash_combine(const FlashParams& p, int D, int batch, hipStream_t stream) {
  if (p.kv_splits < 2 || p.kv_splits > FLASH_MAX_SPLITS) fail(ANIMA_E_INVALID_ARGUMENT, "flash key splits out of range");
  const int64_t rows = (int64_t)batch * p.H * p.Sq;
  const int rpb = 256 / (D / 8);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "attention combine grid too large");
  if (D == 128)
    hipLaunchKernelGGL(flash_combine_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, stream, p, rows);
  else if (D == 384)
    hipLaunchKernelGGL(flash_combine_kernel<384>, dim3((unsigned)blocks), dim3(256), 0, stream, p, rows);
  else
    hipLaunchKernelGGL(flash_combine_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, stream, p, rows);
  ANIMA_HIP(hipGetLastError());
}

// Heads of one query tile on consecutive workgroups (the kernel's block order): 8 for
// single-image launches of at least 128 workgroups over at least 1024 keys whose head
// count 8 divides, else 1.  Measured against 1 (A/B of library builds, medians of 3-5
// rounds): S=4096 self-attention with Q/K norm and RoPE 138.2 -> 137.1 us, S=1024
// self-attention on two key splits 24.6 -> 23.7 us; 4 heads gave 137.0 and 24.9 us, 16
// heads 138.0 and 23.7 us.  With few keys a head's K/V is best shared in one XCD's L2 by
// many workgroups: the adapter attention (32 workgroups) went from 19.35 to 19.6 us with
// 8, and the DiT block's cross attention (4096 queries over 512 keys) from 26.08 to 26.34.
static int flash_v2_head_group(const FlashParams& p, int64_t blocks, bool persist) {
  if (persist || p.nbatch != 1 || p.H % 8 != 0 || blocks < 128 || p.Sk < 1024) return 1;
  return 8;
}

void launch_flash_v2(const FlashParams& p_in, int D, dim3 grid, hipStream_t stream, bool persist) {
  FlashParams p = p_in;
  p.head_group = flash_v2_head_group(p, grid.x, persist);
  // The kernel decodes blockIdx into (split, query tile, batch, head) with these counts
  // (persistent: (query tile, head), batch entries walked in the kernel): a grid of any
  // other size would address rows past the tensors.
  if (p.nbatch < 1 || p.q_tiles < 1 || p.H < 1 || p.H % p.head_group != 0 ||
      (int64_t)grid.x != (int64_t)p.q_tiles * p.H * (persist ? 1 : p.nbatch) * (p.kv_splits > 1 ? p.kv_splits : 1))
    fail(ANIMA_E_INVALID_ARGUMENT, "flash attention grid does not match its tiles, heads and batch");
  if (persist && (p.rope || p.kv_splits > 1 || !flash_v2_persist_fits(p, D)))
    fail(ANIMA_E_INVALID_ARGUMENT, "persistent flash attention takes no Q RoPE, no key splits and Q rows within 2 GiB");
  if (D == 128) {
    if (persist)
      hipLaunchKernelGGL((flash_attention_v2_kernel<128, true>), grid, dim3(F2_NT), 0, stream, p);
    else
      hipLaunchKernelGGL((flash_attention_v2_kernel<128, false>), grid, dim3(F2_NT), 0, stream, p);
  } else if (D == 64) {
    if (persist)
      hipLaunchKernelGGL((flash_attention_v2_kernel<64, true>), grid, dim3(F2_NT), 0, stream, p);
    else
      hipLaunchKernelGGL((flash_attention_v2_kernel<64, false>), grid, dim3(F2_NT), 0, stream, p);
  } else {
    fail(ANIMA_E_UNSUPPORTED, "flash attention requires head_dim 64 or 128");
  }
  ANIMA_HIP(hipGetLastError());
}

bool flash_v2_persist_fits(const FlashParams& p, int D) {
  return p.Sq >= 1 && (int64_t)(p.Sq - 1) * p.q_tok * 2 + D * 2 < ((int64_t)1 << 31) &&
         (int64_t)(p.Sq - 1) * p.o_tok * 2 + D * 2 < ((int64_t)1 << 31);
}

}  // namespace anima
