// Small-M quantized linear (M <= 64 input rows) for gfx950: a weight-streaming GEMM.
//
// With a handful of input rows the GEMM is bound by reading the packed weight
// (LinearExecutor.swift:79-133 routes M=1 through the matvec and small M through
// MPS; here both are one kernel).  Work decomposition:
//   * a wave owns R blocks of 16 weight rows and one K slice; the S waves of a
//     workgroup share the rows and split K, so every workgroup reads its rows'
//     packed bytes exactly once and the grid has N/(16R) workgroups of S waves;
//   * per 128-wide K chunk each lane loads 16 B of W4 (32 B W8, 64 B FP16) of one
//     row -- a whole 64-group's half, so one scale/zero pair -- and dequantizes it
//     in registers with the exact rounding of the reference decoder,
//     half(fma(q, scale, zero)) (q*scale is exact in fp32);
//   * the products run on v_mfma_f32_16x16x32_f16 with the weight as the A
//     operand (16 rows x 32 k) and X^T as B (32 k x 16 input rows).  The lane
//     group g = lane/16 takes k = 32g .. 32g+31 of the chunk, so each 16-byte
//     weight load feeds four MFMAs; X fragments use the same k order;
//   * the S partial sums are reduced in a fixed order through LDS (deterministic),
//     rounded to fp16 once and stored.
#include <algorithm>

#include "linear.hpp"

namespace anima {

struct SmallMParams {
  const half_t* x;       // [M, K] fp16, row stride K
  half_t* y;             // [M, N] fp16, row stride N
  const uint8_t* w;      // packed rows
  const half_t* scale;   // [N, groups]
  const half_t* zero;
  int64_t row_stride;    // bytes (W4/W8) or halfs (FP16)
  int M, N, K, groups;
  int kw;                // K per wave, multiple of 128
};

constexpr int SM_CHUNK = 128;
constexpr int SMALLM_MAX_STEPS = 8;   // steps per wave, each of NCH chunks
constexpr int SM_PARAM_REGS = 8;      // scale (and zero) halfs each thread stages into LDS

template <int STORAGE>
struct SmallMChunk {
  // 32-bit words of one lane's weight bytes for one 128-wide K chunk (32 k values).
  static constexpr int WORDS = STORAGE == ANIMA_STORAGE_W4 ? 4 : (STORAGE == ANIMA_STORAGE_W8 ? 8 : 16);
};

// One weight value: half(fl32(q*s + z)), the reference decoder's two roundings.
// With ONE_ROUNDING the fp32 step is skipped (the compiler may fuse multiply, add and
// conversion into v_fma_mix); the caller only asks for that when q*s + z is exact in
// fp32 (one_rounding_exact), where both give the same bits.
template <bool ONE_ROUNDING>
__device__ __forceinline__ half_t dq1(uint32_t q, half_t s, half_t z) {
  if constexpr (ONE_ROUNDING)
    return (half_t)fmaf((float)q, (float)s, (float)z);
  else
    return f32_to_f16(fmaf((float)q, (float)s, (float)z));
}

// A fragment t (k = 32g + 8t .. +7 of the chunk) from a lane's raw weight words.
template <int STORAGE, bool ONE_ROUNDING>
__device__ __forceinline__ half8v dequant_frag(const uint32_t (&wv)[SmallMChunk<STORAGE>::WORDS], int t, half_t s,
                                               half_t z) {
  half8v a;
  if constexpr (STORAGE == ANIMA_STORAGE_W4) {
    const uint32_t d = wv[t];
    const uint32_t lo = d & 0x0F0F0F0Fu;          // even k: nibbles 0, 2, 4, 6
    const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;   // odd k
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      a[2 * b] = dq1<ONE_ROUNDING>((lo >> (8 * b)) & 0xFFu, s, z);
      a[2 * b + 1] = dq1<ONE_ROUNDING>((hi >> (8 * b)) & 0xFFu, s, z);
    }
  } else if constexpr (STORAGE == ANIMA_STORAGE_W8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t d = wv[2 * t + h];
#pragma unroll
      for (int b = 0; b < 4; ++b) a[4 * h + b] = dq1<ONE_ROUNDING>((d >> (8 * b)) & 0xFFu, s, z);
    }
  } else {
    const u32x4 raw = {wv[4 * t], wv[4 * t + 1], wv[4 * t + 2], wv[4 * t + 3]};
    a = __builtin_bit_cast(half8v, raw);
  }
  return a;
}

// Waves per workgroup: 16 for one m-block (<= 128 VGPRs), 8 otherwise (<= 256).
template <int MB>
constexpr int smallm_max_waves() { return MB == 1 ? 16 : 8; }

// Chunks preloaded per step, bounded by the registers the raw weight words take.
template <int STORAGE, int MB>
constexpr int smallm_max_chunks() {
  return STORAGE == ANIMA_STORAGE_W8 ? 1 : (MB <= 2 ? 2 : 1);
}

template <int STORAGE, int MB, int R, int NCH, int NST, bool DIRECT>
__global__ __launch_bounds__(64 * smallm_max_waves<MB>()) void smallm_gemm_kernel(SmallMParams p) {
  constexpr int WORDS = SmallMChunk<STORAGE>::WORDS;
  // Dynamic LDS: the S x R*MB partial-sum tiles of the final reduction, then the
  // workgroup's scale and zero rows ([16R][groups] halfs each).
  extern __shared__ float red[];   // [S][R*MB][64][4], then scale, zero

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int S = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * R;
  const int kslice = wave * p.kw;
  const int kstop = min(p.K, kslice + p.kw);

  // Rows past N re-read row N-1 (computed, never stored).
  const uint8_t* wrow[R];
#pragma unroll
  for (int rb = 0; rb < R; ++rb) {
    const int n = min(n0 + rb * 16 + r, p.N - 1);
    wrow[rb] = p.w + (int64_t)n * p.row_stride * (STORAGE == ANIMA_STORAGE_FP16 ? 2 : 1);
  }
  // Scale / zero.  With a short slice (DIRECT: at most 4 chunks per wave, K a multiple
  // of 256) each lane loads its own rows' pairs straight into registers: chunk c of the
  // slice uses group kslice/64 + 2c + g/2, so one 8-byte load of four consecutive groups
  // serves two chunks, and the loads go out with the weight loads (one memory round trip
  // before the MFMAs, no barrier).  Otherwise the workgroup's 16R rows are one contiguous
  // run of the [N][groups] arrays, copied into LDS with coalesced loads (lanes read
  // consecutive halfs) rather than one scattered 2-byte load per lane and chunk.
  constexpr int PAIRS = R * MB;
  constexpr int SLICE_CHUNKS = NCH * NST;
  half_t* s_lds = reinterpret_cast<half_t*>(red + S * PAIRS * 4 * 64);
  half_t* z_lds = s_lds + 16 * R * p.groups;
  const int nrows = min(16 * R, p.N - n0);
  const int nparam = nrows * p.groups;
  // Scale/zero halfs per thread: 16R rows x K/64 groups over 64 x S threads, with
  // S x NCH x NST chunks of 128 covering K, is at most ceil(R x NCH x NST / 2) per thread.
  constexpr int PARAM_REGS = std::min(SM_PARAM_REGS, (R * NCH * NST + 1) / 2);
  half_t sreg[PARAM_REGS], zreg[PARAM_REGS];
  // DIRECT: per row block, (SLICE_CHUNKS + 1) / 2 loads of 4 groups (one of 2 groups for a
  // one-chunk slice) of scale and of zero.
  constexpr int DLOADS = (SLICE_CHUNKS + 1) / 2;
  uint64_t sdir[DIRECT ? R : 1][DIRECT ? DLOADS : 1], zdir[DIRECT ? R : 1][DIRECT ? DLOADS : 1];
  if constexpr (DIRECT) {
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
      const int n = min(n0 + rb * 16 + r, p.N - 1);
      const int64_t base = (int64_t)n * p.groups + kslice / 64;
#pragma unroll
      for (int q = 0; q < DLOADS; ++q) {
        if constexpr (SLICE_CHUNKS == 1) {
          sdir[rb][q] = *reinterpret_cast<const uint32_t*>(p.scale + base);
          zdir[rb][q] = *reinterpret_cast<const uint32_t*>(p.zero + base);
        } else {
          sdir[rb][q] = *reinterpret_cast<const uint64_t*>(p.scale + base + 4 * q);
          zdir[rb][q] = *reinterpret_cast<const uint64_t*>(p.zero + base + 4 * q);
        }
      }
    }
  } else if constexpr (STORAGE != ANIMA_STORAGE_FP16) {
    const half_t* sbase = p.scale + (int64_t)n0 * p.groups;
    const half_t* zbase = p.zero + (int64_t)n0 * p.groups;
#pragma unroll
    for (int i = 0; i < PARAM_REGS; ++i) {
      const int e = threadIdx.x + i * (int)blockDim.x;
      const int ec = min(e, nparam - 1);
      sreg[i] = sbase[ec];
      zreg[i] = zbase[ec];
    }
  }
  // X is read through one bounded buffer descriptor over its M x K halfs: lanes of rows
  // past M (and chunks past the slice) get the offset xbytes, so their loads return
  // zeros without touching memory (the load is still issued, which keeps the in-order
  // load counter exact).  Rows past M are 15 of 16 lanes at M = 1.
  const int xbytes = p.M * p.K * 2;
  uint32_t xoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    xoff[mb] = m < p.M ? (uint32_t)m * (uint32_t)p.K * 2u : 0xffffffffu;
  }

  floatx4 acc[R][MB];
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = floatx4{};

  // One step = NCH chunks whose weight words are loaded together.  Steps are
  // double-buffered: the next step's loads are in flight while this step's
  // dequantization and MFMAs run, so a wave pays HBM latency about once.  Every
  // load is unconditional (chunks past the slice re-read its last chunk and are
  // masked through zero X), which keeps the in-order load counter exact: a wait
  // for this step never waits for the next step's loads.
  struct Step {
    uint32_t wv[NCH][R][WORDS];
  };
  constexpr int STEP_K = NCH * SM_CHUNK;
  const int klast = kstop - SM_CHUNK;   // start of the slice's last chunk (every wave has one)

  auto load_step = [&](int step, Step& st) {
    const int kbeg = kslice + step * STEP_K;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int kl = min(kbeg + c * SM_CHUNK, klast) + 32 * g;
#pragma unroll
      for (int rb = 0; rb < R; ++rb) {
        const int64_t boff = STORAGE == ANIMA_STORAGE_W4 ? kl / 2 : (STORAGE == ANIMA_STORAGE_W8 ? kl : 2 * kl);
        const u32x4* src = reinterpret_cast<const u32x4*>(wrow[rb] + boff);
#pragma unroll
        for (int v = 0; v < WORDS / 4; ++v) {
          const u32x4 t4 = __builtin_nontemporal_load(src + v);
          st.wv[c][rb][4 * v] = t4[0];
          st.wv[c][rb][4 * v + 1] = t4[1];
          st.wv[c][rb][4 * v + 2] = t4[2];
          st.wv[c][rb][4 * v + 3] = t4[3];
        }
      }
    }
  };

  // X fragments of chunk c of a step; rows past M and chunks past the slice are
  // loaded from valid addresses and zeroed with a mask (no branch around the load).
  auto load_x = [&](int step, int c, half8v (&xf)[MB][4]) {
    const int kc = kslice + step * STEP_K + c * SM_CHUNK;
    const bool live = kc < kstop;
    const uint32_t kb = (uint32_t)(kc + 32 * g) * 2u;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t base = live && xoff[mb] != 0xffffffffu ? xoff[mb] + kb : (uint32_t)xbytes;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xf[mb][t] = __builtin_bit_cast(half8v, load16_bounded(p.x, xbytes, base + 16u * t));
    }
  };

  // Order per iteration: this step's X fragments (L2), then the next step's weight
  // prefetch (HBM), then the arithmetic.  Loads retire in issue order, so waiting for
  // X and this step's weights never waits for the prefetch.  (Issuing the next step's
  // X with its weights, in a second X buffer, measured no faster.)
  auto compute_step = [&](int step, const Step& st, const half8v (&xs)[NCH][MB][4]) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int kl = min(kslice + step * STEP_K + c * SM_CHUNK, klast) + 32 * g;
      half_t sc[R], zc[R];
#pragma unroll
      for (int rb = 0; rb < R; ++rb) {
        if constexpr (DIRECT) {
          // Slice chunk i = step * NCH + c (chunks past the slice re-read its last one);
          // its group is half (i % 2) * 2 + g / 2 of load i / 2.
          const int i = min(step * NCH + c, (kstop - kslice) / SM_CHUNK - 1);
          const int sh = 16 * ((i & 1) * 2 + (g >> 1));
          sc[rb] = __builtin_bit_cast(half_t, (unsigned short)(sdir[rb][i >> 1] >> sh));
          zc[rb] = __builtin_bit_cast(half_t, (unsigned short)(zdir[rb][i >> 1] >> sh));
        } else if constexpr (STORAGE != ANIMA_STORAGE_FP16) {
          const int li = (rb * 16 + r) * p.groups + (kl >> 6);
          sc[rb] = s_lds[li];
          zc[rb] = z_lds[li];
        } else {
          sc[rb] = zc[rb] = (half_t)0.f;
        }
      }
      constexpr int QBITS = STORAGE == ANIMA_STORAGE_W4 ? 4 : 8;
      bool fast = true;
#pragma unroll
      for (int rb = 0; rb < R; ++rb) fast = fast && one_rounding_exact<QBITS>(sc[rb], zc[rb]);
      if constexpr (NST == 1) {
        // One step: every fragment is dequantised before the first MFMA, so the VALU
        // work overlaps the wait for X (issued after the weights).
        half8v a[R][4];
        if (__all(fast)) {
#pragma unroll
          for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t) a[rb][t] = dequant_frag<STORAGE, true>(st.wv[c][rb], t, sc[rb], zc[rb]);
        } else {
#pragma unroll
          for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t) a[rb][t] = dequant_frag<STORAGE, false>(st.wv[c][rb], t, sc[rb], zc[rb]);
        }
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = mfma16(a[rb][t], xs[c][mb][t], acc[rb][mb]);
      } else {
        // Several steps: each fragment is dequantised right before its MFMAs, which
        // keeps the live A fragments to one (the two-row-block kernels for 49-64 input
        // rows spilled otherwise).  The rounding form is one uniform branch around it.
        auto run = [&](auto one_rounding) __attribute__((always_inline)) {
#pragma unroll
          for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const half8v a = dequant_frag<STORAGE, decltype(one_rounding)::value>(st.wv[c][rb], t, sc[rb], zc[rb]);
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = mfma16(a, xs[c][mb][t], acc[rb][mb]);
            }
        };
        if (__all(fast))
          run(std::true_type{});
        else
          run(std::false_type{});
      }
    }
  };

  // NST steps, fully unrolled (straight-line code keeps every wait exact) and
  // ping-ponged; steps past the slice re-read its last chunk and multiply zero X.
  Step sa, sb;
  half8v xs[NCH][MB][4];
  load_step(0, sa);
  if constexpr (DIRECT) {
    // Everything step 0 needs is in flight at once: weights, scale/zero, X.
#pragma unroll
    for (int c = 0; c < NCH; ++c) load_x(0, c, xs[c]);
  } else {
    // Park the scale/zero copy in LDS (waits only for those loads, issued before the
    // weight loads) and make it visible to every wave.
    if constexpr (STORAGE != ANIMA_STORAGE_FP16) {
#pragma unroll
      for (int i = 0; i < PARAM_REGS; ++i) {
        const int e = threadIdx.x + i * (int)blockDim.x;
        if (e < nparam) {
          s_lds[(e / p.groups) * p.groups + e % p.groups] = sreg[i];
          z_lds[(e / p.groups) * p.groups + e % p.groups] = zreg[i];
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int step = 0; step < NST; ++step) {
    Step& cur = (step & 1) ? sb : sa;
    Step& nxt = (step & 1) ? sa : sb;
    if (!DIRECT || step > 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) load_x(step, c, xs[c]);
    }
    if (step + 1 < NST) load_step(step + 1, nxt);
    compute_step(step, cur, xs);
  }

  // Fixed-order reduction of the S K-slices through LDS: each lane's 4 sums of a
  // (row block, m block) pair are one 16-byte word, and the reading wave issues every
  // slice's read before the first add (the loop runs to the largest S, reads past S
  // predicated off), so the tail is one LDS round trip instead of S dependent ones.
  floatx4* red4 = reinterpret_cast<floatx4*>(red);
#pragma unroll
  for (int pi = 0; pi < PAIRS; ++pi) red4[(wave * PAIRS + pi) * 64 + lane] = acc[pi / MB][pi % MB];
  __syncthreads();
  for (int pi = wave; pi < PAIRS; pi += S) {
    const int rb = pi / MB, mb = pi % MB;
    // NS slots read at once (NS the smallest of 4, 8, 16 that covers S, one uniform
    // branch); slots past S re-read slot S-1 and add +0 instead (no branch per slot).
    // The sum starts at +0, so the extra +0 terms change no bit, not even a zero's sign.
    auto reduce = [&](auto ns) __attribute__((always_inline)) -> floatx4 {
      constexpr int NS = decltype(ns)::value;
      floatx4 part[NS];
#pragma unroll
      for (int w = 0; w < NS; ++w) part[w] = red4[(min(w, S - 1) * PAIRS + pi) * 64 + lane];
      floatx4 sum = floatx4{};
#pragma unroll
      for (int w = 0; w < NS; ++w) sum += w < S ? part[w] : floatx4{};
      return sum;
    };
    constexpr int SMAX = smallm_max_waves<MB>();
    floatx4 sum;
    if (SMAX > 8 && S > 8)
      sum = reduce(std::integral_constant<int, SMAX>{});
    else if (S > 4)
      sum = reduce(std::integral_constant<int, 8>{});
    else
      sum = reduce(std::integral_constant<int, 4>{});
    const float v[4] = {sum[0], sum[1], sum[2], sum[3]};
    // C layout: lane (col = lane%16, rows 4*(lane/16) .. +3) -> y[m = col][n = row]
    const int m = mb * 16 + r;
    const int nb = n0 + rb * 16 + 4 * g;
    if (m < p.M) {
      half_t* yp = p.y + (int64_t)m * p.N + nb;
      if (nb + 3 < p.N && ((reinterpret_cast<uintptr_t>(yp) & 7u) == 0)) {
        *reinterpret_cast<half4v*>(yp) = half4v{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nb + i < p.N) yp[i] = (half_t)v[i];
      }
    }
  }
}

template <int STORAGE, int MB, int R, int NCH, int NST>
static void launch_smallm_t(SmallMParams p, int S, hipStream_t stream) {
  p.kw = NCH * NST * SM_CHUNK;
  const int wgs = (p.N + 16 * R - 1) / (16 * R);
  // Per-lane scale/zero loads: a slice of at most 4 chunks, every wave's slice whole (so
  // its groups stay inside the row), and 8-byte aligned runs of 4 groups (rows of a
  // multiple of 4 groups; a one-chunk slice needs 4-byte runs of 2).
  constexpr bool SHORT = NCH * NST <= 4 && STORAGE != ANIMA_STORAGE_FP16;
  const bool aligned = NCH * NST == 1 ? (p.groups % 2 == 0 && aligned4(p.scale) && aligned4(p.zero))
                                      : (p.groups % 4 == 0 && aligned8(p.scale) && aligned8(p.zero));
  if (SHORT && aligned && p.K % p.kw == 0) {
    const size_t lds = (size_t)S * R * MB * 4 * 64 * sizeof(float);
    hipLaunchKernelGGL((smallm_gemm_kernel<STORAGE, MB, R, NCH, NST, SHORT>), dim3(wgs), dim3(64 * S), lds, stream, p);
  } else {
    const size_t lds = (size_t)S * R * MB * 4 * 64 * sizeof(float) + (size_t)2 * 16 * R * p.groups * sizeof(half_t);
    hipLaunchKernelGGL((smallm_gemm_kernel<STORAGE, MB, R, NCH, NST, false>), dim3(wgs), dim3(64 * S), lds, stream, p);
  }
}

template <int STORAGE, int MB>
constexpr int smallm_rows() { return MB == 2 ? 2 : 1; }

// Waves per workgroup (S) times chunks per wave (NCH x NST) must cover K; the
// fewest chunks per wave wins (the most waves share the dequantization), within
// smallm_max_waves and a reduction buffer (S x R*MB KiB) of at most 64 KiB.
template <int STORAGE, int MB, int R = smallm_rows<STORAGE, MB>()>
static int smallm_steps(int K, int* S) {
  constexpr int NCH = smallm_max_chunks<STORAGE, MB>();
  const int chunks = K / SM_CHUNK;
  const int max_s = std::min(smallm_max_waves<MB>(), 64 / (R * MB));
  const int groups = (K + 63) / 64;
  for (int nst = 1; nst <= SMALLM_MAX_STEPS; nst *= 2) {
    const int per = NCH * nst;
    const int s = (chunks + per - 1) / per;
    // the scale/zero copy: 16R rows x groups halfs over 64*S threads
    const int64_t lds = (int64_t)s * R * MB * 4 * 64 * 4 + (int64_t)2 * 16 * R * groups * 2;
    if (s <= max_s && 16 * R * groups <= SM_PARAM_REGS * 64 * s && lds <= 65536) {
      *S = s;
      return nst;
    }
  }
  return 0;
}

template <int STORAGE, int MB, int R>
static void launch_smallm_rr(const SmallMParams& p, hipStream_t stream) {
  constexpr int NCH = smallm_max_chunks<STORAGE, MB>();
  int S = 0;
  switch (smallm_steps<STORAGE, MB, R>(p.K, &S)) {
    case 1: launch_smallm_t<STORAGE, MB, R, NCH, 1>(p, S, stream); break;
    case 2: launch_smallm_t<STORAGE, MB, R, NCH, 2>(p, S, stream); break;
    case 4: launch_smallm_t<STORAGE, MB, R, NCH, 4>(p, S, stream); break;
    case 8: launch_smallm_t<STORAGE, MB, R, NCH, 8>(p, S, stream); break;
    default: fail(ANIMA_E_UNSUPPORTED, "small-M GEMM: K too large for the weight-streaming kernel");
  }
}

// With 33..64 input rows every workgroup re-reads X for its K slices, so wide N pays
// X traffic per 16 weight rows; two row blocks per wave halve it when N leaves
// enough workgroups (>= 256 of 32 rows).
template <int STORAGE, int MB>
static void launch_smallm_r(const SmallMParams& p, hipStream_t stream) {
  constexpr int R = smallm_rows<STORAGE, MB>();
  if constexpr (MB >= 3 && R == 1 && STORAGE != ANIMA_STORAGE_FP16) {
    int S = 0;
    if (p.N >= 32 * 256 && smallm_steps<STORAGE, MB, 2>(p.K, &S) > 0) {
      launch_smallm_rr<STORAGE, MB, 2>(p, stream);
      return;
    }
  }
  launch_smallm_rr<STORAGE, MB, R>(p, stream);
}

template <int STORAGE>
static void launch_smallm_s(const SmallMParams& p, hipStream_t stream) {
  switch ((p.M + 15) / 16) {
    case 1: launch_smallm_r<STORAGE, 1>(p, stream); break;
    case 2: launch_smallm_r<STORAGE, 2>(p, stream); break;
    case 3: launch_smallm_r<STORAGE, 3>(p, stream); break;
    default: launch_smallm_r<STORAGE, 4>(p, stream); break;
  }
}

template <int STORAGE>
static bool smallm_fits(int M, int K) {
  int S = 0;
  switch ((M + 15) / 16) {
    case 1: return smallm_steps<STORAGE, 1>(K, &S) > 0;
    case 2: return smallm_steps<STORAGE, 2>(K, &S) > 0;
    case 3: return smallm_steps<STORAGE, 3>(K, &S) > 0;
    default: return smallm_steps<STORAGE, 4>(K, &S) > 0;
  }
}

bool smallm_supported(const GemmParams& p, int storage) {
  if (p.M < 1 || p.M > SMALLM_MAX_ROWS || p.K % SM_CHUNK != 0 || !aligned16(p.x) || !aligned16(p.w)) return false;
  if ((int64_t)p.M * p.K * 2 > 0x7fffffff) return false;   // X is addressed with 32-bit buffer offsets
  if (storage == ANIMA_STORAGE_FP16) return p.row_stride % 8 == 0 && smallm_fits<ANIMA_STORAGE_FP16>(p.M, p.K);
  if (p.row_stride % 16 != 0) return false;
  return storage == ANIMA_STORAGE_W4 ? smallm_fits<ANIMA_STORAGE_W4>(p.M, p.K) : smallm_fits<ANIMA_STORAGE_W8>(p.M, p.K);
}

void launch_smallm(const GemmParams& g, int storage, hipStream_t stream) {
  if (g.epilogue != GEMM_STORE) fail(ANIMA_E_UNSUPPORTED, "fused GEMM epilogues need the ping-pong kernel");
  SmallMParams p{};
  p.x = g.x; p.y = g.y; p.w = g.w; p.scale = g.scale; p.zero = g.zero;
  p.row_stride = g.row_stride; p.M = g.M; p.N = g.N; p.K = g.K; p.groups = g.groups;
  if (storage == ANIMA_STORAGE_W4)
    launch_smallm_s<ANIMA_STORAGE_W4>(p, stream);
  else if (storage == ANIMA_STORAGE_W8)
    launch_smallm_s<ANIMA_STORAGE_W8>(p, stream);
  else
    launch_smallm_s<ANIMA_STORAGE_FP16>(p, stream);
  ANIMA_HIP(hipGetLastError());
}


// ---------------------------------------------------------------------------
// Split-K form (W4/W8).  The kernel above gives each 16 weight rows all of X: with
// 33..64 input rows every wave gathers M x K halfs of X from L2 for 16 x K/2 bytes of
// weights, and N = 2048 leaves half the chip without a workgroup.  Here:
//   * a workgroup owns SK_ROWS weight rows (16 per row block) and one K slice; the
//     slice of X (all M rows, zero rows up to 16 * MB) is copied into LDS once with
//     coalesced 16-byte loads, and every wave reads its B fragments there, so an X
//     byte crosses the CU's memory path once per SK_ROWS weight rows;
//   * with four or more chunks per slice, two waves share each row block, one per half
//     of the slice's chunks (two waves per SIMD, so one's dequantisation and LDS reads
//     overlap the other's MFMAs), and add their sums through LDS at the end;
//   * a wave loads all its weight words at once (one 16-byte load per lane and chunk
//     for W4, two for W8) and dequantises them chunk by chunk with the exact rounding
//     of the kernel above (one_rounding_exact, wave-uniform);
//   * slices are chosen so the grid reaches 256 workgroups; with more than one, each
//     writes fp32 partial rows [slice][M][N] and launch_splitk_reduce adds them in
//     slice order (deterministic) and rounds once to fp16.
// MFMA operand layout as above: A = 16 weight rows x 32 k (lane (r, g) holds row r,
// k = chunk + 32g + 8t .. +7 of step t), B = X^T with the same k, C lane (r, g) =
// Y[m = 16mb + r][n = 16w + 4g .. +3].
// ---------------------------------------------------------------------------
constexpr int SK_RWAVES = 4;                 // row blocks per workgroup
constexpr int SK_ROWS = 16 * SK_RWAVES;
template <int NCHK>
constexpr int sk_khalves() { return NCHK >= 4 ? 2 : 1; }
constexpr int SK_MAX_CHUNKS = 8;              // 128-wide K chunks per slice
constexpr int64_t SK_MAX_LDS = 160 * 1024;    // X slice bytes per workgroup

template <int STORAGE, int MB, int NCHK>
__global__ __launch_bounds__(64 * SK_RWAVES * sk_khalves<NCHK>()) void smallm_splitk_kernel(SmallMParams p, float* part,
                                                                                           int rgroups) {
  constexpr int WORDS = SmallMChunk<STORAGE>::WORDS;
  constexpr int QBITS = STORAGE == ANIMA_STORAGE_W4 ? 4 : 8;
  constexpr int KH = sk_khalves<NCHK>();      // waves per row block
  constexpr int NT = 64 * SK_RWAVES * KH;     // threads
  constexpr int CPW = NCHK / KH;              // chunks per wave
  constexpr int KS = NCHK * SM_CHUNK;         // K of the slice
  constexpr int XROW = KS + 8;                // padded LDS row (halfs)
  constexpr int XCH = KS / 8;                 // 16-byte chunks per X row
  static_assert(NCHK % KH == 0 && SK_RWAVES * MB * 64 * 16 <= 16 * MB * XROW * 2, "K halves and their LDS sums fit");
  __shared__ __attribute__((aligned(16))) half_t xs[16 * MB * XROW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rw = wave % SK_RWAVES, kh = wave / SK_RWAVES;
  const int r = lane & 15, g = lane >> 4;
  const int rg = blockIdx.x % rgroups, slice = blockIdx.x / rgroups;
  const int k0 = slice * KS;
  const int nb = rg * SK_ROWS + rw * 16;      // first weight row of this wave
  // Rows past N re-read row N-1 (computed, never stored).
  const int n = min(nb + r, p.N - 1);
  const uint8_t* wrow = p.w + (int64_t)n * p.row_stride;

  uint32_t wv[CPW][WORDS];
  half_t sc[CPW], zc[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int kl = k0 + (kh * CPW + c) * SM_CHUNK + 32 * g;
    const int64_t boff = STORAGE == ANIMA_STORAGE_W4 ? kl / 2 : kl;
    const u32x4* src = reinterpret_cast<const u32x4*>(wrow + boff);
#pragma unroll
    for (int v = 0; v < WORDS / 4; ++v) {
      const u32x4 t4 = __builtin_nontemporal_load(src + v);
      wv[c][4 * v] = t4[0];
      wv[c][4 * v + 1] = t4[1];
      wv[c][4 * v + 2] = t4[2];
      wv[c][4 * v + 3] = t4[3];
    }
    sc[c] = p.scale[(int64_t)n * p.groups + (kl >> 6)];
    zc[c] = p.zero[(int64_t)n * p.groups + (kl >> 6)];
  }
  // The slice of X, 16 loads per thread in flight at a time.  Rows M .. 16 MB - 1 copy
  // row M - 1: they only feed output columns m >= M, which are never stored.
  constexpr int PER = 16 * MB * XCH / NT;
  constexpr int BATCH = PER <= 16 ? PER : (PER % 16 == 0 ? 16 : (PER % 12 == 0 ? 12 : 8));
  static_assert(PER * NT == 16 * MB * XCH && PER % BATCH == 0, "X copy splits evenly");
#pragma unroll
  for (int b0 = 0; b0 < PER; b0 += BATCH) {
    u32x4 v[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int i = threadIdx.x + (b0 + j) * NT;
      const int m = min(i / XCH, p.M - 1), ch = i % XCH;
      v[j] = *reinterpret_cast<const u32x4*>(p.x + (int64_t)m * p.K + k0 + ch * 8);
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int i = threadIdx.x + (b0 + j) * NT;
      *reinterpret_cast<u32x4*>(xs + (i / XCH) * XROW + (i % XCH) * 8) = v[j];
    }
  }
  __syncthreads();

  floatx4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = floatx4{};
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int kc = (kh * CPW + c) * SM_CHUNK;   // chunk start within the slice
    const bool fast = __all(one_rounding_exact<QBITS>(sc[c], zc[c]));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half8v a = fast ? dequant_frag<STORAGE, true>(wv[c], t, sc[c], zc[c])
                            : dequant_frag<STORAGE, false>(wv[c], t, sc[c], zc[c]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const half8v b = *reinterpret_cast<const half8v*>(xs + (mb * 16 + r) * XROW + kc + 32 * g + 8 * t);
        acc[mb] = mfma16(a, b, acc[mb]);
      }
    }
  }
  if constexpr (KH == 2) {
    // The second half's sums go to LDS over the X slice (once every wave is past its
    // reads) and the first half adds them: first half + second half, a fixed order.
    __syncthreads();
    floatx4* red = reinterpret_cast<floatx4*>(xs);
    if (kh == 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) red[(rw * MB + mb) * 64 + lane] = acc[mb];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] += red[(rw * MB + mb) * 64 + lane];
  }

  const int nc = nb + 4 * g;                  // this lane's first output column
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    if (m >= p.M) continue;
    if (part) {
      float* pp = part + ((int64_t)slice * p.M + m) * p.N + nc;
      if (nc + 3 < p.N && (reinterpret_cast<uintptr_t>(pp) & 15u) == 0) {
        *reinterpret_cast<floatx4*>(pp) = acc[mb];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nc + i < p.N) pp[i] = acc[mb][i];
      }
    } else {
      half_t* yp = p.y + (int64_t)m * p.N + nc;
      if (nc + 3 < p.N && (reinterpret_cast<uintptr_t>(yp) & 7u) == 0) {
        *reinterpret_cast<half4v*>(yp) =
            half4v{(half_t)acc[mb][0], (half_t)acc[mb][1], (half_t)acc[mb][2], (half_t)acc[mb][3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nc + i < p.N) yp[i] = (half_t)acc[mb][i];
      }
    }
  }
}

int smallm_splitk_slices(const GemmParams& p, int storage) {
  if (storage != ANIMA_STORAGE_W4 && storage != ANIMA_STORAGE_W8) return 0;
  if (p.epilogue != GEMM_STORE) return 0;
  // With N wide enough for the weight-streaming kernel to give 256 workgroups of 32
  // rows, that kernel is faster (it needs no partial rows); so it is with up to 32
  // input rows while X is under 256 KB.  Past that, each of its workgroups reading all
  // of X (about 0.044 us per KB at 16-row blocks) costs more than the partial rows:
  // M=32 N=2048 K=4096 13.3 -> 8.5 us, M=16 K=8192 13.2 -> 10.9 us, M=8 K=16384
  // 17.4 -> 14.9 us; M=16 K=4096 ties and M=32 N=4096 K=2048 is 5 % slower split.
  if (p.N >= 32 * 256 || (p.M <= 32 && (int64_t)p.M * p.K < 131072)) return 0;
  if (p.M < 1 || p.M > SMALLM_MAX_ROWS || p.K % SM_CHUNK != 0 || !aligned16(p.x) || !aligned16(p.w) ||
      p.row_stride % 16 != 0)
    return 0;
  const int mb = (p.M + 15) / 16, nch = p.K / SM_CHUNK;
  const int64_t rgroups = (p.N + SK_ROWS - 1) / SK_ROWS;
  int best = 0;
  // The fewest slices that give the grid 256 workgroups (else the most there can be),
  // each slice 1, 2, 4 or 8 chunks and its X copy within the LDS budget.
  for (int d = 1; d <= nch; ++d) {
    if (nch % d != 0) continue;
    const int ch = nch / d;
    if (ch > SK_MAX_CHUNKS || (ch & (ch - 1)) != 0) continue;
    if ((int64_t)16 * mb * (ch * SM_CHUNK + 8) * 2 > SK_MAX_LDS) continue;
    if (rgroups * d > 0x7fffffff) break;
    best = d;
    if (rgroups * d >= 256) break;
  }
  return best;
}

template <int STORAGE, int MB, int NCHK>
static void launch_splitk_t(const SmallMParams& sp, float* part, int rgroups, int slices, hipStream_t stream) {
  hipLaunchKernelGGL((smallm_splitk_kernel<STORAGE, MB, NCHK>), dim3((unsigned)(rgroups * slices)),
                     dim3(64 * SK_RWAVES * sk_khalves<NCHK>()), 0, stream, sp, part, rgroups);
}

template <int STORAGE, int MB>
static void launch_splitk_m(const SmallMParams& sp, float* part, int rgroups, int slices, int chunks,
                            hipStream_t stream) {
  switch (chunks) {
    case 1: launch_splitk_t<STORAGE, MB, 1>(sp, part, rgroups, slices, stream); break;
    case 2: launch_splitk_t<STORAGE, MB, 2>(sp, part, rgroups, slices, stream); break;
    case 4: launch_splitk_t<STORAGE, MB, 4>(sp, part, rgroups, slices, stream); break;
    case 8: launch_splitk_t<STORAGE, MB, 8>(sp, part, rgroups, slices, stream); break;
    default: fail(ANIMA_E_UNSUPPORTED, "small-M split-K GEMM: unsupported slice length");
  }
}

template <int STORAGE>
static void launch_splitk_s(const SmallMParams& sp, float* part, int rgroups, int slices, int chunks,
                            hipStream_t stream) {
  switch ((sp.M + 15) / 16) {
    case 1: launch_splitk_m<STORAGE, 1>(sp, part, rgroups, slices, chunks, stream); break;
    case 2: launch_splitk_m<STORAGE, 2>(sp, part, rgroups, slices, chunks, stream); break;
    case 3: launch_splitk_m<STORAGE, 3>(sp, part, rgroups, slices, chunks, stream); break;
    default: launch_splitk_m<STORAGE, 4>(sp, part, rgroups, slices, chunks, stream); break;
  }
}

void launch_smallm_splitk(const GemmParams& g, int storage, hipStream_t stream) {
  const int slices = smallm_splitk_slices(g, storage);
  if (slices < 1 || slices != (g.ksplit > 1 ? g.ksplit : 1))
    fail(ANIMA_E_INVALID_ARGUMENT, "small-M split-K GEMM: slice count does not match the shape");
  if (slices > 1 && !g.part) fail(ANIMA_E_INVALID_ARGUMENT, "small-M split-K GEMM: missing partial rows");
  SmallMParams sp{};
  sp.x = g.x; sp.y = g.y; sp.w = g.w; sp.scale = g.scale; sp.zero = g.zero;
  sp.row_stride = g.row_stride; sp.M = g.M; sp.N = g.N; sp.K = g.K; sp.groups = g.groups;
  const int rgroups = (g.N + SK_ROWS - 1) / SK_ROWS;
  const int chunks = g.K / SM_CHUNK / slices;
  float* part = slices > 1 ? g.part : nullptr;
  if (storage == ANIMA_STORAGE_W4)
    launch_splitk_s<ANIMA_STORAGE_W4>(sp, part, rgroups, slices, chunks, stream);
  else
    launch_splitk_s<ANIMA_STORAGE_W8>(sp, part, rgroups, slices, chunks, stream);
  ANIMA_HIP(hipGetLastError());
  if (slices > 1) launch_splitk_reduce(g.part, g.y, (int64_t)g.M * g.N, slices, stream);
}

}  // namespace anima
