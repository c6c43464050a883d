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

template <int STORAGE>
struct SmallMChunk {
  // 32-bit words of one lane's weight bytes for one 128-wide K chunk (32 k values).
  static constexpr int WORDS = STORAGE == ANIMA_STORAGE_W4 ? 4 : (STORAGE == ANIMA_STORAGE_W8 ? 8 : 16);
};

__device__ __forceinline__ half_t dq1(uint32_t q, float s, float z) {
  return f32_to_f16(fmaf((float)q, s, z));
}

// A fragment t (k = 32g + 8t .. +7 of the chunk) from a lane's raw weight words.
template <int STORAGE>
__device__ __forceinline__ half8v dequant_frag(const uint32_t (&wv)[SmallMChunk<STORAGE>::WORDS], int t, float s,
                                               float z) {
  half8v a;
  if constexpr (STORAGE == ANIMA_STORAGE_W4) {
    const uint32_t d = wv[t];
    const uint32_t lo = d & 0x0F0F0F0Fu;          // even k: nibbles 0, 2, 4, 6
    const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;   // odd k
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      a[2 * b] = dq1((lo >> (8 * b)) & 0xFFu, s, z);
      a[2 * b + 1] = dq1((hi >> (8 * b)) & 0xFFu, s, z);
    }
  } else if constexpr (STORAGE == ANIMA_STORAGE_W8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t d = wv[2 * t + h];
#pragma unroll
      for (int b = 0; b < 4; ++b) a[4 * h + b] = dq1((d >> (8 * b)) & 0xFFu, s, z);
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
  return MB == 1 ? (STORAGE == ANIMA_STORAGE_W4 ? 8 : 4)
                 : (STORAGE == ANIMA_STORAGE_W4 ? 4 : (STORAGE == ANIMA_STORAGE_W8 ? 2 : 1));
}

template <int STORAGE, int MB, int R, int NCH>
__global__ __launch_bounds__(64 * smallm_max_waves<MB>()) void smallm_gemm_kernel(SmallMParams p) {
  constexpr int WORDS = SmallMChunk<STORAGE>::WORDS;
  extern __shared__ float red[];   // [S][R*MB][4][64]

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int S = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * R;
  const int kslice = wave * p.kw;
  const int kstop = min(p.K, kslice + p.kw);

  // Rows past N re-read row N-1 (computed, never stored).
  const uint8_t* wrow[R];
  const half_t* srow[R];
  const half_t* zrow[R];
#pragma unroll
  for (int rb = 0; rb < R; ++rb) {
    const int n = min(n0 + rb * 16 + r, p.N - 1);
    wrow[rb] = p.w + (int64_t)n * p.row_stride * (STORAGE == ANIMA_STORAGE_FP16 ? 2 : 1);
    srow[rb] = p.scale + (int64_t)n * p.groups;
    zrow[rb] = p.zero + (int64_t)n * p.groups;
  }
  const half_t* xrow[MB];
  bool xvalid[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    xvalid[mb] = m < p.M;
    xrow[mb] = p.x + (int64_t)(xvalid[mb] ? m : 0) * p.K;
  }

  floatx4 acc[R][MB];
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = floatx4{};

  for (int kbeg = kslice; kbeg < kstop; kbeg += NCH * SM_CHUNK) {
  // Issue every weight load of this step (NCH chunks) before any arithmetic, so
  // their HBM latency is paid once per step.
  uint32_t wv[NCH][R][WORDS];
  float sc[NCH][R], zc[NCH][R];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int kl = kbeg + c * SM_CHUNK + 32 * g;
    const bool live = kbeg + c * SM_CHUNK < kstop;
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
      const int64_t boff = STORAGE == ANIMA_STORAGE_W4 ? kl / 2 : (STORAGE == ANIMA_STORAGE_W8 ? kl : 2 * kl);
      const u32x4* src = reinterpret_cast<const u32x4*>(wrow[rb] + (live ? boff : 0));
#pragma unroll
      for (int v = 0; v < WORDS / 4; ++v) {
        const u32x4 t4 = __builtin_nontemporal_load(src + v);
        wv[c][rb][4 * v] = t4[0];
        wv[c][rb][4 * v + 1] = t4[1];
        wv[c][rb][4 * v + 2] = t4[2];
        wv[c][rb][4 * v + 3] = t4[3];
      }
      if constexpr (STORAGE != ANIMA_STORAGE_FP16) {
        const int gi = live ? (kl >> 6) : 0;
        sc[c][rb] = (float)srow[rb][gi];
        zc[c][rb] = (float)zrow[rb][gi];
      } else {
        sc[c][rb] = zc[c][rb] = 0.f;
      }
    }
  }

  auto load_x = [&](int c, half8v (&xf)[MB][4]) {
    const int kl = kbeg + c * SM_CHUNK + 32 * g;
    const bool live = kbeg + c * SM_CHUNK < kstop;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xf[mb][t] = (live && xvalid[mb]) ? *reinterpret_cast<const half8v*>(xrow[mb] + kl + 8 * t) : half8v{};
  };

  half8v xa[MB][4], xb[MB][4];
  load_x(0, xa);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    half8v (&xc)[MB][4] = (c & 1) ? xb : xa;
    half8v (&xn)[MB][4] = (c & 1) ? xa : xb;
    if (c + 1 < NCH) load_x(c + 1, xn);
    // A chunk past K has zero X, so its (clamped, in-bounds) weight bytes add nothing.
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const half8v a = dequant_frag<STORAGE>(wv[c][rb], t, sc[c][rb], zc[c][rb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = mfma16(a, xc[mb][t], acc[rb][mb]);
      }
  }
  }

  // Fixed-order reduction of the S K-slices through LDS.
  constexpr int PAIRS = R * MB;
#pragma unroll
  for (int pi = 0; pi < PAIRS; ++pi)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * PAIRS + pi) * 4 + i) * 64 + lane] = acc[pi / MB][pi % MB][i];
  __syncthreads();
  for (int pi = wave; pi < PAIRS; pi += S) {
    const int rb = pi / MB, mb = pi % MB;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
      for (int w = 0; w < S; ++w) s += red[((w * PAIRS + pi) * 4 + i) * 64 + lane];
      v[i] = s;
    }
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

template <int STORAGE, int MB, int R, int NCH>
static void launch_smallm_t(SmallMParams p, hipStream_t stream) {
  // About 2048 waves over the grid, at most smallm_max_waves per workgroup, a K
  // slice per wave of whole steps of NCH chunks, and a reduction buffer
  // (S x R*MB KiB) within 64 KiB of LDS.
  const int wgs = (p.N + 16 * R - 1) / (16 * R);
  const int chunks = p.K / SM_CHUNK;
  const int max_s = std::min(smallm_max_waves<MB>(), 64 / (R * MB));
  const int want_s = std::max(1, std::min(max_s, 2048 / std::max(1, wgs)));
  const int steps = (chunks + NCH - 1) / NCH;
  const int steps_per_wave = (steps + want_s - 1) / want_s;
  p.kw = steps_per_wave * NCH * SM_CHUNK;
  const int S = (p.K + p.kw - 1) / p.kw;
  const size_t lds = (size_t)S * R * MB * 4 * 64 * sizeof(float);
  hipLaunchKernelGGL((smallm_gemm_kernel<STORAGE, MB, R, NCH>), dim3(wgs), dim3(64 * S), lds, stream, p);
}

template <int STORAGE, int MB, int R>
static void launch_smallm_r(const SmallMParams& p, hipStream_t stream) {
  constexpr int NCH = smallm_max_chunks<STORAGE, MB>();
  // Fewer chunks per step when K is short, so waves are not left empty.
  const int chunks = p.K / SM_CHUNK;
  if (NCH >= 8 && chunks <= 16 * 4)
    launch_smallm_t<STORAGE, MB, R, (NCH >= 4 ? 4 : NCH)>(p, stream);
  else
    launch_smallm_t<STORAGE, MB, R, NCH>(p, stream);
}

template <int STORAGE>
static void launch_smallm_s(const SmallMParams& p, hipStream_t stream) {
  const int MB = (p.M + 15) / 16;
  switch (MB) {
    case 1: launch_smallm_r<STORAGE, 1, 1>(p, stream); break;
    case 2: launch_smallm_r<STORAGE, 2, 2>(p, stream); break;
    case 3: launch_smallm_r<STORAGE, 3, 2>(p, stream); break;
    default: launch_smallm_r<STORAGE, 4, 2>(p, stream); break;
  }
}

bool smallm_supported(const GemmParams& p, int storage) {
  if (p.M < 1 || p.M > SMALLM_MAX_ROWS || p.K % SM_CHUNK != 0 || !aligned16(p.x) || !aligned16(p.w)) return false;
  if (storage == ANIMA_STORAGE_FP16) return p.row_stride % 8 == 0;
  return p.row_stride % 16 == 0;
}

void launch_smallm(const GemmParams& g, int storage, hipStream_t stream) {
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

}  // namespace anima
