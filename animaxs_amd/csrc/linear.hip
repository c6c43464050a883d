// Quantized linear for gfx950: W4/W8/FP16-weight MFMA GEMM with the dequant
// fused into the weight-tile load, the standalone dequant kernel and the fp32
// matvec.
//
// Replaces LinearExecutor.encodeMPS / encodeQGEMM (AnimaXS/Runtime/Metal/
// LinearExecutor.swift:137-361) and the Metal kernels dequant_w4_to_half,
// dequant_w8_to_half, copy_half_rows, qgemm_*, w4/w8/fp16_matvec_f32
// (AnimaXS/Shaders/AnimaKernels.metal:19-79, 804-1047).  Weight value
// v = fl32(q*scale + zero) (q*scale is exact, so one rounding), fp16 weight
// RNE16(v): bit-identical to the reference's dequant_*_to_half.
#include <algorithm>
#include <string>

#include "linear.hpp"

namespace anima {

// ===========================================================================
// GEMM: Y[M,N] = X[M,K] deq(W)[N,K]^T.
//
// Workgroup tile 256 (M) x 128 (N) x 64 (K = one quantisation group), 4 waves
// as 2 (N) x 2 (M); each wave owns 64 x 128 of C^T = W X^T computed with
// v_mfma_f32_32x32x16_f16 (weights on M so each lane ends with 4 consecutive
// output columns -> 8-byte stores).  The weight tile is unpacked and
// dequantised in registers (nibble -> v_cvt_f32_ubyte, one FMA, RNE pack) and
// written to LDS as fp16; X and W tiles are double-buffered with an XOR
// swizzle; the next K block's global loads are issued before this block's
// MFMAs.
// ===========================================================================
constexpr int G_BM = 256, G_BN = 128, G_BK = 64, G_NT = 256;

__device__ __forceinline__ half_t dq1(uint32_t q, float s, float z) {
  return f32_to_f16(fmaf((float)q, s, z));
}

// 16 packed bytes of one W4 row (32 K values) -> four fp16 chunks of 8.
__device__ __forceinline__ void dq_w4_16(const u32x4 raw, float s, float z, half8v out[4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = raw[w];
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    half8v o;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      o[2 * b] = dq1((lo >> (8 * b)) & 0xffu, s, z);
      o[2 * b + 1] = dq1((hi >> (8 * b)) & 0xffu, s, z);
    }
    out[w] = o;
  }
}

// 16 packed bytes of one W8 row (16 K values) -> two fp16 chunks of 8.
__device__ __forceinline__ void dq_w8_16(const u32x4 raw, float s, float z, half8v out[2]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = raw[w];
#pragma unroll
    for (int b = 0; b < 4; ++b) out[w >> 1][(w & 1) * 4 + b] = dq1((x >> (8 * b)) & 0xffu, s, z);
  }
}

template <int STORAGE, bool FAST>
__global__ __launch_bounds__(G_NT, 1) void gemm_kernel(GemmParams p, int vec_store) {
  __shared__ __attribute__((aligned(16))) half_t Xs[2][G_BM * G_BK];
  __shared__ __attribute__((aligned(16))) half_t Ws[2][G_BN * G_BK];
  constexpr int XL = G_BM * G_BK / 8 / G_NT;      // 8 X chunks per thread
  constexpr int WL = STORAGE == ANIMA_STORAGE_W4 ? 1 : (STORAGE == ANIMA_STORAGE_W8 ? 2 : 4);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c32 = lane & 31, hh = lane >> 5;
  const int wn = wave & 1, wm = wave >> 1;
  const int ntn = (p.N + G_BN - 1) / G_BN;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int tn = lb % ntn, tm = lb / ntn;
  const int m0 = tm * G_BM, n0 = tn * G_BN;
  const int nk = (p.K + G_BK - 1) / G_BK;

  // One K block's global data in registers.  The fast path keeps two of these so the
  // loads of block kb+2 are in flight while block kb+1 is written to LDS.
  struct Regs {
    half8v xr[XL];
    u32x4 wr[WL];
    float ws_s[WL], ws_z[WL];
  };
  const half8v zero8 = {};
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  auto load_global = [&](int kb, Regs& rg) __attribute__((always_inline)) {
    half8v (&xr)[XL] = rg.xr;
    u32x4 (&wr)[WL] = rg.wr;
    float (&ws_s)[WL] = rg.ws_s;
    float (&ws_z)[WL] = rg.ws_z;
    const int kbase = kb * G_BK;
#pragma unroll
    for (int r = 0; r < XL; ++r) {
      const int c = tid + G_NT * r;
      const int row = c >> 3, ch = c & 7;
      const int m = m0 + row;
      if (FAST) {
        // Rows past M are clamped, not masked: they only feed output rows never stored.
        xr[r] = *reinterpret_cast<const half8v*>(p.x + (int64_t)min(m, p.M - 1) * p.K + kbase + ch * 8);
      } else {
        half8v v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = kbase + ch * 8 + e;
          v[e] = (m < p.M && k < p.K) ? p.x[(int64_t)m * p.K + k] : (half_t)0.f;
        }
        xr[r] = v;
      }
    }
#pragma unroll
    for (int r = 0; r < WL; ++r) {
      const int c = tid + G_NT * r;
      int row, part;
      if (STORAGE == ANIMA_STORAGE_W4) { row = c >> 1; part = c & 1; }
      else if (STORAGE == ANIMA_STORAGE_W8) { row = c >> 2; part = c & 3; }
      else { row = c >> 3; part = c & 7; }
      // Rows past N are clamped in the fast path: they only feed columns never stored.
      const int n = FAST ? min(n0 + row, p.N - 1) : n0 + row;
      if (STORAGE != ANIMA_STORAGE_FP16) {
        if (FAST) {
          ws_s[r] = (float)p.scale[(int64_t)n * p.groups + kb];
          ws_z[r] = (float)p.zero[(int64_t)n * p.groups + kb];
        } else {
          ws_s[r] = n < p.N ? (float)p.scale[(int64_t)n * p.groups + kb] : 0.f;
          ws_z[r] = n < p.N ? (float)p.zero[(int64_t)n * p.groups + kb] : 0.f;
        }
      }
      if (FAST) {
        const uint8_t* src;
        if (STORAGE == ANIMA_STORAGE_W4) src = p.w + (int64_t)n * p.row_stride + kb * 32 + part * 16;
        else if (STORAGE == ANIMA_STORAGE_W8) src = p.w + (int64_t)n * p.row_stride + kbase + part * 16;
        else src = p.w + ((int64_t)n * p.row_stride + kbase + part * 8) * 2;
        wr[r] = *reinterpret_cast<const u32x4*>(src);
      } else {
        // byte-granular path: any row stride / offset / K tail
        uint32_t bytes[4] = {0u, 0u, 0u, 0u};
        if (STORAGE == ANIMA_STORAGE_W4) {
          // 32 K values -> 16 nibble bytes (even K low nibble); out-of-range K -> q = 0, and the
          // value itself is zeroed after dequant (see store_tile)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int k = kbase + part * 32 + 2 * i;
            uint32_t b = 0;
            if (n < p.N && k < p.K) b = p.w[(int64_t)n * p.row_stride + (k >> 1)];
            if (k + 1 >= p.K) b &= 0x0Fu;
            bytes[i >> 2] |= b << (8 * (i & 3));
          }
        } else if (STORAGE == ANIMA_STORAGE_W8) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int k = kbase + part * 16 + i;
            const uint32_t b = (n < p.N && k < p.K) ? p.w[(int64_t)n * p.row_stride + k] : 0u;
            bytes[i >> 2] |= b << (8 * (i & 3));
          }
        } else {
          const half_t* w16 = reinterpret_cast<const half_t*>(p.w);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int k = kbase + part * 8 + i;
            const half_t h = (n < p.N && k < p.K) ? w16[(int64_t)n * p.row_stride + k] : (half_t)0.f;
            const uint32_t hb = __builtin_bit_cast(uint16_t, h);
            bytes[i >> 1] |= hb << (16 * (i & 1));
          }
        }
        wr[r] = u32x4{bytes[0], bytes[1], bytes[2], bytes[3]};
      }
    }
  };

  auto store_tile = [&](int st, int kb, const Regs& rg) __attribute__((always_inline)) {
    const half8v (&xr)[XL] = rg.xr;
    const u32x4 (&wr)[WL] = rg.wr;
    const float (&ws_s)[WL] = rg.ws_s;
    const float (&ws_z)[WL] = rg.ws_z;
    const int kbase = kb * G_BK;
#pragma unroll
    for (int r = 0; r < XL; ++r) {
      const int c = tid + G_NT * r;
      const int row = c >> 3, ch = c & 7;
      *reinterpret_cast<half8v*>(&Xs[st][row * G_BK + ((ch ^ (row & 7)) * 8)]) = xr[r];
    }
#pragma unroll
    for (int r = 0; r < WL; ++r) {
      const int c = tid + G_NT * r;
      if (STORAGE == ANIMA_STORAGE_W4) {
        const int row = c >> 1, part = c & 1;
        half8v o[4];
        dq_w4_16(wr[r], ws_s[r], ws_z[r], o);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!FAST) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (kbase + part * 32 + j * 8 + e >= p.K) o[j][e] = (half_t)0.f;
          }
          const int ch = part * 4 + j;
          *reinterpret_cast<half8v*>(&Ws[st][row * G_BK + ((ch ^ (row & 7)) * 8)]) = o[j];
        }
      } else if (STORAGE == ANIMA_STORAGE_W8) {
        const int row = c >> 2, part = c & 3;
        half8v o[2];
        dq_w8_16(wr[r], ws_s[r], ws_z[r], o);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if (!FAST) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (kbase + part * 16 + j * 8 + e >= p.K) o[j][e] = (half_t)0.f;
          }
          const int ch = part * 2 + j;
          *reinterpret_cast<half8v*>(&Ws[st][row * G_BK + ((ch ^ (row & 7)) * 8)]) = o[j];
        }
      } else {
        const int row = c >> 3, ch = c & 7;
        *reinterpret_cast<u32x4*>(&Ws[st][row * G_BK + ((ch ^ (row & 7)) * 8)]) = wr[r];
      }
    }
  };

  floatx16 acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = floatx16{};

  auto mfma_block = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < G_BK / 16; ++s) {
      half8v wf[2], xf[4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 64 * wn + 32 * t + c32;
        wf[t] = *reinterpret_cast<const half8v*>(&Ws[st][row * G_BK + (((2 * s + hh) ^ (row & 7)) * 8)]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 128 * wm + 32 * t + c32;
        xf[t] = *reinterpret_cast<const half8v*>(&Xs[st][row * G_BK + (((2 * s + hh) ^ (row & 7)) * 8)]);
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma32(wf[a], xf[b], acc[a][b]);
    }
  };

  if (FAST) {
    // Register double buffer, loads two K blocks ahead, every load unconditional (the
    // prefetch past the last block re-reads it) so each wait covers exactly the
    // older block.  Unrolled by two so both register sets stay static.
    Regs ra, rb;
    if (nk > 0) {
      load_global(0, ra);
      load_global(min(1, nk - 1), rb);
      store_tile(0, 0, ra);
    }
    __syncthreads();
    for (int kb = 0; kb < nk; kb += 2) {
      load_global(min(kb + 2, nk - 1), ra);
      mfma_block(0);
      if (kb + 1 < nk) store_tile(1, kb + 1, rb);
      __syncthreads();
      if (kb + 1 >= nk) break;
      load_global(min(kb + 3, nk - 1), rb);
      mfma_block(1);
      if (kb + 2 < nk) store_tile(0, kb + 2, ra);
      __syncthreads();
    }
  } else {
    Regs ra;
    if (nk > 0) {
      load_global(0, ra);
      store_tile(0, 0, ra);
    }
    __syncthreads();
    for (int kb = 0; kb < nk; ++kb) {
      const int st = kb & 1;
      if (kb + 1 < nk) load_global(kb + 1, ra);
      mfma_block(st);
      if (kb + 1 < nk) store_tile(st ^ 1, kb + 1, ra);
      __syncthreads();
    }
  }

#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int m = m0 + 128 * wm + 32 * b + c32;
      if (m >= p.M) continue;
      half_t* yrow = p.y + (int64_t)m * p.N;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int n = n0 + 64 * wn + 32 * a + 8 * jj + 4 * hh;
        const half4v v = {(half_t)acc[a][b][4 * jj], (half_t)acc[a][b][4 * jj + 1], (half_t)acc[a][b][4 * jj + 2],
                          (half_t)acc[a][b][4 * jj + 3]};
        if (vec_store && n + 3 < p.N) {
          *reinterpret_cast<half4v*>(yrow + n) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.N) yrow[n + e] = v[e];
        }
      }
    }
}

// ===========================================================================
// Standalone dequant (dequant_w4_to_half / dequant_w8_to_half): one thread per
// (row, 8 consecutive K); exact reference element formula.
// ===========================================================================
__global__ __launch_bounds__(256) void dequant_kernel(DequantParams p) {
  const int chunks = (p.K + 7) / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)chunks * p.N) return;
  const int r = (int)(idx / chunks);
  const int k0 = (int)(idx % chunks) * 8;
  half_t* out = p.out + (int64_t)r * p.out_stride;
  if (p.storage == ANIMA_STORAGE_FP16) {
    const half_t* w16 = reinterpret_cast<const half_t*>(p.w) + (int64_t)r * p.row_stride;
    for (int k = k0; k < k0 + 8 && k < p.K; ++k) out[k] = w16[k];
    return;
  }
  const uint8_t* row = p.w + (int64_t)r * p.row_stride;
  for (int k = k0; k < k0 + 8 && k < p.K; ++k) {
    uint32_t q;
    if (p.storage == ANIMA_STORAGE_W4) {
      const uint32_t b = row[k >> 1];
      q = (k & 1) == 0 ? (b & 0x0Fu) : (b >> 4);
    } else {
      q = row[k];
    }
    const int64_t g = (int64_t)r * p.groups + k / 64;
    out[k] = dq1(q, (float)p.scale[g], (float)p.zero[g]);
  }
}

// ===========================================================================
// fp32 matvec (w4/w8/fp16_matvec_f32).
//
// Vectorised form: LPR lanes per output row, 64/LPR rows per wave.  Each lane
// reads 16-byte chunks of the packed row (8 fp16 / 16 W8 / 32 W4 weights, always
// inside one 64-column quantisation group) and accumulates x*w with fp32 FMAs; a
// butterfly over the row's LPR lanes sums it.  One launch takes up to MV_BATCH
// independent matvecs of one storage and lane split (the DiT modulation's three
// branches), each with an optional SiLU on the input and bias on the output.
// Rows that are not 16-byte aligned, or whose length is not a multiple of the
// chunk, take the scalar kernel (one wave per row, one weight per lane and step).
// ===========================================================================
template <int STORAGE>
struct MvChunk {
  static constexpr int elems = STORAGE == ANIMA_STORAGE_W4 ? 32 : STORAGE == ANIMA_STORAGE_W8 ? 16 : 8;
};

__device__ __forceinline__ float mv_finish(const MatvecParams& p, int row, float sum) {
  return p.bias ? sum + p.bias[row] : sum;
}

template <int STORAGE, int LPR, int CAP>
__global__ __launch_bounds__(256) void matvec_vec_kernel(MatvecBatchN<CAP> b) {
  constexpr int E = MvChunk<STORAGE>::elems, RPW = 64 / LPR;
  int bi = 0;
#pragma unroll
  for (int j = 1; j < CAP; ++j)
    if (j < b.count && (int)blockIdx.x >= b.first_block[j]) bi = j;
  MatvecParams p;
  if constexpr (CAP == MV_BATCH) {
    p = b.p[0];
    if (bi == 1) p = b.p[1];
    if (bi == 2) p = b.p[2];
  } else {
    p = b.p[bi];   // bi is uniform over the workgroup: scalar loads at a computed offset
  }
  const int lane = threadIdx.x & 63, sub = lane & (LPR - 1);
  const int row = ((int)blockIdx.x - b.first_block[bi]) * (4 * RPW) + (threadIdx.x >> 6) * RPW + lane / LPR;
  float sum = 0.f;
  if (row < p.N) {
    const uint8_t* wrow = p.w + (int64_t)row * p.row_stride * (STORAGE == ANIMA_STORAGE_FP16 ? 2 : 1);
    const int nch = p.K / E;
    for (int c = sub; c < nch; c += LPR) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(wrow + (int64_t)c * 16);
      const int k0 = c * E;
      float xv[E];
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const floatx4 t = *reinterpret_cast<const floatx4*>(p.x + k0 + e);
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[e + u] = p.silu_input ? silu_f32(t[u]) : t[u];
      }
      if (STORAGE == ANIMA_STORAGE_FP16) {
        const half8v wv = __builtin_bit_cast(half8v, raw);
#pragma unroll
        for (int e = 0; e < E; ++e) sum = fmaf(xv[e], (float)wv[e], sum);
      } else {
        const int64_t g = (int64_t)row * p.groups + k0 / 64;
        const float sc = (float)p.scale[g], zr = (float)p.zero[g];
#pragma unroll
        for (int e = 0; e < E; ++e) {
          uint32_t q;
          if (STORAGE == ANIMA_STORAGE_W4)
            q = (raw[e / 8] >> (4 * (e % 8))) & 0x0Fu;
          else
            q = (raw[e / 4] >> (8 * (e % 4))) & 0xFFu;
          sum = fmaf(xv[e], (float)q * sc + zr, sum);
        }
      }
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (row < p.N && sub == 0) p.y[row] = mv_finish(p, row, sum);
}

__global__ __launch_bounds__(256) void matvec_kernel(MatvecParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.N) return;
  float sum = 0.f;
  if (p.storage == ANIMA_STORAGE_FP16) {
    const half_t* w16 = reinterpret_cast<const half_t*>(p.w) + (int64_t)row * p.row_stride;
    for (int k = lane; k < p.K; k += 64) {
      const float x = p.silu_input ? silu_f32(p.x[k]) : p.x[k];
      sum = fmaf(x, (float)w16[k], sum);
    }
  } else {
    const uint8_t* w = p.w + (int64_t)row * p.row_stride;
    for (int k = lane; k < p.K; k += 64) {
      uint32_t q;
      if (p.storage == ANIMA_STORAGE_W4) {
        const uint32_t b = w[k >> 1];
        q = (k & 1) == 0 ? (b & 0x0Fu) : (b >> 4);
      } else {
        q = w[k];
      }
      const int64_t g = (int64_t)row * p.groups + k / 64;
      const float v = (float)q * (float)p.scale[g] + (float)p.zero[g];
      const float x = p.silu_input ? silu_f32(p.x[k]) : p.x[k];
      sum = fmaf(x, v, sum);
    }
  }
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane == 0) p.y[row] = mv_finish(p, row, sum);
}

// ===========================================================================
// Launchers.
// ===========================================================================
template <int S>
static void launch_gemm_t(const GemmParams& p, bool fast, int vec, dim3 grid, hipStream_t stream) {
  if (fast)
    hipLaunchKernelGGL((gemm_kernel<S, true>), grid, dim3(G_NT), 0, stream, p, vec);
  else
    hipLaunchKernelGGL((gemm_kernel<S, false>), grid, dim3(G_NT), 0, stream, p, vec);
}

void launch_gemm(const GemmParams& p, int storage, hipStream_t stream) {
  if (p.M <= 0 || p.N <= 0) return;
  if (pingpong_supported(p, storage)) {
    launch_pingpong(p, storage, stream);
    return;
  }
  if (p.epilogue != GEMM_STORE) fail(ANIMA_E_UNSUPPORTED, "fused GEMM epilogues need the ping-pong kernel");
  const int64_t tiles = (int64_t)((p.M + G_BM - 1) / G_BM) * ((p.N + G_BN - 1) / G_BN);
  if (tiles <= 0) return;
  if (tiles > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "GEMM grid too large");
  const bool x_ok = aligned16(p.x) && (p.K % 8 == 0);
  bool w_ok;
  if (storage == ANIMA_STORAGE_W4)
    w_ok = aligned16(p.w) && (p.row_stride % 16 == 0);
  else if (storage == ANIMA_STORAGE_W8)
    w_ok = aligned16(p.w) && (p.row_stride % 16 == 0);
  else
    w_ok = aligned16(p.w) && (p.row_stride % 8 == 0);
  const bool fast = x_ok && w_ok && (p.K % G_BK == 0);
  const int vec = ((reinterpret_cast<uintptr_t>(p.y) & 7u) == 0 && p.N % 4 == 0) ? 1 : 0;
  const dim3 grid((unsigned)tiles);
  if (storage == ANIMA_STORAGE_W4)
    launch_gemm_t<ANIMA_STORAGE_W4>(p, fast, vec, grid, stream);
  else if (storage == ANIMA_STORAGE_W8)
    launch_gemm_t<ANIMA_STORAGE_W8>(p, fast, vec, grid, stream);
  else
    launch_gemm_t<ANIMA_STORAGE_FP16>(p, fast, vec, grid, stream);
  ANIMA_HIP(hipGetLastError());
}

void launch_dequant(const DequantParams& p, hipStream_t stream) {
  const int64_t total = (int64_t)((p.K + 7) / 8) * p.N;
  if (total <= 0) return;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "dequant grid too large");
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  ANIMA_HIP(hipGetLastError());
}

// Lanes per row for the vectorised matvec: the smallest power of two in [8, 64]
// that covers the row's chunks in one step, or 0 when the row does not vectorise.
static int matvec_lanes(const MatvecParams& p) {
  const int e = p.storage == ANIMA_STORAGE_W4 ? 32 : p.storage == ANIMA_STORAGE_W8 ? 16 : 8;
  const int64_t stride_bytes = p.row_stride * (p.storage == ANIMA_STORAGE_FP16 ? 2 : 1);
  if (p.K % e != 0 || stride_bytes % 16 != 0 || !aligned16(p.w) || !aligned16(p.x)) return 0;
  const int nch = p.K / e;
  int lpr = 8;
  while (lpr < 64 && lpr < nch) lpr *= 2;
  return lpr;
}

template <int STORAGE, int CAP>
static void launch_matvec_vec(const MatvecBatchN<CAP>& b, int lpr, unsigned blocks, hipStream_t stream) {
  switch (lpr) {
    case 8: hipLaunchKernelGGL((matvec_vec_kernel<STORAGE, 8, CAP>), dim3(blocks), dim3(256), 0, stream, b); break;
    case 16: hipLaunchKernelGGL((matvec_vec_kernel<STORAGE, 16, CAP>), dim3(blocks), dim3(256), 0, stream, b); break;
    case 32: hipLaunchKernelGGL((matvec_vec_kernel<STORAGE, 32, CAP>), dim3(blocks), dim3(256), 0, stream, b); break;
    default: hipLaunchKernelGGL((matvec_vec_kernel<STORAGE, 64, CAP>), dim3(blocks), dim3(256), 0, stream, b); break;
  }
}

// One launch of count (1..CAP) matvecs that share storage and lane split lpr.
template <int CAP>
static void launch_matvec_together(const MatvecParams* ps, int count, int lpr, hipStream_t stream) {
  MatvecBatchN<CAP> b{};
  const int rows_per_block = 4 * (64 / lpr);
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) {
    b.p[i] = ps[i];
    b.first_block[i] = (int)blocks;
    blocks += ps[i].N > 0 ? (ps[i].N + rows_per_block - 1) / rows_per_block : 0;
    if (blocks > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "matvec grid too large");
  }
  for (int i = count; i < CAP; ++i) b.first_block[i] = (int)blocks;
  b.count = count;
  if (blocks <= 0) return;
  if (ps[0].storage == ANIMA_STORAGE_W4)
    launch_matvec_vec<ANIMA_STORAGE_W4>(b, lpr, (unsigned)blocks, stream);
  else if (ps[0].storage == ANIMA_STORAGE_W8)
    launch_matvec_vec<ANIMA_STORAGE_W8>(b, lpr, (unsigned)blocks, stream);
  else
    launch_matvec_vec<ANIMA_STORAGE_FP16>(b, lpr, (unsigned)blocks, stream);
  ANIMA_HIP(hipGetLastError());
}

void launch_matvec_batch(const MatvecParams* ps, int count, hipStream_t stream) {
  if (count < 1 || count > MV_BATCH) fail(ANIMA_E_INVALID_ARGUMENT, "matvec batch holds 1 to 3 matvecs");
  const int lpr = matvec_lanes(ps[0]);
  bool together = lpr != 0;
  for (int i = 1; i < count; ++i)
    together = together && ps[i].storage == ps[0].storage && matvec_lanes(ps[i]) == lpr;
  if (!together) {
    for (int i = 0; i < count; ++i) {
      if (ps[i].N <= 0) continue;
      if (matvec_lanes(ps[i]) != 0) {
        launch_matvec_batch(&ps[i], 1, stream);
      } else {
        hipLaunchKernelGGL(matvec_kernel, dim3((unsigned)((ps[i].N + 3) / 4)), dim3(256), 0, stream, ps[i]);
        ANIMA_HIP(hipGetLastError());
      }
    }
    return;
  }
  launch_matvec_together<MV_BATCH>(ps, count, lpr, stream);
}

void launch_matvec_many(const MatvecParams* ps, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int lpr = matvec_lanes(ps[0]);
  bool together = lpr != 0;
  for (int64_t i = 1; i < count; ++i)
    together = together && ps[i].storage == ps[0].storage && matvec_lanes(ps[i]) == lpr;
  for (int64_t i = 0; i < count;) {
    const int cap = together ? MV_BATCH_WIDE : MV_BATCH;
    const int n = (int)std::min<int64_t>(cap, count - i);
    if (together)
      launch_matvec_together<MV_BATCH_WIDE>(ps + i, n, lpr, stream);
    else
      launch_matvec_batch(ps + i, n, stream);
    i += n;
  }
}

void launch_matvec(const MatvecParams& p, hipStream_t stream) {
  if (p.N <= 0) return;
  launch_matvec_batch(&p, 1, stream);
}

// ---------------------------------------------------------------------------
// Read probe: the achievable rate of a plain streaming read of `bytes` bytes, the
// floor a weight-streaming kernel of the same byte count is measured against.  Every
// thread XOR-folds 16-byte nontemporal loads (UNROLL in flight per iteration) and
// each workgroup writes one 16-byte word to `sink`, so the probe reads exactly the
// bytes asked and writes a few KB.
// ---------------------------------------------------------------------------
constexpr int PROBE_THREADS = 256, PROBE_UNROLL = 4, PROBE_MAX_BLOCKS = 2048;

__global__ __launch_bounds__(PROBE_THREADS) void read_probe_kernel(const u32x4* src, int64_t chunks, u32x4* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * PROBE_THREADS;
  int64_t i = (int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x;
  for (; i + (PROBE_UNROLL - 1) * stride < chunks; i += PROBE_UNROLL * stride) {
    u32x4 v[PROBE_UNROLL];
#pragma unroll
    for (int u = 0; u < PROBE_UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u];
  }
  for (; i < chunks; i += stride) acc ^= __builtin_nontemporal_load(src + i);
  __shared__ u32x4 part[PROBE_THREADS];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = PROBE_THREADS / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] ^= part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0];
}

// One 16-byte chunk per thread up to PROBE_MAX_BLOCKS workgroups (small reads spread over
// the whole chip), then grid-stride loops with PROBE_UNROLL loads in flight.
int64_t read_probe_sink_bytes(int64_t bytes) {
  const int64_t chunks = bytes / 16;
  const int64_t blocks = std::min<int64_t>(PROBE_MAX_BLOCKS, std::max<int64_t>(1, (chunks + PROBE_THREADS - 1) / PROBE_THREADS));
  return blocks * 16;
}

void launch_read_probe(const void* src, int64_t bytes, void* sink, hipStream_t stream) {
  const int64_t chunks = bytes / 16;
  if (chunks <= 0) return;
  const int64_t blocks = read_probe_sink_bytes(bytes) / 16;
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)blocks), dim3(PROBE_THREADS), 0, stream,
                     static_cast<const u32x4*>(src), chunks, static_cast<u32x4*>(sink));
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
