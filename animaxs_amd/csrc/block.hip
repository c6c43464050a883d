// DiT block and Qwen layer support kernels and compositions for gfx950.
//
// Kernels restate AnimaXS/Shaders/AnimaKernels.metal: dit_layernorm_modulate_to_half
// (:477-524), gate_add_half_f32 (:624-634), dit_gelu_half_inplace (:312-322),
// silu (:388-397), add_f32 (:649-656), rmsnorm_f32_to_f32 + float_to_half
// (:172-204, :81-88), gated_silu_half (:401-411) and add_half_into_float (:639-647).  The composition follows
// DiTBlockExecutor.encodeAttentionBranch / encodeMLP / encodeModulation
// (AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:1035-1319, :1403-1417) with every
// shape a parameter (the reference hard-wires 1024 tokens).
#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "attention.hpp"
#include "block.hpp"
#include "linear.hpp"
#include "pack.hpp"

namespace anima {

// ---------------------------------------------------------------------------
// Row normalisations.  Wave form: one wave per row, four rows per 256-thread
// workgroup; lane l holds columns 4*(l + 64*e) .. +3 for e < V as float4s, so the
// row stays in registers between the mean, variance and output passes (the
// reference re-reads memory three times) and the sums are wave butterflies with
// no barriers.  Rows longer than 256*V (V <= 16), not a multiple of 4 columns or
// not 16-byte aligned take the workgroup-per-row kernels (one element per thread
// and step, n <= 8192).
// ---------------------------------------------------------------------------
constexpr int LN_NT = 256;
constexpr int LN_MAX_PER_THREAD = 32;  // n <= 8192

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < LN_NT / 64; ++w) t += red[w];
  return t;
}

// dit_layernorm_modulate_to_half (AnimaKernels.metal:477-524):
// half(((x - mean) * rsqrt(var + eps)) * (1 + scale) + shift), var the mean of the
// squared deviations.  With HB (the FinalLayer's fp16 boundaries,
// DiTFinalLayerExecutor.swift:134-157) the residual is read as float(half(x)) and the
// normalised value is rounded through fp16 before the modulation.
template <int V, bool HB>
__global__ __launch_bounds__(256) void layernorm_modulate_wave_kernel(const float* __restrict__ residual,
                                                                      const float* __restrict__ mod,
                                                                      half_t* __restrict__ out, int n, int rows,
                                                                      float eps, int64_t mod_offset) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* x = residual + (int64_t)row * n;
  const float* scale = mod + mod_offset;
  const float* shift = mod;
  floatx4 v[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int c = 4 * (lane + 64 * e);
    v[e] = c < n ? *reinterpret_cast<const floatx4*>(x + c) : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  // Up to 2048 columns the modulation rows go out right behind the row, so their round
  // trip overlaps the row's instead of following the two reductions (wider rows load
  // them at the end, within the registers that keep four waves per SIMD).
  constexpr bool PRE = V <= 8;
  floatx4 sc[PRE ? V : 1], sh[PRE ? V : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int c = 4 * (lane + 64 * e);
      sc[e] = c < n ? *reinterpret_cast<const floatx4*>(scale + c) : floatx4{0.f, 0.f, 0.f, 0.f};
      sh[e] = c < n ? *reinterpret_cast<const floatx4*>(shift + c) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if (HB) {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[e][u] = (float)(half_t)v[e][u];
    }
    s += (v[e][0] + v[e][1]) + (v[e][2] + v[e][3]);
  }
  const float mean = wave_sum(s) / (float)n;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int c = 4 * (lane + 64 * e);
    if (c < n) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float d = v[e][u] - mean;
        sq = fmaf(d, d, sq);
      }
    }
  }
  const float inv = rsqrtf(wave_sum(sq) / (float)n + eps);
  half_t* o = out + (int64_t)row * n;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int c = 4 * (lane + 64 * e);
    if (c < n) {
      const floatx4 sce = PRE ? sc[PRE ? e : 0] : *reinterpret_cast<const floatx4*>(scale + c);
      const floatx4 she = PRE ? sh[PRE ? e : 0] : *reinterpret_cast<const floatx4*>(shift + c);
      half4v h;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float nv = (v[e][u] - mean) * inv;
        if (HB) nv = (float)f32_to_f16(nv);
        h[u] = f32_to_f16(nv * (1.0f + sce[u]) + she[u]);
      }
      *reinterpret_cast<half4v*>(o + c) = h;
    }
  }
}

template <bool HB>
__global__ __launch_bounds__(LN_NT) void layernorm_modulate_kernel(const float* __restrict__ residual,
                                                                   const float* __restrict__ mod, half_t* __restrict__ out,
                                                                   int n, float eps, int64_t mod_offset) {
  __shared__ float red[LN_NT / 64];
  const int64_t row = blockIdx.x;
  const float* x = residual + row * n;
  float v[LN_MAX_PER_THREAD];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < LN_MAX_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * LN_NT;
    v[e] = i < n ? (HB ? (float)(half_t)x[i] : x[i]) : 0.f;
    s += v[e];
  }
  const float mean = block_sum(s, red) / (float)n;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < LN_MAX_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * LN_NT;
    if (i < n) {
      const float c = v[e] - mean;
      sq = fmaf(c, c, sq);
    }
  }
  const float inv = rsqrtf(block_sum(sq, red) / (float)n + eps);
  const float* scale = mod + mod_offset;
  const float* shift = mod;
  half_t* o = out + row * n;
#pragma unroll
  for (int e = 0; e < LN_MAX_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * LN_NT;
    if (i < n) {
      float nv = (v[e] - mean) * inv;
      if (HB) nv = (float)f32_to_f16(nv);
      o[i] = f32_to_f16(nv * (1.0f + scale[i]) + shift[i]);
    }
  }
}

// RMSNorm of an fp32 row with an fp16 weight, stored as fp16: rmsnorm_f32_to_f32
// (AnimaKernels.metal:172-204) followed by float_to_half (:81-88) in one pass.
// out = half(x * rsqrt(mean(x^2) + eps) * w), the product in the reference's order.
template <int V>
__global__ __launch_bounds__(256) void rmsnorm_half_wave_kernel(const float* __restrict__ in,
                                                                const half_t* __restrict__ w,
                                                                half_t* __restrict__ out, int n, int rows, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* x = in + (int64_t)row * n;
  floatx4 v[V];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int c = 4 * (lane + 64 * e);
    v[e] = c < n ? *reinterpret_cast<const floatx4*>(x + c) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) ss = fmaf(v[e][u], v[e][u], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)n + eps);
  half_t* o = out + (int64_t)row * n;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int c = 4 * (lane + 64 * e);
    if (c < n) {
      const half4v wv = *reinterpret_cast<const half4v*>(w + c);
      half4v h;
#pragma unroll
      for (int u = 0; u < 4; ++u) h[u] = f32_to_f16(v[e][u] * inv * (float)wv[u]);
      *reinterpret_cast<half4v*>(o + c) = h;
    }
  }
}

__global__ __launch_bounds__(LN_NT) void rmsnorm_half_kernel(const float* __restrict__ in, const half_t* __restrict__ w,
                                                             half_t* __restrict__ out, int n, float eps) {
  __shared__ float red[LN_NT / 64];
  const int64_t row = blockIdx.x;
  const float* x = in + row * n;
  float v[LN_MAX_PER_THREAD];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < LN_MAX_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * LN_NT;
    v[e] = i < n ? x[i] : 0.f;
    ss = fmaf(v[e], v[e], ss);
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)n + eps);
  half_t* o = out + row * n;
#pragma unroll
  for (int e = 0; e < LN_MAX_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * LN_NT;
    if (i < n) o[i] = f32_to_f16(v[e] * inv * (float)w[i]);
  }
}

// ---------------------------------------------------------------------------
// Elementwise kernels.  Each thread takes a chunk of EW consecutive elements:
// 16-byte accesses (one per 8 fp16, two per 8 fp32) when the launcher found every
// pointer 16-byte aligned (vec != 0) and the chunk is whole, element-wise
// accesses for the last partial chunk and for unaligned buffers.
// ---------------------------------------------------------------------------
constexpr int EW = 8;

__device__ __forceinline__ void load8(const float* p, float (&v)[EW]) {
  const floatx4 a = *reinterpret_cast<const floatx4*>(p), b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    v[u] = a[u];
    v[u + 4] = b[u];
  }
}
__device__ __forceinline__ void store8(float* p, const float (&v)[EW]) {
  *reinterpret_cast<floatx4*>(p) = floatx4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<floatx4*>(p + 4) = floatx4{v[4], v[5], v[6], v[7]};
}

// gate_add_half_f32 (AnimaKernels.metal:624-634): residual += float(branch) * gate[i % n].
// The vector form needs n % 8 == 0 so that a chunk never wraps a row.
__global__ __launch_bounds__(256) void gate_add_kernel(float* __restrict__ residual, const half_t* __restrict__ branch,
                                                       const float* __restrict__ gate, int64_t n, int64_t count,
                                                       int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    const int64_t col = c0 % n;
    float r[EW], g[EW];
    load8(residual + c0, r);
    load8(gate + col, g);
    const half8v b = *reinterpret_cast<const half8v*>(branch + c0);
#pragma unroll
    for (int u = 0; u < EW; ++u) r[u] = fmaf((float)b[u], g[u], r[u]);
    store8(residual + c0, r);
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) residual[i] = fmaf((float)branch[i], gate[i % n], residual[i]);
  }
}

// dit_gelu_half_inplace (AnimaKernels.metal:312-322).
__global__ __launch_bounds__(256) void gelu_kernel(half_t* __restrict__ values, int64_t count, int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    half8v v = *reinterpret_cast<const half8v*>(values + c0);
#pragma unroll
    for (int u = 0; u < EW; ++u) v[u] = gelu_erf_half(v[u]);
    *reinterpret_cast<half8v*>(values + c0) = v;
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) values[i] = gelu_erf_half(values[i]);
  }
}

// silu (AnimaKernels.metal:388-397).
__global__ __launch_bounds__(256) void silu_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t count,
                                                   int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    float v[EW];
    load8(in + c0, v);
#pragma unroll
    for (int u = 0; u < EW; ++u) v[u] = silu_f32(v[u]);
    store8(out + c0, v);
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) out[i] = silu_f32(in[i]);
  }
}

// add_f32 (AnimaKernels.metal:649-656).
__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t count,
                                                  int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    float d[EW], s[EW];
    load8(dst + c0, d);
    load8(src + c0, s);
#pragma unroll
    for (int u = 0; u < EW; ++u) d[u] += s[u];
    store8(dst + c0, d);
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) dst[i] += src[i];
  }
}

// gated_silu_half (AnimaKernels.metal:401-411): SiLU and product in fp32, one rounding.
__global__ __launch_bounds__(256) void gated_silu_kernel(const half_t* __restrict__ gate, const half_t* __restrict__ up,
                                                         half_t* __restrict__ out, int64_t count, int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    const half8v g = *reinterpret_cast<const half8v*>(gate + c0);
    const half8v u = *reinterpret_cast<const half8v*>(up + c0);
    half8v o;
#pragma unroll
    for (int e = 0; e < EW; ++e) o[e] = f32_to_f16(silu_f32((float)g[e]) * (float)u[e]);
    *reinterpret_cast<half8v*>(out + c0) = o;
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) out[i] = f32_to_f16(silu_f32((float)gate[i]) * (float)up[i]);
  }
}

// add_half_into_float (AnimaKernels.metal:639-647).
__global__ __launch_bounds__(256) void add_half_kernel(float* __restrict__ residual, const half_t* __restrict__ branch,
                                                       int64_t count, int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW;
  if (c0 >= count) return;
  if (vec && c0 + EW <= count) {
    float r[EW];
    load8(residual + c0, r);
    const half8v b = *reinterpret_cast<const half8v*>(branch + c0);
#pragma unroll
    for (int u = 0; u < EW; ++u) r[u] += (float)b[u];
    store8(residual + c0, r);
  } else {
    const int64_t end = c0 + EW < count ? c0 + EW : count;
    for (int64_t i = c0; i < end; ++i) residual[i] += (float)branch[i];
  }
}

static dim3 grid_ew(int64_t count) {
  const int64_t b = (count + 256 * EW - 1) / (256 * EW);
  if (b > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "elementwise grid too large");
  return dim3((unsigned)b);
}

// Smallest wave-kernel register depth V (float4s per lane) for a row of n, or 0.
static int wave_depth(int64_t n) {
  if (n % 4 != 0) return 0;
  for (int v = 2; v <= 16; v *= 2)
    if (n <= 256 * v) return v;
  return 0;
}

template <bool HB>
static void launch_layernorm_modulate_t(const float* residual, const float* mod, half_t* out, int64_t n, int64_t rows,
                                        float eps, int64_t mod_offset, hipStream_t stream) {
  const int depth = wave_depth(n);
  if (depth && aligned16(residual) && aligned16(mod) && mod_offset % 4 == 0 && aligned8(out)) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch (depth) {
      case 2: hipLaunchKernelGGL((layernorm_modulate_wave_kernel<2, HB>), grid, dim3(256), 0, stream, residual, mod,
                                 out, (int)n, (int)rows, eps, mod_offset); break;
      case 4: hipLaunchKernelGGL((layernorm_modulate_wave_kernel<4, HB>), grid, dim3(256), 0, stream, residual, mod,
                                 out, (int)n, (int)rows, eps, mod_offset); break;
      case 8: hipLaunchKernelGGL((layernorm_modulate_wave_kernel<8, HB>), grid, dim3(256), 0, stream, residual, mod,
                                 out, (int)n, (int)rows, eps, mod_offset); break;
      default: hipLaunchKernelGGL((layernorm_modulate_wave_kernel<16, HB>), grid, dim3(256), 0, stream, residual, mod,
                                  out, (int)n, (int)rows, eps, mod_offset); break;
    }
  } else {
    hipLaunchKernelGGL((layernorm_modulate_kernel<HB>), dim3((unsigned)rows), dim3(LN_NT), 0, stream, residual, mod,
                       out, (int)n, eps, mod_offset);
  }
  ANIMA_HIP(hipGetLastError());
}

void launch_layernorm_modulate(const float* residual, const float* mod, half_t* out, int64_t n, int64_t rows, float eps,
                               int64_t mod_offset, hipStream_t stream, bool fp16_boundaries) {
  if (n > LN_NT * LN_MAX_PER_THREAD) fail(ANIMA_E_UNSUPPORTED, "layernorm-modulate supports rows of at most 8192");
  if (rows > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "layernorm-modulate rows exceed int32");
  if (rows <= 0 || n <= 0) return;
  if (fp16_boundaries)
    launch_layernorm_modulate_t<true>(residual, mod, out, n, rows, eps, mod_offset, stream);
  else
    launch_layernorm_modulate_t<false>(residual, mod, out, n, rows, eps, mod_offset, stream);
}
void launch_gate_add(float* residual, const half_t* branch, const float* gate, int64_t n, int64_t count,
                     hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(residual) && aligned16(branch) && aligned16(gate) && n % EW == 0;
  hipLaunchKernelGGL(gate_add_kernel, grid_ew(count), dim3(256), 0, stream, residual, branch, gate, n, count, vec);
  ANIMA_HIP(hipGetLastError());
}
void launch_gelu(half_t* values, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  hipLaunchKernelGGL(gelu_kernel, grid_ew(count), dim3(256), 0, stream, values, count, aligned16(values) ? 1 : 0);
  ANIMA_HIP(hipGetLastError());
}
void launch_silu(const float* in, float* out, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(in) && aligned16(out);
  hipLaunchKernelGGL(silu_kernel, grid_ew(count), dim3(256), 0, stream, in, out, count, vec);
  ANIMA_HIP(hipGetLastError());
}
void launch_add(float* dst, const float* src, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(dst) && aligned16(src);
  hipLaunchKernelGGL(add_kernel, grid_ew(count), dim3(256), 0, stream, dst, src, count, vec);
  ANIMA_HIP(hipGetLastError());
}
void launch_rmsnorm_half(const float* in, const half_t* w, half_t* out, int64_t n, int64_t rows, float eps,
                         hipStream_t stream) {
  if (n > LN_NT * LN_MAX_PER_THREAD) fail(ANIMA_E_UNSUPPORTED, "rmsnorm supports rows of at most 8192");
  if (rows > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "rmsnorm rows exceed int32");
  if (rows <= 0 || n <= 0) return;
  const int depth = wave_depth(n);
  if (depth && aligned16(in) && aligned8(w) && aligned8(out)) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch (depth) {
      case 2: hipLaunchKernelGGL(rmsnorm_half_wave_kernel<2>, grid, dim3(256), 0, stream, in, w, out, (int)n,
                                 (int)rows, eps); break;
      case 4: hipLaunchKernelGGL(rmsnorm_half_wave_kernel<4>, grid, dim3(256), 0, stream, in, w, out, (int)n,
                                 (int)rows, eps); break;
      case 8: hipLaunchKernelGGL(rmsnorm_half_wave_kernel<8>, grid, dim3(256), 0, stream, in, w, out, (int)n,
                                 (int)rows, eps); break;
      default: hipLaunchKernelGGL(rmsnorm_half_wave_kernel<16>, grid, dim3(256), 0, stream, in, w, out, (int)n,
                                  (int)rows, eps); break;
    }
  } else {
    hipLaunchKernelGGL(rmsnorm_half_kernel, dim3((unsigned)rows), dim3(LN_NT), 0, stream, in, w, out, (int)n, eps);
  }
  ANIMA_HIP(hipGetLastError());
}
void launch_gated_silu(const half_t* gate, const half_t* up, half_t* out, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(gate) && aligned16(up) && aligned16(out);
  hipLaunchKernelGGL(gated_silu_kernel, grid_ew(count), dim3(256), 0, stream, gate, up, out, count, vec);
  ANIMA_HIP(hipGetLastError());
}
void launch_add_half(float* residual, const half_t* branch, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(residual) && aligned16(branch);
  hipLaunchKernelGGL(add_half_kernel, grid_ew(count), dim3(256), 0, stream, residual, branch, count, vec);
  ANIMA_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// DiT block composition.
// ---------------------------------------------------------------------------
DitBlockExecutor::DitBlockExecutor(anima_ctx* ctx)
    : ctx_(ctx),
      attention_(ctx, anima_attention_config{128, ANIMA_NUMERICS_FP32_SCORES, ANIMA_ATTENTION_BACKEND_AUTO,
                                             ANIMA_LAYOUT_TOKEN_MAJOR, 0, 0}),
      linear_(ctx, anima_linear_config{128, ANIMA_LINEAR_BACKEND_AUTO}) {}

static anima_buffer sub(char* base, int64_t off, int64_t bytes) { return anima_buffer{base + off, bytes}; }

void encode_linear_epilogue(LinearExecutor& lin, anima_buffer input, int64_t input_offset, const anima_qweight& weight,
                            anima_buffer output, int64_t output_offset, int64_t input_rows, int32_t family,
                            int epilogue, float* residual, const float* gate) {
  if (lin.encode_fused(input, input_offset, weight, output, output_offset, input_rows, family, epilogue, residual, gate))
    return;
  lin.encode(input, input_offset, weight, output, output_offset, input_rows, family);
  DeviceGuard guard(lin.context());
  half_t* y = reinterpret_cast<half_t*>(byte_ptr_mut(output, output_offset));
  const int64_t count = input_rows * weight.rows;  // bounded by the output range encode() checked
  if (epilogue == GEMM_GELU)
    launch_gelu(y, count, lin.context()->stream);
  else if (epilogue == GEMM_RESIDUAL_ADD)
    launch_add_half(residual, y, count, lin.context()->stream);
  else
    launch_gate_add(residual, y, gate, weight.rows, count, lin.context()->stream);
}

static MatvecParams matvec_params(const anima_qweight& weight, const float* x, float* y) {
  const QWeightView v = validate_weight(weight, "DiT modulation");
  MatvecParams p{};
  p.w = v.packed; p.scale = v.scale; p.zero = v.zero; p.row_stride = v.row_stride;
  p.x = x; p.y = y;
  p.N = (int)v.rows; p.K = (int)v.cols; p.groups = (int)v.groups; p.storage = v.storage;
  return p;
}

static void modulation_params(const anima_qweight& w1, const anima_qweight& w2, const anima_dit_block_args& a,
                              float* hid, float* mod, MatvecParams* mv1, MatvecParams* mv2) {
  *mv1 = matvec_params(w1, static_cast<const float*>(a.emb.ptr), hid);
  mv1->silu_input = 1;
  *mv2 = matvec_params(w2, hid, mod);
  mv2->bias = static_cast<const float*>(a.adaln_lora.ptr);
}

static void require_buffer(const anima_buffer& b, int64_t bytes, const char* what) {
  if (!b.ptr) fail(ANIMA_E_INVALID_ARGUMENT, std::string(what) + " pointer is null");
  if (b.length < bytes) fail(ANIMA_E_OUT_OF_BOUNDS, std::string(what) + " buffer range is out of bounds");
}

void DitBlockExecutor::check(const anima_dit_block_weights& w, const anima_dit_block_args& a,
                             const CrossKVCache* cache, int64_t block_index) const {
  const int64_t S = a.tokens, dim = a.dim, H = a.heads, hd = a.head_dim, T = a.context_tokens, C = a.context_dim,
                hidden = a.mlp_hidden;
  if (!(S > 0 && dim > 0 && H > 0 && hd > 0 && T > 0 && C > 0 && hidden > 0 && H * hd == dim))
    fail(ANIMA_E_INVALID_SHAPE, "invalid DiT block shape (requires heads * head_dim == dim)");
  if (hd % 2) fail(ANIMA_E_INVALID_SHAPE, "DiT block RoPE requires an even head_dim");
  if (!(a.eps >= 0.f && std::isfinite(a.eps))) fail(ANIMA_E_INVALID_ARGUMENT, "DiT block epsilon must be finite");
  require_buffer(a.residual, checked_product({S, dim, 4}, "DiT block"), "DiT block residual");
  require_buffer(a.emb, checked_product({dim, 4}, "DiT block"), "DiT block emb");
  require_buffer(a.adaln_lora, checked_product({3 * dim, 4}, "DiT block"), "DiT block adaln_lora");
  require_buffer(a.context, checked_product({T, C, 2}, "DiT block"), "DiT block context");
  // [tokens][head_dim/2][2][2] fp32
  require_buffer(a.rope, checked_product({S, hd, 8}, "DiT block"), "DiT block RoPE table");
  const int64_t nb = checked_product({hd, 2}, "DiT block");
  require_buffer(w.self_q_norm, nb, "DiT block self Q norm");
  require_buffer(w.self_k_norm, nb, "DiT block self K norm");
  require_buffer(w.cross_q_norm, nb, "DiT block cross Q norm");
  require_buffer(w.cross_k_norm, nb, "DiT block cross K norm");
  auto need = [&](const anima_qweight& q, int64_t rows, int64_t cols, const char* nm) {
    if (q.rows != rows || q.columns != cols) fail(ANIMA_E_INVALID_SHAPE, std::string(nm) + " shape mismatch");
    (void)validate_weight(q, nm);
  };
  need(w.self_q, dim, dim, "self_q"); need(w.self_k, dim, dim, "self_k"); need(w.self_v, dim, dim, "self_v");
  need(w.self_o, dim, dim, "self_o"); need(w.cross_q, dim, dim, "cross_q"); need(w.cross_k, dim, C, "cross_k");
  need(w.cross_v, dim, C, "cross_v"); need(w.cross_o, dim, dim, "cross_o"); need(w.mlp1, hidden, dim, "mlp1");
  need(w.mlp2, dim, hidden, "mlp2");
  const int64_t lora = w.mod_self_w1.rows;
  need(w.mod_self_w1, lora, dim, "mod_self_w1"); need(w.mod_cross_w1, lora, dim, "mod_cross_w1");
  need(w.mod_mlp_w1, lora, dim, "mod_mlp_w1"); need(w.mod_self_w2, 3 * dim, lora, "mod_self_w2");
  need(w.mod_cross_w2, 3 * dim, lora, "mod_cross_w2"); need(w.mod_mlp_w2, 3 * dim, lora, "mod_mlp_w2");
  if (cache) {
    if (block_index < 0 || block_index >= cache->blocks())
      fail(ANIMA_E_INVALID_ARGUMENT, "cross K/V cache block index out of range");
    if (cache->tokens() != T || cache->dim() != dim)
      fail(ANIMA_E_INVALID_SHAPE, "cross K/V cache shape differs from the block's context tokens or dim");
  }
}

void DitBlockExecutor::encode(const anima_dit_block_weights& w, const anima_dit_block_args& a, CrossKVCache* cache,
                              int64_t block_index) {
  check(w, a, cache, block_index);
  encode_block(w, a, cache, block_index, nullptr, 0);
}

// Modulation matvecs of one branch (DiTBlockExecutor.encodeModulation, :1403-1417):
// SiLU(emb) -> W1 -> hid, then hid -> W2 (+ adaln_lora) -> mod.
static void modulation_params(const anima_qweight& w1, const anima_qweight& w2, const anima_dit_block_args& a,
                              float* hid, float* mod, MatvecParams* mv1, MatvecParams* mv2);

void DitBlockExecutor::encode_block(const anima_dit_block_weights& w, const anima_dit_block_args& a,
                                    CrossKVCache* cache, int64_t block_index, const float* premod,
                                    int64_t mod_stride) {
  const int64_t S = a.tokens, dim = a.dim, H = a.heads, hd = a.head_dim, T = a.context_tokens,
                hidden = a.mlp_hidden;
  const int64_t lora = w.mod_self_w1.rows;

  // Workspace layout (bytes, 256-aligned).
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t o_hid = 0, hid_bytes = al(lora * 4);
  const int64_t o_mod = o_hid + 3 * hid_bytes;
  const int64_t mod_bytes = al(3 * dim * 4);
  const int64_t o_norm = o_mod + 3 * mod_bytes;
  const int64_t act = al(checked_product({S, dim, 2}, "DiT block"));
  const int64_t o_q = o_norm + act, o_k = o_q + act, o_v = o_k + act, o_a = o_v + act, o_b = o_a + act;
  const int64_t ctx_act = al(checked_product({T, dim, 2}, "DiT block"));
  const int64_t o_ck = o_b + act, o_cv = o_ck + ctx_act;
  const int64_t o_h = o_cv + ctx_act;
  const int64_t total = o_h + al(checked_product({S, hidden, 2}, "DiT block"));

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  char* ws = static_cast<char*>(ws_.get(total, stream));
  float* residual = static_cast<float*>(a.residual.ptr);
  anima_buffer norm_b = sub(ws, o_norm, S * dim * 2), q_b = sub(ws, o_q, S * dim * 2), k_b = sub(ws, o_k, S * dim * 2),
               v_b = sub(ws, o_v, S * dim * 2), a_b = sub(ws, o_a, S * dim * 2), br_b = sub(ws, o_b, S * dim * 2),
               ck_b = sub(ws, o_ck, T * dim * 2), cv_b = sub(ws, o_cv, T * dim * 2), h_b = sub(ws, o_h, S * hidden * 2);
  if (cache) {
    ck_b = anima_buffer{cache->k(block_index), T * dim * 2};
    cv_b = anima_buffer{cache->v(block_index), T * dim * 2};
  }
  const bool cache_hit = cache && cache->ready(block_index);

  // Modulation (DiTBlockExecutor.encodeModulation, :1403-1417): SiLU(emb) -> W1 -> W2 -> + adaln_lora,
  // for the three branches at once: one launch for the W1 matvecs (SiLU applied to emb as it is
  // read), one for the W2 matvecs (adaln_lora added to each output).  A forward computes every
  // block's rows up front instead (they depend on emb and adaln_lora alone).
  const anima_qweight* w1s[3] = {&w.mod_self_w1, &w.mod_cross_w1, &w.mod_mlp_w1};
  const anima_qweight* w2s[3] = {&w.mod_self_w2, &w.mod_cross_w2, &w.mod_mlp_w2};
  const float* mods[3];
  if (premod) {
    for (int br = 0; br < 3; ++br) mods[br] = premod + br * mod_stride;
  } else {
    MatvecParams mv1[3], mv2[3];
    for (int br = 0; br < 3; ++br) {
      float* mod = reinterpret_cast<float*>(ws + o_mod + br * mod_bytes);
      float* hid = reinterpret_cast<float*>(ws + o_hid + br * hid_bytes);
      modulation_params(*w1s[br], *w2s[br], a, hid, mod, &mv1[br], &mv2[br]);
      mods[br] = mod;
    }
    launch_matvec_batch(mv1, 3, stream);
    launch_matvec_batch(mv2, 3, stream);
  }

  anima_attention_args att{};
  att.heads = H; att.head_dim = hd; att.key_value_heads = H; att.layout = ANIMA_LAYOUT_TOKEN_MAJOR;
  att.token_stride = dim; att.batch = 1;

  // Self attention (encodeAttentionBranch, :1035-1242).
  launch_layernorm_modulate(residual, mods[0], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  {
    const anima_qweight* ws3[3] = {&w.self_q, &w.self_k, &w.self_v};
    const anima_buffer outs[3] = {q_b, k_b, v_b};
    linear_.encode_group(norm_b, ws3, outs, 3, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  }
  anima_qk_prologue self_pro{};
  self_pro.q_norm_weight = w.self_q_norm; self_pro.k_norm_weight = w.self_k_norm; self_pro.eps = a.eps;
  self_pro.rope = a.rope; self_pro.rope_tokens = S; self_pro.rope_q = 1; self_pro.rope_k = 1;
  att.query = q_b; att.key = k_b; att.value = v_b; att.output = a_b;
  att.query_count = S; att.key_count = S; att.prologue = &self_pro;
  attention_.encode(att);
  encode_linear_epilogue(linear_, a_b, 0, w.self_o, br_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION, GEMM_GATE_ADD,
                         residual, mods[0] + 2 * dim);

  // Cross attention to the context (no RoPE).  The per-head RMSNorm of Q and of the
  // context K runs in the projections' output stage when the tiled GEMM takes them,
  // else as an in-place pass right after; either way Q and K reach the attention
  // normalised, so the cached K is the attention's input itself (CrossKVCache holds
  // the post-norm K, DiTBlockExecutor.swift:1110-1161).
  launch_layernorm_modulate(residual, mods[1], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  linear_.encode_head_rmsnorm(norm_b, 0, w.cross_q, q_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION,
                              static_cast<const half_t*>(w.cross_q_norm.ptr), hd, a.eps);
  if (!cache_hit) {
    const anima_qweight* ws2[2] = {&w.cross_k, &w.cross_v};
    const anima_buffer outs[2] = {ck_b, cv_b};
    const GemmEpilogueArgs ekv[2] = {{GEMM_QK_NORM, static_cast<const half_t*>(w.cross_k_norm.ptr), a.eps},
                                     {GEMM_STORE, nullptr, 0.f}};
    const bool fused = hd == 128 && linear_.encode_group(a.context, ws2, outs, 2, T, ANIMA_FAMILY_ATTENTION_PROJECTION, ekv);
    if (!fused) {
      linear_.encode_group(a.context, ws2, outs, 2, T, ANIMA_FAMILY_ATTENTION_PROJECTION);
      PrologueParams pp{};
      half_t* kx = static_cast<half_t*>(ck_b.ptr);
      pp.in = kx; pp.in_tok = dim; pp.in_head = hd; pp.in_batch = T * dim;
      pp.out = kx; pp.out_tok = dim; pp.out_head = hd; pp.out_batch = T * dim;
      pp.batch = 1; pp.rows = (int)T; pp.heads = (int)H; pp.D = (int)hd;
      pp.norm_w = static_cast<const half_t*>(w.cross_k_norm.ptr); pp.eps = a.eps; pp.rope = nullptr;
      launch_prologue(pp, stream);
    }
    if (cache) cache->mark_ready(block_index);
  }
  att.query = q_b; att.key = ck_b; att.value = cv_b; att.output = a_b;
  att.query_count = S; att.key_count = T; att.prologue = nullptr;
  attention_.encode(att);
  encode_linear_epilogue(linear_, a_b, 0, w.cross_o, br_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION, GEMM_GATE_ADD,
                         residual, mods[1] + 2 * dim);

  // MLP (encodeMLP, :1244-1319): mlp1 -> exact GELU -> mlp2.
  launch_layernorm_modulate(residual, mods[2], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  encode_linear_epilogue(linear_, norm_b, 0, w.mlp1, h_b, 0, S, ANIMA_FAMILY_MLP_UP, GEMM_GELU, nullptr, nullptr);
  encode_linear_epilogue(linear_, h_b, 0, w.mlp2, br_b, 0, S, ANIMA_FAMILY_MLP_DOWN, GEMM_GATE_ADD, residual,
                         mods[2] + 2 * dim);
}

void DitBlockExecutor::forward(const anima_dit_block_weights* blocks, int64_t count, const anima_dit_block_args& a,
                               CrossKVCache* cache) {
  if (!blocks) fail(ANIMA_E_INVALID_ARGUMENT, "DiT forward block array is null");
  if (count <= 0) fail(ANIMA_E_INVALID_SHAPE, "DiT forward needs at least one block");
  if (cache && cache->blocks() < count) fail(ANIMA_E_INVALID_SHAPE, "cross K/V cache holds fewer blocks than the forward");
  // Every block validates before the first launch.
  for (int64_t i = 0; i < count; ++i) check(blocks[i], a, cache, i);
  // The modulation rows depend on emb and adaln_lora alone, so every block's are computed
  // first, MV_BATCH_WIDE matvecs per launch (the same kernel and bits as a block's own
  // 3-matvec launches), in place of two small launches per block.
  const int64_t dim = a.dim;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  int64_t hid_bytes = 0;
  for (int64_t i = 0; i < count; ++i) hid_bytes = std::max<int64_t>(hid_bytes, al(blocks[i].mod_self_w1.rows * 4));
  const int64_t mod_bytes = al(3 * dim * 4), per_block = 3 * (hid_bytes + mod_bytes);
  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  char* mws = static_cast<char*>(mod_ws_.get(checked_product({count, per_block}, "DiT forward"), stream));
  std::vector<MatvecParams> mv1((size_t)(3 * count)), mv2((size_t)(3 * count));
  for (int64_t i = 0; i < count; ++i) {
    const anima_dit_block_weights& w = blocks[i];
    const anima_qweight* w1s[3] = {&w.mod_self_w1, &w.mod_cross_w1, &w.mod_mlp_w1};
    const anima_qweight* w2s[3] = {&w.mod_self_w2, &w.mod_cross_w2, &w.mod_mlp_w2};
    for (int br = 0; br < 3; ++br) {
      float* hid = reinterpret_cast<float*>(mws + i * per_block + br * hid_bytes);
      float* mod = reinterpret_cast<float*>(mws + i * per_block + 3 * hid_bytes + br * mod_bytes);
      modulation_params(*w1s[br], *w2s[br], a, hid, mod, &mv1[3 * i + br], &mv2[3 * i + br]);
    }
  }
  launch_matvec_many(mv1.data(), 3 * count, stream);
  launch_matvec_many(mv2.data(), 3 * count, stream);
  for (int64_t i = 0; i < count; ++i)
    encode_block(blocks[i], a, cache, i, reinterpret_cast<const float*>(mws + i * per_block + 3 * hid_bytes),
                 mod_bytes / 4);
}

// Rebase one template buffer (ptr holds a byte offset into the block's range) onto
// the slot the range was copied to.
void DitBlockExecutor::forward_streamed(WeightStreamer& st, const anima_dit_block_weights* templates,
                                        const void* const* ranges, const int64_t* range_bytes, int64_t count,
                                        const anima_dit_block_args& a, CrossKVCache* cache) {
  if (!templates || !ranges || !range_bytes) fail(ANIMA_E_INVALID_ARGUMENT, "streamed DiT forward array is null");
  if (count <= 0) fail(ANIMA_E_INVALID_SHAPE, "DiT forward needs at least one block");
  if (st.context() != ctx_) fail(ANIMA_E_INVALID_ARGUMENT, "weight streamer belongs to another context");
  if (cache && cache->blocks() < count) fail(ANIMA_E_INVALID_SHAPE, "cross K/V cache holds fewer blocks than the forward");
  // Validate every block against the slot it will land in before anything is queued.
  for (int64_t i = 0; i < count; ++i) {
    if (!ranges[i]) fail(ANIMA_E_INVALID_ARGUMENT, "streamed block range pointer is null");
    if (range_bytes[i] <= 0 || range_bytes[i] > st.capacity())
      fail(ANIMA_E_OUT_OF_BOUNDS, "execution range does not fit the weight slot");
    check(rebase_block(templates[i], st.slot((int)(i % st.slots())), range_bytes[i]), a, cache, i);
  }
  DeviceGuard guard(ctx_);
  // DitForward.loopStep (DitForward.swift:21-35): with two or more slots block i runs from
  // slot i % slots while the copy stream fills the slot of block i+1, last read by block
  // i+1-slots <= i-1, whose release is already queued.  With one slot there is no look-ahead:
  // block i is copied in only after block i-1's release (queued at the end of the previous
  // iteration), so the copy waits for every kernel that still reads the slot.
  st.load(0, ranges[0], range_bytes[0]);
  for (int64_t i = 0; i < count; ++i) {
    const int s = (int)(i % st.slots());
    if (st.slots() == 1) {
      if (i > 0) st.load(0, ranges[i], range_bytes[i]);
    } else if (i + 1 < count) {
      const int ns = (int)((i + 1) % st.slots());
      st.load(ns, ranges[i + 1], range_bytes[i + 1]);
    }
    st.acquire(s);
    encode(rebase_block(templates[i], st.slot(s), range_bytes[i]), a, cache, i);
    st.release(s);
  }
}

CrossKVCache::CrossKVCache(anima_ctx* ctx, int64_t blocks, int64_t tokens, int64_t dim)
    : ctx_(ctx), blocks_(blocks), tokens_(tokens), dim_(dim) {
  if (!(blocks > 0 && tokens > 0 && dim > 0)) fail(ANIMA_E_INVALID_SHAPE, "invalid cross K/V cache shape");
  bytes_ = checked_product({blocks, 2, tokens, dim, 2}, "cross K/V cache");
  ready_.assign((size_t)blocks, 0);
  DeviceGuard guard(ctx_);
  void* p = nullptr;
  ANIMA_HIP(hipMalloc(&p, (size_t)bytes_));
  base_ = static_cast<half_t*>(p);
}

CrossKVCache::~CrossKVCache() {
  if (base_) (void)hipFree(base_);  // hipFree waits for outstanding work on the device
}

WeightStreamer::WeightStreamer(anima_ctx* ctx, int64_t capacity, int slots)
    : ctx_(ctx), capacity_(capacity), slots_(slots) {
  if (capacity <= 0) fail(ANIMA_E_INVALID_SHAPE, "weight ring capacity must be positive");
  if (slots < 1 || slots > 4) fail(ANIMA_E_INVALID_ARGUMENT, "weight slot count must be in 1...4");
  DeviceGuard guard(ctx_);
  try {
    for (int s = 0; s < slots_; ++s) {
      void* p = nullptr;
      ANIMA_HIP(hipMalloc(&p, (size_t)capacity_));
      slot_[s] = static_cast<char*>(p);
      ANIMA_HIP(hipEventCreateWithFlags(&loaded_[s], hipEventDisableTiming));
      ANIMA_HIP(hipEventCreateWithFlags(&released_[s], hipEventDisableTiming));
    }
    ANIMA_HIP(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking));
  } catch (...) {
    this->~WeightStreamer();
    throw;
  }
}

WeightStreamer::~WeightStreamer() {
  if (copy_) {
    (void)hipStreamSynchronize(copy_);
    (void)hipStreamDestroy(copy_);
    copy_ = nullptr;
  }
  for (int s = 0; s < 4; ++s) {
    if (slot_[s]) (void)hipFree(slot_[s]);
    if (loaded_[s]) (void)hipEventDestroy(loaded_[s]);
    if (released_[s]) (void)hipEventDestroy(released_[s]);
    slot_[s] = nullptr;
    loaded_[s] = released_[s] = nullptr;
  }
}

void WeightStreamer::load(int s, const void* src, int64_t bytes) {
  // released_[s] was last recorded after the kernels of the previous block in this slot
  // were queued on the context stream (or never recorded: then the wait is a no-op).
  ANIMA_HIP(hipStreamWaitEvent(copy_, released_[s], 0));
  ANIMA_HIP(hipMemcpyAsync(slot_[s], src, (size_t)bytes, hipMemcpyHostToDevice, copy_));
  ANIMA_HIP(hipEventRecord(loaded_[s], copy_));
}

void WeightStreamer::acquire(int s) { ANIMA_HIP(hipStreamWaitEvent(ctx_->stream, loaded_[s], 0)); }

void WeightStreamer::release(int s) { ANIMA_HIP(hipEventRecord(released_[s], ctx_->stream)); }

// ---------------------------------------------------------------------------
// Qwen encoder layer (QwenLayerExecutor.execute, QwenEncoderMetal.swift:232-304),
// for a batch of right-padded sequences.  The reference transposes Q/K/V to
// head-major and back around the attention (:264-279); here the attention reads
// the projections' token-major rows directly (grouped K/V row stride), the Q
// RMSNorm+RoPE is fused into the flash kernel, and RMSNorm writes fp16 directly.
// ---------------------------------------------------------------------------
QwenLayerExecutor::QwenLayerExecutor(anima_ctx* ctx)
    : ctx_(ctx),
      attention_(ctx, anima_attention_config{128, ANIMA_NUMERICS_FP32_SCORES, ANIMA_ATTENTION_BACKEND_AUTO,
                                             ANIMA_LAYOUT_TOKEN_MAJOR, 0, 0}),
      linear_(ctx, anima_linear_config{128, ANIMA_LINEAR_BACKEND_AUTO}) {}

void QwenLayerExecutor::encode(const anima_qwen_layer_weights& w, const anima_qwen_layer_args& a) {
  const int64_t B = a.batch, S = a.tokens, hidden = a.hidden, H = a.heads, Hkv = a.kv_heads, D = a.head_dim,
                inter = a.intermediate;
  if (!(B > 0 && S > 0 && hidden > 0 && H > 0 && Hkv > 0 && D > 0 && inter > 0 && H % Hkv == 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid Qwen layer shape (heads must be a multiple of kv_heads)");
  if (!(a.eps >= 0.f && std::isfinite(a.eps))) fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer epsilon must be finite");
  const int64_t rows = checked_product({B, S}, "Qwen layer");
  const int64_t qdim = H * D, kvdim = Hkv * D;
  if (D % 2) fail(ANIMA_E_INVALID_SHAPE, "Qwen layer RoPE requires an even head_dim");
  if (checked_product({rows, hidden, 4}, "Qwen layer") > a.residual.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "invalid Qwen layer input buffers");
  if (!a.residual.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer residual pointer is null");
  if (!a.rope.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer requires a RoPE table");
  if (checked_product({S, D, 8}, "Qwen layer") > a.rope.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "Qwen layer RoPE table is shorter than tokens rows");
  if (!w.input_norm.ptr || !w.post_attention_norm.ptr || !w.q_norm.ptr || !w.k_norm.ptr)
    fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer norm weight pointer is null");
  if (w.input_norm.length < checked_product({hidden, 2}, "Qwen layer") ||
      w.post_attention_norm.length < checked_product({hidden, 2}, "Qwen layer") ||
      w.q_norm.length < checked_product({D, 2}, "Qwen layer") || w.k_norm.length < checked_product({D, 2}, "Qwen layer"))
    fail(ANIMA_E_OUT_OF_BOUNDS, "Qwen layer norm weight buffer is too short");
  auto need = [&](const anima_qweight& q, int64_t r, int64_t c, const char* nm) {
    if (q.rows != r || q.columns != c) fail(ANIMA_E_INVALID_SHAPE, std::string("invalid Qwen matrix ") + nm);
  };
  need(w.q, qdim, hidden, "q"); need(w.k, kvdim, hidden, "k"); need(w.v, kvdim, hidden, "v");
  need(w.o, hidden, qdim, "o"); need(w.gate, inter, hidden, "gate"); need(w.up, inter, hidden, "up");
  need(w.down, hidden, inter, "down");

  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t o_norm = 0;
  const int64_t o_q = o_norm + al(checked_product({rows, hidden, 2}, "Qwen layer"));
  const int64_t o_k = o_q + al(checked_product({rows, qdim, 2}, "Qwen layer"));
  const int64_t o_v = o_k + al(checked_product({rows, kvdim, 2}, "Qwen layer"));
  const int64_t o_att = o_v + al(checked_product({rows, kvdim, 2}, "Qwen layer"));
  const int64_t o_proj = o_att + al(checked_product({rows, qdim, 2}, "Qwen layer"));
  const int64_t o_gate = o_proj + al(checked_product({rows, hidden, 2}, "Qwen layer"));
  const int64_t o_up = o_gate + al(checked_product({rows, inter, 2}, "Qwen layer"));
  const int64_t total = o_up + al(checked_product({rows, inter, 2}, "Qwen layer"));

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  char* ws = static_cast<char*>(ws_.get(total, stream));
  float* residual = static_cast<float*>(a.residual.ptr);
  anima_buffer norm_b = sub(ws, o_norm, rows * hidden * 2), q_b = sub(ws, o_q, rows * qdim * 2),
               k_b = sub(ws, o_k, rows * kvdim * 2), v_b = sub(ws, o_v, rows * kvdim * 2),
               att_b = sub(ws, o_att, rows * qdim * 2), proj_b = sub(ws, o_proj, rows * hidden * 2),
               gate_b = sub(ws, o_gate, rows * inter * 2), up_b = sub(ws, o_up, rows * inter * 2);
  half_t* norm = static_cast<half_t*>(norm_b.ptr);

  // Attention branch (:244-282).
  launch_rmsnorm_half(residual, static_cast<const half_t*>(w.input_norm.ptr), norm, hidden, rows, a.eps, stream);
  {
    const anima_qweight* ws3[3] = {&w.q, &w.k, &w.v};
    const anima_buffer outs[3] = {q_b, k_b, v_b};
    linear_.encode_group(norm_b, ws3, outs, 3, rows, ANIMA_FAMILY_ATTENTION_PROJECTION);
  }
  anima_qk_prologue pro{};
  pro.q_norm_weight = w.q_norm; pro.k_norm_weight = w.k_norm; pro.eps = a.eps;
  pro.rope = a.rope; pro.rope_tokens = S; pro.rope_q = 1; pro.rope_k = 1;
  anima_attention_args att{};
  att.query = q_b; att.key = k_b; att.value = v_b; att.output = att_b;
  att.heads = H; att.key_value_heads = Hkv; att.head_dim = D; att.query_count = S; att.key_count = S;
  att.causal = 1; att.layout = ANIMA_LAYOUT_TOKEN_MAJOR; att.token_stride = qdim; att.kv_token_stride = kvdim;
  att.batch = B; att.key_lengths = a.key_lengths; att.key_lengths_on_device = 0; att.prologue = &pro;
  attention_.encode(att);
  encode_linear_epilogue(linear_, att_b, 0, w.o, proj_b, 0, rows, ANIMA_FAMILY_ATTENTION_PROJECTION, GEMM_RESIDUAL_ADD,
                         residual, nullptr);

  // MLP branch (:284-302): gate/up -> SwiGLU (into the gate buffer) -> down.
  launch_rmsnorm_half(residual, static_cast<const half_t*>(w.post_attention_norm.ptr), norm, hidden, rows, a.eps,
                      stream);
  {
    const anima_qweight* ws2[2] = {&w.gate, &w.up};
    const anima_buffer outs[2] = {gate_b, up_b};
    linear_.encode_group(norm_b, ws2, outs, 2, rows, ANIMA_FAMILY_MLP_UP);
  }
  launch_gated_silu(static_cast<const half_t*>(gate_b.ptr), static_cast<const half_t*>(up_b.ptr),
                    static_cast<half_t*>(gate_b.ptr), rows * inter, stream);
  encode_linear_epilogue(linear_, gate_b, 0, w.down, proj_b, 0, rows, ANIMA_FAMILY_MLP_DOWN, GEMM_RESIDUAL_ADD,
                         residual, nullptr);
}

}  // namespace anima
