// DiT input / output stages and the sampler update for gfx950.
//
// Kernels restate AnimaXS/Shaders/AnimaKernels.metal: flow_velocity_to_denoised_f32
// (:1191-1201), euler_step_f32 (:1206-1216), patchify17 (:1225-1246), unpatchify16
// (:1251-1268) and unpatchify_velocity16 (:1276-1297); the timestep kernel computes the
// sinusoid of DiTPreparationExecutor.makeTimestep (DiTPreparationExecutor.swift:137-147)
// on the device and applies rmsnorm_f32_to_f32 (AnimaKernels.metal:172-204) in the same
// workgroup.  The compositions follow DiTPreparationExecutor.execute
// (DiTPreparationExecutor.swift:51-135) and DiTFinalLayerExecutor.execute
// (DiTFinalLayerExecutor.swift:75-186, the fp16Legacy residual boundary) at any even
// latent size and any hidden width up to 8192 (the reference fixes 64x64 and 2048).
#include <cmath>
#include <string>

#include "block.hpp"
#include "dit_io.hpp"

namespace anima {
namespace {

// ---------------------------------------------------------------------------
// Patch layout kernels.  Pure copies: bit-exact by construction.  The grids are one
// thread per (token, channel) pair; the host guarantees tokens * 17 < 2^31.
// ---------------------------------------------------------------------------

// patchify17: thread g writes feature block c of token t (g = t*17 + c), so a
// wavefront stores whole tokens contiguously.  Channels at or past in_channels read
// as zero (the 16-channel latent with the zero padding-mask channel appended).
template <class OutT>
__global__ __launch_bounds__(256) void patchify17_kernel(const float* __restrict__ in, OutT* __restrict__ tokens,
                                                         int in_channels, int H, int W, int T, int vec) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= T * 17) return;
  const int t = g / 17, c = g - t * 17;
  const int pw = W >> 1;
  const int i = t / pw, j = t - i * pw;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (c < in_channels) {
    const float* p = in + ((int64_t)c * H + 2 * i) * W + 2 * j;
    v[0] = p[0];
    v[1] = p[1];
    v[2] = p[W];
    v[3] = p[W + 1];
  }
  OutT* o = tokens + (int64_t)t * 68 + c * 4;
  if (vec) {
    if constexpr (sizeof(OutT) == 2) {
      *reinterpret_cast<half4v*>(o) = half4v{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    } else {
      *reinterpret_cast<floatx4*>(o) = floatx4{v[0], v[1], v[2], v[3]};
    }
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = (OutT)v[u];
  }
}

// unpatchify16: thread g = c*T + t rebuilds channel c of patch t, so consecutive lanes
// store consecutive pixel pairs of one image row.
__global__ __launch_bounds__(256) void unpatchify16_kernel(const float* __restrict__ tokens, float* __restrict__ out,
                                                           int H, int W, int T) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= T * 16) return;
  const int c = g / T, t = g - c * T;
  const int pw = W >> 1;
  const int i = t / pw, j = t - i * pw;
  const float* p = tokens + (int64_t)t * 68 + c * 4;
  float* o = out + ((int64_t)c * H + 2 * i) * W + 2 * j;
  o[0] = p[0];
  o[1] = p[1];
  o[W] = p[2];
  o[W + 1] = p[3];
}

// unpatchify_velocity16: FinalLayer token element (di*2 + dj)*16 + c is pixel
// (2i+di, 2j+dj) of channel c.  InT is fp32 (the reference kernel's input) or fp16
// (the projection output, converted here instead of in a half_to_float pass).
template <class InT>
__global__ __launch_bounds__(256) void unpatchify_velocity16_kernel(const InT* __restrict__ tokens,
                                                                    float* __restrict__ out, int H, int W, int T) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= T * 16) return;
  const int c = g / T, t = g - c * T;
  const int pw = W >> 1;
  const int i = t / pw, j = t - i * pw;
  const InT* p = tokens + (int64_t)t * 64 + c;
  float* o = out + ((int64_t)c * H + 2 * i) * W + 2 * j;
  o[0] = (float)p[0];
  o[1] = (float)p[16];
  o[W] = (float)p[32];
  o[W + 1] = (float)p[48];
}

// ---------------------------------------------------------------------------
// Elementwise fp32 kernels: four consecutive elements per thread, one 16-byte
// access per operand when every pointer is 16-byte aligned (vec), scalar
// accesses for the tail and for unaligned buffers.
// ---------------------------------------------------------------------------

// denoised = x - sigma * velocity (a single rounding: the product and the
// difference are one fused multiply-add).
__global__ __launch_bounds__(256) void flow_denoised_kernel(const float* __restrict__ x, const float* __restrict__ vel,
                                                            float* __restrict__ den, float sigma, int64_t count,
                                                            int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c0 >= count) return;
  if (vec && c0 + 4 <= count) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(x + c0);
    const floatx4 b = *reinterpret_cast<const floatx4*>(vel + c0);
    floatx4 r;
#pragma unroll
    for (int u = 0; u < 4; ++u) r[u] = fmaf(-sigma, b[u], a[u]);
    *reinterpret_cast<floatx4*>(den + c0) = r;
  } else {
    const int64_t end = c0 + 4 < count ? c0 + 4 : count;
    for (int64_t i = c0; i < end; ++i) den[i] = fmaf(-sigma, vel[i], x[i]);
  }
}

// x_next = x + dsigma * (x - denoised) * inv_sigma, inv_sigma = 1/sigma rounded once
// on the host (the reference kernel's `inv`).
__device__ __forceinline__ float euler1(float x, float d, float dsigma, float inv_sigma) {
  return fmaf(dsigma * (x - d), inv_sigma, x);
}

__global__ __launch_bounds__(256) void euler_step_kernel(const float* __restrict__ x, const float* __restrict__ den,
                                                         float* __restrict__ out, float dsigma, float inv_sigma,
                                                         int64_t count, int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c0 >= count) return;
  if (vec && c0 + 4 <= count) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(x + c0);
    const floatx4 b = *reinterpret_cast<const floatx4*>(den + c0);
    floatx4 r;
#pragma unroll
    for (int u = 0; u < 4; ++u) r[u] = euler1(a[u], b[u], dsigma, inv_sigma);
    *reinterpret_cast<floatx4*>(out + c0) = r;
  } else {
    const int64_t end = c0 + 4 < count ? c0 + 4 : count;
    for (int64_t i = c0; i < end; ++i) out[i] = euler1(x[i], den[i], dsigma, inv_sigma);
  }
}

// fp16 -> fp32 (half_to_float, AnimaKernels.metal:90-97), eight elements per thread.
__global__ __launch_bounds__(256) void half_to_float_kernel(const half_t* __restrict__ in, float* __restrict__ out,
                                                            int64_t count, int vec) {
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= count) return;
  if (vec && c0 + 8 <= count) {
    const half8v h = *reinterpret_cast<const half8v*>(in + c0);
    *reinterpret_cast<floatx4*>(out + c0) = floatx4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    *reinterpret_cast<floatx4*>(out + c0 + 4) = floatx4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
  } else {
    const int64_t end = c0 + 8 < count ? c0 + 8 : count;
    for (int64_t i = c0; i < end; ++i) out[i] = (float)in[i];
  }
}

// ---------------------------------------------------------------------------
// Timestep: raw[i] = cos(sigma * f_i), raw[half + i] = sin(sigma * f_i) with
// f_i = exp((-ln(10000) * i) / half) in fp32 (predict2.py Timesteps as restated by
// DiTPreparationExecutor.makeTimestep), then emb = raw * rsqrt(mean(raw^2) + eps) * w
// (rmsnorm_f32_to_f32 with the fp16 t_embedding_norm weight).  One 256-thread
// workgroup; each thread keeps its <= TS_PER_THREAD pairs in registers.
// ---------------------------------------------------------------------------
constexpr int TS_NT = 256;
constexpr int TS_PER_THREAD = 16;  // dim <= 2 * 256 * 16 = 8192

__global__ __launch_bounds__(TS_NT) void timestep_embed_kernel(float sigma, const half_t* __restrict__ w,
                                                               float* __restrict__ raw, float* __restrict__ emb,
                                                               int dim, float eps) {
  __shared__ float red[TS_NT / 64];
  const int half = dim >> 1;
  const float neg_log = -9.21034037197618f;  // -ln(10000) rounded to fp32
  float cs[TS_PER_THREAD], sn[TS_PER_THREAD];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < TS_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * TS_NT;
    cs[e] = 0.f;
    sn[e] = 0.f;
    if (i < half) {
      const float f = expf((neg_log * (float)i) / (float)half);
      const float a = sigma * f;
      cs[e] = cosf(a);
      sn[e] = sinf(a);
      raw[i] = cs[e];
      raw[half + i] = sn[e];
      ss = fmaf(cs[e], cs[e], ss);
      ss = fmaf(sn[e], sn[e], ss);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < TS_NT / 64; ++k) tot += red[k];
  const float inv = rsqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int e = 0; e < TS_PER_THREAD; ++e) {
    const int i = threadIdx.x + e * TS_NT;
    if (i < half) {
      emb[i] = cs[e] * inv * (float)w[i];
      emb[half + i] = sn[e] * inv * (float)w[half + i];
    }
  }
}

dim3 grid_of(int64_t threads) {
  const int64_t b = (threads + 255) / 256;
  if (b > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "elementwise grid too large");
  return dim3((unsigned)b);
}

void half_to_float(const half_t* in, float* out, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(in) && aligned16(out);
  hipLaunchKernelGGL(half_to_float_kernel, grid_of((count + 7) / 8), dim3(256), 0, stream, in, out, count, vec);
  ANIMA_HIP(hipGetLastError());
}

void require_range(const anima_buffer& b, int64_t bytes, const char* what) {
  if (!b.ptr) fail(ANIMA_E_INVALID_ARGUMENT, std::string(what) + " pointer is null");
  if (b.length < bytes) fail(ANIMA_E_OUT_OF_BOUNDS, std::string(what) + " buffer is too small");
}

MatvecParams matvec_of(const QWeightView& v, const float* x, float* y) {
  MatvecParams p{};
  p.w = v.packed; p.scale = v.scale; p.zero = v.zero; p.row_stride = v.row_stride;
  p.x = x; p.y = y;
  p.N = (int)v.rows; p.K = (int)v.cols; p.groups = (int)v.groups; p.storage = v.storage;
  return p;
}

QWeightView matrix(const anima_qweight& w, int64_t rows, int64_t cols, const char* label) {
  const QWeightView v = validate_weight(w, label);
  if (v.rows != rows || v.cols != cols)
    fail(ANIMA_E_INVALID_SHAPE, std::string(label) + " must be [" + std::to_string(rows) + ", " +
                                    std::to_string(cols) + "]");
  return v;
}

char* align256(char* p) { return reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(p) + 255) & ~uintptr_t(255)); }
int64_t round256(int64_t b) { return (b + 255) & ~int64_t(255); }

}  // namespace

// Token count of an even [height, width] grid whose 17-channel patch table fits int32.
int patch_tokens(int64_t height, int64_t width, const char* who) {
  if (!(height > 0 && width > 0 && height % 2 == 0 && width % 2 == 0))
    fail(ANIMA_E_INVALID_SHAPE, std::string(who) + " needs a positive even height and width");
  if (height > 0x7fffffff || width > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, std::string(who) + " size exceeds int32");
  const int64_t t = (height / 2) * (width / 2);  // 17 * height * width == 68 * t
  if (t > 0x7fffffff / 68) fail(ANIMA_E_INVALID_SHAPE, std::string(who) + " latent is too large");
  return (int)t;
}

// ---------------------------------------------------------------------------
// Launchers (shapes validated by the caller).
// ---------------------------------------------------------------------------
void launch_patchify17(const float* input, int in_channels, int64_t height, int64_t width, float* tokens,
                       hipStream_t stream) {
  const int T = patch_tokens(height, width, "patchify17");
  const int vec = aligned16(tokens);
  hipLaunchKernelGGL(patchify17_kernel<float>, grid_of((int64_t)T * 17), dim3(256), 0, stream, input, tokens,
                     in_channels, (int)height, (int)width, T, vec);
  ANIMA_HIP(hipGetLastError());
}

void launch_unpatchify16(const float* tokens, int64_t height, int64_t width, float* output, hipStream_t stream) {
  const int T = patch_tokens(height, width, "unpatchify16");
  hipLaunchKernelGGL(unpatchify16_kernel, grid_of((int64_t)T * 16), dim3(256), 0, stream, tokens, output,
                     (int)height, (int)width, T);
  ANIMA_HIP(hipGetLastError());
}

void launch_unpatchify_velocity16(const float* tokens, int64_t height, int64_t width, float* output,
                                  hipStream_t stream) {
  const int T = patch_tokens(height, width, "unpatchify_velocity16");
  hipLaunchKernelGGL(unpatchify_velocity16_kernel<float>, grid_of((int64_t)T * 16), dim3(256), 0, stream, tokens,
                     output, (int)height, (int)width, T);
  ANIMA_HIP(hipGetLastError());
}

void launch_flow_denoised(const float* x, const float* velocity, float* denoised, float sigma, int64_t count,
                          hipStream_t stream) {
  if (count <= 0) return;
  const int vec = aligned16(x) && aligned16(velocity) && aligned16(denoised);
  hipLaunchKernelGGL(flow_denoised_kernel, grid_of((count + 3) / 4), dim3(256), 0, stream, x, velocity, denoised,
                     sigma, count, vec);
  ANIMA_HIP(hipGetLastError());
}

void launch_euler_step(const float* x, const float* denoised, float* x_next, float sigma, float next_sigma,
                       int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  const float dsigma = next_sigma - sigma;
  const float inv = 1.0f / sigma;
  const int vec = aligned16(x) && aligned16(denoised) && aligned16(x_next);
  hipLaunchKernelGGL(euler_step_kernel, grid_of((count + 3) / 4), dim3(256), 0, stream, x, denoised, x_next, dsigma,
                     inv, count, vec);
  ANIMA_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// DiTPreparationExecutor.execute: patchify (16 latent channels + the zero mask
// channel, stored fp16 as the float_to_half boundary requires) -> x_embedder linear
// (fp16 output) -> fp32 residual; sinusoid + RMSNorm -> emb; t_embed1 matvec on the
// raw sinusoid -> SiLU fused into the t_embed2 matvec's input -> adaln_lora.
// ---------------------------------------------------------------------------
DitPrepareExecutor::DitPrepareExecutor(anima_ctx* ctx)
    : ctx_(ctx), linear_(ctx, anima_linear_config{128, ANIMA_LINEAR_BACKEND_AUTO}) {}

void DitPrepareExecutor::encode(const anima_dit_prepare_weights& w, const anima_dit_prepare_args& a) {
  if (!std::isfinite(a.sigma) || !std::isfinite(a.eps) || a.eps < 0.f)
    fail(ANIMA_E_INVALID_ARGUMENT, "invalid DiT preparation input");
  if (!(a.dim > 0 && a.dim % 2 == 0 && a.dim <= 2 * TS_NT * TS_PER_THREAD))
    fail(ANIMA_E_INVALID_SHAPE, "DiT preparation hidden width must be even and at most 8192");
  const int T = patch_tokens(a.height, a.width, "DiT preparation");
  const int64_t dim = a.dim;
  (void)matrix(w.x_embed, dim, 68, "DiT preparation x_embedder");
  const QWeightView t1 = matrix(w.t_embed1, dim, dim, "DiT preparation t_embedder linear_1");
  const QWeightView t2 = matrix(w.t_embed2, 3 * dim, dim, "DiT preparation t_embedder linear_2");
  require_range(w.t_norm, dim * 2, "DiT preparation t_embedding_norm");
  require_range(a.latent, checked_product({16, a.height, a.width, 4}, "DiT preparation"), "DiT preparation latent");
  require_range(a.residual, checked_product({T, dim, 4}, "DiT preparation"), "DiT preparation residual");
  require_range(a.emb, dim * 4, "DiT preparation embedding");
  require_range(a.adaln_lora, 3 * dim * 4, "DiT preparation adaln_lora");
  if (reinterpret_cast<uintptr_t>(w.t_norm.ptr) & 1u)
    fail(ANIMA_E_MISALIGNED, "DiT preparation t_embedding_norm must be 2-byte aligned");

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  const int64_t patch_bytes = round256((int64_t)T * 68 * 2);
  const int64_t half_bytes = round256(checked_product({T, dim, 2}, "DiT preparation"));
  const int64_t vec_bytes = round256(dim * 4);
  char* ws = align256(static_cast<char*>(ws_.get(patch_bytes + half_bytes + 2 * vec_bytes + 256, stream)));
  half_t* patches = reinterpret_cast<half_t*>(ws);
  half_t* resid_half = reinterpret_cast<half_t*>(ws + patch_bytes);
  float* raw = reinterpret_cast<float*>(ws + patch_bytes + half_bytes);
  float* hidden = reinterpret_cast<float*>(ws + patch_bytes + half_bytes + vec_bytes);

  hipLaunchKernelGGL(patchify17_kernel<half_t>, grid_of((int64_t)T * 17), dim3(256), 0, stream,
                     static_cast<const float*>(a.latent.ptr), patches, 16, (int)a.height, (int)a.width, T,
                     aligned8(patches) ? 1 : 0);
  ANIMA_HIP(hipGetLastError());
  linear_.encode(anima_buffer{patches, (int64_t)T * 68 * 2}, 0, w.x_embed, anima_buffer{resid_half, half_bytes}, 0, T,
                 ANIMA_FAMILY_OTHER);
  half_to_float(resid_half, static_cast<float*>(a.residual.ptr), (int64_t)T * dim, stream);

  hipLaunchKernelGGL(timestep_embed_kernel, dim3(1), dim3(TS_NT), 0, stream, a.sigma,
                     static_cast<const half_t*>(w.t_norm.ptr), raw, static_cast<float*>(a.emb.ptr), (int)dim, a.eps);
  ANIMA_HIP(hipGetLastError());
  const MatvecParams m1 = matvec_of(t1, raw, hidden);
  launch_matvec_batch(&m1, 1, stream);
  MatvecParams m2 = matvec_of(t2, hidden, static_cast<float*>(a.adaln_lora.ptr));
  m2.silu_input = 1;
  launch_matvec_batch(&m2, 1, stream);
}

// ---------------------------------------------------------------------------
// DiTFinalLayerExecutor.execute (fp16Legacy): SiLU(emb) fused into the first
// modulation matvec; adaln_lora[0:2*dim] fused into the second as its bias; one
// LayerNorm + AdaLN pass with both fp16 boundaries (residual and normalised value)
// writing the fp16 projection input; the 64-wide projection; the unpatchify reading
// its fp16 output directly.
// ---------------------------------------------------------------------------
DitFinalExecutor::DitFinalExecutor(anima_ctx* ctx)
    : ctx_(ctx), linear_(ctx, anima_linear_config{128, ANIMA_LINEAR_BACKEND_AUTO}) {}

void DitFinalExecutor::encode(const anima_dit_final_weights& w, const anima_dit_final_args& a) {
  if (!std::isfinite(a.eps) || a.eps < 0.f) fail(ANIMA_E_INVALID_ARGUMENT, "invalid DiT final-layer epsilon");
  if (!(a.dim > 0 && a.dim <= 8192)) fail(ANIMA_E_INVALID_SHAPE, "DiT final-layer hidden width must be 1..8192");
  const int T = patch_tokens(a.height, a.width, "DiT final layer");
  const int64_t dim = a.dim;
  const QWeightView m1 = validate_weight(w.mod_w1, "DiT final adaln_modulation.1");
  if (m1.cols != dim) fail(ANIMA_E_INVALID_SHAPE, "DiT final adaln_modulation.1 must have dim columns");
  const int64_t lora = m1.rows;
  const QWeightView m2 = matrix(w.mod_w2, 2 * dim, lora, "DiT final adaln_modulation.2");
  (void)matrix(w.proj, 64, dim, "DiT final linear");
  require_range(a.residual, checked_product({T, dim, 4}, "DiT final layer"), "DiT final-layer residual");
  require_range(a.emb, dim * 4, "DiT final-layer embedding");
  require_range(a.adaln_lora, 2 * dim * 4, "DiT final-layer adaln_lora");
  require_range(a.velocity, checked_product({16, a.height, a.width, 4}, "DiT final layer"), "DiT final-layer velocity");

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  const int64_t hid_bytes = round256(lora * 4);
  const int64_t mod_bytes = round256(2 * dim * 4);
  const int64_t y_bytes = round256(checked_product({T, dim, 2}, "DiT final layer"));
  const int64_t p_bytes = round256((int64_t)T * 64 * 2);
  char* ws = align256(static_cast<char*>(ws_.get(hid_bytes + mod_bytes + y_bytes + p_bytes + 256, stream)));
  float* hid = reinterpret_cast<float*>(ws);
  float* mod = reinterpret_cast<float*>(ws + hid_bytes);
  half_t* y = reinterpret_cast<half_t*>(ws + hid_bytes + mod_bytes);
  half_t* proj = reinterpret_cast<half_t*>(ws + hid_bytes + mod_bytes + y_bytes);

  MatvecParams p1 = matvec_of(m1, static_cast<const float*>(a.emb.ptr), hid);
  p1.silu_input = 1;
  launch_matvec_batch(&p1, 1, stream);
  MatvecParams p2 = matvec_of(m2, hid, mod);
  p2.bias = static_cast<const float*>(a.adaln_lora.ptr);
  launch_matvec_batch(&p2, 1, stream);
  // shift = mod[0:dim], scale = mod[dim:2*dim] (DiTFinalLayerExecutor.swift:233-252)
  launch_layernorm_modulate(static_cast<const float*>(a.residual.ptr), mod, y, dim, T, a.eps, dim, stream, true);
  linear_.encode(anima_buffer{y, y_bytes}, 0, w.proj, anima_buffer{proj, p_bytes}, 0, T, ANIMA_FAMILY_OTHER);
  hipLaunchKernelGGL(unpatchify_velocity16_kernel<half_t>, grid_of((int64_t)T * 16), dim3(256), 0, stream, proj,
                     static_cast<float*>(a.velocity.ptr), (int)a.height, (int)a.width, T);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
