// DiT block and Qwen layer support kernels and compositions for gfx950.
//
// Kernels restate AnimaXS/Shaders/AnimaKernels.metal: dit_layernorm_modulate_to_half
// (:477-524), gate_add_half_f32 (:624-634), dit_gelu_half_inplace (:312-322),
// silu (:388-397), add_f32 (:649-656), rmsnorm_f32_to_f32 + float_to_half
// (:172-204, :81-88), gated_silu_half (:401-411) and add_half_into_float (:639-647).  The composition follows
// DiTBlockExecutor.encodeAttentionBranch / encodeMLP / encodeModulation
// (AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:1035-1319, :1403-1417) with every
// shape a parameter (the reference hard-wires 1024 tokens).
#include <cmath>
#include <string>

#include "attention.hpp"
#include "block.hpp"
#include "linear.hpp"

namespace anima {

// ---------------------------------------------------------------------------
// LayerNorm (mean-centred, no affine) * (1 + scale) + shift -> fp16.  One
// 256-thread workgroup per row; the row stays in registers between the mean,
// variance and output passes (the reference re-reads memory three times).
// ---------------------------------------------------------------------------
constexpr int LN_NT = 256;
constexpr int LN_MAX_PER_THREAD = 32;  // n <= 8192

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < LN_NT / 64; ++w) t += red[w];
  return t;
}

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
    v[e] = i < n ? x[i] : 0.f;
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
      const float normalized = (v[e] - mean) * inv;
      o[i] = f32_to_f16(normalized * (1.0f + scale[i]) + shift[i]);
    }
  }
}

__global__ __launch_bounds__(256) void gate_add_kernel(float* __restrict__ residual, const half_t* __restrict__ branch,
                                                       const float* __restrict__ gate, int64_t n, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) residual[i] += (float)branch[i] * gate[i % n];
}

__global__ __launch_bounds__(256) void gelu_kernel(half_t* __restrict__ values, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) {
    const float x = (float)values[i];
    values[i] = f32_to_f16(0.5f * x * (1.0f + erff(x * 0.7071067811865475f)));
  }
}

__global__ __launch_bounds__(256) void silu_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) {
    const float x = in[i];
    out[i] = x / (1.0f + expf(-x));
  }
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) dst[i] += src[i];
}

// RMSNorm of an fp32 row with an fp16 weight, stored as fp16: rmsnorm_f32_to_f32
// (AnimaKernels.metal:172-204) followed by float_to_half (:81-88) in one pass.
// out = half(x * rsqrt(mean(x^2) + eps) * w), the product in the reference's order.
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

// gated_silu_half (AnimaKernels.metal:401-411): SiLU and product in fp32, one rounding.
__global__ __launch_bounds__(256) void gated_silu_kernel(const half_t* __restrict__ gate, const half_t* __restrict__ up,
                                                         half_t* __restrict__ out, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) {
    const float x = (float)gate[i];
    out[i] = f32_to_f16((x / (1.0f + expf(-x))) * (float)up[i]);
  }
}

// add_half_into_float (AnimaKernels.metal:639-647).
__global__ __launch_bounds__(256) void add_half_kernel(float* __restrict__ residual, const half_t* __restrict__ branch,
                                                       int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) residual[i] += (float)branch[i];
}

static dim3 grid1d(int64_t count) {
  const int64_t b = (count + 255) / 256;
  if (b > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "elementwise grid too large");
  return dim3((unsigned)b);
}

void launch_layernorm_modulate(const float* residual, const float* mod, half_t* out, int64_t n, int64_t rows, float eps,
                               int64_t mod_offset, hipStream_t stream) {
  if (n > LN_NT * LN_MAX_PER_THREAD) fail(ANIMA_E_UNSUPPORTED, "layernorm-modulate supports rows of at most 8192");
  if (rows > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "layernorm-modulate rows exceed int32");
  hipLaunchKernelGGL(layernorm_modulate_kernel, dim3((unsigned)rows), dim3(LN_NT), 0, stream, residual, mod, out, (int)n,
                     eps, mod_offset);
  ANIMA_HIP(hipGetLastError());
}
void launch_gate_add(float* residual, const half_t* branch, const float* gate, int64_t n, int64_t count,
                     hipStream_t stream) {
  hipLaunchKernelGGL(gate_add_kernel, grid1d(count), dim3(256), 0, stream, residual, branch, gate, n, count);
  ANIMA_HIP(hipGetLastError());
}
void launch_gelu(half_t* values, int64_t count, hipStream_t stream) {
  hipLaunchKernelGGL(gelu_kernel, grid1d(count), dim3(256), 0, stream, values, count);
  ANIMA_HIP(hipGetLastError());
}
void launch_silu(const float* in, float* out, int64_t count, hipStream_t stream) {
  hipLaunchKernelGGL(silu_kernel, grid1d(count), dim3(256), 0, stream, in, out, count);
  ANIMA_HIP(hipGetLastError());
}
void launch_add(float* dst, const float* src, int64_t count, hipStream_t stream) {
  hipLaunchKernelGGL(add_kernel, grid1d(count), dim3(256), 0, stream, dst, src, count);
  ANIMA_HIP(hipGetLastError());
}
void launch_rmsnorm_half(const float* in, const half_t* w, half_t* out, int64_t n, int64_t rows, float eps,
                         hipStream_t stream) {
  if (n > LN_NT * LN_MAX_PER_THREAD) fail(ANIMA_E_UNSUPPORTED, "rmsnorm supports rows of at most 8192");
  if (rows > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "rmsnorm rows exceed int32");
  hipLaunchKernelGGL(rmsnorm_half_kernel, dim3((unsigned)rows), dim3(LN_NT), 0, stream, in, w, out, (int)n, eps);
  ANIMA_HIP(hipGetLastError());
}
void launch_gated_silu(const half_t* gate, const half_t* up, half_t* out, int64_t count, hipStream_t stream) {
  hipLaunchKernelGGL(gated_silu_kernel, grid1d(count), dim3(256), 0, stream, gate, up, out, count);
  ANIMA_HIP(hipGetLastError());
}
void launch_add_half(float* residual, const half_t* branch, int64_t count, hipStream_t stream) {
  hipLaunchKernelGGL(add_half_kernel, grid1d(count), dim3(256), 0, stream, residual, branch, count);
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

void DitBlockExecutor::encode(const anima_dit_block_weights& w, const anima_dit_block_args& a) {
  const int64_t S = a.tokens, dim = a.dim, H = a.heads, hd = a.head_dim, T = a.context_tokens, C = a.context_dim,
                hidden = a.mlp_hidden;
  if (!(S > 0 && dim > 0 && H > 0 && hd > 0 && T > 0 && C > 0 && hidden > 0 && H * hd == dim))
    fail(ANIMA_E_INVALID_SHAPE, "invalid DiT block shape (requires heads * head_dim == dim)");
  if (!(a.eps >= 0.f && std::isfinite(a.eps))) fail(ANIMA_E_INVALID_ARGUMENT, "DiT block epsilon must be finite");
  if (checked_product({S, dim, 4}, "DiT block") > a.residual.length || checked_product({dim, 4}, "DiT block") > a.emb.length ||
      checked_product({3 * dim, 4}, "DiT block") > a.adaln_lora.length ||
      checked_product({T, C, 2}, "DiT block") > a.context.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "DiT block buffer range is out of bounds");
  if (!a.rope) fail(ANIMA_E_INVALID_ARGUMENT, "DiT block requires a RoPE table");
  auto need = [&](const anima_qweight& q, int64_t rows, int64_t cols, const char* nm) {
    if (q.rows != rows || q.columns != cols) fail(ANIMA_E_INVALID_SHAPE, std::string(nm) + " shape mismatch");
  };
  need(w.self_q, dim, dim, "self_q"); need(w.self_k, dim, dim, "self_k"); need(w.self_v, dim, dim, "self_v");
  need(w.self_o, dim, dim, "self_o"); need(w.cross_q, dim, dim, "cross_q"); need(w.cross_k, dim, C, "cross_k");
  need(w.cross_v, dim, C, "cross_v"); need(w.cross_o, dim, dim, "cross_o"); need(w.mlp1, hidden, dim, "mlp1");
  need(w.mlp2, dim, hidden, "mlp2");
  const int64_t lora = w.mod_self_w1.rows;
  need(w.mod_self_w1, lora, dim, "mod_self_w1"); need(w.mod_cross_w1, lora, dim, "mod_cross_w1");
  need(w.mod_mlp_w1, lora, dim, "mod_mlp_w1"); need(w.mod_self_w2, 3 * dim, lora, "mod_self_w2");
  need(w.mod_cross_w2, 3 * dim, lora, "mod_cross_w2"); need(w.mod_mlp_w2, 3 * dim, lora, "mod_mlp_w2");

  // Workspace layout (bytes, 256-aligned).
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t o_silu = 0;
  const int64_t o_hid = o_silu + al(dim * 4);
  const int64_t o_mod = o_hid + al(lora * 4);
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
  anima_buffer silu_b = sub(ws, o_silu, dim * 4), hid_b = sub(ws, o_hid, lora * 4);
  anima_buffer norm_b = sub(ws, o_norm, S * dim * 2), q_b = sub(ws, o_q, S * dim * 2), k_b = sub(ws, o_k, S * dim * 2),
               v_b = sub(ws, o_v, S * dim * 2), a_b = sub(ws, o_a, S * dim * 2), br_b = sub(ws, o_b, S * dim * 2),
               ck_b = sub(ws, o_ck, T * dim * 2), cv_b = sub(ws, o_cv, T * dim * 2), h_b = sub(ws, o_h, S * hidden * 2);

  // Modulation (DiTBlockExecutor.encodeModulation, :1403-1417): SiLU(emb) -> W1 -> W2 -> + adaln_lora.
  launch_silu(static_cast<const float*>(a.emb.ptr), static_cast<float*>(silu_b.ptr), dim, stream);
  const anima_qweight* w1s[3] = {&w.mod_self_w1, &w.mod_cross_w1, &w.mod_mlp_w1};
  const anima_qweight* w2s[3] = {&w.mod_self_w2, &w.mod_cross_w2, &w.mod_mlp_w2};
  float* mods[3];
  for (int br = 0; br < 3; ++br) {
    anima_buffer mod_b = sub(ws, o_mod + br * mod_bytes, 3 * dim * 4);
    mods[br] = static_cast<float*>(mod_b.ptr);
    encode_matvec(ctx_, *w1s[br], silu_b, 0, hid_b, 0);
    encode_matvec(ctx_, *w2s[br], hid_b, 0, mod_b, 0);
    launch_add(mods[br], static_cast<const float*>(a.adaln_lora.ptr), 3 * dim, stream);
  }

  anima_attention_args att{};
  att.heads = H; att.head_dim = hd; att.key_value_heads = H; att.layout = ANIMA_LAYOUT_TOKEN_MAJOR;
  att.token_stride = dim; att.batch = 1;

  // Self attention (encodeAttentionBranch, :1035-1242).
  launch_layernorm_modulate(residual, mods[0], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  linear_.encode(norm_b, 0, w.self_q, q_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(norm_b, 0, w.self_k, k_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(norm_b, 0, w.self_v, v_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  anima_qk_prologue self_pro{w.self_q_norm, w.self_k_norm, a.eps, a.rope, S, 1, 1};
  att.query = q_b; att.key = k_b; att.value = v_b; att.output = a_b;
  att.query_count = S; att.key_count = S; att.prologue = &self_pro;
  attention_.encode(att);
  linear_.encode(a_b, 0, w.self_o, br_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  launch_gate_add(residual, static_cast<const half_t*>(br_b.ptr), mods[0] + 2 * dim, dim, S * dim, stream);

  // Cross attention to the context (no RoPE; per-head RMSNorm on Q and K).
  launch_layernorm_modulate(residual, mods[1], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  linear_.encode(norm_b, 0, w.cross_q, q_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(a.context, 0, w.cross_k, ck_b, 0, T, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(a.context, 0, w.cross_v, cv_b, 0, T, ANIMA_FAMILY_ATTENTION_PROJECTION);
  anima_qk_prologue cross_pro{w.cross_q_norm, w.cross_k_norm, a.eps, nullptr, 0, 0, 0};
  att.query = q_b; att.key = ck_b; att.value = cv_b; att.output = a_b;
  att.query_count = S; att.key_count = T; att.prologue = &cross_pro;
  attention_.encode(att);
  linear_.encode(a_b, 0, w.cross_o, br_b, 0, S, ANIMA_FAMILY_ATTENTION_PROJECTION);
  launch_gate_add(residual, static_cast<const half_t*>(br_b.ptr), mods[1] + 2 * dim, dim, S * dim, stream);

  // MLP (encodeMLP, :1244-1319): mlp1 -> exact GELU -> mlp2.
  launch_layernorm_modulate(residual, mods[2], static_cast<half_t*>(norm_b.ptr), dim, S, a.eps, dim, stream);
  linear_.encode(norm_b, 0, w.mlp1, h_b, 0, S, ANIMA_FAMILY_MLP_UP);
  launch_gelu(static_cast<half_t*>(h_b.ptr), S * hidden, stream);
  linear_.encode(h_b, 0, w.mlp2, br_b, 0, S, ANIMA_FAMILY_MLP_DOWN);
  launch_gate_add(residual, static_cast<const half_t*>(br_b.ptr), mods[2] + 2 * dim, dim, S * dim, stream);
}

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
  if (checked_product({rows, hidden, 4}, "Qwen layer") > a.residual.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "invalid Qwen layer input buffers");
  if (!a.rope) fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer requires a RoPE table");
  if (!w.input_norm || !w.post_attention_norm || !w.q_norm || !w.k_norm)
    fail(ANIMA_E_INVALID_ARGUMENT, "Qwen layer norm weight pointer is null");
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
  launch_rmsnorm_half(residual, static_cast<const half_t*>(w.input_norm), norm, hidden, rows, a.eps, stream);
  linear_.encode(norm_b, 0, w.q, q_b, 0, rows, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(norm_b, 0, w.k, k_b, 0, rows, ANIMA_FAMILY_ATTENTION_PROJECTION);
  linear_.encode(norm_b, 0, w.v, v_b, 0, rows, ANIMA_FAMILY_ATTENTION_PROJECTION);
  anima_qk_prologue pro{w.q_norm, w.k_norm, a.eps, a.rope, S, 1, 1};
  anima_attention_args att{};
  att.query = q_b; att.key = k_b; att.value = v_b; att.output = att_b;
  att.heads = H; att.key_value_heads = Hkv; att.head_dim = D; att.query_count = S; att.key_count = S;
  att.causal = 1; att.layout = ANIMA_LAYOUT_TOKEN_MAJOR; att.token_stride = qdim; att.kv_token_stride = kvdim;
  att.batch = B; att.key_lengths = a.key_lengths; att.key_lengths_on_device = 0; att.prologue = &pro;
  attention_.encode(att);
  linear_.encode(att_b, 0, w.o, proj_b, 0, rows, ANIMA_FAMILY_ATTENTION_PROJECTION);
  launch_add_half(residual, static_cast<const half_t*>(proj_b.ptr), rows * hidden, stream);

  // MLP branch (:284-302): gate/up -> SwiGLU (into the gate buffer) -> down.
  launch_rmsnorm_half(residual, static_cast<const half_t*>(w.post_attention_norm), norm, hidden, rows, a.eps, stream);
  linear_.encode(norm_b, 0, w.gate, gate_b, 0, rows, ANIMA_FAMILY_MLP_UP);
  linear_.encode(norm_b, 0, w.up, up_b, 0, rows, ANIMA_FAMILY_MLP_UP);
  launch_gated_silu(static_cast<const half_t*>(gate_b.ptr), static_cast<const half_t*>(up_b.ptr),
                    static_cast<half_t*>(gate_b.ptr), rows * inter, stream);
  linear_.encode(gate_b, 0, w.down, proj_b, 0, rows, ANIMA_FAMILY_MLP_DOWN);
  launch_add_half(residual, static_cast<const half_t*>(proj_b.ptr), rows * hidden, stream);
}

}  // namespace anima
