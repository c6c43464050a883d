// DiT block support kernels and DiTBlockExecutor analog
// (AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:49-1319); QwenLayerExecutor analog
// (AnimaXS/Runtime/Metal/QwenEncoderMetal.swift:202-304).
#pragma once

#include "attention.hpp"
#include "linear.hpp"

namespace anima {

void launch_layernorm_modulate(const float* residual, const float* mod, half_t* out, int64_t n, int64_t rows, float eps,
                               int64_t mod_offset, hipStream_t stream);
void launch_gate_add(float* residual, const half_t* branch, const float* gate, int64_t n, int64_t count,
                     hipStream_t stream);
void launch_gelu(half_t* values, int64_t count, hipStream_t stream);
void launch_silu(const float* in, float* out, int64_t count, hipStream_t stream);
void launch_add(float* dst, const float* src, int64_t count, hipStream_t stream);
void launch_rmsnorm_half(const float* in, const half_t* w, half_t* out, int64_t n, int64_t rows, float eps,
                         hipStream_t stream);
void launch_gated_silu(const half_t* gate, const half_t* up, half_t* out, int64_t count, hipStream_t stream);
void launch_add_half(float* residual, const half_t* branch, int64_t count, hipStream_t stream);

// lin.encode() followed by gelu (GEMM_GELU) on its output, or by gate_add of its
// output into residual with gate (GEMM_GATE_ADD), fused into the GEMM when the
// tiled kernel takes the shape.  residual / gate ranges are the caller's to check.
void encode_linear_epilogue(LinearExecutor& lin, anima_buffer input, int64_t input_offset, const anima_qweight& weight,
                            anima_buffer output, int64_t output_offset, int64_t input_rows, int32_t family,
                            int epilogue, float* residual, const float* gate);

class DitBlockExecutor {
 public:
  explicit DitBlockExecutor(anima_ctx* ctx);
  void encode(const anima_dit_block_weights& w, const anima_dit_block_args& a);

 private:
  anima_ctx* ctx_;
  AttentionExecutor attention_;
  LinearExecutor linear_;
  Workspace ws_;
};

class QwenLayerExecutor {
 public:
  explicit QwenLayerExecutor(anima_ctx* ctx);
  void encode(const anima_qwen_layer_weights& w, const anima_qwen_layer_args& a);

 private:
  anima_ctx* ctx_;
  AttentionExecutor attention_;
  LinearExecutor linear_;
  Workspace ws_;
};

}  // namespace anima

struct anima_qwen_layer {
  anima::QwenLayerExecutor impl;
  explicit anima_qwen_layer(anima_ctx* c) : impl(c) {}
};

struct anima_dit_block {
  anima::DitBlockExecutor impl;
  explicit anima_dit_block(anima_ctx* c) : impl(c) {}
};
