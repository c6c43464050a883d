// DiT input / output stages and the sampler update: DiTPreparationExecutor
// (AnimaXS/Runtime/Metal/DiTPreparationExecutor.swift:6-135), DiTFinalLayerExecutor
// (AnimaXS/Runtime/Metal/DiTFinalLayerExecutor.swift:21-186) and the elementwise
// kernels of the sampler step (DiffusionSampler.swift:212-250, EulerSampler.swift:42-68).
#pragma once

#include "context.hpp"
#include "linear.hpp"

namespace anima {

// Token count (height/2)*(width/2) of an even grid; fails with INVALID_SHAPE unless
// height and width are positive and even and the 68-wide token table fits int32.
int patch_tokens(int64_t height, int64_t width, const char* who);

// Patch layout of a fp32 [channels][height][width] latent: token t = i*(width/2) + j
// holds the 2x2 patch at (2i, 2j); feature c*4 + di*2 + dj of a 68-wide token is
// pixel (2i+di, 2j+dj) of channel c.
void launch_patchify17(const float* input, int in_channels, int64_t height, int64_t width, float* tokens,
                       hipStream_t stream);
void launch_unpatchify16(const float* tokens, int64_t height, int64_t width, float* output, hipStream_t stream);
void launch_unpatchify_velocity16(const float* tokens, int64_t height, int64_t width, float* output,
                                  hipStream_t stream);
void launch_flow_denoised(const float* x, const float* velocity, float* denoised, float sigma, int64_t count,
                          hipStream_t stream);
void launch_euler_step(const float* x, const float* denoised, float* x_next, float sigma, float next_sigma,
                       int64_t count, hipStream_t stream);

class DitPrepareExecutor {
 public:
  explicit DitPrepareExecutor(anima_ctx* ctx);
  void encode(const anima_dit_prepare_weights& w, const anima_dit_prepare_args& a);

 private:
  anima_ctx* ctx_;
  LinearExecutor linear_;
  Workspace ws_;
};

class DitFinalExecutor {
 public:
  explicit DitFinalExecutor(anima_ctx* ctx);
  void encode(const anima_dit_final_weights& w, const anima_dit_final_args& a);

 private:
  anima_ctx* ctx_;
  LinearExecutor linear_;
  Workspace ws_;
};

}  // namespace anima

struct anima_dit_prepare {
  anima::DitPrepareExecutor impl;
  explicit anima_dit_prepare(anima_ctx* c) : impl(c) {}
};

struct anima_dit_final {
  anima::DitFinalExecutor impl;
  explicit anima_dit_final(anima_ctx* c) : impl(c) {}
};
