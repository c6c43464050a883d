// DiT block support kernels and DiTBlockExecutor analog
// (AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:49-1319); QwenLayerExecutor analog
// (AnimaXS/Runtime/Metal/QwenEncoderMetal.swift:202-304).
#pragma once

#include <algorithm>
#include <vector>

#include "attention.hpp"
#include "linear.hpp"

namespace anima {

// fp16_boundaries: the FinalLayer form (float(half(x)) in, the normalised value rounded
// through fp16 before the modulation).
void launch_layernorm_modulate(const float* residual, const float* mod, half_t* out, int64_t n, int64_t rows, float eps,
                               int64_t mod_offset, hipStream_t stream, bool fp16_boundaries = false);
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

// CrossKVCache (DiTBlockExecutor.swift:19-43): per block, the context's cross-attention
// K (after its per-head RMSNorm) and V, fp16 [context_tokens, dim] each, in one device
// allocation owned by the cache.
class CrossKVCache {
 public:
  CrossKVCache(anima_ctx* ctx, int64_t blocks, int64_t tokens, int64_t dim);
  ~CrossKVCache();
  CrossKVCache(const CrossKVCache&) = delete;
  CrossKVCache& operator=(const CrossKVCache&) = delete;
  half_t* k(int64_t block) const { return base_ + block * 2 * tokens_ * dim_; }
  half_t* v(int64_t block) const { return k(block) + tokens_ * dim_; }
  bool ready(int64_t block) const { return ready_[block] != 0; }
  void mark_ready(int64_t block) { ready_[block] = 1; }
  void reset() { std::fill(ready_.begin(), ready_.end(), 0); }
  int64_t blocks() const { return blocks_; }
  int64_t tokens() const { return tokens_; }
  int64_t dim() const { return dim_; }
  int64_t bytes() const { return bytes_; }

 private:
  anima_ctx* ctx_;
  int64_t blocks_, tokens_, dim_, bytes_;
  half_t* base_ = nullptr;
  std::vector<uint8_t> ready_;
};

// WeightStreamer (WeightStreamer.swift:87-213): `slots` device slots, a copy stream
// and per-slot events (copy done / last reader done).
class WeightStreamer {
 public:
  WeightStreamer(anima_ctx* ctx, int64_t capacity, int slots);
  ~WeightStreamer();
  WeightStreamer(const WeightStreamer&) = delete;
  WeightStreamer& operator=(const WeightStreamer&) = delete;
  int slots() const { return slots_; }
  int64_t capacity() const { return capacity_; }
  char* slot(int s) const { return slot_[s]; }
  // Copy `bytes` from host `src` into slot s on the copy stream once the slot's last
  // reader has finished, and make the slot's "loaded" event follow the copy.
  void load(int s, const void* src, int64_t bytes);
  // Make the context stream wait for slot s's copy / mark slot s read up to here.
  void acquire(int s);
  void release(int s);
  anima_ctx* context() const { return ctx_; }

 private:
  anima_ctx* ctx_;
  int64_t capacity_;
  int slots_;
  char* slot_[4] = {};
  hipStream_t copy_ = nullptr;
  hipEvent_t loaded_[4] = {};
  hipEvent_t released_[4] = {};
};

class DitBlockExecutor {
 public:
  explicit DitBlockExecutor(anima_ctx* ctx);
  // Shape, range and pointer checks of one block (nothing is launched).
  void check(const anima_dit_block_weights& w, const anima_dit_block_args& a, const CrossKVCache* cache,
             int64_t block_index) const;
  void encode(const anima_dit_block_weights& w, const anima_dit_block_args& a, CrossKVCache* cache = nullptr,
              int64_t block_index = 0);
  // DitForward.execute (DitForward.swift:78-112) over resident weights.
  void forward(const anima_dit_block_weights* blocks, int64_t count, const anima_dit_block_args& a,
               CrossKVCache* cache);
  // DitForward.execute with host ranges streamed through `st`'s slots.
  void forward_streamed(WeightStreamer& st, const anima_dit_block_weights* templates, const void* const* ranges,
                        const int64_t* range_bytes, int64_t count, const anima_dit_block_args& a,
                        CrossKVCache* cache);

 private:
  // encode() with the block's three modulation rows ([3][3 * dim] fp32, branch stride
  // mod_stride floats) already computed when premod is not null.
  void encode_block(const anima_dit_block_weights& w, const anima_dit_block_args& a, CrossKVCache* cache,
                    int64_t block_index, const float* premod, int64_t mod_stride);

  anima_ctx* ctx_;
  AttentionExecutor attention_;
  LinearExecutor linear_;
  Workspace ws_;
  Workspace mod_ws_;   // the forward's modulation rows of every block
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

struct anima_cross_kv_cache {
  anima::CrossKVCache impl;
  anima_cross_kv_cache(anima_ctx* c, int64_t blocks, int64_t tokens, int64_t dim) : impl(c, blocks, tokens, dim) {}
};

struct anima_weight_streamer {
  anima::WeightStreamer impl;
  anima_weight_streamer(anima_ctx* c, int64_t capacity, int slots) : impl(c, capacity, slots) {}
};
