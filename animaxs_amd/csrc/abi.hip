// extern "C" entry points of libanima_hip (include/anima_hip.h).  Each converts
// exceptions into an anima_status and the thread-local last-error message; no
// entry point launches anything before its arguments validate.
#include <cmath>
#include <string>

#include "attention.hpp"
#include "block.hpp"
#include "context.hpp"
#include "dit_io.hpp"
#include "linear.hpp"
#include "numerics_probe.hpp"

namespace anima {

static thread_local std::string g_last_error;

void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }

template <class T>
static T* require(T* p, const char* what) {
  if (!p) fail(ANIMA_E_INVALID_ARGUMENT, std::string(what) + " handle is null");
  return p;
}

}  // namespace anima

using namespace anima;

extern "C" {

const char* anima_last_error(void) { return g_last_error.c_str(); }

int32_t anima_abi_version(void) { return ANIMA_HIP_ABI_VERSION; }

// ---------------------------------------------------------------- context
anima_status anima_ctx_create(int32_t device, anima_ctx** out) {
  return guarded([&] {
    require(out, "context output");
    *out = nullptr;
    // The device is bound lazily: nothing touches HIP until the first launch,
    // so validation works (and is tested) on hosts without a GPU.
    if (device < 0) fail(ANIMA_E_INVALID_ARGUMENT, "HIP device index must be >= 0");
    anima_ctx* c = new anima_ctx();
    c->device = device;
    c->stream = nullptr;
    *out = c;
  });
}

anima_status anima_ctx_destroy(anima_ctx* ctx) {
  return guarded([&] { delete ctx; });
}

anima_status anima_ctx_set_stream(anima_ctx* ctx, void* hip_stream) {
  return guarded([&] { require(ctx, "context")->stream = static_cast<hipStream_t>(hip_stream); });
}

anima_status anima_ctx_synchronize(anima_ctx* ctx) {
  return guarded([&] {
    require(ctx, "context");
    DeviceGuard g(ctx);
    ANIMA_HIP(hipStreamSynchronize(ctx->stream));
  });
}

// ---------------------------------------------------------------- attention
anima_status anima_attention_create(anima_ctx* ctx, const anima_attention_config* cfg, anima_attention** out) {
  return guarded([&] {
    require(out, "attention output");
    *out = nullptr;
    require(ctx, "context");
    require(cfg, "attention config");
    *out = new anima_attention(ctx, *cfg);
  });
}

anima_status anima_attention_destroy(anima_attention* attn) {
  return guarded([&] {
    delete attn;  // hipFree needs no current-device switch
  });
}

anima_status anima_attention_encode(anima_attention* attn, const anima_attention_args* args) {
  return guarded([&] { require(attn, "attention")->impl.encode(*require(args, "attention args")); });
}

anima_status anima_attention_encode_noalloc(anima_attention* attn, const anima_attention_args* args) {
  return guarded([&] { require(attn, "attention")->impl.encode_noalloc(*require(args, "attention args")); });
}

anima_status anima_attention_execute(anima_attention* attn, const anima_attention_args* args) {
  return guarded([&] {
    require(attn, "attention")->impl.encode(*require(args, "attention args"));
    DeviceGuard g(attn->impl.context());
    ANIMA_HIP(hipStreamSynchronize(attn->impl.context()->stream));
  });
}

anima_status anima_attention_max_score_scratch_bytes(anima_attention* attn, int64_t key_count, int64_t query_count,
                                                     int64_t* out_bytes) {
  return guarded([&] {
    *require(out_bytes, "output") = require(attn, "attention")->impl.maximum_score_scratch_bytes(key_count, query_count);
  });
}

anima_status anima_attention_workspace_bytes(anima_attention* attn, int64_t* out_bytes) {
  return guarded([&] { *require(out_bytes, "output") = require(attn, "attention")->impl.workspace_bytes(); });
}

// ---------------------------------------------------------------- linear
anima_status anima_linear_create(anima_ctx* ctx, const anima_linear_config* cfg, anima_linear** out) {
  return guarded([&] {
    require(out, "linear output");
    *out = nullptr;
    require(ctx, "context");
    require(cfg, "linear config");
    *out = new anima_linear(ctx, *cfg);
  });
}

anima_status anima_linear_destroy(anima_linear* lin) {
  return guarded([&] {
    delete lin;
  });
}

anima_status anima_linear_encode(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                 const anima_qweight* weight, anima_buffer output, int64_t output_offset,
                                 int64_t input_rows, int32_t family) {
  return guarded([&] {
    require(lin, "linear")->impl.encode(input, input_offset, *require(weight, "weight"), output, output_offset,
                                        input_rows, family);
  });
}

static void check_elementwise(const anima_buffer& b, int64_t count, int64_t elem, const char* what) {
  if (count < 0) fail(ANIMA_E_INVALID_SHAPE, std::string(what) + " count must be >= 0");
  if (checked_product({count, elem}, what) > b.length) fail(ANIMA_E_OUT_OF_BOUNDS, std::string(what) + " buffer range is out of bounds");
  if (count > 0 && !b.ptr) fail(ANIMA_E_INVALID_ARGUMENT, std::string(what) + " buffer pointer is null");
}

anima_status anima_linear_encode_epilogue(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                          const anima_qweight* weight, anima_buffer output, int64_t output_offset,
                                          int64_t input_rows, int32_t family, int32_t epilogue, anima_buffer residual,
                                          anima_buffer gate) {
  return guarded([&] {
    require(lin, "linear");
    const anima_qweight& w = *require(weight, "weight");
    if (epilogue != ANIMA_LINEAR_EPILOGUE_GELU && epilogue != ANIMA_LINEAR_EPILOGUE_GATE_ADD &&
        epilogue != ANIMA_LINEAR_EPILOGUE_RESIDUAL_ADD)
      fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear epilogue");
    float* res = nullptr;
    const float* gt = nullptr;
    if (epilogue != ANIMA_LINEAR_EPILOGUE_GELU) {
      if (!(input_rows > 0 && w.rows > 0)) fail(ANIMA_E_INVALID_SHAPE, "invalid LinearExecutor shape or offset");
      check_elementwise(residual, checked_product({input_rows, w.rows}, "linear epilogue"), 4, "linear residual");
      res = static_cast<float*>(residual.ptr);
    }
    if (epilogue == ANIMA_LINEAR_EPILOGUE_GATE_ADD) {
      check_elementwise(gate, w.rows, 4, "linear gate");
      gt = static_cast<const float*>(gate.ptr);
    }
    const int epi = epilogue == ANIMA_LINEAR_EPILOGUE_GELU       ? GEMM_GELU
                    : epilogue == ANIMA_LINEAR_EPILOGUE_GATE_ADD ? GEMM_GATE_ADD
                                                                 : GEMM_RESIDUAL_ADD;
    encode_linear_epilogue(lin->impl, input, input_offset, w, output, output_offset, input_rows, family, epi, res, gt);
  });
}

anima_status anima_linear_encode_group(anima_linear* lin, anima_buffer input, const anima_qweight* const* weights,
                                       const anima_buffer* outputs, int32_t count, int64_t input_rows,
                                       int32_t family) {
  return guarded([&] {
    require(lin, "linear");
    require(weights, "weights");
    require(outputs, "outputs");
    if (count < 1 || count > 3) fail(ANIMA_E_INVALID_ARGUMENT, "linear group holds 1 to 3 weights");
    for (int i = 0; i < count; ++i) require(weights[i], "weight");
    lin->impl.encode_group(input, weights, outputs, count, input_rows, family);
  });
}

anima_status anima_linear_encode_head_rmsnorm(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                              const anima_qweight* weight, anima_buffer output, int64_t output_offset,
                                              int64_t input_rows, int32_t family, anima_buffer norm_weight,
                                              int64_t head_dim, float eps) {
  return guarded([&] {
    require(lin, "linear");
    const anima_qweight& w = *require(weight, "weight");
    if (head_dim <= 0) fail(ANIMA_E_INVALID_SHAPE, "per-head RMSNorm head_dim must be positive");
    if (!norm_weight.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "per-head RMSNorm weight pointer is null");
    check_elementwise(norm_weight, head_dim, 2, "per-head RMSNorm weight");
    lin->impl.encode_head_rmsnorm(input, input_offset, w, output, output_offset, input_rows, family,
                                  static_cast<const half_t*>(norm_weight.ptr), head_dim, eps);
  });
}

anima_status anima_linear_execute(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                  const anima_qweight* weight, anima_buffer output, int64_t output_offset,
                                  int64_t input_rows, int32_t family) {
  return guarded([&] {
    require(lin, "linear")->impl.encode(input, input_offset, *require(weight, "weight"), output, output_offset,
                                        input_rows, family);
    DeviceGuard g(lin->impl.context());
    ANIMA_HIP(hipStreamSynchronize(lin->impl.context()->stream));
  });
}

anima_status anima_matvec_encode(anima_ctx* ctx, const anima_qweight* weight, anima_buffer input_f32,
                                 int64_t input_offset, anima_buffer output_f32, int64_t output_offset) {
  return guarded([&] {
    encode_matvec(require(ctx, "context"), *require(weight, "weight"), input_f32, input_offset, output_f32,
                  output_offset);
  });
}

anima_status anima_dequant_to_half_encode(anima_ctx* ctx, const anima_qweight* weight, anima_buffer output,
                                          int64_t output_offset, int64_t out_row_stride) {
  return guarded([&] {
    encode_dequant(require(ctx, "context"), *require(weight, "weight"), output, output_offset, out_row_stride);
  });
}

anima_status anima_read_probe_encode(anima_ctx* ctx, anima_buffer src, int64_t src_offset, int64_t bytes,
                                     anima_buffer sink) {
  return guarded([&] {
    require(ctx, "context");
    if (bytes < 0 || bytes % 16 != 0) fail(ANIMA_E_INVALID_SHAPE, "read probe: bytes must be a non-negative multiple of 16");
    if (src_offset < 0 || (src_offset & 15) != 0 || !src.ptr || ((uintptr_t)src.ptr & 15u) != 0)
      fail(ANIMA_E_MISALIGNED, "read probe: the source must be 16-byte aligned");
    if (checked_end(src_offset, bytes, "read probe") > src.length)
      fail(ANIMA_E_OUT_OF_BOUNDS, "read probe: source range is out of bounds");
    if (bytes == 0) return;
    if (!sink.ptr || ((uintptr_t)sink.ptr & 15u) != 0 || sink.length < read_probe_sink_bytes(bytes))
      fail(ANIMA_E_OUT_OF_BOUNDS, "read probe: sink must be 16-byte aligned and hold anima_read_probe_sink_bytes bytes");
    DeviceGuard g(ctx);
    launch_read_probe(static_cast<const char*>(src.ptr) + src_offset, bytes, sink.ptr, ctx->stream);
  });
}

int64_t anima_read_probe_sink_bytes(int64_t bytes) { return bytes > 0 ? read_probe_sink_bytes(bytes) : 0; }

// ---------------------------------------------------------------- numerical-health probes

anima_status anima_numerics_probe_reset_encode(anima_ctx* ctx, anima_buffer stats, int32_t slots) {
  return guarded([&] {
    require(ctx, "context");
    if (slots < 0) fail(ANIMA_E_INVALID_SHAPE, "numerics probe: slots must be >= 0");
    check_elementwise(stats, (int64_t)slots * ANIMA_PROBE_SLOT_UINTS, 4, "numerics probe stats");
    if (((uintptr_t)stats.ptr & 3u) != 0) fail(ANIMA_E_MISALIGNED, "numerics probe: stats must be 4-byte aligned");
    if (slots == 0) return;
    DeviceGuard g(ctx);
    launch_numerics_probe_reset(static_cast<uint32_t*>(stats.ptr), slots, ctx->stream);
  });
}

anima_status anima_numerics_probe_encode(anima_ctx* ctx, anima_buffer values, int64_t offset, int64_t count,
                                         int32_t dtype, anima_buffer stats, int32_t slot) {
  return guarded([&] {
    require(ctx, "context");
    if (dtype != ANIMA_PROBE_F16 && dtype != ANIMA_PROBE_F32)
      fail(ANIMA_E_INVALID_ARGUMENT, "numerics probe: dtype must be ANIMA_PROBE_F16 or ANIMA_PROBE_F32");
    if (count < 0 || offset < 0) fail(ANIMA_E_INVALID_SHAPE, "numerics probe: count and offset must be >= 0");
    if (count >= (int64_t)ANIMA_PROBE_NO_INDEX)
      fail(ANIMA_E_INVALID_SHAPE, "numerics probe: count must be below 0xFFFFFFFF");
    if (slot < 0) fail(ANIMA_E_INVALID_ARGUMENT, "numerics probe: slot must be >= 0");
    const int64_t elem = dtype == ANIMA_PROBE_F16 ? 2 : 4;
    check_elementwise(values, checked_end(offset, count, "numerics probe"), elem, "numerics probe values");
    check_elementwise(stats, ((int64_t)slot + 1) * ANIMA_PROBE_SLOT_UINTS, 4, "numerics probe stats");
    if (((uintptr_t)stats.ptr & 3u) != 0) fail(ANIMA_E_MISALIGNED, "numerics probe: stats must be 4-byte aligned");
    if (((uintptr_t)values.ptr & (uintptr_t)(elem - 1)) != 0)
      fail(ANIMA_E_MISALIGNED, "numerics probe: values must be aligned to their element size");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_numerics_probe(static_cast<const char*>(values.ptr) + offset * elem, count, dtype == ANIMA_PROBE_F16,
                          static_cast<uint32_t*>(stats.ptr) + (int64_t)slot * ANIMA_PROBE_SLOT_UINTS, ctx->stream);
  });
}

// ---------------------------------------------------------------- DiT block support kernels

anima_status anima_layernorm_modulate_to_half_encode(anima_ctx* ctx, anima_buffer residual, anima_buffer modulation,
                                                     anima_buffer output, int64_t n, int64_t rows, float eps,
                                                     int64_t modulation_offset) {
  return guarded([&] {
    require(ctx, "context");
    if (n <= 0 || rows <= 0 || modulation_offset < 0) fail(ANIMA_E_INVALID_SHAPE, "invalid layernorm-modulate shape");
    check_elementwise(residual, checked_product({rows, n}, "layernorm"), 4, "layernorm residual");
    check_elementwise(output, checked_product({rows, n}, "layernorm"), 2, "layernorm output");
    check_elementwise(modulation, std::max(n, checked_end(modulation_offset, n, "layernorm")), 4, "layernorm modulation");
    DeviceGuard g(ctx);
    launch_layernorm_modulate(static_cast<const float*>(residual.ptr), static_cast<const float*>(modulation.ptr),
                              static_cast<half_t*>(output.ptr), n, rows, eps, modulation_offset, ctx->stream);
  });
}

anima_status anima_gate_add_half_f32_encode(anima_ctx* ctx, anima_buffer residual, anima_buffer branch,
                                            anima_buffer gate, int64_t n, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    if (n <= 0) fail(ANIMA_E_INVALID_SHAPE, "gate width must be positive");
    check_elementwise(residual, count, 4, "gate_add residual");
    check_elementwise(branch, count, 2, "gate_add branch");
    check_elementwise(gate, n, 4, "gate_add gate");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_gate_add(static_cast<float*>(residual.ptr), static_cast<const half_t*>(branch.ptr),
                    static_cast<const float*>(gate.ptr), n, count, ctx->stream);
  });
}

anima_status anima_gelu_half_inplace_encode(anima_ctx* ctx, anima_buffer values, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    check_elementwise(values, count, 2, "gelu");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_gelu(static_cast<half_t*>(values.ptr), count, ctx->stream);
  });
}

anima_status anima_silu_f32_encode(anima_ctx* ctx, anima_buffer input, anima_buffer output, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    check_elementwise(input, count, 4, "silu input");
    check_elementwise(output, count, 4, "silu output");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_silu(static_cast<const float*>(input.ptr), static_cast<float*>(output.ptr), count, ctx->stream);
  });
}

anima_status anima_add_f32_encode(anima_ctx* ctx, anima_buffer destination, anima_buffer source, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    check_elementwise(destination, count, 4, "add destination");
    check_elementwise(source, count, 4, "add source");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_add(static_cast<float*>(destination.ptr), static_cast<const float*>(source.ptr), count, ctx->stream);
  });
}

anima_status anima_rmsnorm_f32_to_half_encode(anima_ctx* ctx, anima_buffer input, anima_buffer weight,
                                              anima_buffer output, int64_t n, int64_t rows, float eps) {
  return guarded([&] {
    require(ctx, "context");
    if (n <= 0 || rows <= 0) fail(ANIMA_E_INVALID_SHAPE, "invalid rmsnorm shape");
    if (!(eps >= 0.f && std::isfinite(eps))) fail(ANIMA_E_INVALID_ARGUMENT, "rmsnorm epsilon must be finite");
    check_elementwise(input, checked_product({rows, n}, "rmsnorm"), 4, "rmsnorm input");
    check_elementwise(weight, n, 2, "rmsnorm weight");
    check_elementwise(output, checked_product({rows, n}, "rmsnorm"), 2, "rmsnorm output");
    DeviceGuard g(ctx);
    launch_rmsnorm_half(static_cast<const float*>(input.ptr), static_cast<const half_t*>(weight.ptr),
                        static_cast<half_t*>(output.ptr), n, rows, eps, ctx->stream);
  });
}

anima_status anima_gated_silu_half_encode(anima_ctx* ctx, anima_buffer gate, anima_buffer up, anima_buffer output,
                                          int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    check_elementwise(gate, count, 2, "gated_silu gate");
    check_elementwise(up, count, 2, "gated_silu up");
    check_elementwise(output, count, 2, "gated_silu output");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_gated_silu(static_cast<const half_t*>(gate.ptr), static_cast<const half_t*>(up.ptr),
                      static_cast<half_t*>(output.ptr), count, ctx->stream);
  });
}

anima_status anima_add_half_into_float_encode(anima_ctx* ctx, anima_buffer residual, anima_buffer branch,
                                              int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    check_elementwise(residual, count, 4, "add_half residual");
    check_elementwise(branch, count, 2, "add_half branch");
    if (count == 0) return;
    DeviceGuard g(ctx);
    launch_add_half(static_cast<float*>(residual.ptr), static_cast<const half_t*>(branch.ptr), count, ctx->stream);
  });
}

// ---------------------------------------------------------------- Qwen layer
anima_status anima_qwen_layer_create(anima_ctx* ctx, anima_qwen_layer** out) {
  return guarded([&] {
    require(out, "layer output");
    *out = nullptr;
    *out = new anima_qwen_layer(require(ctx, "context"));
  });
}

anima_status anima_qwen_layer_destroy(anima_qwen_layer* layer) {
  return guarded([&] { delete layer; });
}

anima_status anima_qwen_layer_encode(anima_qwen_layer* layer, const anima_qwen_layer_weights* w,
                                     const anima_qwen_layer_args* args) {
  return guarded([&] {
    require(layer, "layer")->impl.encode(*require(w, "layer weights"), *require(args, "layer args"));
  });
}

// ---------------------------------------------------------------- DiT block
anima_status anima_dit_block_create(anima_ctx* ctx, anima_dit_block** out) {
  return guarded([&] {
    require(out, "block output");
    *out = nullptr;
    *out = new anima_dit_block(require(ctx, "context"));
  });
}

anima_status anima_dit_block_destroy(anima_dit_block* blk) {
  return guarded([&] { delete blk; });
}

anima_status anima_dit_block_encode(anima_dit_block* blk, const anima_dit_block_weights* w,
                                    const anima_dit_block_args* args) {
  return guarded([&] { require(blk, "block")->impl.encode(*require(w, "block weights"), *require(args, "block args")); });
}

anima_status anima_dit_block_encode_cached(anima_dit_block* blk, const anima_dit_block_weights* w,
                                           const anima_dit_block_args* args, anima_cross_kv_cache* cache,
                                           int64_t block_index) {
  return guarded([&] {
    require(blk, "block")->impl.encode(*require(w, "block weights"), *require(args, "block args"),
                                       cache ? &cache->impl : nullptr, block_index);
  });
}

anima_status anima_dit_forward_encode(anima_dit_block* blk, const anima_dit_block_weights* blocks,
                                      int64_t block_count, const anima_dit_block_args* args,
                                      anima_cross_kv_cache* cache) {
  return guarded([&] {
    require(blk, "block")->impl.forward(blocks, block_count, *require(args, "block args"),
                                        cache ? &cache->impl : nullptr);
  });
}

anima_status anima_dit_forward_encode_streamed(anima_dit_block* blk, anima_weight_streamer* streamer,
                                               const anima_dit_block_weights* templates,
                                               const void* const* host_ranges, const int64_t* range_bytes,
                                               int64_t block_count, const anima_dit_block_args* args,
                                               anima_cross_kv_cache* cache) {
  return guarded([&] {
    require(blk, "block")->impl.forward_streamed(require(streamer, "weight streamer")->impl, templates, host_ranges,
                                                 range_bytes, block_count, *require(args, "block args"),
                                                 cache ? &cache->impl : nullptr);
  });
}

// ---------------------------------------------------------------- cross K/V cache, weight streamer
anima_status anima_cross_kv_cache_create(anima_ctx* ctx, int64_t blocks, int64_t context_tokens, int64_t dim,
                                         anima_cross_kv_cache** out) {
  return guarded([&] {
    require(out, "cache output");
    *out = nullptr;
    require(ctx, "context");
    if (!(blocks > 0 && context_tokens > 0 && dim > 0)) fail(ANIMA_E_INVALID_SHAPE, "invalid cross K/V cache shape");
    *out = new anima_cross_kv_cache(ctx, blocks, context_tokens, dim);
  });
}

anima_status anima_cross_kv_cache_destroy(anima_cross_kv_cache* cache) {
  return guarded([&] { delete cache; });
}

anima_status anima_cross_kv_cache_reset(anima_cross_kv_cache* cache) {
  return guarded([&] { require(cache, "cross K/V cache")->impl.reset(); });
}

anima_status anima_cross_kv_cache_is_ready(const anima_cross_kv_cache* cache, int64_t block, int32_t* ready) {
  return guarded([&] {
    const CrossKVCache& c = require(cache, "cross K/V cache")->impl;
    if (block < 0 || block >= c.blocks()) fail(ANIMA_E_INVALID_ARGUMENT, "cross K/V cache block index out of range");
    *require(ready, "output") = c.ready(block) ? 1 : 0;
  });
}

anima_status anima_cross_kv_cache_bytes(const anima_cross_kv_cache* cache, int64_t* bytes) {
  return guarded([&] { *require(bytes, "output") = require(cache, "cross K/V cache")->impl.bytes(); });
}

anima_status anima_weight_streamer_create(anima_ctx* ctx, int64_t capacity, int32_t slots,
                                          anima_weight_streamer** out) {
  return guarded([&] {
    require(out, "streamer output");
    *out = nullptr;
    require(ctx, "context");
    if (capacity <= 0) fail(ANIMA_E_INVALID_SHAPE, "weight ring capacity must be positive");
    if (slots < 1 || slots > 4) fail(ANIMA_E_INVALID_ARGUMENT, "weight slot count must be in 1...4");
    *out = new anima_weight_streamer(ctx, capacity, slots);
  });
}

anima_status anima_weight_streamer_destroy(anima_weight_streamer* streamer) {
  return guarded([&] { delete streamer; });
}

// ---------------------------------------------------------------- DiT input / output and sampler

static void check_sampler(const anima_buffer& b, int64_t count, const char* message) {
  if (!b.ptr) fail(ANIMA_E_INVALID_ARGUMENT, message);
  if (checked_product({count, 4}, "sampler") > b.length) fail(ANIMA_E_OUT_OF_BOUNDS, message);
}

static int64_t latent_floats(int64_t channels, int64_t height, int64_t width, const char* who) {
  (void)patch_tokens(height, width, who);
  return checked_product({channels, height, width}, who);
}

anima_status anima_patchify17_encode(anima_ctx* ctx, anima_buffer input, int64_t channels, int64_t height,
                                     int64_t width, anima_buffer tokens) {
  return guarded([&] {
    require(ctx, "context");
    if (channels != 16 && channels != 17) fail(ANIMA_E_INVALID_SHAPE, "patchify17 reads 16 or 17 channels");
    const int64_t n = latent_floats(channels, height, width, "patchify17");
    check_elementwise(input, n, 4, "patchify17 input");
    check_elementwise(tokens, checked_product({height / 2, width / 2, 68}, "patchify17"), 4, "patchify17 tokens");
    DeviceGuard g(ctx);
    launch_patchify17(static_cast<const float*>(input.ptr), (int)channels, height, width,
                      static_cast<float*>(tokens.ptr), ctx->stream);
  });
}

anima_status anima_unpatchify16_encode(anima_ctx* ctx, anima_buffer tokens, int64_t height, int64_t width,
                                       anima_buffer output) {
  return guarded([&] {
    require(ctx, "context");
    const int64_t n = latent_floats(16, height, width, "unpatchify16");
    check_elementwise(tokens, checked_product({height / 2, width / 2, 68}, "unpatchify16"), 4, "unpatchify16 tokens");
    check_elementwise(output, n, 4, "unpatchify16 output");
    DeviceGuard g(ctx);
    launch_unpatchify16(static_cast<const float*>(tokens.ptr), height, width, static_cast<float*>(output.ptr),
                        ctx->stream);
  });
}

anima_status anima_unpatchify_velocity16_encode(anima_ctx* ctx, anima_buffer tokens, int64_t height, int64_t width,
                                                anima_buffer output) {
  return guarded([&] {
    require(ctx, "context");
    const int64_t n = latent_floats(16, height, width, "unpatchify_velocity16");
    check_elementwise(tokens, n, 4, "unpatchify_velocity16 tokens");  // [T, 64] holds 16*H*W values
    check_elementwise(output, n, 4, "unpatchify_velocity16 output");
    DeviceGuard g(ctx);
    launch_unpatchify_velocity16(static_cast<const float*>(tokens.ptr), height, width,
                                 static_cast<float*>(output.ptr), ctx->stream);
  });
}

anima_status anima_flow_velocity_to_denoised_encode(anima_ctx* ctx, anima_buffer x, anima_buffer velocity,
                                                    anima_buffer denoised, float sigma, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    const char* msg = "invalid FLOW conversion input";
    if (count <= 0 || !std::isfinite(sigma)) fail(ANIMA_E_INVALID_ARGUMENT, msg);
    check_sampler(x, count, msg);
    check_sampler(velocity, count, msg);
    check_sampler(denoised, count, msg);
    DeviceGuard g(ctx);
    launch_flow_denoised(static_cast<const float*>(x.ptr), static_cast<const float*>(velocity.ptr),
                         static_cast<float*>(denoised.ptr), sigma, count, ctx->stream);
  });
}

anima_status anima_euler_step_encode(anima_ctx* ctx, anima_buffer x, anima_buffer denoised, anima_buffer x_next,
                                     float sigma, float next_sigma, int64_t count) {
  return guarded([&] {
    require(ctx, "context");
    const char* msg = "invalid Euler sampler buffer or sigma";
    if (count <= 0 || !std::isfinite(sigma) || !(sigma > 0.f) || !std::isfinite(next_sigma))
      fail(ANIMA_E_INVALID_ARGUMENT, msg);
    check_sampler(x, count, msg);
    check_sampler(denoised, count, msg);
    check_sampler(x_next, count, msg);
    DeviceGuard g(ctx);
    launch_euler_step(static_cast<const float*>(x.ptr), static_cast<const float*>(denoised.ptr),
                      static_cast<float*>(x_next.ptr), sigma, next_sigma, count, ctx->stream);
  });
}

anima_status anima_dit_prepare_create(anima_ctx* ctx, anima_dit_prepare** out) {
  return guarded([&] {
    require(out, "DiT preparation output");
    *out = nullptr;
    *out = new anima_dit_prepare(require(ctx, "context"));
  });
}

anima_status anima_dit_prepare_destroy(anima_dit_prepare* prep) {
  return guarded([&] { delete prep; });
}

anima_status anima_dit_prepare_encode(anima_dit_prepare* prep, const anima_dit_prepare_weights* w,
                                      const anima_dit_prepare_args* args) {
  return guarded([&] {
    require(prep, "DiT preparation")->impl.encode(*require(w, "DiT preparation weights"),
                                                  *require(args, "DiT preparation args"));
  });
}

anima_status anima_dit_final_create(anima_ctx* ctx, anima_dit_final** out) {
  return guarded([&] {
    require(out, "DiT final-layer output");
    *out = nullptr;
    *out = new anima_dit_final(require(ctx, "context"));
  });
}

anima_status anima_dit_final_destroy(anima_dit_final* fin) {
  return guarded([&] { delete fin; });
}

anima_status anima_dit_final_encode(anima_dit_final* fin, const anima_dit_final_weights* w,
                                    const anima_dit_final_args* args) {
  return guarded([&] {
    require(fin, "DiT final layer")->impl.encode(*require(w, "DiT final-layer weights"),
                                                 *require(args, "DiT final-layer args"));
  });
}

}  // extern "C"
