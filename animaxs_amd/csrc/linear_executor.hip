// Host side of the linear executor: LinearExecutor.validate
// (AnimaXS/Runtime/Metal/LinearExecutor.swift:412-438) and dispatch.
#include <cmath>
#include <string>

#include "attention.hpp"
#include "linear.hpp"

namespace anima {

QWeightView validate_weight(const anima_qweight& w, const char* who) {
  const std::string name(who);
  if (w.storage != ANIMA_STORAGE_W4 && w.storage != ANIMA_STORAGE_W8 && w.storage != ANIMA_STORAGE_FP16)
    fail(ANIMA_E_UNSUPPORTED, name + " requires W4, W8, or FP16 weights");
  if (!(w.rows > 0 && w.columns > 0 && w.packed_offset >= 0 && w.scale_offset >= 0 && w.zero_offset >= 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid " + name + " shape or offset");
  const int64_t min_stride = w.storage == ANIMA_STORAGE_W4 ? (w.columns + 1) / 2 : w.columns;
  if (w.packed_row_stride < min_stride) fail(ANIMA_E_INVALID_SHAPE, "packed linear row stride is too small");
  if (w.rows > 0x7fffffff || w.columns > 0x7fffffff)
    fail(ANIMA_E_INVALID_SHAPE, name + " dimension exceeds int32");
  const int64_t elem = w.storage == ANIMA_STORAGE_FP16 ? 2 : 1;
  const int64_t packed_bytes = checked_product({w.rows, w.packed_row_stride, elem}, "LinearExecutor");
  const int64_t groups = (w.columns + 63) / 64;
  if (checked_end(w.packed_offset, packed_bytes, "LinearExecutor") > w.packed.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "LinearExecutor buffer range is out of bounds");
  if (!w.packed.ptr) fail(ANIMA_E_INVALID_ARGUMENT, name + " weight pointer is null");
  QWeightView v{};
  v.storage = w.storage;
  v.packed = reinterpret_cast<const uint8_t*>(byte_ptr(w.packed, w.packed_offset));
  v.rows = w.rows;
  v.cols = w.columns;
  v.row_stride = w.packed_row_stride;
  v.groups = groups;
  if (w.storage == ANIMA_STORAGE_FP16) {
    if (w.packed_offset & 1) fail(ANIMA_E_MISALIGNED, "FP16 weight offset must be 2-byte aligned");
    return v;
  }
  const int64_t param_bytes = checked_product({w.rows, groups, 2}, "LinearExecutor");
  if (checked_end(w.scale_offset, param_bytes, "LinearExecutor") > w.scale.length ||
      checked_end(w.zero_offset, param_bytes, "LinearExecutor") > w.zero.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "LinearExecutor buffer range is out of bounds");
  if (!w.scale.ptr || !w.zero.ptr) fail(ANIMA_E_INVALID_ARGUMENT, name + " scale/zero pointer is null");
  if ((w.scale_offset | w.zero_offset) & 1) fail(ANIMA_E_MISALIGNED, "scale/zero offsets must be 2-byte aligned");
  v.scale = reinterpret_cast<const half_t*>(byte_ptr(w.scale, w.scale_offset));
  v.zero = reinterpret_cast<const half_t*>(byte_ptr(w.zero, w.zero_offset));
  return v;
}

LinearExecutor::LinearExecutor(anima_ctx* ctx, const anima_linear_config& cfg) : ctx_(ctx), cfg_(cfg) {
  if (cfg.tile_rows <= 0) fail(ANIMA_E_INVALID_ARGUMENT, "linear tile rows must be positive");
  if (cfg.backend < ANIMA_LINEAR_BACKEND_AUTO || cfg.backend > ANIMA_LINEAR_BACKEND_DEQUANT_THEN_GEMM)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear backend");
}

GemmParams LinearExecutor::prepare(anima_buffer input, int64_t input_offset, const QWeightView& w,
                                   anima_buffer output, int64_t output_offset, int64_t input_rows) const {
  if (!(input_rows > 0 && input_offset >= 0 && output_offset >= 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid LinearExecutor shape or offset");
  const int64_t in_bytes = checked_product({input_rows, w.cols, 2}, "LinearExecutor");
  const int64_t out_bytes = checked_product({input_rows, w.rows, 2}, "LinearExecutor");
  if (checked_end(input_offset, in_bytes, "LinearExecutor") > input.length ||
      checked_end(output_offset, out_bytes, "LinearExecutor") > output.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "LinearExecutor buffer range is out of bounds");
  if (!input.ptr || !output.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "LinearExecutor buffer pointer is null");
  if ((input_offset | output_offset) & 1) fail(ANIMA_E_MISALIGNED, "LinearExecutor offsets must be 2-byte aligned");
  if (input_rows > 0x7fffffff) fail(ANIMA_E_INVALID_SHAPE, "LinearExecutor input rows exceed int32");
  GemmParams p{};
  p.x = reinterpret_cast<const half_t*>(byte_ptr(input, input_offset));
  p.y = reinterpret_cast<half_t*>(byte_ptr_mut(output, output_offset));
  p.M = (int)input_rows;
  p.N = (int)w.rows;
  p.K = (int)w.cols;
  p.groups = (int)w.groups;
  p.w = w.packed;
  p.scale = w.scale;
  p.zero = w.zero;
  p.row_stride = w.row_stride;
  return p;
}

void LinearExecutor::encode(anima_buffer input, int64_t input_offset, const anima_qweight& weight,
                            anima_buffer output, int64_t output_offset, int64_t input_rows, int32_t family) {
  if (family < ANIMA_FAMILY_OTHER || family > ANIMA_FAMILY_MLP_DOWN)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear family");
  if (!(input_rows > 0 && input_offset >= 0 && output_offset >= 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid LinearExecutor shape or offset");
  const QWeightView w = validate_weight(weight, "LinearExecutor");
  GemmParams p = prepare(input, input_offset, w, output, output_offset, input_rows);

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  if (cfg_.backend == ANIMA_LINEAR_BACKEND_DEQUANT_THEN_GEMM && w.storage != ANIMA_STORAGE_FP16) {
    // Reference default shape: dequantise the whole weight once into fp16
    // scratch (LinearExecutor.swift:146-193), then the fp16 GEMM.
    const int64_t stride = (w.cols + 7) / 8 * 8;
    half_t* scratch = static_cast<half_t*>(ws_.get(checked_product({w.rows, stride, 2}, "LinearExecutor"), stream));
    DequantParams dp{};
    dp.w = w.packed; dp.scale = w.scale; dp.zero = w.zero; dp.row_stride = w.row_stride;
    dp.out = scratch; dp.out_stride = stride; dp.N = (int)w.rows; dp.K = (int)w.cols;
    dp.groups = (int)w.groups; dp.storage = w.storage;
    launch_dequant(dp, stream);
    p.w = reinterpret_cast<const uint8_t*>(scratch);
    p.scale = nullptr;
    p.zero = nullptr;
    p.row_stride = stride;
    launch_gemm(p, ANIMA_STORAGE_FP16, stream);
    return;
  }
  const int slices = cfg_.backend == ANIMA_LINEAR_BACKEND_AUTO ? smallm_splitk_slices(p, w.storage) : 0;
  if (slices > 0) {
    p.ksplit = slices;
    if (slices > 1)
      p.part = static_cast<float*>(ws_.get(checked_product({(int64_t)slices, p.M, p.N, 4}, "LinearExecutor"), stream));
    launch_smallm_splitk(p, w.storage, stream);
    return;
  }
  if (smallm_supported(p, w.storage)) {
    launch_smallm(p, w.storage, stream);
    return;
  }
  const int ks = pingpong_ksplit(p, w.storage);
  if (ks > 1) {
    p.ksplit = ks;
    p.part = static_cast<float*>(ws_.get(checked_product({(int64_t)ks, p.M, p.N, 4}, "LinearExecutor"), stream));
  }
  launch_gemm(p, w.storage, stream);
}

bool LinearExecutor::encode_group(anima_buffer input, const anima_qweight* const* weights, const anima_buffer* outputs,
                                  int count, int64_t input_rows, int32_t family, const GemmEpilogueArgs* epi) {
  if (count < 1 || count > PG_GROUP) fail(ANIMA_E_INVALID_ARGUMENT, "linear group holds 1 to 3 weights");
  if (family < ANIMA_FAMILY_OTHER || family > ANIMA_FAMILY_MLP_DOWN)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear family");
  if (!(input_rows > 0)) fail(ANIMA_E_INVALID_SHAPE, "invalid LinearExecutor shape or offset");
  GemmParams ps[PG_GROUP];
  int storage = -1;
  bool together = cfg_.backend == ANIMA_LINEAR_BACKEND_AUTO;
  for (int i = 0; i < count; ++i) {
    const QWeightView w = validate_weight(*weights[i], "LinearExecutor");
    ps[i] = prepare(input, 0, w, outputs[i], 0, input_rows);
    // A weight encode() would split over K runs on its own, and so does, in a group of two
    // or more, one encode() would run in the M-split form (a single launch takes that form
    // itself), so the bits match encode().
    together = together && !smallm_supported(ps[i], w.storage) && pingpong_supported(ps[i], w.storage) &&
               pingpong_ksplit(ps[i], w.storage) == 1 && (count == 1 || !pingpong_msplit(ps[i], w.storage)) &&
               (i == 0 || (w.storage == storage && ps[i].K == ps[0].K));
    storage = w.storage;
  }
  if (epi) {
    for (int i = 0; i < count; ++i) {
      if (epi[i].epilogue != GEMM_STORE && epi[i].epilogue != GEMM_QK_NORM)
        fail(ANIMA_E_INVALID_ARGUMENT, "grouped linears take plain or Q/K-norm output stages");
      if (epi[i].epilogue == GEMM_QK_NORM) {
        together = together && epi[i].norm_w && aligned16(epi[i].norm_w) && ps[i].N % 128 == 0;
        ps[i].epilogue = GEMM_QK_NORM;
        ps[i].norm_w = epi[i].norm_w;
        ps[i].eps = epi[i].eps;
      }
    }
    if (!together) return false;
  }
  if (!together) {
    for (int i = 0; i < count; ++i) encode(input, 0, *weights[i], outputs[i], 0, input_rows, family);
    return true;
  }
  DeviceGuard guard(ctx_);
  launch_pingpong_group(ps, count, storage, ctx_->stream);
  return true;
}

bool LinearExecutor::encode_fused(anima_buffer input, int64_t input_offset, const anima_qweight& weight,
                                  anima_buffer output, int64_t output_offset, int64_t input_rows, int32_t family,
                                  int epilogue, float* residual, const float* gate) {
  if (family < ANIMA_FAMILY_OTHER || family > ANIMA_FAMILY_MLP_DOWN)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear family");
  if (epilogue != GEMM_GELU && epilogue != GEMM_GATE_ADD && epilogue != GEMM_RESIDUAL_ADD)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown linear epilogue");
  if (!(input_rows > 0 && input_offset >= 0 && output_offset >= 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid LinearExecutor shape or offset");
  const QWeightView w = validate_weight(weight, "LinearExecutor");
  GemmParams p = prepare(input, input_offset, w, output, output_offset, input_rows);
  if (cfg_.backend != ANIMA_LINEAR_BACKEND_AUTO || smallm_supported(p, w.storage) || !pingpong_supported(p, w.storage))
    return false;
  // The split decision is the one encode() makes, so the bits match encode() + the step.
  const int ks = pingpong_ksplit(p, w.storage);
  if (ks > 1 && epilogue != GEMM_RESIDUAL_ADD) return false;
  p.epilogue = epilogue;
  p.residual = residual;
  p.gate = gate;
  DeviceGuard guard(ctx_);
  if (ks > 1) {
    p.ksplit = ks;
    p.part = static_cast<float*>(ws_.get(checked_product({(int64_t)ks, p.M, p.N, 4}, "LinearExecutor"), ctx_->stream));
  }
  launch_pingpong(p, w.storage, ctx_->stream);
  return true;
}

void LinearExecutor::encode_head_rmsnorm(anima_buffer input, int64_t input_offset, const anima_qweight& weight,
                                         anima_buffer output, int64_t output_offset, int64_t input_rows,
                                         int32_t family, const half_t* norm_w, int64_t head_dim, float eps) {
  if (!(head_dim > 0 && weight.rows > 0 && weight.rows % head_dim == 0))
    fail(ANIMA_E_INVALID_SHAPE, "per-head RMSNorm requires weight rows to be a multiple of head_dim");
  if (head_dim > 512) fail(ANIMA_E_UNSUPPORTED, "per-head RMSNorm supports head_dim <= 512");
  if (!(eps >= 0.f && std::isfinite(eps))) fail(ANIMA_E_INVALID_ARGUMENT, "RMSNorm epsilon must be finite and >= 0");
  if (!norm_w) fail(ANIMA_E_INVALID_ARGUMENT, "per-head RMSNorm weight pointer is null");
  if (head_dim == 128 && input_offset == 0 && output_offset == 0) {
    const anima_qweight* ws1[1] = {&weight};
    const GemmEpilogueArgs epi[1] = {{GEMM_QK_NORM, norm_w, eps}};
    if (encode_group(input, ws1, &output, 1, input_rows, family, epi)) return;
  }
  encode(input, input_offset, weight, output, output_offset, input_rows, family);
  // In place on the [rows, weight.rows] output just written (ranges checked by encode()):
  // every element is read and rewritten by the same lane.
  DeviceGuard guard(ctx_);
  PrologueParams pp{};
  half_t* y = reinterpret_cast<half_t*>(byte_ptr_mut(output, output_offset));
  pp.in = y; pp.in_tok = weight.rows; pp.in_head = head_dim; pp.in_batch = input_rows * weight.rows;
  pp.out = y; pp.out_tok = weight.rows; pp.out_head = head_dim; pp.out_batch = input_rows * weight.rows;
  pp.batch = 1; pp.rows = (int)input_rows; pp.heads = (int)(weight.rows / head_dim); pp.D = (int)head_dim;
  pp.norm_w = norm_w; pp.eps = eps; pp.rope = nullptr;
  launch_prologue(pp, ctx_->stream);
}

void encode_matvec(anima_ctx* ctx, const anima_qweight& weight, anima_buffer input, int64_t input_offset,
                   anima_buffer output, int64_t output_offset) {
  const QWeightView w = validate_weight(weight, "matvec");
  if (!(input_offset >= 0 && output_offset >= 0)) fail(ANIMA_E_INVALID_SHAPE, "invalid matvec shape or offset");
  if (checked_end(input_offset, checked_product({w.cols, 4}, "matvec"), "matvec") > input.length ||
      checked_end(output_offset, checked_product({w.rows, 4}, "matvec"), "matvec") > output.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "matvec buffer range is out of bounds");
  if (!input.ptr || !output.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "matvec buffer pointer is null");
  if ((input_offset | output_offset) & 3) fail(ANIMA_E_MISALIGNED, "matvec offsets must be 4-byte aligned");
  DeviceGuard guard(ctx);
  MatvecParams p{};
  p.w = w.packed; p.scale = w.scale; p.zero = w.zero; p.row_stride = w.row_stride;
  p.x = reinterpret_cast<const float*>(byte_ptr(input, input_offset));
  p.y = reinterpret_cast<float*>(byte_ptr_mut(output, output_offset));
  p.N = (int)w.rows; p.K = (int)w.cols; p.groups = (int)w.groups; p.storage = w.storage;
  launch_matvec(p, ctx->stream);
}

void encode_dequant(anima_ctx* ctx, const anima_qweight& weight, anima_buffer output, int64_t output_offset,
                    int64_t out_row_stride) {
  const QWeightView w = validate_weight(weight, "dequant");
  if (!(output_offset >= 0 && out_row_stride >= w.cols))
    fail(ANIMA_E_INVALID_SHAPE, "invalid dequant output stride or offset");
  const int64_t out_bytes =
      checked_product({w.rows - 1, out_row_stride, 2}, "dequant") + checked_product({w.cols, 2}, "dequant");
  if (checked_end(output_offset, out_bytes, "dequant") > output.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "dequant buffer range is out of bounds");
  if (!output.ptr) fail(ANIMA_E_INVALID_ARGUMENT, "dequant buffer pointer is null");
  if (output_offset & 1) fail(ANIMA_E_MISALIGNED, "dequant output offset must be 2-byte aligned");
  DeviceGuard guard(ctx);
  DequantParams p{};
  p.w = w.packed; p.scale = w.scale; p.zero = w.zero; p.row_stride = w.row_stride;
  p.out = reinterpret_cast<half_t*>(byte_ptr_mut(output, output_offset));
  p.out_stride = out_row_stride;
  p.N = (int)w.rows; p.K = (int)w.cols; p.groups = (int)w.groups; p.storage = w.storage;
  launch_dequant(p, ctx->stream);
}

}  // namespace anima
