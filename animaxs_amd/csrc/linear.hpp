// LinearExecutor for gfx950 (AnimaXS/Runtime/Metal/LinearExecutor.swift:43-459).
#pragma once

#include "context.hpp"

namespace anima {

struct GemmParams {
  const half_t* x;        // [M, K] row-major fp16
  half_t* y;              // [M, N] row-major fp16
  const uint8_t* w;       // packed [N, row_stride] (bytes; halfs for FP16 storage)
  const half_t* scale;    // [N, groups]
  const half_t* zero;     // [N, groups]
  int64_t row_stride;     // bytes (W4/W8) or halfs (FP16)
  int M, N, K, groups;
  // Output stage (ping-pong kernel only; the others require GEMM_STORE):
  //   GEMM_STORE     y = half(acc)
  //   GEMM_GELU      y = half(gelu_erf(half(acc)))   (dit_gelu_half_inplace fused)
  //   GEMM_GATE_ADD  residual[m, n] += float(half(acc)) * gate[n]; y is not written
  //                  (gate_add_half_f32 fused)
  //   GEMM_RESIDUAL_ADD  residual[m, n] += float(half(acc)); y is not written
  //                  (add_half_into_float fused)
  //   GEMM_QK_NORM   y = half(the per-head (128 columns) RMSNorm of half(acc) times
  //                  norm_w): the attention's Q/K RMSNorm prologue fused, for projections
  //                  without RoPE (the RoPE'd form, with a table row per token, cost more
  //                  in the output stage than the prologue kernel it replaced)
  int epilogue;
  float* residual;        // [M, N] fp32, GEMM_GATE_ADD / GEMM_RESIDUAL_ADD
  const float* gate;      // [N] fp32, GEMM_GATE_ADD
  // Split K (ping-pong kernel, GEMM_STORE or GEMM_RESIDUAL_ADD, single problem): ksplit workgroups per
  // tile each sum K / ksplit and write fp32 rows to part [ksplit][M][N]; a second
  // kernel adds them in split order and rounds once.
  int ksplit;
  float* part;
  const half_t* norm_w;   // [128] fp16, GEMM_QK_NORM
  float eps;
};

enum GemmEpilogue { GEMM_STORE = 0, GEMM_GELU = 1, GEMM_GATE_ADD = 2, GEMM_RESIDUAL_ADD = 3, GEMM_QK_NORM = 4 };

// Output stage of one member of a grouped linear (GEMM_STORE or GEMM_QK_NORM).
struct GemmEpilogueArgs {
  int epilogue;
  const half_t* norm_w;
  float eps;
};

// Up to PG_GROUP independent GEMMs of one K and storage in one ping-pong launch
// (the Q/K/V projections of one input): logical tiles [first_tile[i],
// first_tile[i+1]) compute problem i.
constexpr int PG_GROUP = 3;
struct GemmGroup {
  GemmParams p[PG_GROUP];
  int first_tile[PG_GROUP];
  int vec[PG_GROUP];      // 16-byte output accesses allowed
  int count;
};

struct MatvecParams {
  const uint8_t* w;
  const half_t* scale;
  const half_t* zero;
  int64_t row_stride;
  const float* x;
  float* y;
  int N, K, groups, storage;
  int silu_input;         // use x / (1 + exp(-x)) in place of x (silu kernel fused)
  const float* bias;      // optional [N]: y = sum + bias (add_f32 fused)
};

// Up to CAP independent matvecs in one launch; blocks [first_block[i],
// first_block[i+1]) compute matvec i.
template <int CAP>
struct MatvecBatchN {
  MatvecParams p[CAP];
  int first_block[CAP];
  int count;
};
constexpr int MV_BATCH = 3;
using MatvecBatch = MatvecBatchN<MV_BATCH>;
// Wide batches (about 2 KB of kernel arguments): the modulation matvecs of up to 8 DiT
// blocks, 3 branches each, in one launch.
constexpr int MV_BATCH_WIDE = 24;

struct DequantParams {
  const uint8_t* w;
  const half_t* scale;
  const half_t* zero;
  int64_t row_stride;
  half_t* out;
  int64_t out_stride;
  int N, K, groups, storage;
};

// Exponent of the unit in the last place of an fp16 value, as a biased field (1..31).
__device__ __forceinline__ int fp16_unit_exponent(half_t v) {
  const int e = (__builtin_bit_cast(uint16_t, v) >> 10) & 31;
  return e < 1 ? 1 : e;
}

// True when q*s + z is exactly representable in fp32 for every code q < 2^QBITS.
// q*s is an integer of at most QBITS+11 bits times s's unit, z one of at most 11
// bits times its own unit; their sum spans at most 24 bits exactly when the unit
// exponents differ by d = u(s) - u(z) with -12 <= d <= 12 - QBITS (or when s or z
// is zero).
// Written without short-circuits so that it compiles to straight-line code.
template <int QBITS>
__device__ __forceinline__ bool one_rounding_exact(half_t s, half_t z) {
  const bool zero = ((__builtin_bit_cast(uint16_t, s) & 0x7fff) == 0) | ((__builtin_bit_cast(uint16_t, z) & 0x7fff) == 0);
  const int d = fp16_unit_exponent(s) - fp16_unit_exponent(z);
  return zero | ((d >= -12) & (d <= 12 - QBITS));
}

// Validated, resolved view of an anima_qweight.
struct QWeightView {
  int storage;
  const uint8_t* packed;
  const half_t* scale;
  const half_t* zero;
  int64_t rows, cols, row_stride, groups;
};

// LinearExecutor.validate (LinearExecutor.swift:412-438) for the weight part;
// input/output ranges are checked by the callers.
QWeightView validate_weight(const anima_qweight& w, const char* who);

void launch_gemm(const GemmParams& p, int storage, hipStream_t stream);

// Ping-pong W4/W8 GEMM (linear_pingpong.hip): K a multiple of 64, 16-byte aligned X
// and weight rows, buffers below 2 GiB.  launch_gemm routes to it when it applies.
bool pingpong_supported(const GemmParams& p, int storage);
void launch_pingpong(const GemmParams& p, int storage, hipStream_t stream);
// K splits the ping-pong kernel uses for this plain GEMM (1: none): when its tiles
// fill less than half the chip, as many splits of >= 16 K blocks as keep the grid
// within 256 workgroups (shorter splits lose more to the partial rows than they gain).
int pingpong_ksplit(const GemmParams& p, int storage);
// count (1..PG_GROUP) ping-pong GEMMs sharing K and storage in one launch.
void launch_pingpong_group(const GemmParams* ps, int count, int storage, hipStream_t stream);
// Whether a single launch of p runs the M-split form (256-row tiles, no K split between
// the wave groups); its sums differ from the K-split form's in the last place, so a
// grouped launch containing such a problem runs it on its own.
bool pingpong_msplit(const GemmParams& p, int storage);

// Weight-streaming GEMM for M <= SMALLM_MAX_ROWS (linear_smallm.hip); requires K a
// multiple of 128 and 16-byte aligned X and weight rows.
constexpr int SMALLM_MAX_ROWS = 64;
bool smallm_supported(const GemmParams& p, int storage);
void launch_smallm(const GemmParams& p, int storage, hipStream_t stream);
// Split-K form for W4/W8 (linear_smallm.hip): the number of K slices it runs this GEMM
// with (0: it does not apply).  With more than one slice the caller passes
// p.part = [slices][M][N] fp32 and p.ksplit = slices; launch_smallm_splitk adds the
// slices in order (launch_splitk_reduce) into p.y.
int smallm_splitk_slices(const GemmParams& p, int storage);
void launch_smallm_splitk(const GemmParams& p, int storage, hipStream_t stream);
// y[i] = half(sum_s part[s * count + i]) for i < count, slices added in order.
void launch_splitk_reduce(const float* part, half_t* y, int64_t count, int ksplit, hipStream_t stream);
void launch_matvec(const MatvecParams& p, hipStream_t stream);
// count (1..MV_BATCH) matvecs; one launch when they share storage and lane split.
void launch_matvec_batch(const MatvecParams* ps, int count, hipStream_t stream);
// Any count of matvecs: one launch per MV_BATCH_WIDE of them when all share storage and
// lane split, else launch_matvec_batch per MV_BATCH.  Same bits per matvec either way.
void launch_matvec_many(const MatvecParams* ps, int64_t count, hipStream_t stream);
void launch_dequant(const DequantParams& p, hipStream_t stream);
// Plain streaming read of `bytes` (a multiple of 16, 16-byte aligned); one 16-byte word per
// workgroup goes to sink (read_probe_sink_bytes(bytes) bytes).
int64_t read_probe_sink_bytes(int64_t bytes);
void launch_read_probe(const void* src, int64_t bytes, void* sink, hipStream_t stream);

class LinearExecutor {
 public:
  LinearExecutor(anima_ctx* ctx, const anima_linear_config& cfg);
  void encode(anima_buffer input, int64_t input_offset, const anima_qweight& weight, anima_buffer output,
              int64_t output_offset, int64_t input_rows, int32_t family);
  // encode() with a fused output stage (GEMM_GELU or GEMM_GATE_ADD, see GemmParams)
  // when the ping-pong kernel takes the shape under the automatic backend; returns
  // false, having encoded nothing, otherwise.  residual is [input_rows, weight.rows]
  // fp32 and gate [weight.rows] fp32, both ranges checked by the caller.
  bool encode_fused(anima_buffer input, int64_t input_offset, const anima_qweight& weight, anima_buffer output,
                    int64_t output_offset, int64_t input_rows, int32_t family, int epilogue, float* residual,
                    const float* gate);
  // count (1..PG_GROUP) linears of one input, each into its own output, as one
  // ping-pong launch when every one of them takes that kernel (same K and storage);
  // otherwise encode() for each in turn.
  // With epi (one per weight): the output stages run in the GEMM and encode_group
  // returns true; if the group cannot run as one ping-pong launch it encodes nothing
  // and returns false.  Without epi it always encodes and returns true.
  bool encode_group(anima_buffer input, const anima_qweight* const* weights, const anima_buffer* outputs, int count,
                    int64_t input_rows, int32_t family, const GemmEpilogueArgs* epi = nullptr);
  // encode() followed by the per-head RMSNorm of the output (rmsnorm_heads_half,
  // AnimaKernels.metal:660-689) over heads of head_dim columns with the fp16 weight
  // norm_w: in the ping-pong GEMM's output stage when it takes the shape and
  // head_dim is 128, else as a second, in-place pass.  norm_w's range is the
  // caller's to check.
  void encode_head_rmsnorm(anima_buffer input, int64_t input_offset, const anima_qweight& weight, anima_buffer output,
                           int64_t output_offset, int64_t input_rows, int32_t family, const half_t* norm_w,
                           int64_t head_dim, float eps);
  anima_ctx* context() const { return ctx_; }

 private:
  GemmParams prepare(anima_buffer input, int64_t input_offset, const QWeightView& w, anima_buffer output,
                     int64_t output_offset, int64_t input_rows) const;
  anima_ctx* ctx_;
  anima_linear_config cfg_;
  Workspace ws_;
};

void encode_matvec(anima_ctx* ctx, const anima_qweight& weight, anima_buffer input, int64_t input_offset,
                   anima_buffer output, int64_t output_offset);
void encode_dequant(anima_ctx* ctx, const anima_qweight& weight, anima_buffer output, int64_t output_offset,
                    int64_t out_row_stride);

}  // namespace anima

struct anima_linear {
  anima::LinearExecutor impl;
  anima_linear(anima_ctx* c, const anima_linear_config& cfg) : impl(c, cfg) {}
};
