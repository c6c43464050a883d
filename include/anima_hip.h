/*
 * anima_hip.h — C ABI of libanima_hip, the MI355X (gfx950) attention and
 * quantized-linear hot path of AnimaXS.
 *
 * The ABI replaces the reference's Swift/Metal operator executors:
 *   AttentionExecutor   AnimaXS/Runtime/Metal/AttentionExecutor.swift:77-848
 *   LinearExecutor      AnimaXS/Runtime/Metal/LinearExecutor.swift:43-459
 *   QuantDecoders       AnimaXS/Runtime/Animapk/QuantDecoders.swift:17-164
 * plus the DiT-block support kernels of AnimaXS/Shaders/AnimaKernels.metal that
 * DiTBlockExecutor (AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:1035-1319) encodes
 * around them.
 *
 * Conventions (mirroring the reference):
 *   - A Metal buffer + byte offset becomes an anima_buffer {device pointer, byte
 *     length} + byte offset; every range is validated against the length before
 *     anything is launched (AttentionExecutor.validate, LinearExecutor.validate).
 *   - *_encode appends work to the context's HIP stream (the analog of encoding
 *     into a caller-owned MTLCommandBuffer); *_execute = encode + stream
 *     synchronize (the async execute of the reference).
 *   - Executors own their scratch workspaces and are NOT re-entrant
 *     (AttentionExecutor.swift:70): one caller at a time per executor.
 *   - Failures return a non-zero anima_status; anima_last_error() returns the
 *     thread-local message.  Nothing silently falls back.
 *   - Plain C types only: no torch, no HIP types in signatures (streams are
 *     passed as void* holding a hipStream_t).
 */
#ifndef ANIMA_HIP_H
#define ANIMA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANIMA_HIP_ABI_VERSION 4

/* Status codes.  The reference throws AnimapkError.validation(String)
 * (Runtime/Animapk/MappedFile.swift:14) for every failure; the codes split that
 * one error by cause. */
typedef enum anima_status {
  ANIMA_OK = 0,
  ANIMA_E_INVALID_SHAPE = 1,   /* non-positive / inconsistent dimensions */
  ANIMA_E_OUT_OF_BOUNDS = 2,   /* a byte range exceeds its buffer */
  ANIMA_E_OVERFLOW = 3,        /* a size product or range end overflows int64 */
  ANIMA_E_MISALIGNED = 4,      /* offsets / strides violate the alignment contract */
  ANIMA_E_UNSUPPORTED = 5,     /* valid request this backend refuses (loudly) */
  ANIMA_E_DEVICE = 6,          /* HIP runtime error */
  ANIMA_E_INVALID_ARGUMENT = 7, /* null handle / unknown enum value */
  ANIMA_E_FORMAT = 8,          /* a .animapk header, JSON or layout violates ANMA v1 */
  ANIMA_E_IO = 9               /* a file could not be opened or mapped */
} anima_status;

/* Thread-local message of the last failure on this thread ("" after success). */
const char* anima_last_error(void);
/* ABI version (ANIMA_HIP_ABI_VERSION of the built library). */
int32_t anima_abi_version(void);

/* ------------------------------------------------------------------------- */
/* Device buffers: MTLBuffer analog.                                          */
/* ------------------------------------------------------------------------- */
typedef struct anima_buffer {
  void* ptr;        /* device pointer (hipMalloc'ed or any device-visible pointer) */
  int64_t length;   /* bytes addressable from ptr */
} anima_buffer;

/* ------------------------------------------------------------------------- */
/* Context: MetalContext analog (Runtime/Metal/MetalContext.swift:14-81).     */
/* ------------------------------------------------------------------------- */
typedef struct anima_ctx anima_ctx;

/* MetalContext.init (MetalContext.swift:24-42): binds HIP device `device`; the
 * context starts on the device's null stream. */
anima_status anima_ctx_create(int32_t device, anima_ctx** out);
anima_status anima_ctx_destroy(anima_ctx* ctx);
/* Replace the stream all *_encode calls append to (the command buffer analog). */
anima_status anima_ctx_set_stream(anima_ctx* ctx, void* hip_stream);
/* Wait for all work encoded on the context stream (command buffer completion). */
anima_status anima_ctx_synchronize(anima_ctx* ctx);

/* ------------------------------------------------------------------------- */
/* Attention: AttentionExecutor (AttentionExecutor.swift:77-848).              */
/* ------------------------------------------------------------------------- */

/* AttentionInputLayout (AttentionExecutor.swift:55-64). */
typedef enum anima_layout {
  ANIMA_LAYOUT_HEAD_MAJOR = 0,  /* [batch][heads][rows][head_dim], tight */
  ANIMA_LAYOUT_TOKEN_MAJOR = 1  /* [batch][rows][token_stride]; head h at columns h*head_dim */
} anima_layout;

/* AttentionNumerics (AttentionExecutor.swift:5-12).  As in the reference, what
 * LEGACY means depends on the backend.  The reference's metalFlash and
 * streamingMPS backends keep fp32 scores and softmax state under legacy numerics
 * (:179-203), and so do AUTO, FLASH and GENERIC here (the flash kernels round P
 * to fp16 for the PV product on the matrix cores).  Its MPS score-tile backends
 * round the scaled scores and the normalised probabilities to fp16 between
 * passes (:221-301, 412-496); ANIMA_ATTENTION_BACKEND_LEGACY_MPS keeps those
 * rounding points.  FP32_SCORES selects fp32 scores on every backend (the
 * reference's encodeFP32 ignores the backend).  BF16_COMPUTE is refused with
 * ANIMA_E_UNSUPPORTED. */
typedef enum anima_attention_numerics {
  ANIMA_NUMERICS_LEGACY = 0,
  ANIMA_NUMERICS_FP32_SCORES = 1,
  ANIMA_NUMERICS_BF16_COMPUTE = 2
} anima_attention_numerics;

/* DiTAttentionBackend (AttentionExecutor.swift:29-44) re-cut for MI355X:
 * AUTO picks the MFMA flash kernel when its contract holds (head_dim 64/128/384,
 * 16-byte aligned rows) and the generic fp32 kernel otherwise; FLASH demands the
 * MFMA kernel and fails loudly when the shape is outside it (the metalFlash gate,
 * :685-705); GENERIC forces the generic kernel (the fp32 diagnostic path);
 * LEGACY_MPS is the legacyHeadMajorMPS / stridedTokenMajorMPS pair: under LEGACY
 * numerics it stores fp16 scaled scores and fp16 normalised probabilities, as
 * the MPS passes and attention_softmax_rows (AnimaKernels.metal:1051-1100) do
 * (one workgroup per query row, a compatibility path, not a fast one); under
 * FP32_SCORES it runs the generic kernel. */
typedef enum anima_attention_backend {
  ANIMA_ATTENTION_BACKEND_AUTO = 0,
  ANIMA_ATTENTION_BACKEND_FLASH = 1,
  ANIMA_ATTENTION_BACKEND_GENERIC = 2,
  ANIMA_ATTENTION_BACKEND_LEGACY_MPS = 3
} anima_attention_backend;

/* AttentionExecutor.init (AttentionExecutor.swift:97-110). */
typedef struct anima_attention_config {
  int32_t tile_rows;      /* query rows per tile; > 0 (reference default 128) */
  int32_t numerics;       /* anima_attention_numerics */
  int32_t backend;        /* anima_attention_backend */
  int32_t layout;         /* anima_layout default of encode() */
  int64_t token_stride;   /* half elements per token row for TOKEN_MAJOR */
  int32_t flash_rows;     /* query rows per flash workgroup: 0 = auto (256 whenever 64 key
                             rows span < 2 GiB, else 128), 128 or 256 */
} anima_attention_config;

typedef struct anima_attention anima_attention;

anima_status anima_attention_create(anima_ctx* ctx, const anima_attention_config* cfg,
                                    anima_attention** out);
anima_status anima_attention_destroy(anima_attention* attn);

/* Fused per-head Q/K prologue: RMSNorm with a shared [head_dim] fp16 weight
 * (rmsnorm_heads_half, AnimaKernels.metal:660-689) and/or split-half RoPE on the
 * pairs (p, p+head_dim/2) from an fp32 [tokens][head_dim/2][2][2] table of
 * [cos,-sin,sin,cos] blocks (rms_rope_split_half, AnimaKernels.metal:696-729;
 * rms_rope_adapter64, :733-763).  Each table or weight is a device buffer whose
 * length is checked before launch; a NULL ptr disables that step.  Query row r
 * uses row r of `rope`; key row r uses row r of `k_rope` when its ptr is set (the
 * LLM adapter's cross attention rotates its context keys with the context's own
 * positions, LLMAdapterMetal.swift:336-340, 383-397), else row r of `rope`. */
typedef struct anima_qk_prologue {
  anima_buffer q_norm_weight;  /* fp16 [head_dim] (ptr NULL: no Q RMSNorm) */
  anima_buffer k_norm_weight;  /* fp16 [head_dim] (ptr NULL: no K RMSNorm) */
  float eps;                   /* RMSNorm epsilon (DiT and Qwen use 1e-6) */
  anima_buffer rope;           /* fp32 [rope_tokens][head_dim/2][2][2] (ptr NULL: no RoPE) */
  int64_t rope_tokens;         /* rows of `rope` (>= query_count, and >= key_count when it serves K) */
  int32_t rope_q;              /* apply RoPE to Q (1) */
  int32_t rope_k;              /* apply RoPE to K (1) */
  anima_buffer k_rope;         /* optional fp32 [k_rope_tokens][head_dim/2][2][2] for K */
  int64_t k_rope_tokens;       /* rows of `k_rope` (>= key_count) */
} anima_qk_prologue;

/* AttentionExecutor.encode (AttentionExecutor.swift:122-133).  The first block of
 * fields is exactly the reference's parameter list; the rest are extensions whose
 * zero values reproduce the reference behaviour (batch 1, no key mask, scale
 * 1/sqrt(head_dim), no prologue). */
typedef struct anima_attention_args {
  anima_buffer query;  int64_t query_offset;
  anima_buffer key;    int64_t key_offset;
  anima_buffer value;  int64_t value_offset;
  anima_buffer output; int64_t output_offset;
  int64_t heads;
  int64_t query_count;
  int64_t key_count;
  int64_t head_dim;
  int64_t key_value_heads;     /* 0 -> heads; GQA map kv = h / (heads/key_value_heads) */
  int32_t causal;              /* requires query_count == key_count */
  int32_t layout;              /* -1 -> executor default, else anima_layout */
  int64_t token_stride;        /* TOKEN_MAJOR row stride in halfs (0 -> executor default) */
  /* --- extensions --- */
  int64_t batch;               /* 0 or 1 -> single sequence; batches are contiguous */
  const int32_t* key_lengths;  /* per-batch valid key count or NULL (all keys) */
  int32_t key_lengths_on_device; /* 0: host array, validated 1..key_count; 1: device
                                    array, clamped to [1, key_count] by the kernel */
  float scale;                 /* 0 -> 1/sqrt(head_dim) (AttentionExecutor.swift:153) */
  const anima_qk_prologue* prologue; /* NULL -> none */
  int64_t kv_token_stride;     /* TOKEN_MAJOR K/V row stride in halfs: 0 -> the reference contract
                                  (K/V share token_stride, key_value_heads == heads); otherwise
                                  key_value_heads * head_dim, which admits grouped-query heads
                                  with token-major [rows, heads*D] Q/O and [rows, kv_heads*D] K/V
                                  (the Qwen projections' natural layout, no transposes). */
} anima_attention_args;

anima_status anima_attention_encode(anima_attention* attn, const anima_attention_args* args);
anima_status anima_attention_execute(anima_attention* attn, const anima_attention_args* args);
/* No counterpart in the reference: anima_attention_encode for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, validation, kernels and results; the
 * workspace (K/Q prologue rows, key-split partial rows) comes from a static per-device
 * array of at most 64 MiB instead of the executor's own allocations, and the call
 * makes no hipMalloc, hipFree or other allocating call.  A request whose workspace
 * exceeds 64 MiB fails with ANIMA_E_UNSUPPORTED before anything is launched.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race. */
anima_status anima_attention_encode_noalloc(anima_attention* attn, const anima_attention_args* args);
/* AttentionExecutor.maximumScoreScratchBytes (AttentionExecutor.swift:112-120):
 * the score scratch the reference's query-tiled path would need (fp16 legacy /
 * fp32 scores) for min(tile_rows, query_count) x key_count.  The flash kernels
 * here keep no score tile; the figure is reported for API parity. query_count<=0
 * means "unbounded" (nil in the reference). */
anima_status anima_attention_max_score_scratch_bytes(anima_attention* attn, int64_t key_count,
                                                     int64_t query_count, int64_t* out_bytes);
/* Bytes of device workspace the executor currently holds. */
anima_status anima_attention_workspace_bytes(anima_attention* attn, int64_t* out_bytes);

/* ------------------------------------------------------------------------- */
/* Quantized linear: LinearExecutor (LinearExecutor.swift:43-459).             */
/* ------------------------------------------------------------------------- */

/* StorageDtype codes (Runtime/Animapk/AnimapkTensor.swift:4-9). */
typedef enum anima_storage {
  ANIMA_STORAGE_W4 = 0,
  ANIMA_STORAGE_W8 = 1,
  ANIMA_STORAGE_FP16 = 2,
  ANIMA_STORAGE_FP32 = 3
} anima_storage;

/* QuantizedLinearWeightBuffers (LinearExecutor.swift:18-29): a packed [rows=N,
 * columns=K] matrix; W4 packs the even K index in the low nibble; fp16 scale and
 * zero per (row, 64-wide K group), groups reset at every row; value =
 * q*scale + zero.  FP16 storage reuses the struct with packed_row_stride = K
 * halfs' worth of bytes / 2 (stride counted in elements, as the reference). */
typedef struct anima_qweight {
  int32_t storage;             /* anima_storage (W4, W8 or FP16) */
  anima_buffer packed; int64_t packed_offset;
  anima_buffer scale;  int64_t scale_offset;
  anima_buffer zero;   int64_t zero_offset;
  int64_t rows;                /* N (output features) */
  int64_t columns;             /* K (input features) */
  int64_t packed_row_stride;   /* bytes per row for W4/W8, halfs per row for FP16 */
} anima_qweight;

/* DiTLinearBackend (LinearExecutor.swift:43-75) re-cut for MI355X: AUTO = fused
 * dequant-in-registers MFMA GEMM (small-M rows use the group-scaled weight-stream
 * kernel); DEQUANT_THEN_GEMM = the reference default shape (dequantize the whole
 * weight to fp16 scratch, then an fp16 MFMA GEMM). */
typedef enum anima_linear_backend {
  ANIMA_LINEAR_BACKEND_AUTO = 0,
  ANIMA_LINEAR_BACKEND_FUSED = 1,
  ANIMA_LINEAR_BACKEND_DEQUANT_THEN_GEMM = 2
} anima_linear_backend;

/* DiTLinearFamily (LinearExecutor.swift:10-15); informational tag. */
typedef enum anima_linear_family {
  ANIMA_FAMILY_OTHER = 0,
  ANIMA_FAMILY_ATTENTION_PROJECTION = 1,
  ANIMA_FAMILY_MLP_UP = 2,
  ANIMA_FAMILY_MLP_DOWN = 3
} anima_linear_family;

typedef struct anima_linear_config {
  int32_t tile_rows;   /* > 0 (reference default 128); informational for the fused kernels */
  int32_t backend;     /* anima_linear_backend */
} anima_linear_config;

typedef struct anima_linear anima_linear;

anima_status anima_linear_create(anima_ctx* ctx, const anima_linear_config* cfg, anima_linear** out);
anima_status anima_linear_destroy(anima_linear* lin);

/* LinearExecutor.encode (LinearExecutor.swift:79-88): output[M,N] fp16 =
 * input[M,K] fp16 x deq(weight)[N,K]^T, fp32 accumulation; input and output are
 * tight row-major. */
anima_status anima_linear_encode(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                 const anima_qweight* weight, anima_buffer output,
                                 int64_t output_offset, int64_t input_rows, int32_t family);
anima_status anima_linear_execute(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                  const anima_qweight* weight, anima_buffer output,
                                  int64_t output_offset, int64_t input_rows, int32_t family);

/* Extension, no reference entry point: a linear followed by the DiT block's next
 * elementwise step, which DiTBlockExecutor encodes as two dispatches
 * (DiTBlockExecutor.swift:1180-1242 output projection + gate_add_half_f32,
 * :1244-1319 mlp1 + dit_gelu_half_inplace).
 *   ANIMA_LINEAR_EPILOGUE_GELU:     output = half(gelu_erf(linear(input)))
 *   ANIMA_LINEAR_EPILOGUE_GATE_ADD: residual[r, n] += float(linear(input)[r, n]) * gate[n]
 *                                   (residual fp32 [input_rows, weight.rows], gate fp32
 *                                   [weight.rows]); output is scratch the call may
 *                                   leave unwritten.
 *   ANIMA_LINEAR_EPILOGUE_RESIDUAL_ADD: residual[r, n] += float(linear(input)[r, n]) (the
 *                                   Qwen layer's add_half_into_float, QwenEncoderMetal.swift:
 *                                   280-302); gate is ignored, output as above.
 * Results equal anima_linear_encode followed by anima_gelu_half_inplace_encode /
 * anima_gate_add_half_f32_encode / anima_add_half_into_float_encode bit for bit: the tiled GEMM applies the step in
 * its output stage when it takes the shape, otherwise the two kernels run in turn.
 * residual and gate are ignored for ANIMA_LINEAR_EPILOGUE_GELU. */
typedef enum anima_linear_epilogue {
  ANIMA_LINEAR_EPILOGUE_GELU = 1,
  ANIMA_LINEAR_EPILOGUE_GATE_ADD = 2,
  ANIMA_LINEAR_EPILOGUE_RESIDUAL_ADD = 3
} anima_linear_epilogue;
anima_status anima_linear_encode_epilogue(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                          const anima_qweight* weight, anima_buffer output,
                                          int64_t output_offset, int64_t input_rows, int32_t family,
                                          int32_t epilogue, anima_buffer residual, anima_buffer gate);

/* Extension, no reference entry point: count (1..3) linears of one input, each into
 * its own output -- the Q/K/V (or gate/up) projections that DiTBlockExecutor and
 * QwenEncoderMetal encode one after another on the same normalised input
 * (DiTBlockExecutor.swift:1035-1105, QwenEncoderMetal.swift:244-262).  Results equal
 * count anima_linear_encode calls bit for bit; when every weight takes the tiled
 * W4/W8 GEMM with the same K and storage, the linears run as one launch. */
anima_status anima_linear_encode_group(anima_linear* lin, anima_buffer input, const anima_qweight* const* weights,
                                       const anima_buffer* outputs, int32_t count, int64_t input_rows,
                                       int32_t family);

/* Extension, no reference entry point: a linear followed by the per-head RMSNorm
 * that DiTBlockExecutor encodes on the cross-attention Q and context-K projections
 * (linear.encode + encodeRMSHeads / rmsnorm_heads_half, DiTBlockExecutor.swift:
 * 1103-1161, AnimaKernels.metal:660-689): output[r, h*head_dim + d] =
 * half(y[d] * rsqrt(mean_d(y^2) + eps) * norm_weight[d]) with y = half(linear(input))
 * restricted to head h.  weight.rows must be a multiple of head_dim; norm_weight is
 * fp16 [head_dim].  The tiled GEMM applies the norm in its output stage for
 * head_dim 128; otherwise the GEMM runs, then the norm in place. */
anima_status anima_linear_encode_head_rmsnorm(anima_linear* lin, anima_buffer input, int64_t input_offset,
                                              const anima_qweight* weight, anima_buffer output,
                                              int64_t output_offset, int64_t input_rows, int32_t family,
                                              anima_buffer norm_weight, int64_t head_dim, float eps);

/* M=1 fp32 matvec w4_matvec_f32 / w8_matvec_f32 / fp16_matvec_f32
 * (AnimaKernels.metal:804-933; DiTQuantizedWeightFactory.matvecKernel,
 * LinearExecutor.swift:520-528): output_f32[N] = deq(W)[N,K] . input_f32[K]. */
anima_status anima_matvec_encode(anima_ctx* ctx, const anima_qweight* weight,
                                 anima_buffer input_f32, int64_t input_offset,
                                 anima_buffer output_f32, int64_t output_offset);

/* Standalone dequant dequant_w4_to_half / dequant_w8_to_half
 * (AnimaKernels.metal:19-66): out[r*out_row_stride + k] = RNE16(q*s + z) for
 * k < columns; out_row_stride in halfs (>= columns). */
anima_status anima_dequant_to_half_encode(anima_ctx* ctx, const anima_qweight* weight,
                                          anima_buffer output, int64_t output_offset,
                                          int64_t out_row_stride);

/* No counterpart in the reference (a measurement probe, like its diagnostics):
 * a plain streaming read of `bytes` bytes of src (16-byte aligned, a multiple of
 * 16) that writes anima_read_probe_sink_bytes(bytes) bytes to sink.  It times the
 * achievable rate of reading a given number of bytes, the floor a weight-streaming
 * GEMM of the same byte count is compared with. */
anima_status anima_read_probe_encode(anima_ctx* ctx, anima_buffer src, int64_t src_offset, int64_t bytes,
                                     anima_buffer sink);
int64_t anima_read_probe_sink_bytes(int64_t bytes);

/* ------------------------------------------------------------------------- */
/* CPU decoders: QuantDecoders (QuantDecoders.swift:17-164).                   */
/* scale/zero are raw binary16 payloads; outputs are fp32.                     */
/* ------------------------------------------------------------------------- */
anima_status anima_dequant_w4(const uint8_t* data, const uint16_t* scale, const uint16_t* zero,
                              int64_t k, int64_t group_size, float* out);            /* :23-48 */
anima_status anima_dequant_w4_matrix(const uint8_t* data, const uint16_t* scale,
                                     const uint16_t* zero, int64_t rows, int64_t cols,
                                     int64_t group_size, float* out);                 /* :54-87 */
anima_status anima_dequant_w8(const uint8_t* data, const uint16_t* scale, const uint16_t* zero,
                              int64_t k, int64_t group_size, float* out);            /* :90-114 */
anima_status anima_dequant_w8_matrix(const uint8_t* data, const uint16_t* scale,
                                     const uint16_t* zero, int64_t rows, int64_t cols,
                                     int64_t group_size, float* out);                 /* :117-147 */
anima_status anima_fp16_to_float32(const uint16_t* bits, int64_t count, float* out);  /* :150-163 */

/* ------------------------------------------------------------------------- */
/* RoPE tables (CPU): fp32 [tokens][head_dim/2][2][2] of [cos,-sin,sin,cos].   */
/* ------------------------------------------------------------------------- */
/* DitRoPE.generate (Runtime/Text/DitRoPE.swift:58-107), any T/H/W grid,
 * head_dim 128 (t/h/w dims 44/42/42).  out holds T*H*W*64*4 floats. */
anima_status anima_rope_dit3d(int64_t T, int64_t H, int64_t W, float* out);
/* QwenEncoderMetal.makeRope (Runtime/Metal/QwenEncoderMetal.swift:126-143):
 * angle = pos / theta^(2j/head_dim).  out holds tokens*(head_dim/2)*4 floats. */
anima_status anima_rope_neox(int64_t tokens, int64_t head_dim, float theta, float* out);

/* ------------------------------------------------------------------------- */
/* DiT block support kernels (AnimaKernels.metal), fp32 residual stream.       */
/* ------------------------------------------------------------------------- */
/* dit_layernorm_modulate_to_half (AnimaKernels.metal:477-524): out_f16[r,i] =
 * half(LN(residual[r])[i] * (1 + modulation[modulation_offset + i]) + modulation[i]). */
anima_status anima_layernorm_modulate_to_half_encode(anima_ctx* ctx, anima_buffer residual,
                                                     anima_buffer modulation, anima_buffer output,
                                                     int64_t n, int64_t rows, float eps,
                                                     int64_t modulation_offset);
/* gate_add_half_f32 (AnimaKernels.metal:624-634): residual[i] += float(branch[i]) * gate[i % n]. */
anima_status anima_gate_add_half_f32_encode(anima_ctx* ctx, anima_buffer residual,
                                            anima_buffer branch, anima_buffer gate, int64_t n,
                                            int64_t count);
/* dit_gelu_half_inplace (AnimaKernels.metal:312-322), exact-erf GELU in fp32. */
anima_status anima_gelu_half_inplace_encode(anima_ctx* ctx, anima_buffer values, int64_t count);
/* silu (AnimaKernels.metal:388-397), fp32. */
anima_status anima_silu_f32_encode(anima_ctx* ctx, anima_buffer input, anima_buffer output,
                                   int64_t count);
/* add_f32 (AnimaKernels.metal:649-656): destination[i] += source[i]. */
anima_status anima_add_f32_encode(anima_ctx* ctx, anima_buffer destination, anima_buffer source,
                                  int64_t count);

/* ------------------------------------------------------------------------- */
/* DiT block: DiTBlockExecutor.execute (DiTBlockExecutor.swift:155-282) for one  */
/* block at any square token count, fp32 residual updated in place.            */
/* ------------------------------------------------------------------------- */
typedef struct anima_dit_block_weights {
  anima_qweight self_q, self_k, self_v, self_o;
  anima_qweight cross_q, cross_k, cross_v, cross_o;
  anima_qweight mlp1, mlp2;
  /* modulation W1 [256, dim] and W2 [3*dim, 256] per branch (fp16/W4/W8) */
  anima_qweight mod_self_w1, mod_self_w2, mod_cross_w1, mod_cross_w2, mod_mlp_w1, mod_mlp_w2;
  anima_buffer self_q_norm, self_k_norm;    /* fp16 [head_dim] each, required */
  anima_buffer cross_q_norm, cross_k_norm;  /* fp16 [head_dim] each, required */
} anima_dit_block_weights;

typedef struct anima_dit_block_args {
  anima_buffer residual;       /* fp32 [tokens, dim], updated in place */
  anima_buffer emb;            /* fp32 [dim] timestep embedding */
  anima_buffer adaln_lora;     /* fp32 [3*dim] */
  anima_buffer context;        /* fp16 [context_tokens, context_dim] */
  anima_buffer rope;           /* fp32 [tokens][head_dim/2][2][2] (anima_rope_dit3d) */
  int64_t tokens, dim, heads, head_dim, context_tokens, context_dim, mlp_hidden;
  float eps;
} anima_dit_block_args;

typedef struct anima_dit_block anima_dit_block;
anima_status anima_dit_block_create(anima_ctx* ctx, anima_dit_block** out);
anima_status anima_dit_block_destroy(anima_dit_block* blk);
anima_status anima_dit_block_encode(anima_dit_block* blk, const anima_dit_block_weights* w,
                                    const anima_dit_block_args* args);

/* CrossKVCache (DiTBlockExecutor.swift:19-43, used at :1110-1161): the cross-
 * attention K (after its per-head RMSNorm) and V of every block, computed from the
 * fixed context the first time a block runs and reused, exactly, by every later
 * sampler step of the same generation.  One device allocation of
 * blocks * 2 * context_tokens * dim fp16 owned by the cache; the attention reads
 * the cached rows in place (the reference copies them back into scratch).  The
 * cache belongs to one prompt: call reset when the context changes. */
typedef struct anima_cross_kv_cache anima_cross_kv_cache;
anima_status anima_cross_kv_cache_create(anima_ctx* ctx, int64_t blocks, int64_t context_tokens, int64_t dim,
                                         anima_cross_kv_cache** out);
anima_status anima_cross_kv_cache_destroy(anima_cross_kv_cache* cache);
/* Every block misses again on its next run (a new prompt). */
anima_status anima_cross_kv_cache_reset(anima_cross_kv_cache* cache);
anima_status anima_cross_kv_cache_is_ready(const anima_cross_kv_cache* cache, int64_t block, int32_t* ready);
anima_status anima_cross_kv_cache_bytes(const anima_cross_kv_cache* cache, int64_t* bytes);

/* anima_dit_block_encode as block `block_index` of a forward that shares `cache`
 * (NULL: no cache, identical to anima_dit_block_encode).  On a miss the block
 * projects the context into the cache slot and marks it ready; on a hit it skips
 * the context K/V projections and their norm.  Hit and miss give identical bits. */
anima_status anima_dit_block_encode_cached(anima_dit_block* blk, const anima_dit_block_weights* w,
                                           const anima_dit_block_args* args, anima_cross_kv_cache* cache,
                                           int64_t block_index);

/* DitForward.execute (DitForward.swift:78-112): blocks[0..block_count) in order over
 * the residual, weights resident in device memory (the whole W4 DiT is ~1 GB, so on
 * this part every block stays in HBM and nothing is streamed).  cache may be NULL. */
anima_status anima_dit_forward_encode(anima_dit_block* blk, const anima_dit_block_weights* blocks,
                                      int64_t block_count, const anima_dit_block_args* args,
                                      anima_cross_kv_cache* cache);

/* WeightStreamer (WeightStreamer.swift:87-213) for callers that keep the packed
 * blocks in host memory: `slots` (1..4) device slots of `capacity` bytes and a copy
 * stream.  Block i's host range is copied into slot i % slots on the copy stream
 * while earlier blocks compute; an event per slot makes the compute stream wait
 * for the copy, and the copy for the last block that read the slot, so a slot is
 * never overwritten in flight (the reference's markInFlight/complete, enforced on
 * the device instead of by host waits).  The copies are queued with
 * hipMemcpyAsync, so every host range must stay valid (mapped, not freed) until
 * the forward's stream work has completed (anima_ctx_synchronize).  Only pinned
 * ranges (hipHostMalloc) copy while earlier blocks compute; pageable memory, such
 * as the pages of a memory-mapped .animapk, is staged by the HIP runtime and the
 * copy then blocks the host and does not overlap with compute. */
typedef struct anima_weight_streamer anima_weight_streamer;
anima_status anima_weight_streamer_create(anima_ctx* ctx, int64_t capacity, int32_t slots,
                                          anima_weight_streamer** out);
anima_status anima_weight_streamer_destroy(anima_weight_streamer* streamer);

/* DitForward.execute with streamed weights.  templates[i] describes block i with
 * every device pointer (qweight packed/scale/zero ptr, norm ptr) holding a byte
 * offset from the start of host_ranges[i] instead of an address, and lengths
 * ignored: the library rebases them onto the slot the range lands in
 * (DiTQuantizedWeightFactory.makeMatrix binds ring + tensor offset the same way,
 * LinearExecutor.swift:467-518).  range_bytes[i] <= the streamer's capacity. */
anima_status anima_dit_forward_encode_streamed(anima_dit_block* blk, anima_weight_streamer* streamer,
                                               const anima_dit_block_weights* templates,
                                               const void* const* host_ranges, const int64_t* range_bytes,
                                               int64_t block_count, const anima_dit_block_args* args,
                                               anima_cross_kv_cache* cache);

/* ------------------------------------------------------------------------- */
/* DiT input / output and the sampler update (AnimaKernels.metal:1191-1297).   */
/* Latents are fp32 [channels][height][width]; tokens are the 2x2 patches in   */
/* row-major patch order, token t = (height/2 row, width/2 column).             */
/* ------------------------------------------------------------------------- */
/* patchify17 (AnimaKernels.metal:1218-1243): tokens[t][c*4 + di*2 + dj] =
 * input[c][2i+di][2j+dj] for 17 channels.  channels = 17 reads the mask channel
 * from input; channels = 16 treats it as zeros (the zero padding-mask channel that
 * DiTPreparationExecutor appends, DiTPreparationExecutor.swift:82-89).  tokens is
 * fp32 [(height/2)*(width/2)][68]. */
anima_status anima_patchify17_encode(anima_ctx* ctx, anima_buffer input, int64_t channels, int64_t height,
                                     int64_t width, anima_buffer tokens);
/* unpatchify16 (AnimaKernels.metal:1247-1268): the first 16 channels of [T][68]
 * tokens back to fp32 [16][height][width]. */
anima_status anima_unpatchify16_encode(anima_ctx* ctx, anima_buffer tokens, int64_t height, int64_t width,
                                       anima_buffer output);
/* unpatchify_velocity16 (AnimaKernels.metal:1273-1296): FinalLayer tokens fp32
 * [T][64] with element (di*2 + dj)*16 + c to fp32 [16][height][width]. */
anima_status anima_unpatchify_velocity16_encode(anima_ctx* ctx, anima_buffer tokens, int64_t height,
                                                int64_t width, anima_buffer output);
/* flow_velocity_to_denoised_f32 (AnimaKernels.metal:1191-1201): denoised = x - sigma * velocity. */
anima_status anima_flow_velocity_to_denoised_encode(anima_ctx* ctx, anima_buffer x, anima_buffer velocity,
                                                    anima_buffer denoised, float sigma, int64_t count);
/* EulerSampler.encodeStep + euler_step_f32 (EulerSampler.swift:43-70,
 * AnimaKernels.metal:1206-1216): x_next = x + (next_sigma - sigma) * (x - denoised) * (1/sigma);
 * sigma must be finite and > 0, next_sigma finite. */
anima_status anima_euler_step_encode(anima_ctx* ctx, anima_buffer x, anima_buffer denoised, anima_buffer x_next,
                                     float sigma, float next_sigma, int64_t count);

/* DiTPreparationExecutor.execute (DiTPreparationExecutor.swift:51-135) at any even
 * latent size: patchify the 16-channel latent with a zero mask channel, embed the
 * patches (x_embedder linear [dim, 68]) into the fp32 residual, and for sigma build
 * the sinusoidal timestep t (cos / sin halves, dit_source_oracle Timesteps), emb =
 * RMSNorm(t) * t_norm and adaln_lora = t_embed2 . SiLU(t_embed1 . t). */
typedef struct anima_dit_prepare_weights {
  anima_qweight x_embed;    /* [dim, 68] */
  anima_qweight t_embed1;   /* [dim, dim] */
  anima_qweight t_embed2;   /* [3*dim, dim] */
  anima_buffer t_norm;      /* fp16 [dim] */
} anima_dit_prepare_weights;

typedef struct anima_dit_prepare_args {
  anima_buffer latent;      /* fp32 [16][height][width] */
  int64_t height, width;    /* even */
  float sigma;              /* finite */
  anima_buffer residual;    /* out fp32 [(height/2)*(width/2)][dim] */
  anima_buffer emb;         /* out fp32 [dim] */
  anima_buffer adaln_lora;  /* out fp32 [3*dim] */
  int64_t dim;              /* even */
  float eps;                /* RMSNorm epsilon (1e-6) */
} anima_dit_prepare_args;

typedef struct anima_dit_prepare anima_dit_prepare;
anima_status anima_dit_prepare_create(anima_ctx* ctx, anima_dit_prepare** out);
anima_status anima_dit_prepare_destroy(anima_dit_prepare* prep);
anima_status anima_dit_prepare_encode(anima_dit_prepare* prep, const anima_dit_prepare_weights* w,
                                      const anima_dit_prepare_args* args);

/* DiTFinalLayerExecutor.execute (DiTFinalLayerExecutor.swift:75-186, W4 fp16
 * boundary): modulation = mod_w2 . (mod_w1 . SiLU(emb)) + adaln_lora[0 : 2*dim]
 * split into (shift, scale); x = half(residual); n = half(LayerNorm(x)) with fp32
 * statistics; y = half(n * (1 + scale) + shift); velocity = unpatchify_velocity16(
 * float(half(proj . y))). */
typedef struct anima_dit_final_weights {
  anima_qweight mod_w1;     /* [lora, dim] */
  anima_qweight mod_w2;     /* [2*dim, lora] */
  anima_qweight proj;       /* [64, dim] */
} anima_dit_final_weights;

typedef struct anima_dit_final_args {
  anima_buffer residual;    /* fp32 [(height/2)*(width/2)][dim] */
  anima_buffer emb;         /* fp32 [dim] */
  anima_buffer adaln_lora;  /* fp32 [>= 2*dim]; its first 2*dim values are added */
  anima_buffer velocity;    /* out fp32 [16][height][width] */
  int64_t height, width, dim;
  float eps;                /* LayerNorm epsilon (1e-6) */
} anima_dit_final_args;

typedef struct anima_dit_final anima_dit_final;
anima_status anima_dit_final_create(anima_ctx* ctx, anima_dit_final** out);
anima_status anima_dit_final_destroy(anima_dit_final* fin);
anima_status anima_dit_final_encode(anima_dit_final* fin, const anima_dit_final_weights* w,
                                    const anima_dit_final_args* args);

/* ------------------------------------------------------------------------- */
/* .animapk (ANMA v1) packs: AnimapkFile (Runtime/Animapk/AnimapkFile.swift:15-185), */
/* AnimapkHeader (AnimapkHeader.swift:5-69), the tensor_meta JSON          */
/* (AnimapkTensor.swift:90-173) and the execution ranges of                */
/* AnimapkRangeLocator.swift:38-261.  The file is mapped read-only on the  */
/* host; every name and pointer the calls return stays valid until         */
/* anima_pack_close.                                                       */
/* ------------------------------------------------------------------------- */
typedef struct anima_pack anima_pack;

typedef struct anima_pack_info {
  int32_t version;           /* 1 */
  int32_t component;         /* header code: 1 dit, 2 te, 3 vae */
  int64_t alignment;         /* 16384 */
  int64_t tensor_count;
  int64_t json_offset, json_size;
  int64_t table_offset, table_bytes;
  int64_t payload_offset;
  int64_t file_size;
  int32_t record_size;       /* 128 */
  int32_t quant_group;       /* JSON quant.group, -1 when absent */
  const char* quant_scheme;  /* JSON quant.scheme, NULL when absent */
  const char* component_name;/* JSON component ("dit", "te", "vae") */
} anima_pack_info;

/* One tensor_meta entry.  Offsets: blob_* are absolute file offsets; data_*,
 * scale_* and zero_* are relative to the blob (scale/zero -1 when absent). */
typedef struct anima_pack_tensor {
  const char* name;
  int32_t storage;           /* ANIMA_STORAGE_* from storage_dtype ("w4" ... "fp32") */
  int32_t rank;              /* <= 8 */
  int64_t shape[8];
  int64_t blob_offset, blob_size;
  int64_t data_offset, data_size;
  int64_t scale_offset, scale_size;
  int64_t zero_offset, zero_size;
  int64_t block_index;       /* -1 when absent */
  uint32_t crc32;
  int32_t has_crc32;
  const char* logical_dtype;
  const char* quantization_format;  /* NULL when absent */
} anima_pack_tensor;

/* A contiguous file range holding every blob of one execution unit (a DiT block,
 * the final layer, the preparation tensors): AnimapkExecutionRange. */
typedef struct anima_pack_range {
  int64_t logical_index;
  int64_t file_offset;       /* 16 KiB aligned */
  int64_t length;
  int64_t tensor_count;
  const void* host;          /* the mapped bytes of [file_offset, file_offset + length) */
} anima_pack_range;

/* AnimapkFile.init: header, JSON, per-tensor and table cross-match validation
 * (ANIMA_E_FORMAT with the reference's message on a violation, ANIMA_E_IO when
 * the file cannot be opened or mapped). */
anima_status anima_pack_open(const char* path, anima_pack** out);
anima_status anima_pack_close(anima_pack* pack);
anima_status anima_pack_get_info(const anima_pack* pack, anima_pack_info* out);
/* Tensors in JSON order (index 0 .. tensor_count-1), or by full name
 * (ANIMA_E_INVALID_ARGUMENT "missing tensor <name>" when absent). */
anima_status anima_pack_tensor_at(const anima_pack* pack, int64_t index, anima_pack_tensor* out);
anima_status anima_pack_find(const anima_pack* pack, const char* name, anima_pack_tensor* out);
/* AnimapkFile.crc32MismatchCount: tensors whose data CRC-32 (zlib) differs from
 * the JSON value (tensors without one count as matching). */
anima_status anima_pack_crc32_mismatch_count(const anima_pack* pack, int64_t* out);
/* AnimapkFile.bytes(in:): the mapped bytes of an absolute file range. */
anima_status anima_pack_bytes(const anima_pack* pack, int64_t offset, int64_t length, const void** out);
/* AnimapkRangeBuilder.executionRanges: for i < count the range of every tensor
 * named "<prefix><i>." ..., in logical order; physical ranges must not overlap. */
anima_status anima_pack_execution_ranges(const anima_pack* pack, const char* prefix, int64_t count,
                                         anima_pack_range* out);

/* Weight templates of one execution unit: every anima_qweight has packed /
 * scale / zero = {NULL, range length} with *_offset relative to the range start
 * (DiTQuantizedWeightFactory.makeMatrix, LinearExecutor.swift:467-518), and every
 * norm buffer {(void*)offset, bytes}.  anima_dit_forward_encode_streamed takes
 * block templates as they are; the *_rebase calls turn a template into device
 * weights once the range has been copied to `base`. */
/* DiT block i (BlockWeights, DiTBlockExecutor.swift:1864-1917: 20 tensors). */
anima_status anima_pack_dit_block(const anima_pack* pack, int64_t block, anima_dit_block_weights* tmpl,
                                  anima_pack_range* range);
/* DiTPreparationLocator + DiTPreparationWeights (DiTPreparationExecutor.swift:297-323). */
anima_status anima_pack_dit_prepare(const anima_pack* pack, int64_t dim, anima_dit_prepare_weights* tmpl,
                                    anima_pack_range* range);
/* DiTFinalLayerLocator + FinalWeights (DiTFinalLayerExecutor.swift:394-420). */
anima_status anima_pack_dit_final(const anima_pack* pack, int64_t dim, anima_dit_final_weights* tmpl,
                                  anima_pack_range* range);
/* Template -> weights in a device copy of the range at `base` (range_bytes long);
 * an offset outside the range fails with ANIMA_E_OUT_OF_BOUNDS. */
anima_status anima_dit_block_weights_rebase(const anima_dit_block_weights* tmpl, void* base, int64_t range_bytes,
                                            anima_dit_block_weights* out);
anima_status anima_dit_prepare_weights_rebase(const anima_dit_prepare_weights* tmpl, void* base,
                                              int64_t range_bytes, anima_dit_prepare_weights* out);
anima_status anima_dit_final_weights_rebase(const anima_dit_final_weights* tmpl, void* base, int64_t range_bytes,
                                            anima_dit_final_weights* out);

/* ------------------------------------------------------------------------- */
/* Qwen encoder layer: QwenLayerExecutor.execute (QwenEncoderMetal.swift:232-304)  */
/* for a batch of right-padded sequences, fp32 residual updated in place.        */
/* ------------------------------------------------------------------------- */
/* rmsnorm_f32_to_f32 (AnimaKernels.metal:172-204) followed by float_to_half
 * (:81-88), fused: out[r][i] = half(in[r][i] * rsqrt(mean(in[r]^2) + eps) * w[i]). */
anima_status anima_rmsnorm_f32_to_half_encode(anima_ctx* ctx, anima_buffer input,
                                              anima_buffer weight, anima_buffer output,
                                              int64_t n, int64_t rows, float eps);
/* gated_silu_half (AnimaKernels.metal:401-411): out = half(silu(gate) * up), fp32 maths. */
anima_status anima_gated_silu_half_encode(anima_ctx* ctx, anima_buffer gate, anima_buffer up,
                                          anima_buffer output, int64_t count);
/* add_half_into_float (AnimaKernels.metal:639-647): residual[i] += float(branch[i]). */
anima_status anima_add_half_into_float_encode(anima_ctx* ctx, anima_buffer residual,
                                              anima_buffer branch, int64_t count);

typedef struct anima_qwen_layer_weights {
  anima_qweight q, k, v, o, gate, up, down;  /* W8 in the reference; W4/W8/FP16 accepted */
  anima_buffer input_norm;           /* fp16 [hidden], required */
  anima_buffer post_attention_norm;  /* fp16 [hidden], required */
  anima_buffer q_norm;               /* fp16 [head_dim], required */
  anima_buffer k_norm;               /* fp16 [head_dim], required */
} anima_qwen_layer_weights;

typedef struct anima_qwen_layer_args {
  anima_buffer residual;        /* fp32 [batch][tokens][hidden], updated in place */
  anima_buffer rope;            /* fp32 [tokens][head_dim/2][2][2] (anima_rope_neox) */
  const int32_t* key_lengths;   /* host, per sequence, 1..tokens; NULL = every token valid */
  int64_t batch, tokens, hidden, heads, kv_heads, head_dim, intermediate;
  float eps;
} anima_qwen_layer_args;

typedef struct anima_qwen_layer anima_qwen_layer;
anima_status anima_qwen_layer_create(anima_ctx* ctx, anima_qwen_layer** out);
anima_status anima_qwen_layer_destroy(anima_qwen_layer* layer);
anima_status anima_qwen_layer_encode(anima_qwen_layer* layer, const anima_qwen_layer_weights* w,
                                     const anima_qwen_layer_args* args);

/* ------------------------------------------------------------------------- */
/* Numerical-health probes: NumericalMonitor (NumericalMonitor.swift:21-53,   */
/* 136-170, 205-212, 320-358), the stats ABI of AnimaKernels.metal:1578-1600  */
/* and the standalone passes probe_f16_stats / probe_f32_stats (:1921-2040).  */
/* ------------------------------------------------------------------------- */
/* stats holds one uint32 quad per slot: [0] flags (ANIMA_PROBE_FLAG_*), [1] max |v| over
 * the finite values as fp32 bits (0 when there is none), [2] index of the first element
 * that set a flag (ANIMA_PROBE_NO_INDEX when none did), [3] reserved.  A pass ORs its
 * flags into [0] and takes the max of [1] and the min of [2] with relaxed atomics, so
 * passes accumulate into a slot (also concurrently) until the slot is reset. */
#define ANIMA_PROBE_SLOT_UINTS 4
#define ANIMA_PROBE_FLAG_NAN 0x1u
#define ANIMA_PROBE_FLAG_POS_INF 0x2u
#define ANIMA_PROBE_FLAG_NEG_INF 0x4u
#define ANIMA_PROBE_FLAG_HALF_OVERFLOW 0x8u   /* finite |v| > 65504 */
#define ANIMA_PROBE_NO_INDEX 0xFFFFFFFFu

typedef enum anima_probe_dtype {
  ANIMA_PROBE_F16 = 0,  /* probe_f16_stats, NumericalMonitor.encodeProbe (:320-338) */
  ANIMA_PROBE_F32 = 1   /* probe_f32_stats, NumericalMonitor.encodeProbeF32 (:340-358) */
} anima_probe_dtype;

/* beginRun (NumericalMonitor.swift:205-212): slots [0, slots) of stats (4-byte aligned,
 * slots * 16 bytes) become 0, 0, ANIMA_PROBE_NO_INDEX, 0.  A kernel on the context's
 * stream (no memset), so it may be recorded in a HIP graph. */
anima_status anima_numerics_probe_reset_encode(anima_ctx* ctx, anima_buffer stats, int32_t slots);
/* encodeProbe / encodeProbeF32 (NumericalMonitor.swift:320-358): one pass over `count`
 * values of `dtype` starting `offset` elements into `values`, accumulated into slot
 * `slot` of stats.  The first index counts from that start.  count 0 does nothing;
 * count must be below ANIMA_PROBE_NO_INDEX (the index word). */
anima_status anima_numerics_probe_encode(anima_ctx* ctx, anima_buffer values, int64_t offset, int64_t count,
                                         int32_t dtype, anima_buffer stats, int32_t slot);

#ifdef __cplusplus
}
#endif

#endif /* ANIMA_HIP_H */
