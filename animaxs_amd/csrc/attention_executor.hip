// Host side of the attention executor: the validation contract of
// AttentionExecutor.validate (AnimaXS/Runtime/Metal/AttentionExecutor.swift:778-847)
// plus the batch / key-length / prologue extensions, and kernel dispatch.
#include <cmath>
#include <mutex>
#include <string>

#include "attention.hpp"

namespace anima {

AttentionExecutor::AttentionExecutor(anima_ctx* ctx, const anima_attention_config& cfg)
    : ctx_(ctx), cfg_(cfg) {
  if (cfg.tile_rows <= 0) fail(ANIMA_E_INVALID_ARGUMENT, "attention tile rows must be positive");
  if (cfg.numerics < ANIMA_NUMERICS_LEGACY || cfg.numerics > ANIMA_NUMERICS_BF16_COMPUTE)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown attention numerics");
  if (cfg.backend < ANIMA_ATTENTION_BACKEND_AUTO || cfg.backend > ANIMA_ATTENTION_BACKEND_LEGACY_MPS)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown attention backend");
  if (cfg.layout != ANIMA_LAYOUT_HEAD_MAJOR && cfg.layout != ANIMA_LAYOUT_TOKEN_MAJOR)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown attention layout");
  if (cfg.flash_rows != 0 && cfg.flash_rows != 128 && cfg.flash_rows != 256)
    fail(ANIMA_E_INVALID_ARGUMENT, "flash_rows must be 0 (auto), 128 or 256");
}

int64_t AttentionExecutor::maximum_score_scratch_bytes(int64_t key_count, int64_t query_count) const {
  if (key_count <= 0) fail(ANIMA_E_INVALID_SHAPE, "attention key count must be positive");
  const int64_t tile = query_count > 0 ? std::min<int64_t>(cfg_.tile_rows, query_count) : cfg_.tile_rows;
  const int64_t elem = cfg_.numerics == ANIMA_NUMERICS_LEGACY ? 2 : 4;
  return checked_product({tile, key_count, elem}, "attention");
}

static int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Static workspace of anima_attention_encode_noalloc, for callers that cannot
// allocate (code under graph capture, tight serving loops).  Every GPU the library
// runs on holds one copy until the process ends.  Each call uses it from offset 0:
// K prologue rows, then Q prologue rows, then key-split partial rows, all written by
// the call's own kernels before they are read (nothing has to start at zero).  Calls
// that overlap on one GPU share it and race.
// ---------------------------------------------------------------------------
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(64) << 20;
static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mutex;
static char* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of `scratch` on `device` (which must be current): resolved once per
// device with hipGetSymbolAddress.  The array's own name is a host-side stand-in,
// never a device address, so only this pointer reaches kernels.
static char* noalloc_scratch(int device) {
  if (device < 0 || device >= NOALLOC_MAX_DEVICES)
    fail(ANIMA_E_UNSUPPORTED, "allocation-free attention supports device indices below 64");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    ANIMA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) fail(ANIMA_E_DEVICE, "hipGetSymbolAddress returned a null scratch address");
    g_scratch_ptr[device] = static_cast<char*>(ptr);
  }
  return g_scratch_ptr[device];
}

void AttentionExecutor::encode(const anima_attention_args& a) { encode_impl(a, false); }

void AttentionExecutor::encode_noalloc(const anima_attention_args& a) { encode_impl(a, true); }

void AttentionExecutor::encode_impl(const anima_attention_args& a, bool no_alloc) {
  const int layout = a.layout < 0 ? cfg_.layout : a.layout;
  if (layout != ANIMA_LAYOUT_HEAD_MAJOR && layout != ANIMA_LAYOUT_TOKEN_MAJOR)
    fail(ANIMA_E_INVALID_ARGUMENT, "unknown attention layout");
  const bool token_major = layout == ANIMA_LAYOUT_TOKEN_MAJOR;
  const int64_t ts = token_major ? (a.token_stride > 0 ? a.token_stride : cfg_.token_stride) : 0;
  const int64_t H = a.heads, Sq = a.query_count, Sk = a.key_count, D = a.head_dim;
  const int64_t kvh = a.key_value_heads == 0 ? H : a.key_value_heads;
  const int64_t B = a.batch == 0 ? 1 : a.batch;
  // K/V row stride: the reference contract shares token_stride; the extension
  // kv_token_stride = kv_heads * head_dim admits grouped-query heads.
  const int64_t kts = token_major ? (a.kv_token_stride > 0 ? a.kv_token_stride : ts) : 0;

  // ---- AttentionExecutor.validate (:778-825) ----
  if (!(H > 0 && Sq > 0 && Sk > 0 && D > 0 && kvh > 0 && H % kvh == 0 && a.query_offset >= 0 &&
        a.key_offset >= 0 && a.value_offset >= 0 && a.output_offset >= 0 && (!a.causal || Sq == Sk) &&
        B > 0))
    fail(ANIMA_E_INVALID_SHAPE, "invalid attention shape, offset, or causal dimensions");
  if (token_major) {
    if (a.kv_token_stride < 0) fail(ANIMA_E_INVALID_SHAPE, "kv_token_stride must be >= 0");
    if (a.kv_token_stride == 0) {
      if (!(ts > 0 && D <= ts && ts % D == 0 && H * D == ts && kvh == H))
        fail(ANIMA_E_INVALID_SHAPE,
             "P4 token-major attention requires tokenStride == heads * headDim and keyValueHeads == heads");
    } else if (!(ts > 0 && H * D == ts && kvh * D == kts)) {
      fail(ANIMA_E_INVALID_SHAPE,
           "grouped token-major attention requires tokenStride == heads * headDim and "
           "kvTokenStride == keyValueHeads * headDim");
    }
    if (a.query_offset % 16 || a.key_offset % 16 || a.value_offset % 16 || a.output_offset % 16 || (ts * 2) % 16 ||
        (kts * 2) % 16)
      fail(ANIMA_E_MISALIGNED, "P4 token-major attention requires 16-byte-aligned offsets and row stride");
  }
  int64_t q_bytes, k_bytes;
  if (token_major) {
    q_bytes = checked_product({B, Sq, ts, 2}, "attention");
    k_bytes = checked_product({B, Sk, kts, 2}, "attention");
  } else {
    q_bytes = checked_product({B, H, Sq, D, 2}, "attention");
    k_bytes = checked_product({B, kvh, Sk, D, 2}, "attention");
  }
  if (checked_end(a.query_offset, q_bytes, "attention") > a.query.length ||
      checked_end(a.key_offset, k_bytes, "attention") > a.key.length ||
      checked_end(a.value_offset, k_bytes, "attention") > a.value.length ||
      checked_end(a.output_offset, q_bytes, "attention") > a.output.length)
    fail(ANIMA_E_OUT_OF_BOUNDS, "attention buffer range is out of bounds");
  if (!a.query.ptr || !a.key.ptr || !a.value.ptr || !a.output.ptr)
    fail(ANIMA_E_INVALID_ARGUMENT, "attention buffer pointer is null");
  if ((a.query_offset | a.key_offset | a.value_offset | a.output_offset) & 1)
    fail(ANIMA_E_MISALIGNED, "attention offsets must be multiples of the 2-byte fp16 element");
  if (Sq > 0x7fffffff || Sk > 0x7fffffff || H > 0x7fffffff || D > 0x7fffffff)
    fail(ANIMA_E_INVALID_SHAPE, "attention dimension exceeds int32");

  // ---- numerics / extensions ----
  if (cfg_.numerics == ANIMA_NUMERICS_BF16_COMPUTE)
    fail(ANIMA_E_UNSUPPORTED, "bf16_compute attention numerics are not supported on MI355X; select legacy or fp32 scores");
  const float scale = a.scale == 0.f ? (float)(1.0 / std::sqrt((double)D)) : a.scale;
  if (!std::isfinite(scale)) fail(ANIMA_E_INVALID_ARGUMENT, "attention scale must be finite");

  FlashParams p{};
  if (a.key_lengths) {
    if (a.key_lengths_on_device) {
      p.key_lengths_dev = a.key_lengths;
    } else {
      if (B > MAX_HOST_BATCH)
        fail(ANIMA_E_UNSUPPORTED, "host key lengths support batch <= 64; pass device key lengths");
      for (int64_t b = 0; b < B; ++b) {
        const int32_t L = a.key_lengths[b];
        if (L < 1 || L > Sk) fail(ANIMA_E_INVALID_SHAPE, "attention key length out of range (1..keyCount)");
        p.host_lengths[b] = L;
      }
      p.use_host_lengths = 1;
    }
  }

  const anima_qk_prologue* pro = a.prologue;
  const half_t* q_norm = nullptr;
  const half_t* k_norm = nullptr;
  const float* rope_q = nullptr;
  const float* rope_k = nullptr;
  float eps = 0.f;
  if (pro) {
    eps = pro->eps;
    if (!std::isfinite(eps) || eps < 0.f) fail(ANIMA_E_INVALID_ARGUMENT, "RMSNorm epsilon must be finite and >= 0");
    const int64_t w_bytes = checked_product({D, 2}, "attention prologue");
    if (pro->q_norm_weight.ptr) {
      if (pro->q_norm_weight.length < w_bytes)
        fail(ANIMA_E_OUT_OF_BOUNDS, "Q RMSNorm weight holds fewer than head_dim fp16 values");
      q_norm = static_cast<const half_t*>(pro->q_norm_weight.ptr);
    }
    if (pro->k_norm_weight.ptr) {
      if (pro->k_norm_weight.length < w_bytes)
        fail(ANIMA_E_OUT_OF_BOUNDS, "K RMSNorm weight holds fewer than head_dim fp16 values");
      k_norm = static_cast<const half_t*>(pro->k_norm_weight.ptr);
    }
    const bool want_q = pro->rope.ptr && pro->rope_q;
    const bool want_k = pro->rope_k && (pro->k_rope.ptr || pro->rope.ptr);
    if (want_q || want_k) {
      if (D % 2) fail(ANIMA_E_INVALID_SHAPE, "RoPE requires an even head_dim");
      // [tokens][D/2][2][2] fp32 = 8 * D bytes per token.
      const int64_t row_bytes = checked_product({D, 8}, "attention prologue");
      if (want_q) {
        if (pro->rope_tokens < Sq) fail(ANIMA_E_OUT_OF_BOUNDS, "RoPE table has fewer rows than query_count");
        if (checked_product({pro->rope_tokens, row_bytes}, "attention prologue") > pro->rope.length)
          fail(ANIMA_E_OUT_OF_BOUNDS, "RoPE table buffer is shorter than rope_tokens rows");
        rope_q = static_cast<const float*>(pro->rope.ptr);
      }
      if (want_k) {
        if (pro->k_rope.ptr) {
          if (pro->k_rope_tokens < Sk) fail(ANIMA_E_OUT_OF_BOUNDS, "K RoPE table has fewer rows than key_count");
          if (checked_product({pro->k_rope_tokens, row_bytes}, "attention prologue") > pro->k_rope.length)
            fail(ANIMA_E_OUT_OF_BOUNDS, "K RoPE table buffer is shorter than k_rope_tokens rows");
          rope_k = static_cast<const float*>(pro->k_rope.ptr);
        } else {
          if (pro->rope_tokens < Sk) fail(ANIMA_E_OUT_OF_BOUNDS, "RoPE table has fewer rows than key_count");
          if (checked_product({pro->rope_tokens, row_bytes}, "attention prologue") > pro->rope.length)
            fail(ANIMA_E_OUT_OF_BOUNDS, "RoPE table buffer is shorter than rope_tokens rows");
          rope_k = static_cast<const float*>(pro->rope.ptr);
        }
      }
    }
  }

  // ---- strides (elements) ----
  const half_t* qp = reinterpret_cast<const half_t*>(byte_ptr(a.query, a.query_offset));
  const half_t* kp = reinterpret_cast<const half_t*>(byte_ptr(a.key, a.key_offset));
  const half_t* vp = reinterpret_cast<const half_t*>(byte_ptr(a.value, a.value_offset));
  half_t* op = reinterpret_cast<half_t*>(byte_ptr_mut(a.output, a.output_offset));
  int64_t q_tok, q_head, q_batch, k_tok, k_head, k_batch;
  if (token_major) {
    q_tok = ts; q_head = D; q_batch = Sq * ts;
    k_tok = kts; k_head = D; k_batch = Sk * kts;
  } else {
    q_tok = D; q_head = Sq * D; q_batch = H * Sq * D;
    k_tok = D; k_head = Sk * D; k_batch = kvh * Sk * D;
  }

  const bool flash_shape = (D == 64 || D == 128 || D == 384);
  const bool rows_aligned = aligned16(qp) && aligned16(kp) && aligned16(vp) && aligned16(op) && (q_tok % 8 == 0) &&
                            (k_tok % 8 == 0) && (q_head % 8 == 0) && (k_head % 8 == 0) && (q_batch % 8 == 0) &&
                            (k_batch % 8 == 0);
  bool use_flash;
  switch (cfg_.backend) {
    case ANIMA_ATTENTION_BACKEND_FLASH:
      if (!(flash_shape && rows_aligned))
        fail(ANIMA_E_UNSUPPORTED,
             "flash attention requires head_dim 64, 128 or 384 and 16-byte-aligned rows, offsets and strides");
      use_flash = true;
      break;
    case ANIMA_ATTENTION_BACKEND_GENERIC:
    case ANIMA_ATTENTION_BACKEND_LEGACY_MPS:
      use_flash = false;
      break;
    default:
      use_flash = flash_shape && rows_aligned;
  }
  // The wide (head_dim 384) kernel reads Q as it is; the prologue kernel normalises it.
  const bool q_fusable = use_flash && D != 384 && (!q_norm || aligned16(q_norm)) && (!rope_q || aligned16(rope_q));
  const bool need_q_pro = (q_norm || rope_q) && !q_fusable;
  const bool need_k_pro = (k_norm || rope_k);

  const int64_t k_ws = need_k_pro ? round_up(checked_product({B, kvh, Sk, D, 2}, "attention"), 256) : 0;
  const int64_t q_ws = need_q_pro ? round_up(checked_product({B, H, Sq, D, 2}, "attention"), 256) : 0;

  // The whole plan is fixed before anything is launched: the prologues write dense
  // head-major rows, so the flash kernel reads those strides; the key-split decision
  // depends on them.
  const half_t* k_in = kp;
  const half_t* q_in = qp;
  const int64_t k_in_tok = k_tok, k_in_head = k_head, k_in_batch = k_batch;
  const int64_t q_in_tok = q_tok, q_in_head = q_head, q_in_batch = q_batch;
  if (need_k_pro) {
    k_tok = D; k_head = Sk * D; k_batch = kvh * Sk * D;
  }
  if (need_q_pro) {
    q_tok = D; q_head = Sq * D; q_batch = H * Sq * D;
  }
  p.q = qp; p.k = kp; p.v = vp; p.o = op;
  p.q_tok = q_tok; p.q_head = q_head; p.q_batch = q_batch;
  p.k_tok = k_tok; p.k_head = k_head; p.k_batch = k_batch;
  if (token_major) {
    p.v_tok = kts; p.v_head = D; p.v_batch = Sk * kts;
    p.o_tok = ts; p.o_head = D; p.o_batch = Sq * ts;
  } else {
    p.v_tok = D; p.v_head = Sk * D; p.v_batch = kvh * Sk * D;
    p.o_tok = D; p.o_head = Sq * D; p.o_batch = H * Sq * D;
  }
  p.Sq = (int)Sq; p.Sk = (int)Sk; p.H = (int)H; p.group = (int)(H / kvh);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.scale = scale;
  p.causal = a.causal ? 1 : 0;
  p.eps = eps;
  if (use_flash && !need_q_pro) {
    p.q_norm_w = q_norm;
    p.rope = rope_q;
  }
  const int splits = use_flash ? flash_kv_splits(p, (int)D, (int)B, cfg_.flash_rows) : 1;
  const int64_t part = splits > 1 ? round_up(flash_split_bytes(p, (int)D, (int)B, splits), 256) : 0;

  DeviceGuard guard(ctx_);
  hipStream_t stream = ctx_->stream;
  char* ws = nullptr;
  char* pw = nullptr;
  if (no_alloc) {
    const int64_t total = k_ws + q_ws + part;
    if (total > NOALLOC_SCRATCH_BYTES)
      fail(ANIMA_E_UNSUPPORTED, "attention needs " + std::to_string(total) +
                                    " bytes of workspace; the allocation-free entry point holds at most " +
                                    std::to_string(NOALLOC_SCRATCH_BYTES) + " bytes (use anima_attention_encode)");
    char* base = noalloc_scratch(ctx_->device);
    ws = base;
    pw = base + k_ws + q_ws;
  } else {
    if (k_ws + q_ws > 0) ws = static_cast<char*>(ws_.get(k_ws + q_ws, stream));
    if (part > 0) pw = static_cast<char*>(split_ws_.get(part, stream));
  }

  if (need_k_pro) {
    PrologueParams pp{};
    pp.in = k_in; pp.in_tok = k_in_tok; pp.in_head = k_in_head; pp.in_batch = k_in_batch;
    pp.out = reinterpret_cast<half_t*>(ws);
    pp.out_tok = D; pp.out_head = Sk * D; pp.out_batch = kvh * Sk * D;
    pp.batch = (int)B; pp.rows = (int)Sk; pp.heads = (int)kvh; pp.D = (int)D;
    pp.norm_w = k_norm; pp.eps = eps; pp.rope = rope_k;
    launch_prologue(pp, stream);
    p.k = pp.out;
  }
  if (need_q_pro) {
    PrologueParams pp{};
    pp.in = q_in; pp.in_tok = q_in_tok; pp.in_head = q_in_head; pp.in_batch = q_in_batch;
    pp.out = reinterpret_cast<half_t*>(ws + k_ws);
    pp.out_tok = D; pp.out_head = Sq * D; pp.out_batch = H * Sq * D;
    pp.batch = (int)B; pp.rows = (int)Sq; pp.heads = (int)H; pp.D = (int)D;
    pp.norm_w = q_norm; pp.eps = eps; pp.rope = rope_q;
    launch_prologue(pp, stream);
    p.q = pp.out;
  }
  if (use_flash) {
    if (splits > 1) {
      p.kv_splits = splits;
      p.part_o = pw;
      p.part_ml = reinterpret_cast<float*>(pw + flash_split_o_bytes(p, (int)D, (int)B, splits));
    }
    launch_flash(p, (int)D, (int)B, cfg_.flash_rows, stream);
  } else if (cfg_.backend == ANIMA_ATTENTION_BACKEND_LEGACY_MPS && cfg_.numerics == ANIMA_NUMERICS_LEGACY) {
    launch_legacy_mps(p, (int)D, (int)B, stream);
  } else {
    launch_generic(p, (int)D, (int)B, stream);
  }
}

}  // namespace anima
