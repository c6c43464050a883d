// AttentionExecutor for gfx950 (AnimaXS/Runtime/Metal/AttentionExecutor.swift:77-848).
#pragma once

#include "context.hpp"

namespace anima {

constexpr int MAX_HOST_BATCH = 64;  // host key lengths travel inside the kernel arguments

struct FlashParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  int64_t q_tok, q_head, q_batch;  // element strides
  int64_t k_tok, k_head, k_batch;
  int64_t v_tok, v_head, v_batch;
  int64_t o_tok, o_head, o_batch;
  int Sq, Sk, H, group;
  int q_tiles;
  int head_group;                  // 256-row kernel: heads one query tile takes on consecutive
                                   // workgroups (set by launch_flash_v2)
  float scale_log2;                // scale * log2(e)
  float scale;                     // the softmax scale itself (MPS-rounding kernel)
  int causal;
  const int* key_lengths_dev;      // device lengths (clamped in-kernel) or null
  int use_host_lengths;
  int host_lengths[MAX_HOST_BATCH];
  const half_t* q_norm_w;          // fused Q RMSNorm weight or null
  float eps;
  const float* rope;               // fused Q RoPE table or null
  // Key splits (256-row and head-dim-384 kernels, non-causal, no key lengths): workgroup
  // split s takes keys [s*kv_chunk, (s+1)*kv_chunk) and writes its normalised O rows in fp16
  // to part_o ([split][batch][head][Sq][D]) and (running max in log2 units, row sum) in fp32
  // to part_ml ([split][batch][head][Sq][2]); flash_combine_kernel merges them into o.
  int kv_splits;                   // 0 or 1: no split
  int nbatch;                      // batch count (partial row index)
  int kv_chunk;                    // keys per split, a multiple of 64
  void* part_o;                    // key splits: fp16 O_s / l_s rows [split][batch][head][Sq][D] for every
                                   // head_dim, then (256-byte aligned) part_ml
  float* part_ml;
};

struct PrologueParams {
  const half_t* in;
  int64_t in_tok, in_head, in_batch;
  half_t* out;                     // element strides below (the attention uses dense
  int64_t out_tok, out_head, out_batch;  // head-major [batch][heads][rows][D])
  int batch, rows, heads, D;
  const half_t* norm_w;
  float eps;
  const float* rope;
};

void launch_flash(FlashParams p, int D, int batch, int flash_rows, hipStream_t stream);
// Key splits launch_flash will use for this shape (1: none); the caller provides
// p.part_o / p.part_ml of flash_split_bytes() when it returns more than 1.
int flash_kv_splits(const FlashParams& p, int D, int batch, int flash_rows);
int64_t flash_split_bytes(const FlashParams& p, int D, int batch, int splits);
int64_t flash_split_o_bytes(const FlashParams& p, int D, int batch, int splits);

// 256-row flash variant (attention_v2.hip); p.q_tiles counts 256-row tiles.
constexpr int FLASH_V2_ROWS = 256;
// Wide-head (head_dim 384) flash kernel (attention_wide.hip): 128 query rows per
// workgroup, p.q_tiles counts 128-row tiles.
constexpr int FLASH_WIDE_ROWS = 128;
// Most key splits of one attention call (flash_kv_splits); the merge holds them all.
constexpr int FLASH_MAX_SPLITS = 8;
void launch_flash_wide(const FlashParams& p, int D, dim3 grid, hipStream_t stream);
// persist: grid of q_tiles x H workgroups, each walking the batch entries of its query
// tile and head (no Q RoPE, no key splits, flash_v2_persist_fits).
void launch_flash_v2(const FlashParams& p, int D, dim3 grid, hipStream_t stream, bool persist = false);
bool flash_v2_persist_fits(const FlashParams& p, int D);
void launch_flash_combine(const FlashParams& p, int D, int batch, hipStream_t stream);
void launch_generic(const FlashParams& p, int D, int batch, hipStream_t stream);
void launch_legacy_mps(const FlashParams& p, int D, int batch, hipStream_t stream);
void launch_prologue(const PrologueParams& p, hipStream_t stream);

class AttentionExecutor {
 public:
  AttentionExecutor(anima_ctx* ctx, const anima_attention_config& cfg);
  void encode(const anima_attention_args& a);
  // encode() with its workspace taken from the library's static per-device scratch
  // (at most 64 MiB) instead of the executor's allocations: no hipMalloc/hipFree.
  void encode_noalloc(const anima_attention_args& a);
  int64_t maximum_score_scratch_bytes(int64_t key_count, int64_t query_count) const;
  int64_t workspace_bytes() const { return ws_.capacity() + split_ws_.capacity(); }
  anima_ctx* context() const { return ctx_; }

 private:
  void encode_impl(const anima_attention_args& a, bool no_alloc);
  anima_ctx* ctx_;
  anima_attention_config cfg_;
  Workspace ws_;
  Workspace split_ws_;   // key-split partial rows (fp32 O, max, row sum)
};

}  // namespace anima

struct anima_attention {
  anima::AttentionExecutor impl;
  anima_attention(anima_ctx* c, const anima_attention_config& cfg) : impl(c, cfg) {}
};
