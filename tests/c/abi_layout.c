/* A C caller of include/anima_hip.h, compiled by tests/test_abi_c.py with the host C
 * compiler.  It prints, as JSON:
 *   - "layout": offset and size of every field of every struct the header declares,
 *     as the C compiler lays them out (a Swift or C binding imports the header itself,
 *     so this is the layout the Python ctypes mirror must match);
 *   - "rejections": the status and message of requests that fail validation, made
 *     through the C entry points themselves (no device work: every one fails before
 *     a launch, and the context binds its device lazily).
 */
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include "anima_hip.h"

static int first = 1;
#define SEP() (first ? (first = 0, "") : ",\n")
#define FIELD(S, f) printf("%s  \"%s.%s\": [%zu, %zu]", SEP(), #S, #f, offsetof(S, f), sizeof(((S*)0)->f))
#define SIZE(S) printf("%s  \"%s\": [0, %zu]", SEP(), #S, sizeof(S))

static void json_string(const char* s) {
  putchar('"');
  for (; *s; ++s) {
    if (*s == '"' || *s == '\\') putchar('\\');
    putchar(*s);
  }
  putchar('"');
}

static int rfirst = 1;
static void rejection(const char* name, anima_status st) {
  printf("%s  [", rfirst ? "" : ",\n");
  rfirst = 0;
  json_string(name);
  printf(", %d, ", (int)st);
  json_string(anima_last_error());
  printf("]");
}

int main(void) {
  printf("{\"abi_version\": %d,\n\"layout\": {\n", anima_abi_version());
  SIZE(anima_buffer);
  FIELD(anima_buffer, ptr); FIELD(anima_buffer, length);

  SIZE(anima_attention_config);
  FIELD(anima_attention_config, tile_rows); FIELD(anima_attention_config, numerics);
  FIELD(anima_attention_config, backend); FIELD(anima_attention_config, layout);
  FIELD(anima_attention_config, token_stride); FIELD(anima_attention_config, flash_rows);

  SIZE(anima_qk_prologue);
  FIELD(anima_qk_prologue, q_norm_weight); FIELD(anima_qk_prologue, k_norm_weight); FIELD(anima_qk_prologue, eps);
  FIELD(anima_qk_prologue, rope); FIELD(anima_qk_prologue, rope_tokens); FIELD(anima_qk_prologue, rope_q);
  FIELD(anima_qk_prologue, rope_k); FIELD(anima_qk_prologue, k_rope); FIELD(anima_qk_prologue, k_rope_tokens);

  SIZE(anima_attention_args);
  FIELD(anima_attention_args, query); FIELD(anima_attention_args, query_offset);
  FIELD(anima_attention_args, key); FIELD(anima_attention_args, key_offset);
  FIELD(anima_attention_args, value); FIELD(anima_attention_args, value_offset);
  FIELD(anima_attention_args, output); FIELD(anima_attention_args, output_offset);
  FIELD(anima_attention_args, heads); FIELD(anima_attention_args, query_count);
  FIELD(anima_attention_args, key_count); FIELD(anima_attention_args, head_dim);
  FIELD(anima_attention_args, key_value_heads); FIELD(anima_attention_args, causal);
  FIELD(anima_attention_args, layout); FIELD(anima_attention_args, token_stride);
  FIELD(anima_attention_args, batch); FIELD(anima_attention_args, key_lengths);
  FIELD(anima_attention_args, key_lengths_on_device); FIELD(anima_attention_args, scale);
  FIELD(anima_attention_args, prologue); FIELD(anima_attention_args, kv_token_stride);

  SIZE(anima_qweight);
  FIELD(anima_qweight, storage); FIELD(anima_qweight, packed); FIELD(anima_qweight, packed_offset);
  FIELD(anima_qweight, scale); FIELD(anima_qweight, scale_offset); FIELD(anima_qweight, zero);
  FIELD(anima_qweight, zero_offset); FIELD(anima_qweight, rows); FIELD(anima_qweight, columns);
  FIELD(anima_qweight, packed_row_stride);

  SIZE(anima_linear_config);
  FIELD(anima_linear_config, tile_rows); FIELD(anima_linear_config, backend);

  SIZE(anima_dit_block_weights);
  FIELD(anima_dit_block_weights, self_q); FIELD(anima_dit_block_weights, self_k);
  FIELD(anima_dit_block_weights, self_v); FIELD(anima_dit_block_weights, self_o);
  FIELD(anima_dit_block_weights, cross_q); FIELD(anima_dit_block_weights, cross_k);
  FIELD(anima_dit_block_weights, cross_v); FIELD(anima_dit_block_weights, cross_o);
  FIELD(anima_dit_block_weights, mlp1); FIELD(anima_dit_block_weights, mlp2);
  FIELD(anima_dit_block_weights, mod_self_w1); FIELD(anima_dit_block_weights, mod_self_w2);
  FIELD(anima_dit_block_weights, mod_cross_w1); FIELD(anima_dit_block_weights, mod_cross_w2);
  FIELD(anima_dit_block_weights, mod_mlp_w1); FIELD(anima_dit_block_weights, mod_mlp_w2);
  FIELD(anima_dit_block_weights, self_q_norm); FIELD(anima_dit_block_weights, self_k_norm);
  FIELD(anima_dit_block_weights, cross_q_norm); FIELD(anima_dit_block_weights, cross_k_norm);

  SIZE(anima_dit_block_args);
  FIELD(anima_dit_block_args, residual); FIELD(anima_dit_block_args, emb); FIELD(anima_dit_block_args, adaln_lora);
  FIELD(anima_dit_block_args, context); FIELD(anima_dit_block_args, rope); FIELD(anima_dit_block_args, tokens);
  FIELD(anima_dit_block_args, dim); FIELD(anima_dit_block_args, heads); FIELD(anima_dit_block_args, head_dim);
  FIELD(anima_dit_block_args, context_tokens); FIELD(anima_dit_block_args, context_dim);
  FIELD(anima_dit_block_args, mlp_hidden); FIELD(anima_dit_block_args, eps);

  SIZE(anima_qwen_layer_weights);
  FIELD(anima_qwen_layer_weights, q); FIELD(anima_qwen_layer_weights, k); FIELD(anima_qwen_layer_weights, v);
  FIELD(anima_qwen_layer_weights, o); FIELD(anima_qwen_layer_weights, gate); FIELD(anima_qwen_layer_weights, up);
  FIELD(anima_qwen_layer_weights, down); FIELD(anima_qwen_layer_weights, input_norm);
  FIELD(anima_qwen_layer_weights, post_attention_norm); FIELD(anima_qwen_layer_weights, q_norm);
  FIELD(anima_qwen_layer_weights, k_norm);

  SIZE(anima_qwen_layer_args);
  FIELD(anima_qwen_layer_args, residual); FIELD(anima_qwen_layer_args, rope);
  FIELD(anima_qwen_layer_args, key_lengths); FIELD(anima_qwen_layer_args, batch);
  FIELD(anima_qwen_layer_args, tokens); FIELD(anima_qwen_layer_args, hidden); FIELD(anima_qwen_layer_args, heads);
  FIELD(anima_qwen_layer_args, kv_heads); FIELD(anima_qwen_layer_args, head_dim);
  FIELD(anima_qwen_layer_args, intermediate); FIELD(anima_qwen_layer_args, eps);

  SIZE(anima_dit_prepare_weights);
  FIELD(anima_dit_prepare_weights, x_embed); FIELD(anima_dit_prepare_weights, t_embed1);
  FIELD(anima_dit_prepare_weights, t_embed2); FIELD(anima_dit_prepare_weights, t_norm);

  SIZE(anima_dit_prepare_args);
  FIELD(anima_dit_prepare_args, latent); FIELD(anima_dit_prepare_args, height); FIELD(anima_dit_prepare_args, width);
  FIELD(anima_dit_prepare_args, sigma); FIELD(anima_dit_prepare_args, residual); FIELD(anima_dit_prepare_args, emb);
  FIELD(anima_dit_prepare_args, adaln_lora); FIELD(anima_dit_prepare_args, dim); FIELD(anima_dit_prepare_args, eps);

  SIZE(anima_dit_final_weights);
  FIELD(anima_dit_final_weights, mod_w1); FIELD(anima_dit_final_weights, mod_w2); FIELD(anima_dit_final_weights, proj);

  SIZE(anima_dit_final_args);
  FIELD(anima_dit_final_args, residual); FIELD(anima_dit_final_args, emb); FIELD(anima_dit_final_args, adaln_lora);
  FIELD(anima_dit_final_args, velocity); FIELD(anima_dit_final_args, height); FIELD(anima_dit_final_args, width);
  FIELD(anima_dit_final_args, dim); FIELD(anima_dit_final_args, eps);

  SIZE(anima_pack_info);
  FIELD(anima_pack_info, version); FIELD(anima_pack_info, component); FIELD(anima_pack_info, alignment);
  FIELD(anima_pack_info, tensor_count); FIELD(anima_pack_info, json_offset); FIELD(anima_pack_info, json_size);
  FIELD(anima_pack_info, table_offset); FIELD(anima_pack_info, table_bytes); FIELD(anima_pack_info, payload_offset);
  FIELD(anima_pack_info, file_size); FIELD(anima_pack_info, record_size); FIELD(anima_pack_info, quant_group);
  FIELD(anima_pack_info, quant_scheme); FIELD(anima_pack_info, component_name);

  SIZE(anima_pack_tensor);
  FIELD(anima_pack_tensor, name); FIELD(anima_pack_tensor, storage); FIELD(anima_pack_tensor, rank);
  FIELD(anima_pack_tensor, shape); FIELD(anima_pack_tensor, blob_offset); FIELD(anima_pack_tensor, blob_size);
  FIELD(anima_pack_tensor, data_offset); FIELD(anima_pack_tensor, data_size); FIELD(anima_pack_tensor, scale_offset);
  FIELD(anima_pack_tensor, scale_size); FIELD(anima_pack_tensor, zero_offset); FIELD(anima_pack_tensor, zero_size);
  FIELD(anima_pack_tensor, block_index); FIELD(anima_pack_tensor, crc32); FIELD(anima_pack_tensor, has_crc32);
  FIELD(anima_pack_tensor, logical_dtype); FIELD(anima_pack_tensor, quantization_format);

  SIZE(anima_pack_range);
  FIELD(anima_pack_range, logical_index); FIELD(anima_pack_range, file_offset); FIELD(anima_pack_range, length);
  FIELD(anima_pack_range, tensor_count); FIELD(anima_pack_range, host);
  printf("\n},\n\"rejections\": [\n");

  /* Requests that must fail validation, through the C entry points. */
  char fake[16];
  const anima_buffer big = {fake, 1 << 20};
  anima_ctx* ctx = NULL;
  rejection("ctx_create", anima_ctx_create(0, &ctx));
  rejection("ctx_create_negative", anima_ctx_create(-1, NULL));

  anima_attention_config acfg = {128, ANIMA_NUMERICS_FP32_SCORES, ANIMA_ATTENTION_BACKEND_AUTO,
                                 ANIMA_LAYOUT_HEAD_MAJOR, 0, 0};
  anima_attention* attn = NULL;
  rejection("attention_create", anima_attention_create(ctx, &acfg, &attn));
  anima_attention_args a;
  memset(&a, 0, sizeof a);
  a.query = a.key = a.value = a.output = big;
  a.heads = 2; a.query_count = 4; a.key_count = 4; a.head_dim = 64; a.layout = -1;
  a.causal = 1; a.key_count = 5;
  rejection("attention_causal_counts", anima_attention_encode(attn, &a));
  a.causal = 0; a.key_count = 4;
  a.layout = ANIMA_LAYOUT_TOKEN_MAJOR; a.token_stride = 100;
  rejection("attention_token_major_stride", anima_attention_encode(attn, &a));
  a.layout = -1; a.token_stride = 0;
  anima_qk_prologue pro;
  memset(&pro, 0, sizeof pro);
  pro.eps = 1e-6f;
  pro.q_norm_weight.ptr = fake; pro.q_norm_weight.length = 64 * 2 - 2;
  a.prologue = &pro;
  rejection("attention_short_q_norm", anima_attention_encode(attn, &a));
  pro.q_norm_weight.length = 64 * 2;
  pro.rope.ptr = fake; pro.rope.length = 4 * 64 * 8 - 4; pro.rope_tokens = 4; pro.rope_q = 1;
  rejection("attention_short_rope", anima_attention_encode(attn, &a));
  a.prologue = NULL;
  a.output.length = 2 * 4 * 64 * 2 - 2;
  rejection("attention_output_range", anima_attention_encode(attn, &a));
  rejection("attention_null_handle", anima_attention_encode(NULL, &a));

  anima_linear_config lcfg = {128, ANIMA_LINEAR_BACKEND_AUTO};
  anima_linear* lin = NULL;
  rejection("linear_create", anima_linear_create(ctx, &lcfg, &lin));
  anima_qweight w;
  memset(&w, 0, sizeof w);
  w.storage = ANIMA_STORAGE_W4; w.packed = w.scale = w.zero = big;
  w.rows = 8; w.columns = 64; w.packed_row_stride = 31;
  rejection("linear_stride", anima_linear_encode(lin, big, 0, &w, big, 0, 4, ANIMA_FAMILY_OTHER));
  w.packed_row_stride = 32; w.storage = ANIMA_STORAGE_FP32;
  rejection("linear_storage", anima_linear_encode(lin, big, 0, &w, big, 0, 4, ANIMA_FAMILY_OTHER));
  w.storage = ANIMA_STORAGE_W4; w.scale.length = 15;
  rejection("linear_scale_range", anima_linear_encode(lin, big, 0, &w, big, 0, 4, ANIMA_FAMILY_OTHER));

  anima_cross_kv_cache* cache = NULL;
  rejection("cache_shape", anima_cross_kv_cache_create(ctx, 0, 512, 2048, &cache));
  anima_weight_streamer* st = NULL;
  rejection("streamer_slots", anima_weight_streamer_create(ctx, 1 << 20, 9, &st));
  rejection("rope_dit3d_shape", anima_rope_dit3d(0, 1, 1, NULL));
  rejection("euler_sigma", anima_euler_step_encode(ctx, big, big, big, 0.0f, 0.5f, 4));
  rejection("patchify_odd", anima_patchify17_encode(ctx, big, 17, 3, 4, big));
  anima_dit_prepare* prep = NULL;
  rejection("prepare_create", anima_dit_prepare_create(ctx, &prep));
  anima_dit_prepare_weights pw;
  memset(&pw, 0, sizeof pw);
  anima_dit_prepare_args pa;
  memset(&pa, 0, sizeof pa);
  pa.sigma = 1.0f / 0.0f;
  rejection("prepare_sigma", anima_dit_prepare_encode(prep, &pw, &pa));
  anima_dit_prepare_destroy(prep);
  anima_pack* pack = NULL;
  rejection("pack_missing", anima_pack_open("/nonexistent/dir/x.animapk", &pack));

  anima_linear_destroy(lin);
  anima_attention_destroy(attn);
  anima_ctx_destroy(ctx);
  printf("\n]}\n");
  return 0;
}
