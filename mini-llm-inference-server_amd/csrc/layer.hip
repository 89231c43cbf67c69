// One layer of the paged hot path in one host call: KV append (RoPE optionally fused), decode + merge,
// prefill, in that order on one stream (reference TorchRefBackend.forward = write_kv + paged_attention,
// src/minillm/attention/torch_ref.py:46-48).  The launches and their results are those of the separate
// entry points; what changes is the host's cost per layer, one foreign call instead of three or four.
#include "common.h"

extern "C" int mllm_attention_forward(const mllm_layer_step* s, const void* q, int64_t q_stride_tok,
                                      int64_t q_stride_head, const void* k, int64_t k_stride_tok,
                                      int64_t k_stride_head, const void* v, int64_t v_stride_tok,
                                      int64_t v_stride_head, const void* cos, const void* sin, int64_t cs_stride_tok,
                                      void* q_rot, void* k_cache, void* v_cache, float k_scale, float v_scale,
                                      void* out, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(s, MLLM_ERR_INVALID, "mllm_attention_forward: null step");
  MLLM_REQUIRE(s->kv_fp8 || (k_scale == 1.f && v_scale == 1.f), MLLM_ERR_INVALID,
               "mllm_attention_forward: k_scale / v_scale apply to fp8 pools only");
  MLLM_REQUIRE(!cos == !sin && (!cos || q_rot), MLLM_ERR_INVALID,
               "mllm_attention_forward: cos, sin and q_rot go together");
  const bool fp8 = s->kv_fp8 != 0;
  const int64_t slots = s->num_blocks * s->block_size;
  const int64_t row = (int64_t)s->num_heads * s->head_dim;  // q_rot and out: contiguous [N, H, Dh]
  int rc;
  const void* qa = q;
  int64_t qa_st = q_stride_tok, qa_sh = q_stride_head;
  if (cos) {
    rc = fp8 ? mllm_rope_kv_append_fp8(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v, v_stride_tok,
                                       v_stride_head, cos, sin, cs_stride_tok, s->num_heads, s->num_kv_heads,
                                       s->head_dim, s->dtype, q_rot, row, s->head_dim, k_cache, v_cache, slots,
                                       s->slot_mapping, s->num_tokens, k_scale, v_scale, stream)
             : mllm_rope_kv_append(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v, v_stride_tok,
                                   v_stride_head, cos, sin, cs_stride_tok, s->num_heads, s->num_kv_heads, s->head_dim,
                                   s->dtype, q_rot, row, s->head_dim, k_cache, v_cache, slots, s->slot_mapping,
                                   s->num_tokens, stream);
    qa = q_rot;
    qa_st = row;
    qa_sh = s->head_dim;
  } else {
    rc = fp8 ? mllm_kv_append_fp8(k, k_stride_tok, k_stride_head, v, v_stride_tok, v_stride_head, s->dtype, k_cache,
                                  v_cache, slots, s->num_kv_heads, s->head_dim, s->slot_mapping, s->num_tokens,
                                  k_scale, v_scale, stream)
             : mllm_kv_append(k, k_stride_tok, k_stride_head, v, v_stride_tok, v_stride_head, s->dtype, k_cache,
                              v_cache, s->dtype, slots, s->num_kv_heads, s->head_dim, s->slot_mapping, s->num_tokens,
                              stream);
  }
  if (rc != MLLM_OK) return rc;
  if (s->num_decode_work > 0) {
    rc = fp8 ? mllm_paged_decode_fp8(qa, qa_st, qa_sh, k_cache, v_cache, s->num_blocks, s->block_size, s->num_heads,
                                     s->num_kv_heads, s->head_dim, s->qo_indptr, s->kv_indptr, s->kv_indices,
                                     s->seq_lens, s->decode_work, s->num_decode_work, s->merge_work,
                                     s->num_merge_work, s->pages_per_split, s->softmax_scale, s->dtype, k_scale,
                                     v_scale, out, row, s->head_dim, s->workspace, s->workspace_bytes, stream)
             : mllm_paged_decode(qa, qa_st, qa_sh, k_cache, v_cache, s->num_blocks, s->block_size, s->num_heads,
                                 s->num_kv_heads, s->head_dim, s->qo_indptr, s->kv_indptr, s->kv_indices, s->seq_lens,
                                 s->decode_work, s->num_decode_work, s->merge_work, s->num_merge_work,
                                 s->pages_per_split, s->softmax_scale, s->dtype, out, row, s->head_dim, s->workspace,
                                 s->workspace_bytes, stream);
    if (rc != MLLM_OK) return rc;
    rc = mllm_merge_splits(s->merge_work, s->num_merge_work, s->num_decode_work, s->num_heads, s->head_dim,
                           s->qo_indptr, s->dtype, out, row, s->head_dim, s->workspace, s->workspace_bytes, stream);
    if (rc != MLLM_OK) return rc;
  }
  if (s->num_prefill_work > 0) {
    rc = fp8 ? mllm_paged_prefill_fp8(qa, qa_st, qa_sh, k_cache, v_cache, s->num_blocks, s->block_size,
                                      s->num_heads, s->num_kv_heads, s->head_dim, s->qo_indptr, s->kv_indptr,
                                      s->kv_indices, s->seq_lens, s->prefill_work, s->num_prefill_work,
                                      s->q_tile_tokens, s->softmax_scale, s->dtype, k_scale, v_scale, out, row,
                                      s->head_dim, stream)
             : mllm_paged_prefill(qa, qa_st, qa_sh, k_cache, v_cache, s->num_blocks, s->block_size, s->num_heads,
                                  s->num_kv_heads, s->head_dim, s->qo_indptr, s->kv_indptr, s->kv_indices,
                                  s->seq_lens, s->prefill_work, s->num_prefill_work, s->q_tile_tokens,
                                  s->softmax_scale, s->dtype, out, row, s->head_dim, stream);
  }
  return rc;
}
