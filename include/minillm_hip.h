/*
 * minillm_hip.h — C ABI of the MI355X (gfx950) paged-attention library.
 *
 * Every entry point takes raw device pointers, explicit sizes and element strides, and a HIP stream
 * (passed as void*), launches asynchronously on that stream and never synchronises the host.  The
 * library never allocates device memory: the caller (PyTorch, in the host package) owns every buffer,
 * including the decode workspace whose size mllm_decode_workspace_bytes() reports.  The one device
 * memory of its own is the fixed scratch array of mllm_paged_decode_noalloc (64 MiB per GPU, part of
 * the loaded code object).
 *
 * Status: 0 on success, negative on failure; mllm_last_error() then returns a per-thread message.
 *   MLLM_ERR_INVALID     malformed arguments            (the Python wrapper raises ValueError)
 *   MLLM_ERR_UNSUPPORTED shape or dtype not supported   (ValueError)
 *   MLLM_ERR_HIP         a HIP launch or runtime error  (RuntimeError)
 *
 * The pool layout is the reference's (cache/paged.py:24-31): per layer, separate K and V tensors
 * [num_blocks, block_size, Hkv, Dh], contiguous (NHD: token-major inside a block); the flat slot of
 * token p of a sequence is block_ids[p / block_size] * block_size + p % block_size.
 */
#ifndef MINILLM_HIP_H
#define MINILLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLLM_ABI_VERSION 4

#define MLLM_OK 0
#define MLLM_ERR_INVALID (-1)
#define MLLM_ERR_UNSUPPORTED (-2)
#define MLLM_ERR_HIP (-3)

/* element types (torch.float32, torch.float16, torch.bfloat16) */
#define MLLM_DTYPE_F32 0
#define MLLM_DTYPE_F16 1
#define MLLM_DTYPE_BF16 2

/* ABI version of the loaded library (MLLM_ABI_VERSION at build time). */
int mllm_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mllm_last_error(void);

/*
 * Ragged metadata build, on the GPU.
 * Replaces the host loops and eleven host->device copies of AttentionMetadata.build
 * (reference src/minillm/attention/metadata.py:70-103) with one upload of the block manager's tables
 * and two launches.
 *
 * Inputs (device, int32): num_cached[S], num_new[S] (reference SeqStep, metadata.py:27-33), and each
 * sequence's block table in CSR form: table_indptr[S+1] into table_ids[].  The caller has checked that
 * every table holds its sequence (metadata.py:75-76 raises ValueError otherwise) and passes
 * table_width = max table length.
 * Outputs (device), bit-identical in dtype and value to the reference fields (metadata.py:93-102):
 *   int64 positions[N], slot_mapping[N], block_tables[S * table_width] (row-major, padded with 0),
 *         logits_index[S]
 *   int32 qo_indptr[S+1], seq_lens[S], block_tables_i32[S * table_width], kv_indptr[S+1],
 *         kv_indices[sum ceil(len/bs)], kv_last_page_len[S]
 * N = sum num_new.  Any output pointer may be NULL to skip that field, except qo_indptr and kv_indptr.
 */
int mllm_build_metadata(const int32_t* num_cached, const int32_t* num_new, const int32_t* table_indptr,
                        const int32_t* table_ids, int32_t num_seqs, int32_t block_size, int32_t table_width,
                        int64_t* positions, int64_t* slot_mapping, int64_t* block_tables, int64_t* logits_index,
                        int32_t* qo_indptr, int32_t* seq_lens, int32_t* block_tables_i32, int32_t* kv_indptr,
                        int32_t* kv_indices, int32_t* kv_last_page_len, void* stream);

/*
 * The same build from a device-resident mirror of the block manager's tables (the reference rebuilds
 * and uploads every table each step, metadata.py:82-83,101):
 * tables[rows x table_stride] holds one request per row; sequence s of the step reads row seq_rows[s],
 * whose first seq_num_blocks[s] entries are its block_ids.  Only num_cached, num_new, seq_rows and
 * seq_num_blocks travel with the step.  Outputs as mllm_build_metadata, bit-identical.
 */
int mllm_build_metadata_rows(const int32_t* num_cached, const int32_t* num_new, const int32_t* seq_rows,
                             const int32_t* seq_num_blocks, const int32_t* tables, int32_t table_stride,
                             int32_t num_seqs, int32_t block_size, int32_t table_width, int64_t* positions,
                             int64_t* slot_mapping, int64_t* block_tables, int64_t* logits_index, int32_t* qo_indptr,
                             int32_t* seq_lens, int32_t* block_tables_i32, int32_t* kv_indptr, int32_t* kv_indices,
                             int32_t* kv_last_page_len, void* stream);

/*
 * Keeps the resident mirror current: for i < num_updates, tables[updates[2 i]] = updates[2 i + 1] (flat
 * index, block id); indices outside [0, table_size) are skipped.  The step's newly allocated blocks
 * are its only updates, so a decode step sends a few ids instead of every table.
 */
int mllm_update_block_tables(int32_t* tables, int64_t table_size, const int32_t* updates, int32_t num_updates,
                             void* stream);

/*
 * KV append: scatter N new K and V rows into the pool at slot_mapping.
 * Replaces write_kv (reference src/minillm/attention/paged_torch_ref.py:23-28), i.e.
 *   k_cache.view(-1, Hkv, Dh).index_copy_(0, slot_mapping, k.to(k_cache.dtype)), same for v.
 * k, v: [N, Hkv, Dh] with element strides (stride_tok, stride_head) and unit stride on Dh.
 * The value conversion when src_dtype != cache_dtype rounds to nearest even, as torch's .to() does.
 * Bit-exact.  Slots outside [0, num_slots) are not written.
 */
int mllm_kv_append(const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v, int64_t v_stride_tok,
                   int64_t v_stride_head, int32_t src_dtype, void* k_cache, void* v_cache, int32_t cache_dtype,
                   int64_t num_slots, int32_t num_kv_heads, int32_t head_dim, const int64_t* slot_mapping,
                   int64_t num_tokens, void* stream);

/*
 * Rotary embedding fused with the KV append (the step right before the attention path): the model's
 * RoPE of q and k (reference src/minillm/model/llama.py:58-72, apply_rotary with the "rotate half"
 * pairing of dims d and d + Dh/2) and write_kv (paged_torch_ref.py:23-28) in one launch:
 *   q_out[n, h]                   = q[n, h] * cos[n] + rotate_half(q[n, h]) * sin[n]
 *   k_cache[slot_mapping[n], h']  = k[n, h'] * cos[n] + rotate_half(k[n, h']) * sin[n]
 *   v_cache[slot_mapping[n], h']  = v[n, h']
 * cos / sin: [N, Dh] rows of the model's full-width tables (RotaryEmbedding output, dtype `dtype`).
 * Bit-exact with those torch expressions on 16-bit tensors: each product is rounded to `dtype`, then
 * the sum.  q/k/v/q_out: [N, heads, Dh] with element strides (tok, head); all buffers share `dtype`
 * (BF16 or F16), rows 16-byte aligned, head_dim a multiple of 16.  Slots outside [0, num_slots) are
 * not written.
 */
int mllm_rope_kv_append(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
                        int64_t k_stride_tok, int64_t k_stride_head, const void* v, int64_t v_stride_tok,
                        int64_t v_stride_head, const void* cos, const void* sin, int64_t cs_stride_tok,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype, void* q_out,
                        int64_t q_out_stride_tok, int64_t q_out_stride_head, void* k_cache, void* v_cache,
                        int64_t num_slots, const int64_t* slot_mapping, int64_t num_tokens, void* stream);

/*
 * Per-step work plan (the analogue of FlashInfer's plan(), which the reference runs once per step:
 * src/minillm/attention/flashinfer_backend.py:44-64).  Built on the GPU from qo_indptr / kv_indptr /
 * seq_lens (tokens per row, cached + new).
 *   decode rows (num_new == 1): their pages, rows in sequence order, form one stream of T pages, cut into
 *     nb = ceil(T / pages_per_split) bins; bin b holds pages floor(b T / nb) .. floor((b + 1) T / nb) - 1
 *     (stream-K: one decode workgroup per bin, equal work for every wavefront).  A row's part inside a
 *     bin is a segment.  decode_work[num_decode_work] (int4 records) receives:
 *       [0]                       {nb, segments, partial slots, 0} (overflow: {0, records, merges, -1})
 *       [1 + b]                   {first segment, end segment, 1 + nb, -} of bin b
 *       [1 + nb + 2 g], [.. + 1]  segment g: {first page's index in kv_indices, pages, first page within
 *                                 the row, row length}, {qo_indptr[seq], partial slot or -1, seq, 0}
 *     A row cut into several segments gets consecutive partial slots, one per segment, and an int4
 *     {seq, first slot, segments, 0}, in sequence order -> merge_work[num_merge_work]; a row inside one
 *     bin gets slot -1 (its segment writes the output).  1 + nb + 2 segments <= num_decode_work and
 *     segments <= nb + rows - 1; cut rows <= min(rows, nb - 1).
 *   multi-token rows: one item per tile of q_tile_tokens new tokens, 8 int32 each:
 *     {seq, first_new_token, qo_indptr[seq], new tokens of seq, cached tokens of seq, kv_indptr[seq],
 *      keys visible to the tile's last token, 64-key tiles they span} -> prefill_work[8 * num_prefill_work],
 *     across all rows in decreasing number of those tiles (the prefill kernel's work per item).
 * The caller computes the capacities from the facts the plan itself counts: the decode rows' page
 * counts kv_indptr[s + 1] - kv_indptr[s] (which may exceed ceil(seq_len / block_size) when a page list
 * runs past the row's last token), the number of decode rows, and the new-token counts; it fills the
 * buffers with -1 beforehand.  A step whose decode plan does not fit num_decode_work records or
 * num_merge_work merges gets no decode work at all: the header then reads {0, records needed, merges
 * needed, -1} (a step with no decode pages reads {0, 0, 0, 0}), so the decode and merge kernels never
 * index past a workspace sized for num_decode_work partial slots, and a caller that reads the header
 * sees the overflow.  Prefill items past num_prefill_work are dropped.  pages_per_split <= 192.
 */
int mllm_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* seq_lens, int32_t num_seqs,
              int32_t pages_per_split, int32_t q_tile_tokens, int32_t* decode_work, int32_t num_decode_work,
              int32_t* merge_work, int32_t num_merge_work, int32_t* prefill_work, int32_t num_prefill_work,
              void* stream);

/*
 * mllm_plan with the split size read from device memory at run time (*pages_per_split, clamped to
 * [min_pages_per_split, 192]).  No counterpart in the reference: it serves HIP-graph capture of decode steps
 * (the reference's planned M8, docs/distributed_inference_plan.md:309), where one captured plan launch
 * re-plans every replayed step.  The caller checks on the host that a staged step's items fit the
 * capacities at the split size it stages (or runs that step without the graph), so no item is dropped;
 * items past a step's own stay as the caller pre-filled them (-1).
 */
int mllm_plan_dev(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* seq_lens, int32_t num_seqs,
                  const int32_t* pages_per_split, int32_t min_pages_per_split, int32_t q_tile_tokens,
                  int32_t* decode_work, int32_t num_decode_work, int32_t* merge_work, int32_t num_merge_work,
                  int32_t* prefill_work, int32_t num_prefill_work, void* stream);

/* Bytes of the fp32 split-KV partials a plan of num_decode_work records can need: (num_decode_work - 1) / 2
 * partial slots (every slot is a segment of a cut row, and each segment takes two records after the
 * header), each (m, l, acc[Dh]) for num_heads heads. */
int64_t mllm_decode_workspace_bytes(int32_t num_decode_work, int32_t num_heads, int32_t head_dim);

/*
 * Paged decode attention: one new token per row, over its whole context in the pool
 * (reference src/minillm/attention/paged_torch_ref.py:47-59, decode branch; FlashInfer
 * BatchDecodeWithPagedKVCacheWrapper, flashinfer_backend.py:55-58).  One workgroup per (bin of the plan,
 * KV-head group) streams the bin's row segments on bf16/fp16 MFMA with an fp32 online softmax; the grid
 * covers (num_decode_work - 1) / 3 bins, and workgroups past the plan's own exit at once.  Scale softmax_scale (1/sqrt(Dh) in the
 * reference); query head h reads KV head h / (H / Hkv).
 * q/out: [N, H, Dh] with element strides (tok, head), unit stride on Dh; only the rows of decode
 * sequences are read and written.  A row inside one bin gets its output here; a row cut across bins
 * writes fp32 partials (m, l, acc) into the workspace, which mllm_merge_splits then combines, so the
 * two calls go back to back on one stream.  head_dim 128, block_size a multiple of 16,
 * H / Hkv <= 16, dtype F16 or BF16; num_merge_work (from mllm_plan) only sizes the workspace check.
 */
int mllm_paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                      const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                      int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr, const int32_t* kv_indptr,
                      const int32_t* kv_indices, const int32_t* seq_lens, const int32_t* decode_work,
                      int32_t num_decode_work, const int32_t* merge_work, int32_t num_merge_work,
                      int32_t pages_per_split, float softmax_scale, int32_t dtype, void* out, int64_t out_stride_tok,
                      int64_t out_stride_head, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Log-sum-exp merge of the split-KV partials mllm_paged_decode left in the workspace, one
 * {seq, first partial slot, segments, 0} merge item (mllm_plan) per row cut into several segments:
 *   out = sum_j 2^(m_j - M) acc_j / sum_j 2^(m_j - M) l_j,  M = max_j m_j   (exp2 domain).
 * This is the same combine FlashInfer's split-KV decode performs after its chunks.
 */
int mllm_merge_splits(const int32_t* merge_work, int32_t num_merge_work, int32_t num_decode_work, int32_t num_heads,
                      int32_t head_dim, const int32_t* qo_indptr, int32_t dtype, void* out, int64_t out_stride_tok,
                      int64_t out_stride_head, const void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mllm_paged_decode followed by mllm_merge_splits, allocating nothing: no counterpart in the reference.
 * It is for callers that cannot allocate device memory (code under HIP-graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split-KV partials go to a fixed 64 MiB (67,108,864-byte)
 * device array of this library instead of a caller workspace: each GPU the library runs on holds its
 * own copy until the process ends, looked up on the first call on that device (the current device;
 * the stream must belong to it).  A step whose partials need more
 * (mllm_decode_workspace_bytes(num_decode_work, H, Dh) > 64 MiB when num_merge_work > 0; 8,066 plan
 * records at H = 32, Dh = 128) is rejected with MLLM_ERR_INVALID.  Calls that overlap on one GPU (other streams or
 * threads) share the array and race; calls in order on one stream do not.  Arguments and results are
 * mllm_paged_decode's and mllm_merge_splits' (16-bit pools), bit for bit.
 */
int mllm_paged_decode_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                              const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                              const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                              const int32_t* decode_work, int32_t num_decode_work, const int32_t* merge_work,
                              int32_t num_merge_work, int32_t pages_per_split, float softmax_scale, int32_t dtype,
                              void* out, int64_t out_stride_tok, int64_t out_stride_head, void* stream);

/*
 * Ragged prefill / mixed attention for rows with several new tokens (reference paged_torch_ref.py:61-73;
 * FlashInfer BatchPrefillWithPagedKVCacheWrapper, flashinfer_backend.py:59-63): causal within each new
 * chunk, bottom-right aligned over the cached prefix, K/V read through kv_indices.  QK^T and PV on
 * bf16/fp16 MFMA (32x32x16) with fp32 online softmax; the H/Hkv query heads of one KV head share
 * each K/V tile.  Work items from mllm_plan (prefill_work) with q_tile_tokens = 256 / (H / Hkv): one
 * workgroup of 8 wavefronts per (item, KV head), one per CU; or q_tile_tokens = 128 / (H / Hkv):
 * workgroups of 4 wavefronts, two per CU (for steps of few items: one workgroup's prologue and output
 * drain run under the other's main loop).  Other q_tile_tokens values are rejected.
 * Same shape limits as mllm_paged_decode, and H / Hkv must divide 32; q, out and their row strides
 * 16-byte aligned.
 */
int mllm_paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                       const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* seq_lens, const int32_t* prefill_work,
                       int32_t num_prefill_work, int32_t q_tile_tokens, float softmax_scale, int32_t dtype,
                       void* out, int64_t out_stride_tok, int64_t out_stride_head, void* stream);

/*
 * The step-constant arguments of mllm_attention_forward: shapes, the step's metadata (AttentionMetadata's
 * device fields), its work plan (mllm_plan) and the decode workspace.  The caller fills one per step and
 * passes its address to every layer's call; the library reads it during each call only.
 */
typedef struct mllm_layer_step {
  int64_t num_blocks;          /* blocks of each pool */
  int64_t num_tokens;          /* N: new tokens of the step (rows of q, k, v, out) */
  const int64_t* slot_mapping; /* [N] */
  const int32_t* qo_indptr;    /* [S + 1] */
  const int32_t* kv_indptr;    /* [S + 1] */
  const int32_t* kv_indices;
  const int32_t* seq_lens;     /* [S], int32 */
  const int32_t* decode_work;  /* the plan's three lists and their capacities */
  const int32_t* merge_work;
  const int32_t* prefill_work;
  void* workspace;             /* decode partials, >= mllm_decode_workspace_bytes(num_decode_work, H, Dh)
                                  when num_merge_work > 0 */
  int64_t workspace_bytes;
  int32_t num_decode_work, num_merge_work, num_prefill_work;
  int32_t pages_per_split, q_tile_tokens;
  int32_t num_heads, num_kv_heads, head_dim, block_size;
  int32_t dtype;               /* q, k, v, cos, sin, q_rot, out: MLLM_DTYPE_BF16 or MLLM_DTYPE_F16 */
  int32_t kv_fp8;              /* 0: pools of `dtype`; 1: fp8 e4m3fn pools with k_scale / v_scale */
  float softmax_scale;
} mllm_layer_step;

/*
 * One layer's whole hot path in one call (reference TorchRefBackend.forward = write_kv + paged_attention,
 * src/minillm/attention/torch_ref.py:46-48; the backend's forward, base.py:35-45): on `stream`, the KV
 * append of k and v at slot_mapping (mllm_kv_append / _fp8), or with cos and sin given the model's RoPE
 * of q and k fused into it (mllm_rope_kv_append / _fp8, the rotated q written to q_rot, which attention
 * then reads); then the decode rows' split-KV attention and merge (mllm_paged_decode / _fp8 +
 * mllm_merge_splits) and the multi-token rows' prefill (mllm_paged_prefill / _fp8), the same launches
 * with the same results as those calls in that order.  q, k, v: [N, heads, Dh] with element strides
 * (tok, head); cos / sin: [N, Dh] rows with stride cs_stride_tok, or NULL; q_rot (when cos is given) and
 * out: contiguous [N, H, Dh].  k_scale / v_scale apply to fp8 pools and must be 1 otherwise.  One host
 * call instead of three to four, for steps whose launches cost the host more than the GPU's work.
 */
int mllm_attention_forward(const mllm_layer_step* step, const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                           const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                           int64_t v_stride_tok, int64_t v_stride_head, const void* cos, const void* sin,
                           int64_t cs_stride_tok, void* q_rot, void* k_cache, void* v_cache, float k_scale,
                           float v_scale, void* out, void* stream);

/*
 * Contiguous causal attention, the backend's `prefill` method (reference
 * src/minillm/attention/torch_ref.py:20-44 and base.py:19-33): q [B, H, Tq, Dh], k/v [B, Hkv, Tk, Dh]
 * with element strides (batch, head, token) and unit stride on Dh; query i sits at position
 * Tk - Tq + i and sees keys 0 .. Tk - Tq + i.  key_valid [B, Tk] (one byte per key, strides
 * (batch, token), NULL for none) further limits the keys to the real ones, and a query with no real
 * key sees its own position only.  fp32/fp16/bf16, head_dim <= 256, fp32 softmax.
 */
int mllm_dense_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
                         int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         const uint8_t* key_valid, int64_t kv_sb, int64_t kv_st, int32_t batch, int32_t num_heads,
                         int32_t num_kv_heads, int32_t q_len, int32_t kv_len, int32_t head_dim, float softmax_scale,
                         int32_t dtype, void* out, int64_t o_sb, int64_t o_sh, int64_t o_st, void* stream);

/*
 * fp8 KV pool.  No counterpart in the reference's code: it is the reference's planned fp8 KV cache
 * (docs/distributed_inference_plan.md:310, milestone M9b), which halves the bytes decode streams.
 * The pool has the layout above with one byte per element, OCP float8 e4m3fn (torch.float8_e4m3fn),
 * and one scale per tensor (per layer, one for K and one for V):
 *   stored  = e4m3fn(float(x) * (1.0f / scale))   round to nearest even; magnitudes above 464 and
 *                                                  non-finite inputs store NaN (torch's cast)
 *   value   = float(stored) * scale
 * q, k, v, cos, sin and out stay in `dtype` (BF16 or F16).  Attention reads the pool's exact values
 * (every e4m3fn value is exact in bf16 and fp16), applies k_scale to the scores and v_scale to the
 * output, and otherwise matches the 16-bit entry points above, with the same shape limits.
 */

/* KV append into an fp8 pool (write_kv with the quantizing cast); head_dim a multiple of 16, rows
 * 16-byte aligned.  Bit-exact with torch's (x.float() * (1 / scale)).to(torch.float8_e4m3fn). */
int mllm_kv_append_fp8(const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                       int64_t v_stride_tok, int64_t v_stride_head, int32_t src_dtype, void* k_cache, void* v_cache,
                       int64_t num_slots, int32_t num_kv_heads, int32_t head_dim, const int64_t* slot_mapping,
                       int64_t num_tokens, float k_scale, float v_scale, void* stream);

/* mllm_rope_kv_append into an fp8 pool: the rotated k (rounded to `dtype`) and v are quantized. */
int mllm_rope_kv_append_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
                            int64_t k_stride_tok, int64_t k_stride_head, const void* v, int64_t v_stride_tok,
                            int64_t v_stride_head, const void* cos, const void* sin, int64_t cs_stride_tok,
                            int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype, void* q_out,
                            int64_t q_out_stride_tok, int64_t q_out_stride_head, void* k_cache, void* v_cache,
                            int64_t num_slots, const int64_t* slot_mapping, int64_t num_tokens, float k_scale,
                            float v_scale, void* stream);

/* mllm_paged_decode over an fp8 pool; mllm_merge_splits combines its partials unchanged. */
int mllm_paged_decode_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                          const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                          int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr, const int32_t* kv_indptr,
                          const int32_t* kv_indices, const int32_t* seq_lens, const int32_t* decode_work,
                          int32_t num_decode_work, const int32_t* merge_work, int32_t num_merge_work,
                          int32_t pages_per_split, float softmax_scale, int32_t dtype, float k_scale, float v_scale,
                          void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* mllm_paged_prefill over an fp8 pool. */
int mllm_paged_prefill_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                           const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr, const int32_t* kv_indptr,
                           const int32_t* kv_indices, const int32_t* seq_lens, const int32_t* prefill_work,
                           int32_t num_prefill_work, int32_t q_tile_tokens, float softmax_scale, int32_t dtype,
                           float k_scale, float v_scale, void* out, int64_t out_stride_tok, int64_t out_stride_head,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINILLM_HIP_H */
