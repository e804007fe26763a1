/*
 * ernie_kv.h -- C ABI of the MI355X (gfx950) ERNIE 5.5 attention KV-cache path.
 *
 * Every entry point takes device pointers, sizes and strides (in elements
 * unless marked "bytes"), enqueues its kernels on `stream` (a hipStream_t,
 * NULL = default stream) and returns 0 on success or a nonzero status
 * (1 invalid argument, 2 launch failure, 3 workspace too small);
 * ekv_last_error() names the failure.  Nothing here allocates device memory:
 * callers pass outputs and workspaces, as the reference's layers preallocate
 * `out`, `o_padded` and the top-k buffers.  No entry point synchronizes the
 * host.
 *
 * Data formats
 *   bf16          uint16_t bit patterns.
 *   fp8 page      64 token rows of `dim` e4m3fn bytes, then 64 fp32 scales
 *                 (values first, then scales -- the page layout of
 *                 src/vllm_ernie/models/ernie5_5/nvidia/attention.py:852-860);
 *                 pages `page_stride` bytes apart.  Latent rows: dim 512/576.
 *                 Indexer K rows: dim 128 (128 fp8 + 4-byte scale = 132 B per
 *                 token, attention.py:933-935).
 *   slot          block_table[seq][pos / 64] * 64 + pos % 64; negative = skip
 *                 (attention.py:845-847).
 *   quant rule    per-token scale 2^ceil(log2(max(amax,1e-10) * (1/448))),
 *                 values clamp(x / scale, +-448) rounded to nearest-even e4m3fn
 *                 (attention.py:221-227, 317-319); scale stored as fp32.
 *
 * Citations are path:line into the baidu/vLLM-ERNIE tree
 * (src/vllm_ernie/models/ernie5_5/...).
 */
#ifndef ERNIE_KV_H_
#define ERNIE_KV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread. */
const char* ekv_last_error(void);
/* ABI revision of this header (1). */
int ekv_abi_version(void);

/*
 * Latent append with fused fp8 quantization.  rows [num_tokens, row_stride]
 * bf16 (dim in {128, 512, 576}) -> the fp8 page row of slot_mapping[t].
 * Replaces the latent write MLAAttention performs on
 * `mla_attn(q, kv_c_normed, k_pe)` (nvidia/attention.py:1226, inputs built at
 * :1186-1190), the concat_and_cache-style write vLLM runs for it.
 */
int ekv_kv_append_quant(const uint16_t* rows, int64_t row_stride, int32_t num_tokens, int32_t dim,
                        const int64_t* slot_mapping, uint8_t* cache, int64_t page_stride /*bytes*/,
                        int64_t num_pages, void* stream);

/*
 * Indexer K-cache insert: k [num_tokens, k_stride] bf16 (128 wide, after
 * LayerNorm, RoPE and Hadamard) -> 128 fp8 + fp32 scale per token.
 * Replaces the K insert of SparseAttnIndexer (nvidia/attention.py:942-953,
 * `skip_k_cache_insert=False` path; FP4 writer counterpart at :831-860).
 */
int ekv_indexer_k_insert(const uint16_t* k, int64_t k_stride, int32_t num_tokens,
                         const int64_t* slot_mapping, uint8_t* kcache, int64_t page_stride /*bytes*/,
                         int64_t num_pages, void* stream);

/*
 * HCA 128->1 compressor.  For each sequence b (tokens qsl[b]..qsl[b+1]-1 at
 * consecutive positions from positions[qsl[b]]), compresses every 128-token
 * span that completes in this call from kv_score rows ([kv | score], bf16,
 * 2*dim wide) of this call and of the state ring, and writes the fp8 row to
 * compressed slot comp_block_table[b][j/64]*64 + j%64.  ape [128, dim] fp32,
 * norm_w [dim] fp32, cos_sin [max_spans, 64] fp32 (cos | sin at position
 * 128*j).  Must be called before ekv_hca_append of the same step.
 * Replaces Ernie5_5Compressor.forward -> DeepseekCompressor.forward
 * (nvidia/attention.py:398-408; weights compressor.fused_wkv_wgate,
 * nvidia/model.py:684-685).
 */
int ekv_hca_compress(const uint16_t* kv_score, int64_t kvs_stride, const int64_t* positions,
                     const int32_t* qsl, int32_t num_seqs, int32_t max_query_len, int32_t dim,
                     const uint16_t* state, const int32_t* state_slot, int32_t num_state,
                     const float* ape, const float* norm_w, float eps, const float* cos_sin,
                     int32_t max_spans, const int32_t* comp_block_table, int32_t comp_bt_stride,
                     uint8_t* pool, int64_t page_stride /*bytes*/, int64_t num_pages, void* stream);

/*
 * HCA append: quantize latent rows into slot_mapping slots, into the window
 * ring (the last `ring` positions of each sequence, ring slot
 * ring_pages[b][(p % ring)/64]*64 + (p % ring)%64) and copy the kv_score rows
 * of the last 256 positions into the state ring state[state_slot[b]][p % 256].
 * ring_pages / state may be NULL.  Replaces the SWA write of
 * DeepseekV4Attention._prepare_and_attn_fn (nvidia/attention.py:494-505).
 */
int ekv_hca_append(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                   int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                   const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                   int32_t num_seqs, uint8_t* pool, int64_t page_stride /*bytes*/, int64_t num_pages,
                   const int32_t* ring_pages, int32_t ring_stride, int32_t ring, uint16_t* state,
                   const int32_t* state_slot, int32_t num_state, void* stream);

/* ekv_hca_append into a pool of bf16 rows (64 rows of dim bf16 values a
 * page, page_stride >= 128 * dim bytes): rows stored as given.  The bf16 KV
 * row of the non-fp8 HCA class (nvidia/attention.py:542-558). */
int ekv_hca_append_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                        int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                        const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                        int32_t num_seqs, uint16_t* pool, int64_t page_stride /*bytes*/, int64_t num_pages,
                        const int32_t* ring_pages, int32_t ring_stride, int32_t ring, uint16_t* state,
                        const int32_t* state_slot, int32_t num_state, void* stream);

/*
 * The whole HCA write of one step in one call: ekv_hca_compress followed by
 * ekv_hca_append with the same arguments, both on `stream` (same bytes in the
 * pool and the state ring).  comp_block_table must not be NULL; ring_pages /
 * state may be.  workspace (16-byte aligned, at least
 * ekv_hca_write_workspace_size(num_seqs, dim) bytes, zero-filled once before
 * its first use and left zero by every call; pass the same workspace_bytes on
 * every call that shares it) may be NULL; with it, decode-sized calls
 * (max_query_len < 128) compress each completed span with dim / 64 workgroups
 * instead of one, and longer calls whose workspace holds
 * num_seqs * (max_query_len / 128 + 1) spans compress each span with D / 64
 * one-wave workgroups -- same bytes either way.  Calls that share a
 * workspace must not overlap.  Replaces the cache-write half of
 * DeepseekV4Attention._prepare_and_attn_fn (nvidia/attention.py:494-505) with
 * its compressor call (Ernie5_5Compressor.forward, nvidia/attention.py:398-408).
 */
int ekv_hca_write(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score, int64_t kvs_stride,
                  int32_t num_tokens, int32_t dim, const int64_t* slot_mapping, const int64_t* positions,
                  const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs, int32_t max_query_len,
                  uint16_t* state, const int32_t* state_slot, int32_t num_state, const float* ape,
                  const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                  const int32_t* comp_block_table, int32_t comp_bt_stride, const int32_t* ring_pages,
                  int32_t ring_stride, int32_t ring, uint8_t* pool, int64_t page_stride /*bytes*/,
                  int64_t num_pages, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of an ekv_hca_write workspace that holds num_spans spans of width
 * dim (<= 576): a call needs one per sequence, and one per sequence and span
 * slot (num_seqs * (max_query_len / 128 + 1)) for the prefill split (no
 * counterpart in the reference, whose compressor is unfused). */
int64_t ekv_hca_write_workspace_size(int32_t num_spans, int32_t dim);

/*
 * ekv_hca_write followed by ekv_hca_decode_indices of the same tokens
 * (req_ids = token_seq, query_start_loc = qsl, slot_mapping = the call's
 * slots, the given ring_pages) with the same results; decode-sized calls
 * (max_query_len < 128) build the index rows in the write's launch.  The
 * cache-write and index halves of DeepseekV4Attention._prepare_and_attn_fn
 * (nvidia/attention.py:471-539) in one call.
 */
int ekv_hca_write_step(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score, int64_t kvs_stride,
                       int32_t num_tokens, int32_t dim, const int64_t* slot_mapping, const int64_t* positions,
                       const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs, int32_t max_query_len,
                       uint16_t* state, const int32_t* state_slot, int32_t num_state, const float* ape,
                       const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                       const int32_t* comp_block_table, int32_t comp_bt_stride, const int32_t* ring_pages,
                       int32_t ring_stride, int32_t ring, uint8_t* pool, int64_t page_stride /*bytes*/,
                       int64_t num_pages, void* workspace, int64_t workspace_bytes, int32_t window,
                       int32_t* idx_out, int64_t idx_stride, int32_t width, int32_t* lengths, void* stream);

/*
 * ekv_hca_write / ekv_hca_write_step for a pool of bf16 rows (the plain KV
 * row of the non-fp8 HCA class, Ernie5_5HCAFlashInferAttention, which
 * select_ernie5_5_hca_cls picks for a non-fp8 kv_cache_dtype,
 * nvidia/attention.py:542-558): a page is 64 rows of dim bf16 values
 * (page_stride >= 128 * dim bytes; exactly that for the flat-row view the
 * sparse decode reads, nvidia/attention.py:761-763).  Latent and window-ring
 * rows are stored as given; a compressed row is the fp32 result rounded to
 * bf16 (nearest even) instead of quantized.  Everything else as the fp8
 * entry points.
 */
int ekv_hca_write_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                       int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                       const int64_t* positions, const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs,
                       int32_t max_query_len, uint16_t* state, const int32_t* state_slot, int32_t num_state,
                       const float* ape, const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                       const int32_t* comp_block_table, int32_t comp_bt_stride, const int32_t* ring_pages,
                       int32_t ring_stride, int32_t ring, uint16_t* pool, int64_t page_stride /*bytes*/,
                       int64_t num_pages, void* workspace, int64_t workspace_bytes, void* stream);
int ekv_hca_write_step_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                            int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                            const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                            int32_t num_seqs, int32_t max_query_len, uint16_t* state, const int32_t* state_slot,
                            int32_t num_state, const float* ape, const float* norm_w, float eps,
                            const float* cos_sin, int32_t max_spans, const int32_t* comp_block_table,
                            int32_t comp_bt_stride, const int32_t* ring_pages, int32_t ring_stride, int32_t ring,
                            uint16_t* pool, int64_t page_stride /*bytes*/, int64_t num_pages, void* workspace,
                            int64_t workspace_bytes, int32_t window, int32_t* idx_out, int64_t idx_stride,
                            int32_t width, int32_t* lengths, void* stream);

/*
 * HCA decode index rows: [compressed slots 0..n_c-1 | window slots of
 * positions p-w+1..p | -1 ...] with n_c = (p+1)/128, w = min(p+1, window),
 * and the row lengths.  Window slots are ring slots; with query_start_loc
 * [B+1] and slot_mapping [T] of the call (both or neither), positions at or
 * after the first call position of the row's request take that token's
 * slot_mapping slot instead (a prefill chunk longer than the ring reads its
 * own rows).  Replaces the compressed+window index construction inside
 * DeepseekV4Attention (nvidia/attention.py:471-539).
 */
int ekv_hca_decode_indices(const int64_t* positions, const int32_t* req_ids, int32_t num_tokens,
                           const int32_t* comp_block_table, int32_t comp_bt_stride,
                           const int32_t* ring_pages, int32_t ring_stride, int32_t ring, int32_t window,
                           const int32_t* query_start_loc, const int64_t* slot_mapping, int32_t* out,
                           int64_t out_stride, int32_t width, int32_t* lengths, void* stream);

/*
 * merge_swa_topk: out[t] = [topk[t][:n] | seq-w .. seq-1 | -1 ...] with
 * seq = positions[t]+1, n = min(max(seq-window,0), topk_width),
 * w = min(seq, window).  Replaces merge_swa_topk / _merge_swa_topk_kernel
 * (nvidia/attention.py:582-641).
 */
int ekv_merge_swa_topk(const int32_t* topk, int64_t topk_stride, int32_t* out, int64_t out_stride,
                       const int64_t* positions, int32_t num_tokens, int32_t topk_width,
                       int32_t out_width, int32_t window, void* stream);

/*
 * Orthonormal Walsh-Hadamard transform of 128-wide bf16 rows (Sylvester
 * order, times 1/sqrt(128)).  Replaces hadamard_rows / ops.hadacore_transform
 * (nvidia/attention.py:102-108).
 */
int ekv_hadamard_rows(const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, int32_t rows,
                      int32_t dim, void* stream);

/*
 * Indexer prep: k_out = hadamard(rope(k_norm(k))), q_out = hadamard(rope(q))
 * for q [T, heads, 128] and k [T, 128] bf16, with k_norm the LayerNorm
 * (ln_w, ln_b fp32 [128], eps) and rope the NeoX rotation of dims 0..63 by
 * row positions[t] of cos_sin [cos_sin_rows, 64] fp32 (cos 32 | sin 32;
 * positions outside the table leave the row unrotated).  Outputs contiguous
 * bf16.  Replaces the head of Ernie5_5Indexer.forward before the fp8
 * quantization: k_norm, rotary_emb, hadamard_rows (nvidia/attention.py:
 * 955-969; module setup :912-922).
 */
int ekv_indexer_prep(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride, const uint16_t* k,
                     int64_t k_stride, int32_t num_tokens, int32_t heads, const float* ln_w, const float* ln_b,
                     float eps, const float* cos_sin, int32_t cos_sin_rows, const int64_t* positions,
                     uint16_t* q_out, uint16_t* k_out, void* stream);

/*
 * Indexer q quant: q [T, heads, 128] bf16 -> fp8 with a per-(token, head)
 * UE8M0 scale folded into the head weights:
 *   w_out = (w * q_scale) * 128^-0.5 * 64^-0.5.
 * Also writes q's int8 digit planes [T, 3, heads, 128] (may be NULL) used by
 * the exact scorer.  Replaces per_token_group_quant_fp8(..., use_ue8m0=True)
 * and the weight fold (nvidia/attention.py:925, 976-980).
 */
int ekv_indexer_q_quant(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                        const void* weights, int32_t weights_is_bf16, int64_t w_stride,
                        int32_t num_tokens, int32_t heads, uint8_t* q_fp8, float* w_out,
                        int8_t* q_digits, void* stream);

/*
 * DSA decode prologue in one launch, with the results of ekv_indexer_k_insert
 * (k rows into kcache), ekv_kv_append_quant (latent rows of width dim into
 * cache; both at slot_mapping), ekv_indexer_q_quant and
 * ekv_indexer_windowed_lengths with the same arguments.  With cos_sin
 * non-null, q and k are the raw indexer projections and ekv_indexer_prep
 * (ln_w, ln_b, eps, cos_sin, cos_sin_rows, positions) runs first on them, in
 * the same launch.  No single reference function does all of this: it
 * replaces, for a decode step, the head of Ernie5_5Indexer.forward
 * (k_norm, rotary_emb, hadamard_rows, q quant; nvidia/attention.py:955-980),
 * the indexer K insert (nvidia/attention.py:942-953), the MLA latent append
 * [vLLM concat_and_cache_mla] and the metadata lengths
 * (nvidia/attention.py:669-675).
 */
int ekv_dsa_decode_prologue(const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride,
                            int64_t k_num_pages, const uint16_t* latent, int64_t latent_stride, int32_t dim,
                            uint8_t* cache, int64_t page_stride, int64_t num_pages, const int64_t* slot_mapping,
                            int32_t num_tokens, const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                            const void* weights, int32_t weights_is_bf16, int64_t w_stride, int32_t heads,
                            uint8_t* q_fp8, float* w_out, int8_t* q_digits, const int64_t* positions,
                            int32_t window, int32_t* lengths, const float* ln_w, const float* ln_b, float eps,
                            const float* cos_sin, int32_t cos_sin_rows, void* stream);

/*
 * Windowed indexer lengths out[t] = max(positions[t] + 1 - window, 0).
 * Replaces the decode seq_lens rewrite of Ernie5_5IndexerMetadataBuilder.build
 * (nvidia/attention.py:669-675), per query row.
 */
int ekv_indexer_windowed_lengths(const int64_t* positions, int32_t num_tokens, int32_t window,
                                 int32_t* out, void* stream);

/*
 * Exact lightning-indexer scores: for query row t (request req_ids[t]) and
 * every token s < lengths[t],
 *   score = kscale_s * sum_h w[t,h] * relu(q[t,h] . k[s])
 * with the dot product exact and a fixed fp32 head-sum order.
 * Replaces the paged MQA logits of SparseAttnIndexer (DeepGEMM,
 * nvidia/attention.py:56-61, 677-685, 982-984).
 */
int ekv_indexer_score(const int8_t* q_digits, const float* w, const uint8_t* kcache,
                      int64_t page_stride /*bytes*/, int64_t num_pages, const int32_t* block_table,
                      int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                      int32_t num_tokens, int32_t max_len, float* scores, int64_t scores_stride,
                      void* stream);

/*
 * Exact top-k of each score row (first lengths[t] entries): the k largest by
 * (score desc, index asc), written in ascending index order, -1 padded.
 * Replaces the top-k inside SparseAttnIndexer (nvidia/attention.py:942-953)
 * that fills indexer_topk_buffer (nvidia/model.py:71-79).
 */
int ekv_topk_select(const float* scores, int64_t scores_stride, const int32_t* lengths,
                    int32_t num_tokens, int32_t max_len, int32_t* out, int64_t out_stride, int32_t k,
                    void* stream);

/*
 * Workspace bytes the ekv_indexer_topk family needs (shared by its stages).
 * The workspace must be zero-filled once, when it is allocated: its first
 * bytes hold counters that every call expects zero and leaves zero (the
 * first 4 bytes count bound waits that timed out, cumulatively).  A
 * workspace sized for (T, L) serves every call with fewer rows or tokens.
 */
int64_t ekv_indexer_topk_workspace_size(int32_t num_tokens, int32_t max_len);

/*
 * Indexer top-k, stage 1 of 2: fp8-MFMA filter over every token s <
 * lengths[t] with an error bound, then the candidates (tokens whose upper
 * bound reaches the k-th largest lower bound), scored exactly, into
 * `workspace`.  When the shape does not allow that in one launch, this stage
 * leaves the upper bounds and the bound in `workspace` and stage 2 scores the
 * candidates.  q_fp8 [T, 64, 128], q_digits [T, 3, 64, 128] and the folded
 * weights come from ekv_indexer_q_quant.  (Paged MQA logits of
 * SparseAttnIndexer, nvidia/attention.py:56-61, 677-685, 982-984.)
 */
int ekv_indexer_filter(const uint8_t* q_fp8, const int8_t* q_digits, const float* w, const uint8_t* kcache,
                       int64_t page_stride /*bytes*/, int64_t num_pages, const int32_t* block_table,
                       int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                       int32_t num_tokens, int32_t max_len, int32_t k, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * Indexer top-k, stage 2 of 2 (same workspace and arguments): scores the
 * candidates exactly (as ekv_indexer_score) if stage 1 did not, and writes
 * the exact top-k: the k largest by (score desc, index asc), in ascending
 * index order, -1 padded.  Replaces the top-k of SparseAttnIndexer
 * (nvidia/attention.py:942-953) that fills indexer_topk_buffer
 * (nvidia/model.py:71-79).  With merged_out non-null it also writes what
 * ekv_merge_swa_topk would make of the result (merged_width entries per row,
 * from positions and window), saving that launch; with merged_slots != 0 those
 * entries are cache slots block_table[req][i / 64] * 64 + i % 64 (-1 when
 * unmapped), the global indices the decode kernel of FlashMLASparseImpl
 * takes [vLLM: the request-to-global index conversion before
 * flash_mla_with_kvcache, nvidia/attention.py:737-748].
 */
int ekv_indexer_select(const int8_t* q_digits, const float* w, const uint8_t* kcache,
                       int64_t page_stride /*bytes*/, int64_t num_pages, const int32_t* block_table,
                       int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                       int32_t num_tokens, int32_t max_len, int32_t* topk_out, int64_t out_stride,
                       int32_t k, void* workspace, int64_t workspace_bytes, int32_t* merged_out,
                       int64_t merged_stride, int32_t merged_width, const int64_t* positions,
                       int32_t window, int32_t merged_slots, void* stream);

/*
 * Both stages in one call: the SparseAttnIndexer decode path
 * (nvidia/attention.py:942-953, 982-984).  When the filter runs as one launch
 * the exact select runs inside that launch too: the workgroups of each row
 * agree on the top-k threshold through counters in `workspace` and write the
 * output directly.  Same results as ekv_indexer_filter + ekv_indexer_select.
 */
int ekv_indexer_topk(const uint8_t* q_fp8, const int8_t* q_digits, const float* w, const uint8_t* kcache,
                     int64_t page_stride /*bytes*/, int64_t num_pages, const int32_t* block_table,
                     int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                     int32_t num_tokens, int32_t max_len, int32_t* topk_out, int64_t out_stride,
                     int32_t k, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * ekv_indexer_topk with ekv_indexer_select's merged output (merge_swa_topk
 * of the result, optionally as cache slots): the indexer half of
 * Ernie5_5DSAAttention._indexer_and_attn (nvidia/attention.py:1205-1226:
 * SparseAttnIndexer filling topk_indices_buffer, then merge_swa_topk at
 * :582-641), one launch when the filter plan allows it.
 */
int ekv_indexer_topk_merged(const uint8_t* q_fp8, const int8_t* q_digits, const float* w,
                            const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                            const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                            const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                            int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                            int32_t* merged_out, int64_t merged_stride, int32_t merged_width,
                            const int64_t* positions, int32_t window, int32_t merged_slots, void* stream);

/*
 * Diagnostic, no counterpart in the reference: bytes at the front of a
 * top-k workspace that hold the one-launch path's per-row counters (zero
 * between calls).
 */
int64_t ekv_indexer_topk_counter_bytes(void);

/*
 * Test hook, no counterpart in the reference: polls a one-launch top-k
 * workgroup makes while it waits for the rest of its row before it gives up
 * (the row is then selected by its last workgroup alone; still exact).
 * polls < 0 restores the default.  Returns the previous value.  Process-wide;
 * not for concurrent use with top-k calls.
 */
int32_t ekv_indexer_set_spin_limit(int32_t polls);

/* Workspace bytes ekv_sparse_mla_decode needs. */
int64_t ekv_sparse_mla_decode_workspace_size(int32_t num_tokens, int32_t heads, int32_t width);

/*
 * Sparse MLA decode with attention sink.  q [T, heads, dim] bf16 (dim 512 or
 * 576, heads a multiple of 16, <= 64); cache fp8 pages (cache_bf16 = 0) or
 * bf16 flat rows [num_pages*64, dim] (cache_bf16 = 1); indices [T, width]
 * global slots, or request-local token indices when block_table != NULL
 * (converted in-kernel, -1 kept); lengths [T] optional; sinks [heads] fp32
 * optional (natural-log units, enters the denominator only).
 *   out [T, heads, 512] bf16, lse [T, heads] fp32 = log sum_j exp(s_j).
 * Replaces Ernie5_5FlashMLASparseImpl._fp8_flash_mla_kernel /
 * _bf16_flash_mla_kernel -> flash_mla_with_kvcache / flash_mla_sparse_fwd
 * (nvidia/attention.py:701-790) and the logical->global conversion behind
 * record_logical_topk_ready (nvidia/attention.py:1225).
 */
int ekv_sparse_mla_decode(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                          int32_t num_tokens, int32_t heads, int32_t dim, const uint8_t* cache,
                          int32_t cache_bf16, int64_t page_stride /*bytes*/, int64_t num_pages,
                          const int32_t* indices, int64_t idx_stride, int32_t width,
                          const int32_t* lengths, const int32_t* block_table, int64_t bt_stride,
                          const int32_t* req_ids, const float* sinks, float scale, uint16_t* out,
                          int64_t out_tok_stride, int64_t out_head_stride, float* lse,
                          int64_t lse_stride, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * x * sigmoid(gate) (bf16 roundings of torch's `x * torch.sigmoid(gate)`)
 * quantized to fp8 e4m3 in 1 x 128 groups with UE8M0 scales: x, gate
 * [num_rows, hidden] bf16 (hidden a multiple of 512), out [num_rows,
 * out_stride] fp8, scale int32 at scale[pack * scale_stride + row] holding
 * the biased exponents (e + 127) of groups 4 pack .. 4 pack + 3 in bytes
 * 0..3 (DeepGEMM's packed column-major layout; scale_stride >= num_rows).
 * Replaces sigmoid_mul_quant_fp8 / _sigmoid_mul_quant_kernel
 * (nvidia/attention.py:288-361).
 */
int ekv_sigmoid_mul_quant_fp8(const uint16_t* x, int64_t x_stride, const uint16_t* gate, int64_t gate_stride,
                              int32_t num_rows, int32_t hidden, uint8_t* out, int64_t out_stride, int32_t* scale,
                              int64_t scale_stride, void* stream);

/*
 * VHA head mixing + inverse RoPE + fp8 quant of the HCA attention output:
 * y = mix @ o[t] (o [T, heads >= 64 padded, 512] bf16 with the given
 * strides, mix [64, 64] bf16, fp32 accumulation), the interleaved pairs of
 * channels nope_dim .. 511 rotated back by the row positions[t] of cos_sin
 * ([P, cs_stride] fp32: cos rope_dim/2 | sin rope_dim/2), then a UE8M0
 * fp8 quant per (head, 128 channels).  out fp8 [n_groups, T, (64 /
 * n_groups) * 512]; scale int32 [n_groups, 64 / n_groups, aligned_tokens]
 * with the biased exponent of channel chunk c in byte c; scale rows
 * T .. aligned_tokens - 1 are zeroed.  Replaces vha_inv_rope_fp8_quant /
 * _vha_inv_rope_quant_kernel (nvidia/attention.py:166-285).
 */
int ekv_vha_inv_rope_fp8_quant(const uint16_t* o, int64_t o_tok_stride, int64_t o_head_stride, int32_t num_tokens,
                               int32_t heads, const uint16_t* mix, const int64_t* positions, const float* cos_sin,
                               int64_t cs_stride, int32_t n_groups, int32_t nope_dim, int32_t rope_dim, uint8_t* out,
                               int32_t* scale, int32_t aligned_tokens, void* stream);

/*
 * Diagnostic, no counterpart in the reference: the indexer filter's fp8-MFMA
 * dot products out[s][h] = q[h] . k[s] of e4m3fn codes (q [64][128],
 * k [num_keys][128], num_keys a multiple of 16, out [num_keys][64] fp32),
 * computed by the same MFMA call and operand layout as ekv_indexer_filter.
 * Lets a caller check, on the device at hand, the error bound the filter's
 * candidate test assumes (|dot - exact| <= 2^-8 * 448^2 per head).
 */
int ekv_indexer_filter_dots(const uint8_t* q_codes, const uint8_t* k_codes, int32_t num_keys, float* out,
                            void* stream);

/*
 * ekv_sparse_mla_decode without a workspace argument: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split partials go to a 64 MiB device array inside the library (one per
 * GPU, held until the process ends); a call needing more
 * (ekv_sparse_mla_decode_workspace_size > 64 MiB, e.g. beyond ~150 query
 * rows of 2176 entries at 64 heads) fails with status 1.  Calls that overlap
 * on one GPU (different streams) race on that array.  Allocates nothing.
 */
int ekv_sparse_mla_decode_noalloc(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                  int32_t num_tokens, int32_t heads, int32_t dim, const uint8_t* cache,
                                  int32_t cache_bf16, int64_t page_stride /*bytes*/, int64_t num_pages,
                                  const int32_t* indices, int64_t idx_stride, int32_t width,
                                  const int32_t* lengths, const int32_t* block_table, int64_t bt_stride,
                                  const int32_t* req_ids, const float* sinks, float scale, uint16_t* out,
                                  int64_t out_tok_stride, int64_t out_head_stride, float* lse,
                                  int64_t lse_stride, void* stream);

/* The 256-entry byte -> packed signed base-64 digit table the scorer uses. */
int ekv_fp8_digit_table(uint32_t* table, void* stream);

/* ---------------------------------------------------------------------------
 * MXFP4 indexer (use_fp4_kv).  Key rows are 68 bytes: 64 bytes of packed
 * e2m1 values (even element in the low nibble) and 4 E8M0 scale bytes, one
 * per 32 values; a 64-token page holds all values first (row r at 64 r), then
 * all scale bytes (row r at 64 * 64 + 4 r).  Quantization per 32-value group:
 * scale = 2^ceil(log2(amax / 6)), values to the nearest e2m1 with ties to the
 * larger magnitude.
 * ------------------------------------------------------------------------- */

/*
 * MXFP4 quantization of rows r = tok * heads + h of x (bf16 at
 * x + tok * x_tok_stride + h * x_head_stride, dim values, dim % 32 == 0):
 * dim / 2 packed bytes at values + r * values_stride, dim / 32 scale bytes at
 * scales + r * scales_stride.  Replaces downcast_to_mxfp(x, axis=-1) as
 * _quantize_fp4 calls it (nvidia/attention.py:990-1008).
 */
int ekv_mxfp4_quant(const uint16_t* x, int64_t x_tok_stride, int64_t x_head_stride, int32_t num_tokens,
                    int32_t heads, int32_t dim, uint8_t* values, int64_t values_stride, uint8_t* scales,
                    int64_t scales_stride, void* stream);

/*
 * Indexer q for the MXFP4 path: q [T, heads, 128] bf16 -> q_values
 * [T, heads, 64] and q_scales [T, heads] (the four scale bytes of a head as
 * one int32), and w_out [T, heads] = fl32(weights * fl32(128^-0.5 * 64^-0.5))
 * (no q scale is folded on this path).  Replaces the q half of
 * _quantize_fp4 and the weight scaling (nvidia/attention.py:969-974,
 * 990-995, 1022-1025).
 */
int ekv_indexer_q_quant_fp4(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                            const void* weights, int32_t weights_is_bf16, int64_t w_stride, int32_t num_tokens,
                            int32_t heads, uint8_t* q_values, int32_t* q_scales, float* w_out, void* stream);

/*
 * MXFP4 indexer K insert: k [num_tokens, k_stride] bf16 (128 wide) quantized
 * and written to the page row of slot_mapping[t] (negative slots skipped).
 * Replaces the k half of _quantize_fp4: downcast_to_mxfp then
 * _store_indexer_fp4 (nvidia/attention.py:999-1021, 831-860).
 */
int ekv_indexer_k_insert_fp4(const uint16_t* k, int64_t k_stride, int32_t num_tokens,
                             const int64_t* slot_mapping, uint8_t* kcache, int64_t page_stride /*bytes*/,
                             int64_t num_pages, void* stream);

/*
 * Store of already quantized MXFP4 rows (64 value bytes at
 * values + t * values_stride, 4 scale bytes at scales + t * scales_stride)
 * into the page row of slot_mapping[t]; negative slots skipped.  Replaces
 * _store_indexer_fp4 (nvidia/attention.py:831-860).
 */
int ekv_indexer_store_fp4(const uint8_t* values, int64_t values_stride, const uint8_t* scales,
                          int64_t scales_stride, int32_t num_tokens, const int64_t* slot_mapping,
                          uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages, void* stream);

/*
 * The MXFP4 counterpart of ekv_dsa_decode_prologue, in one launch: with
 * cos_sin non-null ekv_indexer_prep of q and k first, then
 * ekv_indexer_k_insert_fp4 of k at slot_mapping, ekv_indexer_q_quant_fp4 of q
 * and weights (values [T, heads, 64], scale words [T, heads], folded weights),
 * ekv_kv_append_quant of the latent rows and ekv_indexer_windowed_lengths --
 * the same bytes as those calls.  Replaces, for a decode step with
 * use_fp4_indexer_cache, the head of Ernie5_5Indexer.forward with
 * _quantize_fp4 (nvidia/attention.py:955-1025), the latent append [vLLM
 * concat_and_cache_mla] and the metadata lengths (nvidia/attention.py:669-675).
 */
int ekv_dsa_decode_prologue_fp4(const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride,
                                int64_t k_num_pages, const uint16_t* latent, int64_t latent_stride, int32_t dim,
                                uint8_t* cache, int64_t page_stride, int64_t num_pages, const int64_t* slot_mapping,
                                int32_t num_tokens, const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                const void* weights, int32_t weights_is_bf16, int64_t w_stride, int32_t heads,
                                uint8_t* q_values, int32_t* q_scales, float* w_out, const int64_t* positions,
                                int32_t window, int32_t* lengths, const float* ln_w, const float* ln_b, float eps,
                                const float* cos_sin, int32_t cos_sin_rows, void* stream);

/*
 * Exact MXFP4 indexer scores, as ekv_indexer_score for 68-byte key rows: per
 * head, block sums D_b of the integers 2 * e2m1 (exact), T_b =
 * fl32(D_b * 2^(sq_b + sk_b - 256)), dot = ((T_0 + T_1) + T_2) + T_3 in fp32,
 * score = sum_h fl32(w_h * relu(dot)) in the fixed head order, + 0.
 * Replaces the FP4 paged MQA logits of SparseAttnIndexer(use_fp4_cache=True)
 * (nvidia/attention.py:942-953, 982-984).
 */
int ekv_indexer_score_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                          const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                          const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                          const int32_t* lengths, int32_t num_tokens, int32_t max_len, float* scores,
                          int64_t scores_stride, void* stream);

/*
 * ekv_dsa_decode_prologue followed by ekv_indexer_topk_merged over the keys
 * in kcache (block_table .. merged_slots as there; lengths, q_fp8, w_out and
 * q_digits are the prologue's outputs, which the top-k reads), with the same
 * outputs as the two calls.  max_new_rows is the most query rows any one
 * sequence has in the call (its newest positions; 1 for plain decode).  When
 * 1 <= max_new_rows <= window no row scores a key the call appends, and when
 * the top-k also runs as one launch that selects (64 heads, merged output)
 * the prologue is folded into that launch: each workgroup prepares and
 * quantizes its row's q itself, and one workgroup per row appends the new
 * rows and writes the prologue's outputs while the row's bound is computed.
 * Otherwise the two calls run.  Replaces
 * the head of Ernie5_5DSAAttention._indexer_and_attn (nvidia/attention.py:
 * 1205-1226: Ernie5_5Indexer.forward's prep, K insert and SparseAttnIndexer
 * top-k (:942-984), the latent append [vLLM concat_and_cache_mla] and
 * merge_swa_topk (:582-641)).
 */
int ekv_dsa_decode_prologue_topk_merged(
    const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride, int64_t k_num_pages,
    const uint16_t* latent, int64_t latent_stride, int32_t dim, uint8_t* cache, int64_t page_stride,
    int64_t num_pages, const int64_t* slot_mapping, int32_t num_tokens, const uint16_t* q, int64_t q_tok_stride,
    int64_t q_head_stride, const void* weights, int32_t weights_is_bf16, int64_t w_stride, int32_t heads,
    uint8_t* q_fp8, float* w_out, int8_t* q_digits, const int64_t* positions, int32_t window,
    int32_t max_new_rows, int32_t* lengths, const float* ln_w, const float* ln_b, float eps, const float* cos_sin,
    int32_t cos_sin_rows, const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids, int32_t max_len,
    int32_t* topk_out, int64_t out_stride, int32_t k_top, void* workspace, int64_t workspace_bytes,
    int32_t* merged_out, int64_t merged_stride, int32_t merged_width, int32_t merged_slots, void* stream);

/*
 * 1 when ekv_dsa_decode_prologue_topk_merged of num_tokens rows of at most
 * max_len keys (64 heads, 1 <= max_new_rows <= window, merged output) runs
 * as one launch on the current device, else 0 (the two calls run).  No counterpart in the
 * reference: a plan query, as ekv_indexer_topk_workspace_size is.
 */
int32_t ekv_dsa_decode_prologue_folds(int32_t num_tokens, int32_t max_len);

/*
 * MXFP4 counterparts of ekv_indexer_filter / _select / _topk / _topk_merged (same workspace,
 * ekv_indexer_topk_workspace_size): the filter runs the scaled fp4 MFMA over
 * every token with an error bound, the candidates are scored exactly as
 * ekv_indexer_score_fp4, and the select writes the exact top-k (lowest index
 * first on ties), optionally merged as ekv_indexer_select describes.
 * Replaces SparseAttnIndexer with use_fp4_cache=True (nvidia/attention.py:
 * 942-953, 982-984).
 */
int ekv_indexer_filter_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                           const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                           const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                           const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t k,
                           void* workspace, int64_t workspace_bytes, void* stream);
int ekv_indexer_select_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                           const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                           const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                           const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                           int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                           int32_t* merged_out, int64_t merged_stride, int32_t merged_width,
                           const int64_t* positions, int32_t window, int32_t merged_slots, void* stream);
int ekv_indexer_topk_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                         const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                         const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                         const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                         int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes, void* stream);
int ekv_indexer_topk_merged_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                const uint8_t* kcache, int64_t page_stride /*bytes*/, int64_t num_pages,
                                const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                                int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                                int32_t* merged_out, int64_t merged_stride, int32_t merged_width,
                                const int64_t* positions, int32_t window, int32_t merged_slots, void* stream);

/*
 * Diagnostic, no counterpart in the reference: the MXFP4 filter's MFMA dot
 * products out[s][h] = q[h] . k[s] of dequantized e2m1 rows (q_values
 * [64][64], q_scales [64] words, k_values [num_keys][64], k_scales [num_keys]
 * words, num_keys a multiple of 16), by the same MFMA call and operand layout
 * as ekv_indexer_filter_fp4, to check the error bound its candidate test
 * assumes on the device at hand.
 */
int ekv_indexer_filter_dots_fp4(const uint8_t* q_values, const int32_t* q_scales, const uint8_t* k_values,
                                const int32_t* k_scales, int32_t num_keys, float* out, void* stream);

/* ---------------------------------------------------------------------------
 * Upstream page format at the KV-connector boundary.  fp8_ds_mla is the fp8
 * KV dtype of vLLM's FlashMLA sparse backend, on which the reference's DSA
 * layers run (nvidia/attention.py:551-558, 792-795): a 576-wide latent row is
 * 656 bytes -- 512 e4m3fn codes (dims 0..511), 4 fp32 scales (scale t for
 * dims 128t..128t+127), 64 bf16 values (dims 512..575) -- 64 token-major rows
 * per page, page stride a multiple of the packed block alignment 9216
 * (nvidia/attention.py:561-571), e.g. 46080.  This library's latent page is
 * 64 rows of 576 codes, then 64 fp32 power-of-two row scales.  The indexer
 * pages already have DeepGEMM's layout (values, then scales) and need no
 * transcoding.  No reference function corresponds: the reference moves
 * fp8_ds_mla blocks as they are; these let a connector move this library's
 * pages in that format.
 * ------------------------------------------------------------------------- */

/*
 * Export: page src_pages[i] of `cache` (this library's 576-wide latent pages)
 * -> page dst_pages[i] (i when dst_pages is NULL) of `out` in fp8_ds_mla.
 * Lossless: codes 0..511 copied, the row scale in the four tile slots, dims
 * 512..575 as exact bf16.  Page ids out of range are skipped.
 */
int ekv_export_fp8_ds_mla_pages(const uint8_t* cache, int64_t page_stride /*bytes*/, int64_t num_pages,
                                const int32_t* src_pages, int32_t n, uint8_t* out,
                                int64_t out_page_stride /*bytes*/, int64_t out_num_pages,
                                const int32_t* dst_pages, void* stream);

/*
 * Import: fp8_ds_mla page src_pages[i] of `src` -> page dst_pages[i] (i when
 * NULL) of `cache`: each row dequantized in fp32 (code * tile scale, bf16 as
 * is), then quantized as ekv_kv_append_quant does (one UE8M0 scale per row,
 * round to nearest even).  Pages that ekv_export_fp8_ds_mla_pages wrote come
 * back with the same values (the same bytes, except rows whose largest code is
 * 224: half the scale, doubled codes).  Page ids out of range are skipped.
 */
int ekv_import_fp8_ds_mla_pages(const uint8_t* src, int64_t src_page_stride /*bytes*/, int64_t src_num_pages,
                                const int32_t* src_pages, int32_t n, uint8_t* cache,
                                int64_t page_stride /*bytes*/, int64_t num_pages, const int32_t* dst_pages,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ERNIE_KV_H_ */
