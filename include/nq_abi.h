/*
 * nq_abi.h -- C ABI of the MI355X-native serving hot path for Qwen3-TTS.
 *
 * Every entry point:
 *   - takes device pointers, element strides and sizes, plus a hipStream_t
 *     passed as `void *` (0 = the null stream);
 *   - never allocates, never synchronises, and is safe to record into a
 *     hipGraph (no memset/memcpy nodes are issued);
 *   - returns 0 on success or a negative NQ_ERR_* code; nq_status_string()
 *     names it.  Argument errors are detected on the host before any launch.
 *
 * Tensor layouts use element strides (not bytes).  "bf16" buffers hold
 * bfloat16 bit patterns (uint16_t).  Reference citations name the file and
 * line of nari-labs/nari-qwen3-tts (src/nari_qwen3_tts/...) whose behaviour
 * the entry point replaces.
 */
#ifndef NQ_ABI_H
#define NQ_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NQ_ABI_VERSION 1

enum nq_status {
    NQ_OK = 0,
    NQ_ERR_INVALID_ARGUMENT = -1, /* shape / contract violation -> ValueError */
    NQ_ERR_UNSUPPORTED = -2,      /* dtype / size outside the kernels' range -> TypeError */
    NQ_ERR_LAUNCH = -3,           /* HIP launch or runtime failure -> RuntimeError */
    NQ_ERR_CAPACITY = -4,         /* too few free KV pages -> KVAllocationError */
    NQ_ERR_STATE = -5             /* device KV state differs from the host ledger -> RuntimeError */
};

/* dtype codes for logits and activations */
enum nq_dtype { NQ_F32 = 0, NQ_BF16 = 1 };

int nq_abi_version(void);
const char *nq_status_string(int status);

/*
 * Ragged KV metadata on the GPU.
 * Replaces PagedTalkerKV._metadata (executor/talker_kv.py:403-483) together
 * with the page choice of PagedKVAllocator.reserve (executor/cache.py:135-184):
 * new pages are the lowest free pages, taken in row order.
 *
 * Real rows r < n_rows: prior sequence length seq_len[r], position_start
 * pos_start[r], advance[r] >= 1 new tokens, prior_pages[r] pages already listed
 * in page_table[table_row[r] * table_stride + 0 .. prior_pages[r]).  New pages
 * are read from free_pages[0 ..) (sorted ascending) and appended to the same
 * page_table row.  expect_pages (may be NULL) lists the pages the host ledger's
 * reservation took, in row order; when the pages read from free_pages differ
 * from it, status[0] is NQ_ERR_STATE (the metadata is still written).
 * Rows n_rows .. capture_rows-1 are padding rows that use scratch_pages[row].  Outputs (device):
 *   qo_indptr[capture_rows+1] (only when prefill != 0; may be NULL otherwise),
 *   kv_indptr[capture_rows+1], kv_indices[kv_indices_capacity],
 *   last_page_len[capture_rows], position_ids / write_pages / write_offsets
 *   [token_capacity] (int64).
 * status[0] receives NQ_OK, NQ_ERR_CAPACITY or NQ_ERR_STATE, status[1] the
 * number of free pages consumed.  grid_blocks = 0 picks a default launch width.
 */
int nq_plan_ragged(const int32_t *seq_len, const int32_t *pos_start, const int32_t *advance,
                   const int32_t *prior_pages, const int32_t *table_row, int n_rows,
                   int capture_rows, int token_capacity, int page_size, int prefill,
                   int32_t *page_table, int64_t table_stride, const int32_t *free_pages,
                   int n_free, const int32_t *expect_pages, const int32_t *scratch_pages, int n_scratch,
                   int32_t *qo_indptr, int32_t *kv_indptr, int32_t *kv_indices,
                   int64_t kv_indices_capacity, int32_t *last_page_len, int64_t *position_ids,
                   int64_t *write_pages, int64_t *write_offsets, int32_t *status,
                   int grid_blocks, void *stream);

/*
 * Return pages to the device copy of the sorted free list: out[0, n_free +
 * n_returned) = the sorted union of free_pages[0, n_free) and returned[0,
 * n_returned), both sorted ascending and distinct (out must not alias either).
 * The device side of PagedKVAllocator's page returns (executor/cache.py:
 * 129-133 remove_request, :208-211 discard), so the free list the planner
 * reads never has to be uploaded from the host again.  A returned page that is
 * already free sets status[0] (may be NULL) to NQ_ERR_INVALID_ARGUMENT and is
 * dropped.
 */
int nq_free_list_merge(const int32_t *free_pages, int n_free, const int32_t *returned, int n_returned,
                       int32_t *out, int32_t *status, void *stream);

/*
 * One decode step's report in one small device buffer, so the host reads it
 * with a single copy per decision (replaces the per-row
 * `int(tokens[index].item()) == codec_eos_token_id` reads of
 * engine/pipeline.py:585-593 and makes the step fail closed):
 *   report[0] = plan_status[0] (the planner's NQ_OK / NQ_ERR_CAPACITY),
 *   report[1] = merge_status[0] (nq_free_list_merge), report[2] =
 *               attention_status[0], report[3] = embed_status[0]: each of
 *               these three is then reset to NQ_OK for the next step (any of
 *               the four status pointers may be NULL: reported as NQ_OK),
 *   report[4] = number of tokens outside [0, vocab), report[5..7] = 0,
 *   report[NQ_REPORT_HEAD + r] = tokens[r] == eos_id, r < rows.
 * One workgroup; graph-capturable.
 */
#define NQ_REPORT_HEAD 8
int nq_step_report(const int32_t *plan_status, int32_t *merge_status, int32_t *attention_status,
                   int32_t *embed_status, const int64_t *tokens, int rows, int64_t eos_id, int64_t vocab,
                   int32_t *report, void *stream);

/*
 * Work decomposition for nq_paged_attention, computed on the GPU from the
 * ragged metadata.  Replaces the host-side plan() of the FlashInfer wrappers
 * (executor/talker_kv.py:175-223 prefill, :259-303 decode).
 * qo_indptr may be NULL (pure decode: row r owns query r).  Rows with one
 * query become 16-token key blocks (page id resolved from kv_indices) that
 * the attention launch splits evenly over its waves; rows with several
 * queries get, per query, its causal key range (bottom-right aligned: query i
 * of a row with qo_len queries sees keys < kv_len - qo_len + i + 1) split
 * into chunks whose size the plan picks on the GPU from the total work.
 * Writes into `workspace` (size from nq_attention_workspace_bytes for the same
 * maxima).  max_pages bounds the pages of all rows together (the length of
 * kv_indices).  position_ids / write_pages / write_offsets ([max_query_tokens]
 * int64, the RoPE positions and K/V write slots of the same metadata) may be
 * NULL; nq_paged_decode_rope_attention needs a plan that was given them (it
 * reads each decode row's position and write slot from the plan).
 */
int64_t nq_attention_workspace_bytes(int max_query_tokens, int max_pages, int page_size,
                                     int num_qo_heads, int num_kv_heads, int head_dim);
int nq_attention_plan(const int32_t *qo_indptr, const int32_t *kv_indptr,
                      const int32_t *last_page_len, const int32_t *kv_indices,
                      const int64_t *position_ids, const int64_t *write_pages,
                      const int64_t *write_offsets, int n_rows,
                      int max_query_tokens, int max_pages, int page_size, int num_qo_heads,
                      int num_kv_heads, int head_dim, void *workspace, int64_t workspace_bytes,
                      void *stream);

/*
 * Paged GQA attention for mixed decode (qo_len == 1) and causal prefill
 * (qo_len > 1, bottom-right aligned) rows over one layer of the paged cache.
 * Replaces BatchDecodeWithPagedKVCacheWrapper.run / BatchPrefillWith-
 * PagedKVCacheWrapper.run as used by executor/talker_kv.py:225-226,305-306.
 * q: bf16 [tokens, num_qo_heads, head_dim] with strides (q_s0, q_s1, 1).
 * cache: bf16 layer view; element (page, kind, slot, kv_head, d) at
 *   page*c_page + kind*c_kind + slot*c_slot + kv_head*c_head + d
 *   (kind 0 = K, 1 = V; the reference layout is [pages, 2, ps, Hkv, D]).
 * out: bf16 [tokens, num_qo_heads, head_dim] with strides (o_s0, o_s1, 1).
 * The plan in `workspace` must come from nq_attention_plan for the same
 * metadata and the same (max_query_tokens, max_pages).  `parts` selects the
 * launches: NQ_ATTN_DECODE (rows with one query: stream + merge kernels),
 * NQ_ATTN_PREFILL (rows with several queries), or both.  The two parts read
 * the same plan and write disjoint output rows, so a caller may issue them on
 * two streams to run them concurrently; NQ_ATTN_DECODE alone promises the plan
 * holds no row with more than one query.  NQ_ATTN_BESIDE_PREFILL (with
 * NQ_ATTN_DECODE) says the prefill part runs concurrently on another stream:
 * decode launches of more than 64 rows then take twelve-wave workgroups
 * instead of sixteen, which leaves each CU room that the prefill tiles use
 * (the K/V span split follows the workgroup size, so results agree with a
 * launch without the flag to rounding, not bit for bit).  status (device int32, may be NULL) is set to
 * NQ_ERR_INVALID_ARGUMENT when a page id outside [0, num_pages) is met (that
 * page is skipped).
 */
enum nq_attention_parts { NQ_ATTN_DECODE = 1, NQ_ATTN_PREFILL = 2, NQ_ATTN_BESIDE_PREFILL = 4 };
int nq_paged_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                       int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head,
                       int num_pages, const int32_t *kv_indices, int page_size, int num_qo_heads,
                       int num_kv_heads, int head_dim, float sm_scale, uint16_t *out, int64_t o_s0,
                       int64_t o_s1, int max_query_tokens, int max_pages, int parts,
                       void *workspace, int64_t workspace_bytes, int32_t *status, void *stream);

/*
 * nq_attention_plan for attention launches that run only `parts` (the
 * nq_attention_parts flags nq_paged_attention takes).  Without NQ_ATTN_DECODE
 * the rows of one query are planned into the prefill part as well, so a
 * single NQ_ATTN_PREFILL launch serves the whole batch and no decode launch
 * is needed; with it the plan is nq_attention_plan's.  No counterpart in the
 * reference, whose prefill and decode batches go to separate FlashInfer
 * wrappers (P/executor/talker_kv.py:140-306): it lets a prefill binding skip
 * the decode launch that only a batch mixing both kinds of row needs.
 */
int nq_attention_plan_parts(const int32_t *qo_indptr, const int32_t *kv_indptr,
                            const int32_t *last_page_len, const int32_t *kv_indices,
                            const int64_t *position_ids, const int64_t *write_pages,
                            const int64_t *write_offsets, int n_rows, int max_query_tokens,
                            int max_pages, int page_size, int num_qo_heads, int num_kv_heads,
                            int head_dim, int parts, void *workspace, int64_t workspace_bytes,
                            void *stream);

/*
 * nq_attention_plan followed by nq_paged_attention (positions and write slots
 * not planned, so not usable before nq_paged_decode_rope_attention), with the
 * plan and partials in the library's own static device scratch instead of a
 * caller workspace: this call allocates nothing, never synchronises and issues
 * no memset.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under hipGraph capture that forbids it, tight
 * serving loops, harnesses without an allocator).  Limit: the workspace that
 * nq_attention_workspace_bytes reports for (max_query_tokens, max_pages, ...)
 * must not exceed NQ_NOALLOC_SCRATCH_BYTES (32 MiB per GPU, held until the
 * process ends; a 128-row decode batch over a 32768-page pool needs about 22
 * MiB), else NQ_ERR_INVALID_ARGUMENT before any launch.  Every call on one GPU
 * shares that GPU's scratch: calls that overlap on one GPU (two streams, two
 * threads) race; calls in stream order do not.
 */
#define NQ_NOALLOC_SCRATCH_BYTES (32ll << 20)
int nq_paged_attention_noalloc(const int32_t *qo_indptr, const int32_t *kv_indptr,
                               const int32_t *last_page_len, const int32_t *kv_indices, int n_rows,
                               const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                               int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head,
                               int num_pages, int page_size, int num_qo_heads, int num_kv_heads,
                               int head_dim, float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                               int max_query_tokens, int max_pages, int parts, int32_t *status,
                               void *stream);

/*
 * Code-predictor short-cache attention: one query per row over the first
 * valid_length positions of a dense per-row cache.
 * Replaces decode_attn_nhd_short_cache (model/kernels.py:408-520).
 * Element (row, kind, pos, kv_head, d) of the cache sits at
 *   row*c_row + kind*c_kind + pos*c_pos + kv_head*c_head + d.
 */
int nq_cp_short_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                          int64_t c_row, int64_t c_kind, int64_t c_pos, int64_t c_head,
                          int rows, int valid_length, int num_qo_heads, int num_kv_heads,
                          int head_dim, float sm_scale, uint16_t *out, int64_t o_s0,
                          int64_t o_s1, void *stream);

/*
 * The code predictor's per-layer q/k norm + RoPE + dense K/V write and its
 * short-cache attention in one launch: nq_qkv_partials_norm_rope_kv_write in
 * dense mode (from the packed QKV projection's split-K planes [splits, rows,
 * (Hq + 2 Hkv) * head_dim]; rotated q to q_out, K and V into cache position
 * cache_position) followed by nq_cp_short_attention over valid_length =
 * cache_position + 1, with the same bits as the two calls.  Replaces
 * paired_qk_norm_rope_dense_cache_ (model/kernels.py:163-248, 335-405) and
 * decode_attn_nhd_short_cache (model/kernels.py:408-463) as the code
 * predictor's attention calls them in sequence (model/components.py:294-345).
 * head_dim 64 or 128 with 1 or 2
 * query heads per kv head; other shapes return NQ_ERR_UNSUPPORTED.
 */
int nq_cp_rope_short_attention(const float *partials, int splits, int rows, const uint16_t *q_weight,
                               const uint16_t *k_weight, const int64_t *positions, int64_t pos_stride,
                               float eps, float rope_theta, int round_to_input, uint16_t *q_out,
                               int64_t q_s0, int64_t q_s1, uint16_t *cache, int64_t c_row, int64_t c_kind,
                               int64_t c_pos, int64_t c_head, int cache_position, int num_qo_heads,
                               int num_kv_heads, int head_dim, float sm_scale, uint16_t *out,
                               int64_t o_s0, int64_t o_s1, void *stream);

/*
 * Fused per-head RMSNorm + rotate-half RoPE of q and k (in place), with K and
 * V written into the cache.
 * Replaces paired_qk_norm_rope_paged_cache_ (model/kernels.py:15-160) and,
 * with write_pages == NULL, paired_qk_norm_rope_dense_cache_ (model/kernels.py:
 * 163-248, 335-405): the destination "page" is then the token index and the
 * slot is the constant `cache_position`.  With cache == NULL nothing is
 * written (paired_qk_norm_rope_, model/kernels.py:275-332).
 * round_to_input != 0 rounds the normalised values to bf16 before RoPE
 * (model/kernels.py:65-67).  positions: int64 with stride pos_stride.
 */
int nq_qk_norm_rope_kv_write(uint16_t *q, int64_t q_s0, int64_t q_s1, uint16_t *k,
                             int64_t k_s0, int64_t k_s1, const uint16_t *v, int64_t v_s0,
                             int64_t v_s1, const uint16_t *q_weight, const uint16_t *k_weight,
                             const int64_t *positions, int64_t pos_stride, int tokens,
                             int num_qo_heads, int num_kv_heads, int head_dim, float eps,
                             float rope_theta, int round_to_input, uint16_t *cache,
                             int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head,
                             const int64_t *write_pages, const int64_t *write_offsets,
                             int cache_position, void *stream);

/*
 * nq_qk_norm_rope_kv_write reading q, k and v straight from the fp32 split-K
 * partial planes [splits, tokens, (Hq + 2 Hkv) * D] that nq_linear leaves with
 * NQ_EPI_PARTIALS (packed QKV projection, model/layers.py:296-306): every
 * value is the plane-order sum rounded to bf16, exactly the bf16 projection
 * output.  Rotated q goes to q_out, rotated k to k_out (may be NULL) and the
 * cache, v to the cache.  The paged / dense cache addressing is that of
 * nq_qk_norm_rope_kv_write.
 */
int nq_qkv_partials_norm_rope_kv_write(const float *partials, int splits, int tokens, uint16_t *q_out,
                                       int64_t q_s0, int64_t q_s1, uint16_t *k_out, int64_t k_s0,
                                       int64_t k_s1, const uint16_t *q_weight, const uint16_t *k_weight,
                                       const int64_t *positions, int64_t pos_stride, int num_qo_heads,
                                       int num_kv_heads, int head_dim, float eps, float rope_theta,
                                       int round_to_input, uint16_t *cache, int64_t c_page,
                                       int64_t c_kind, int64_t c_slot, int64_t c_head,
                                       const int64_t *write_pages, const int64_t *write_offsets,
                                       int cache_position, void *stream);

/*
 * Fused sampler with caller-supplied uniforms, one row per workgroup:
 * optional logit masks, repetition penalty on seen ids (x>0 ? x/r : x*r),
 * division by temperature, top-k (value desc, id asc), top-p nucleus and an
 * inverse-CDF draw from uniforms[row] in [0,1).  Rows with temperature == 0
 * take the argmax of the penalised logits (lowest id on ties).
 * Replaces sample_talker_cuda_graph (executor/sampling.py:156-198),
 * sample_logits_cuda_graph (:201-239), the fused code-predictor kernel
 * (:242-336) and the penalty/greedy rules of sample_logits_stateless
 * (model/sampling.py:55-65,127-225); the seen-mask update of
 * TalkerExecutor._sample (executor/talker.py:373) when update_seen != 0, and
 * the logit masks of TalkerExecutor.forward_logits (executor/talker.py:
 * 173-183, 240-243) when mask_from < vocab.
 * logits: dtype NQ_F32 or NQ_BF16, [rows, vocab] with row stride logits_s0.
 * seen: uint8/bool [rows, vocab] (row stride seen_s0) or NULL.
 * top_k: int32 (<= 0 means the whole vocabulary).  Masks: ids >= mask_from
 * except eos_id become -inf; eos_id becomes -inf where suppress_eos[row] != 0
 * (suppress_eos may be NULL).  tokens: int64 [rows].  vocab <= 4096 (else
 * NQ_ERR_UNSUPPORTED).
 */
int nq_sample(const void *logits, int logits_dtype, int64_t logits_s0, int rows, int vocab,
              const float *temperature, const int32_t *top_k, const float *top_p,
              const float *repetition_penalty, uint8_t *seen, int64_t seen_s0,
              const float *uniforms, int mask_from, int eos_id, const uint8_t *suppress_eos,
              int update_seen, int64_t *tokens, void *stream);

/*
 * nq_sample with row r's uniform drawn inside the kernel from its (seed,
 * offset) counter exactly as nq_uniforms_from_counter computes it (the
 * reference draws the talker's uniform from its stateless (seed, offset) pair
 * in the same sampling call, executor/sampling.py:183-195): one launch
 * instead of two, same tokens.
 */
int nq_sample_counter(const void *logits, int logits_dtype, int64_t logits_s0, int rows, int vocab,
                      const float *temperature, const int32_t *top_k, const float *top_p,
                      const float *repetition_penalty, uint8_t *seen, int64_t seen_s0, const int64_t *seed,
                      int64_t seed_stride, const int64_t *offset, int64_t offset_stride, int mask_from,
                      int eos_id, const uint8_t *suppress_eos, int update_seen, int64_t *tokens, void *stream);

/*
 * nq_sample_counter reading the logits from a projection's fp32 split-K
 * planes [splits][rows][row_stride] (nq_linear with NQ_EPI_PARTIALS): each
 * logit is the planes' sum in plane order rounded to bf16, the value
 * nq_linear's own reduction stores, so the tokens are those of nq_linear
 * followed by nq_sample_counter, in one launch instead of two (the talker's
 * codec-head logits and their draw, executor/talker.py:173-183, 240-243,
 * 373).  The bf16 logits also go to logits_out (row stride out_s0) when it is
 * not NULL.  splits in [1, 64].
 */
int nq_sample_counter_planes(const float *planes, int splits, int64_t row_stride, int rows, int vocab,
                             const float *temperature, const int32_t *top_k, const float *top_p,
                             const float *repetition_penalty, uint8_t *seen, int64_t seen_s0, const int64_t *seed,
                             int64_t seed_stride, const int64_t *offset, int64_t offset_stride, int mask_from,
                             int eos_id, const uint8_t *suppress_eos, int update_seen, uint16_t *logits_out,
                             int64_t out_s0, int64_t *tokens, void *stream);

/*
 * Uniform draws in [0,1) from (seed, offset) counters with Philox-4x32-10
 * (Salmon et al., SC'11): key = seed, counter = (offset, 0); u = (x0 >> 8) * 2^-24.
 * Stands in for the stateless (seed, offset) draws of the reference
 * (executor/sampling.py:183-195,281; contract/rng.py:32-43).
 */
int nq_uniforms_from_counter(const int64_t *seed, int64_t seed_stride, const int64_t *offset,
                             int64_t offset_stride, int rows, float *uniforms, void *stream);

/*
 * Residual add + RMSNorm in place: residual += hidden; hidden = rmsnorm(residual).
 * Replaces flashinfer.norm.fused_add_rmsnorm as called by qwen3_tts_add_rmsnorm
 * (model/layers.py:43-79).  bf16 [rows, width], contiguous rows.
 */
int nq_add_rmsnorm(uint16_t *hidden, uint16_t *residual, const uint16_t *weight, int rows,
                   int width, float eps, void *stream);

/*
 * The talker step's input: residual[r] = bf16(addend[r] + table[ids[r]])
 * (the codec-step embedding plus the text embedding of materialize_decode,
 * executor/talker.py:256-262) and out[r] = rmsnorm(residual[r]) * weight (the
 * first layer's input norm, model/layers.py:82-115), in one launch; the same
 * bits as the add, then nq_rmsnorm.  table [num_embeddings, width] (row stride
 * table_s0), addend [rows, width] (row stride addend_s0), residual and out
 * contiguous; bf16, 16-byte aligned.  An id outside [0, num_embeddings) reads
 * row 0 and stores NQ_ERR_INVALID_ARGUMENT in *status (status may be NULL).
 * With addend == NULL the residual is the gathered row itself (the code
 * predictor's projected codec embedding as the next input,
 * executor/code_predictor.py:72-88, then the first input norm).
 */
int nq_embed_add_rmsnorm(const int64_t *ids, const uint16_t *table, int64_t table_s0, int64_t num_embeddings,
                         const uint16_t *addend, int64_t addend_s0, const uint16_t *weight, int rows, int width,
                         float eps, uint16_t *residual, uint16_t *out, int32_t *status, void *stream);

/*
 * Talker prefill input embedding and the first input norm in one launch
 * (TalkerExecutor.materialize_prefill, executor/talker.py:246-254, then the
 * first layer's input RMSNorm): residual[r] = text[text_ids[r]] +
 * codec[codec_ids[r]] (a bf16 add) where mask[r] != 0, else text[text_ids[r]];
 * out[r] = rmsnorm(residual[r]) * weight.  bf16 [rows, width], residual / out
 * contiguous; an id outside its table reads row 0 and stores
 * NQ_ERR_INVALID_ARGUMENT in *status (may be NULL).
 */
int nq_prefill_embed_rmsnorm(const int64_t *text_ids, const uint16_t *text_table, int64_t text_s0,
                             int64_t text_rows, const int64_t *codec_ids, const uint16_t *codec_table,
                             int64_t codec_s0, int64_t codec_rows, const uint8_t *mask, const uint16_t *weight,
                             int rows, int width, float eps, uint16_t *residual, uint16_t *out, int32_t *status,
                             void *stream);

/*
 * out[r] = first_table[first_ids[r]] + tables[0][ids[0][r]] + ... +
 * tables[groups-1][ids[groups-1][r]], added in group order with every partial
 * sum rounded to bf16: the code predictor's codec_sum (layer-0 embedding plus
 * the codec embedding of each group's token, executor/code_predictor.py:
 * 159-235 and model/components.py:254-411) in one launch, the same bits as
 * adding the rows one at a time in bf16.  ids[g][r] at ids + g * ids_s0 +
 * r * ids_s1; table g, row t at tables + g * table_s0 + t * table_s1.  bf16,
 * 16-byte aligned rows; width % 8 == 0.  An id outside its table reads row 0
 * and stores NQ_ERR_INVALID_ARGUMENT in *status (status may be NULL).
 */
int nq_gather_sum_rows(const int64_t *first_ids, const uint16_t *first_table, int64_t first_s0, int64_t first_rows,
                       const int64_t *ids, int64_t ids_s0, int64_t ids_s1, const uint16_t *tables, int64_t table_s0,
                       int64_t table_s1, int64_t table_rows, int groups, int rows, int width, uint16_t *out,
                       int64_t out_s0, int32_t *status, void *stream);

/*
 * out = rmsnorm(x) (model/layers.py:82-115).  bf16 [rows, width]; out may alias x.
 */
int nq_rmsnorm(const uint16_t *x, const uint16_t *weight, uint16_t *out, int rows, int width,
               float eps, void *stream);

/*
 * out[r, j] = silu(gate_up[r, j]) * gate_up[r, width + j]
 * (qwen3_tts_silu_and_mul, model/layers.py:28-40).  bf16, contiguous rows.
 */
int nq_silu_mul(const uint16_t *gate_up, uint16_t *out, int rows, int width, void *stream);

/*
 * Skinny projection Y[M, N] = X[M, K] . W[N, K]^T in bf16 with fp32
 * accumulation for M <= 128 activation rows (decode buckets), with the
 * consumer of the projection fused in.  Replaces the nn.Linear projections of
 * the talker layer run by torch/hipBLASLt (model/layers.py:195-270: packed
 * QKV, o_proj, gate_up, down; the codec head, executor/talker.py:231-262)
 * and, through `epilogue`, the kernel that follows each of them:
 *   NQ_EPI_NONE        out = bf16(Y + bias) (bias [N] bf16 or NULL: the
 *                      biased nn.Linear, one rounding like a GEMM epilogue)
 *   NQ_EPI_ADD_RMSNORM residual = bf16(residual + bf16(Y));
 *                      out = rmsnorm(residual) * norm_weight  (the fused
 *                      add-RMSNorm of model/layers.py:43-79; N <= 8192)
 *   NQ_EPI_SILU_MUL    out[M, N/2] = silu(bf16(Y[:, :N/2])) * bf16(Y[:, N/2:])
 *                      (qwen3_tts_silu_and_mul, model/layers.py:28-40)
 *   NQ_EPI_PARTIALS    Y is left as S = nq_linear_splits(M, N, K) fp32 planes
 *                      [S, M, N] at the start of `workspace` (for a consumer
 *                      that sums them itself).
 * K is cut into S slices whose fp32 partial planes are always summed in
 * slice order, so the result is deterministic and the same for every
 * epilogue.  Requires N % 64 == 0 and K % 512 == 0 (K % 256 when M > 64):
 * otherwise NQ_ERR_UNSUPPORTED (nq_linear_splits returns -1).  Row strides in
 * elements; x, w, out, residual, norm_weight 16-byte aligned.
 * nq_linear_workspace_bytes gives the workspace size (0 = none needed).
 */
enum nq_epilogue { NQ_EPI_NONE = 0, NQ_EPI_ADD_RMSNORM = 1, NQ_EPI_SILU_MUL = 2, NQ_EPI_PARTIALS = 3 };
int nq_linear_splits(int M, int N, int K);
int64_t nq_linear_workspace_bytes(int M, int N, int K, int epilogue);
int nq_linear(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M, int N, int K,
              int epilogue, const uint16_t *bias, uint16_t *out, int64_t o_s0, uint16_t *residual,
              const uint16_t *norm_weight, float eps, void *workspace, int64_t workspace_bytes,
              void *stream);

/*
 * Decode attention with the q/k norm + RoPE + K/V write fused in, for bindings
 * whose rows are all decode rows: the work of nq_qkv_partials_norm_rope_kv_write
 * (from the packed QKV projection's split-K planes [splits, tokens, (Hq + 2 Hkv)
 * D]) followed by nq_paged_attention with NQ_ATTN_DECODE, in one kernel (the
 * TalkerAttentionContext.attend path, executor/talker_kv.py:104-129 with
 * model/kernels.py:15-91, for decode bindings).  Uses the plan of
 * nq_attention_plan: rows are dealt whole to 256 workgroups (sorted by length,
 * snake order; rows longer than a workgroup's share are cut, and the last
 * arriving piece of a cut row merges it), so partial results merge inside a
 * workgroup.  Each decode row's position and K/V write slot come from the
 * plan, which must have been given the same positions / write_pages /
 * write_offsets as this call (a plan without them makes every K/V write
 * invalid: status NQ_ERR_INVALID_ARGUMENT).  The rotated q is not stored
 * (attend returns the attention output only).  head_dim 128 with 1 or 2 query
 * heads per kv head; other shapes return NQ_ERR_UNSUPPORTED and the caller runs
 * the two entry points it replaces.
 */
int nq_paged_decode_rope_attention(const float *partials, int splits, int tokens, const uint16_t *q_weight,
                                   const uint16_t *k_weight, const int64_t *positions, float eps,
                                   float rope_theta, int round_to_input, uint16_t *cache, int64_t c_page,
                                   int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages,
                                   const int64_t *write_pages, const int64_t *write_offsets,
                                   const int32_t *kv_indices, int page_size, int num_qo_heads, int num_kv_heads,
                                   int head_dim, float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                                   int max_query_tokens, int max_pages, void *workspace, int64_t workspace_bytes,
                                   int32_t *status, void *stream);

/*
 * FP8 (OCP e4m3fn) block quantization of a bf16 weight matrix w [N, K] into
 * codes q [N, K] and fp32 scales [N / 128, K / 128]: per 128 x 128 block,
 * scale = 2^ceil(log2(max(max|w|, 1e-4) / 448)) and q = e4m3fn(w / scale)
 * rounded to nearest even.  Replaces quantize_fp8_weight_blocks
 * (model/layers.py:10-25) as run by GatedMLP.initialize_fp8_gate_up_weight
 * (model/layers.py:226-239).  N, K multiples of 128 (else
 * NQ_ERR_INVALID_ARGUMENT, the reference's ValueError); strides in elements.
 */
int nq_quantize_fp8_blocks(const uint16_t *w, int64_t w_s0, int N, int K, uint8_t *q, int64_t q_s0,
                           float *scales, int64_t s_s0, void *stream);

/*
 * Activation quantization of the block-scaled FP8 GEMM: bf16 x [M, K] ->
 * codes q [M, K] and fp32 scales [M, K / 128], per row and 128 columns
 * scale = max|x| / 448 (1 for an all-zero group), q = e4m3fn(x / scale).  The
 * bf16-input half of flashinfer fp8_blockscale_gemm_sm90 as called at
 * model/layers.py:253-261 (published DeepGEMM / DeepSeek-V3 1 x 128 scheme).
 */
int nq_quantize_fp8_rows(const uint16_t *x, int64_t x_s0, int M, int K, uint8_t *q, int64_t q_s0,
                         float *scales, int64_t s_s0, void *stream);

/*
 * nq_add_rmsnorm with the normalised row stored quantized (codes xq [rows,
 * width], scales sx [rows, width / 128], as nq_quantize_fp8_rows of the bf16
 * result) instead of in `hidden`: the post-attention add-RMSNorm feeding the
 * FP8 gate/up projection (model/components.py:56-63 into GatedMLP.forward,
 * model/layers.py:264-270).  width % 128 == 0.
 */
int nq_add_rmsnorm_fp8(const uint16_t *hidden, uint16_t *residual, const uint16_t *weight, int rows,
                       int width, float eps, uint8_t *xq, int64_t xq_s0, float *sx, int64_t sx_s0,
                       void *stream);

/*
 * nq_linear with NQ_EPI_ADD_RMSNORM whose normalised output is stored as
 * nq_add_rmsnorm_fp8 stores it: the o_proj + post-attention add-RMSNorm of a
 * talker layer with FP8 gate/up.  N % 128 == 0; workspace as
 * nq_linear_workspace_bytes(M, N, K, NQ_EPI_ADD_RMSNORM).
 */
int nq_linear_add_rmsnorm_fp8(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M,
                              int N, int K, uint16_t *residual, const uint16_t *norm_weight, float eps,
                              uint8_t *xq, int64_t xq_s0, float *sx, int64_t sx_s0, void *workspace,
                              int64_t workspace_bytes, void *stream);

/*
 * Block-scaled FP8 projection for M <= 128 rows: Y[m, n] = sum over 128-wide
 * K blocks kb of sx[m, kb] * sw[n / 128, kb] * (q_x[m, kb] . q_w[n, kb]) with
 * fp32 accumulation (flashinfer fp8_blockscale_gemm_sm90 as called by
 * GatedMLP._project_gate_up, model/layers.py:241-262), epilogues as
 * nq_linear: NQ_EPI_NONE (out = bf16(Y)), NQ_EPI_SILU_MUL (the SwiGLU of the
 * gate/up output, model/layers.py:264-270) or NQ_EPI_PARTIALS.  N % 128 == 0,
 * K % 1024 == 0 (K % 512 when M > 64); codes 16-byte aligned with strides
 * multiple of 16 bytes; scale strides in elements.
 */
int nq_linear_fp8_splits(int M, int N, int K);
int64_t nq_linear_fp8_workspace_bytes(int M, int N, int K, int epilogue);
int nq_linear_fp8(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, const uint8_t *wq,
                  int64_t w_s0, const float *sw, int64_t sw_s0, int M, int N, int K, int epilogue,
                  uint16_t *out, int64_t o_s0, void *workspace, int64_t workspace_bytes, void *stream);

/*
 * Gate/up with the SwiGLU fused, for the talker's MLP shape (M <= 64 rows,
 * K = 2048, I % 24 == 0; else NQ_ERR_UNSUPPORTED and the caller uses
 * nq_linear_fp8 with NQ_EPI_SILU_MUL): out[M, I] = silu(bf16(gate)) *
 * bf16(up) of the block-scaled FP8 product (GatedMLP.forward with FP8
 * gate/up, model/layers.py:241-270), whole dot products per workgroup (no
 * split-K planes, no second kernel).  The weight codes are the
 * nq_quantize_fp8_blocks codes with their rows interleaved by
 * nq_fp8_pack_swiglu (the block scales stay those of the [gate; up] layout).
 */
int nq_fp8_pack_swiglu(const uint8_t *q, int64_t q_s0, int I, int K, uint8_t *packed, int64_t p_s0,
                       void *stream);

/*
 * bf16 gate/up with the SwiGLU fused, for the code predictor's MLP shape
 * (K = 1024, I % 24 == 0, any row count in blocks of 64; else
 * NQ_ERR_UNSUPPORTED and the caller uses nq_linear with NQ_EPI_SILU_MUL):
 * out[M, I] = silu(bf16(gate)) * bf16(up) of x[M, K] . W^T (GatedMLP.forward,
 * model/layers.py:264-270, as the code predictor's MLP runs it), whole dot
 * products per workgroup (no split-K planes, no second kernel), summing K in
 * four 256-wide quarters in order: the bits of nq_linear + NQ_EPI_SILU_MUL
 * wherever that cuts K into 256-wide slices (128 rows).  `packed` holds the [gate; up] rows [2I, K]
 * interleaved by nq_fp8_pack_swiglu applied to the bf16 rows as bytes (row
 * length 2K bytes, strides in bytes).
 */
int nq_linear_swiglu(const uint16_t *x, int64_t x_s0, int M, const uint16_t *packed, int64_t w_s0, int I, int K,
                     uint16_t *out, int64_t o_s0, void *stream);
int nq_linear_fp8_swiglu(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, int M,
                         const uint8_t *packed, int64_t w_s0, const float *sw, int64_t sw_s0, int I, int K,
                         uint16_t *out, int64_t o_s0, void *stream);

/*
 * Prefill-sized projections (the talker layer's QKV / o / gate_up / down,
 * model/layers.py:195-317, at the prefill captures' token counts,
 * planner/catalog.py:262-314): tiled MFMA GEMMs for any M >= 1 (128 x 128
 * tiles, LDS-staged 64-wide K slices with two slices of global loads in
 * flight, XCD-grouped tiles; K split into S slices when the tiles alone would
 * leave CUs idle).  The argument meanings, epilogues and workspace rules are
 * those of nq_linear / nq_linear_add_rmsnorm_fp8 (NQ_EPI_SILU_MUL on
 * [gate; up] weights, NQ_EPI_PARTIALS leaving S fp32 planes [S, M, N] at the
 * workspace start); N % 128 == 0 (I % 64 == 0 for SwiGLU), K % 64 == 0,
 * 16-byte aligned X / W with row strides % 8 elements, else
 * NQ_ERR_UNSUPPORTED.  nq_tgemm_splits is S (-1 for unsupported shapes);
 * nq_tgemm_workspace_bytes is the workspace an epilogue needs.
 *
 * nq_tgemm_fp8_swiglu: the block-scaled FP8 gate/up + SwiGLU of
 * nq_linear_fp8_swiglu (same codes, scales, interleaved weight rows and
 * output) for any M; K % 128 == 0 and I % 128 == 0.
 */
int nq_tgemm_splits(int M, int N, int K);
int64_t nq_tgemm_workspace_bytes(int M, int N, int K, int epilogue);
int nq_tgemm(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M, int N, int K, int epilogue,
             uint16_t *out, int64_t o_s0, uint16_t *residual, const uint16_t *norm_weight, float eps,
             void *workspace, int64_t workspace_bytes, void *stream);
int nq_tgemm_add_rmsnorm_fp8(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M, int N, int K,
                             uint16_t *residual, const uint16_t *norm_weight, float eps, uint8_t *xq, int64_t xq_s0,
                             float *sx, int64_t sx_s0, void *workspace, int64_t workspace_bytes, void *stream);
int nq_tgemm_fp8_swiglu(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, int M,
                        const uint8_t *packed, int64_t w_s0, const float *sw, int64_t sw_s0, int I, int K,
                        uint16_t *out, int64_t o_s0, void *stream);

/*
 * fp32 GEMM with fused epilogues for the codec decoder (fp32 throughout,
 * executor/build.py:91-95), replacing torch's addmm / matmul / gelu / the
 * residual-scale adds of model/incremental_codec.py's transformer, ConvNeXt and
 * im2col convolutions:
 *   out[m, n] = res[m, n] + scale[n] * act(sum_k X[r(m), k] W[n, k] + bias[n])
 * with res / scale / bias optional (NULL), act 0 (none) or 1 (GELU, erf form),
 * r(m) = x_rows[m] when x_rows != NULL else m; out may alias res.  K % 4 == 0,
 * N % 4 == 0, 16-byte aligned operands and row strides % 4, else
 * NQ_ERR_UNSUPPORTED.
 *
 * precision names torch's float32 matmul precisions: NQ_MATMUL_HIGHEST, fp32
 * products on MFMA; NQ_MATMUL_HIGH, the reference's serving policy
 * (model/checkpoint.py:46-49 sets torch.set_float32_matmul_precision("high")):
 * each operand as the sum of two bf16 (hi = bf16(v), lo = bf16(v - hi)) and
 * each product as hi*hi + hi*lo + lo*hi on bf16 MFMA with fp32 sums, within
 * 3 * 2^-16 of the fp32 product.
 *
 * nq_row_norm: RMSNorm (b == NULL: x * rsqrt(mean(x^2) + eps) * w) or
 * LayerNorm ((x - mean) * rsqrt(var + eps) * w + b) of fp32 rows, width % 4 ==
 * 0 and <= 1024.
 *
 * nq_codec_last_rows: rows[b] = max(off[b + 1] * u - 1, 0), the row of each
 * stream's last fresh frame at a stage with u rows per frame.
 */
enum nq_matmul_precision { NQ_MATMUL_HIGHEST = 0, NQ_MATMUL_HIGH = 1 };
int nq_sgemm(const float *x, int64_t x_s0, const int32_t *x_rows, const float *w, int64_t w_s0, int M, int N, int K,
             const float *bias, int act, const float *res, int64_t r_s0, const float *scale, float *out, int64_t o_s0,
             int precision, void *stream);
int nq_row_norm(const float *x, int64_t x_s0, int rows, int width, const float *w, const float *b, float eps,
                float *out, int64_t o_s0, void *stream);
int nq_codec_last_rows(const int32_t *off, int B, int u, int32_t *rows, void *stream);

/*
 * Incremental codec-decoder step (fp32, channels-last [T, C]).  Replaces the
 * stateful pieces of Qwen3TTSIncrementalDecoder (model/incremental_codec.py):
 * the fresh rows of B streams are concatenated; stream b owns frames
 * [offsets[b], offsets[b+1]) (device int32 [B+1]) and, at a stage with u
 * samples per frame, rows [offsets[b]*u, offsets[b+1]*u).  Stream b's state
 * lives in slot slots[b] of the state arrays.
 *
 * nq_codec_embed_sum: out[t] = sum_q books[q][codes[t*Q + q]] (the codebook
 *   sum of quantizer.decode); ids outside [0, V) set *status (device int32,
 *   may be NULL) to NQ_ERR_INVALID_ARGUMENT and are skipped.
 * nq_codec_causal_conv: causal Conv1d with per-stream left history
 *   (_causal_conv, :58-88): w [Cout, Cin/groups, K], groups 1 or Cin
 *   (depthwise), history [slots, (K-1)*dilation, Cin] holding post-activation
 *   inputs.  Optional SnakeBeta on the input (act_alpha/act_beta: log-scale
 *   per-channel parameters, x + sin(e^a x)^2 / e^b) and a residual added to the
 *   output.  The history is advanced in place after the convolution; histories
 *   of more than 4096 values per stream ((K-1)*dilation*Cin) are refused
 *   (NQ_ERR_UNSUPPORTED) before any launch.
 * nq_codec_causal_transconv: causal ConvTranspose1d with kernel 2*stride and
 *   a stride-long bias-free overlap carry (_causal_transconv, :90-138):
 *   w [Cin, Cout, 2*stride], overlap [slots, stride, Cout]; optional SnakeBeta
 *   on the input; output rows at u_in*stride samples per frame.
 * nq_codec_window_attention: per-head RMSNorm + RoPE of q and k (positions =
 *   frame_pos[slot] + fresh index), attention over the R = window-1 retained
 *   and the fresh frames inside the sliding window, with retained slot j
 *   valid when j >= R - ctx_len[slot]; then the retained K/V
 *   ([slots, R, H, D] per layer, slot stride state_slot_stride) advance in
 *   place (_pre_transformer, :193-381).  q, k, v rows share stride ld; the
 *   fresh k rows are left rotated (q is only read).  One launch, one workgroup
 *   per (stream, head); D must be 16, 32 or 64, window <= 32, and the
 *   operands 16-byte aligned with strides % 4 == 0, else NQ_ERR_UNSUPPORTED.
 * nq_codec_advance: frame_pos[slot] += F; ctx_len[slot] = min(R, ctx + F)
 *   (:375-380), once per step after the last layer.
 * nq_codec_pcm16: wav = clamp(x, -1, 1); pcm = round-half-even(wav * 32767)
 *   (executor/codec.py:236-238); either output may be NULL.
 */
int nq_codec_embed_sum(const int32_t *codes, int T, int Q, const float *books, int V, int C, float *out,
                       int32_t *status, void *stream);
int nq_codec_causal_conv(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                         const int32_t *slots, float *history, const float *w, const float *bias, int Cin,
                         int Cout, int K, int dilation, int groups, const float *act_alpha,
                         const float *act_beta, const float *residual, int64_t ldres, float *out,
                         int64_t ldo, void *stream);

/*
 * nq_codec_residual_unit: one decoder residual unit of C <= 32 channels in one
 * launch (plus the history update of its K-tap convolution),
 *   out = x + conv1x1_w2(snake_a2(causal_conv_w1(snake_a1(x), dilation) + b1)) + b2,
 * with the same per-stream history rules as nq_codec_causal_conv for the
 * K-tap convolution (history [slots, (K-1)*dilation, C] of snake_a1(x),
 * advanced in place).  Replaces the residual unit of the upstream decoder block
 * as the adapter runs it (model/incremental_codec.py:58-88 for the causal
 * convolutions): two convolutions whose intermediate tensor never reaches
 * memory.  precision NQ_MATMUL_HIGHEST: fp32 products on the vector ALUs, the
 * bits of the two nq_codec_causal_conv launches.  NQ_MATMUL_HIGH (the
 * decoder's default, as the reference's convolutions run under cuDNN's TF32
 * default): for C = 16 and 32 both convolutions as implicit GEMMs on bf16 MFMA
 * with the split products of nq_sgemm's NQ_MATMUL_HIGH (each product within
 * 3 * 2^-16 of fp32, fp32 sums; x, out and history 16-byte aligned with ldx,
 * ldo % 4 == 0); C = 8 keeps the fp32 products.
 * w1 [C, C, K], w2 [C, C, 1]; out must not alias x.  C must be 8, 16 or 32.
 */
int nq_codec_residual_unit(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                           const int32_t *slots, float *history, int C, int K, int dilation, const float *w1,
                           const float *b1, const float *a1_alpha, const float *a1_beta, const float *w2,
                           const float *b2, const float *a2_alpha, const float *a2_beta, float *out, int64_t ldo,
                           int precision, void *stream);
int nq_codec_causal_transconv(const float *x, int64_t ldx, int64_t T_in, const int32_t *offsets, int B,
                              int u_in, int stride_s, const int32_t *slots, float *overlap, const float *w,
                              const float *bias, int Cin, int Cout, const float *act_alpha,
                              const float *act_beta, float *out, int64_t ldo, void *stream);
int nq_codec_window_attention(float *q, float *k, const float *v, int64_t ld, int T, int H, int D,
                              const float *q_norm, const float *k_norm, float eps, float rope_theta,
                              const int32_t *offsets, int B, const int32_t *slots, const int64_t *frame_pos,
                              const int32_t *ctx_len, float *state_k, float *state_v,
                              int64_t state_slot_stride, int R, int window, float *out, int64_t ldo,
                              void *stream);
int nq_codec_advance(const int32_t *offsets, int B, const int32_t *slots, int64_t *frame_pos,
                     int32_t *ctx_len, int R, void *stream);
int nq_codec_pcm16(const float *x, int64_t n, float *wav, int16_t *pcm, void *stream);

/*
 * GEMM form of the wide convolutions.  nq_codec_im2col gathers the operand a
 * conv (or transconv) becomes one GEMM over: conv rows hold the K taps of the
 * (activated) input, history included, as a[t, k*Cin + ci]; transconv rows
 * hold [act(x[t]), act(x[t-1])] (zeros before a stream's first fresh frame;
 * K must be 2).  Cin % 4 == 0.  After the GEMM, nq_codec_history_update
 * advances a conv's history, and nq_codec_transconv_overlap adds the stored
 * overlap to each stream's first `stride` output rows and stores the new one,
 * new_overlap [B, stride * Cout] = (last fresh frame, activated) x (the
 * kernel's second half), which the caller computes with a small GEMM.
 */
int nq_codec_im2col(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                    const int32_t *slots, const float *history, int Cin, int K, int dilation, int transconv,
                    const float *act_alpha, const float *act_beta, float *a, int64_t lda, void *stream);
int nq_codec_history_update(const float *x, int64_t ldx, const int32_t *offsets, int B, int u,
                            const int32_t *slots, float *history, int C, int pad, const float *act_alpha,
                            const float *act_beta, void *stream);
int nq_codec_transconv_overlap(const int32_t *offsets, int B, int u_in, int stride_s,
                               const int32_t *slots, float *overlap, const float *new_overlap, int Cout,
                               float *out, int64_t ldo, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_ABI_H */
