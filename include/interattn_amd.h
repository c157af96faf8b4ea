/*
 * interattn_amd -- C ABI of the MI355X (gfx950) condition-block sparse
 * decode-attention library.
 *
 * Every entry point takes plain device pointers, sizes and strides, launches
 * asynchronously on the given HIP stream (NULL = the default stream), never
 * allocates device memory, never synchronises, and returns 0 on success or a
 * non-zero IA_ERR_* code.  ia_last_error() returns the message of the last
 * failure on the calling thread.  Scratch memory comes from a caller-owned
 * workspace whose size is given by the matching *_workspace_size() function,
 * 256-byte aligned; its contents need no initialisation, except for
 * ia_sparse_topk_decode (zero-filled once, see there).  Calls that share one
 * workspace must not overlap.  Multi-step work (score -> select, split-K partials
 * -> merge) is ordered by kernel boundaries on the caller's stream, except inside
 * ia_sparse_topk_decode, whose one launch hands data between workgroups through
 * flags with bounded waits.
 *
 * Reference paths below are relative to the reference repository root;
 * CBT = llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl,
 * CBG = llama/script/analysis/condition_block_gen.
 */
#ifndef INTERATTN_AMD_H
#define INTERATTN_AMD_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define IA_API __attribute__((visibility("default")))
#else
#define IA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum {
  IA_F32 = 0,
  IA_BF16 = 1,
  IA_FP8_E4M3 = 2, /* OCP e4m3fn, dequantised as code * scale[page, kv_head] */
};

/* Error codes. */
enum {
  IA_OK = 0,
  IA_ERR_INVALID = 1,     /* argument outside the supported contract */
  IA_ERR_UNSUPPORTED = 2, /* valid combination with no kernel instance */
  IA_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  IA_ERR_LAUNCH = 4,      /* HIP reported a launch error */
};

/*
 * A paged K/V source.  Row (token) t of page p for kv head h starts at
 *   k + (p * k_page_stride + h * k_head_stride + t * k_token_stride) elements
 * and holds head_dim contiguous elements; the same for v.  Logical token i of
 * batch entry b lives in page block_table[b * bt_stride + i / page_size] at row
 * i % page_size (only the first bt_cols entries of a row are ever read).
 * block_table == NULL means the identity table (page = i /
 * page_size), which describes the reference's contiguous padded prompt view
 * [Hkv, nb, B, D] (CBT/core.py:383-408) with page_size = B.  Page ids outside
 * [0, n_pages) are skipped (they contribute nothing) instead of being read.
 * For IA_FP8_E4M3, k_scale/v_scale hold one float per (page, kv head) at
 * scale[p * scale_page_stride + h].  Optionally (fp8 only, else NULL) seq_scale
 * holds the same two scales gathered per sequence: the (k, v) pair of logical page
 * lp of batch entry b, kv head h at
 *   seq_scale[b * seq_scale_b_stride + h * seq_scale_h_stride + 2 * lp + {0, 1}]
 * for every lp < bt_cols (identity table: lp < n_pages), equal to
 * (k_scale, v_scale)[block_table[b, lp], h] wherever that page id is valid.  The
 * pairs of a block's consecutive pages then share a cache line, so the finalize
 * reads one line per selected block instead of two per page; the per-page arrays
 * are still required (the summary kernels read them).  The pointer and both strides
 * must be even (8-byte pairs).
 */
typedef struct ia_paged_kv {
  const void* k;
  const void* v;
  int32_t dtype;
  int32_t page_size; /* tokens per page; a multiple of 16 */
  int64_t n_pages;
  int64_t k_page_stride, k_head_stride, k_token_stride;
  int64_t v_page_stride, v_head_stride, v_token_stride;
  const int32_t* block_table;
  int64_t bt_stride;
  int64_t bt_cols; /* valid entries per block-table row; pages past it are skipped */
  const float* k_scale;
  const float* v_scale;
  int64_t scale_page_stride;
  const float* seq_scale; /* optional, fp8: per-sequence (k, v) scale pairs (see above) */
  int64_t seq_scale_b_stride, seq_scale_h_stride;
} ia_paged_kv;

/* Query / output geometry: q[b, row, :] at q + b * q_batch_stride + row * q_row_stride,
 * rows = n_q_heads, row h*G+g attends kv head h (G = n_q_heads / n_kv_heads). */
typedef struct ia_decode_shape {
  int32_t batch;
  int32_t n_q_heads;
  int32_t n_kv_heads;
  int32_t head_dim; /* 64 or 128 */
  int64_t q_batch_stride;
  int64_t q_row_stride;
  int32_t q_dtype; /* IA_F32 or IA_BF16 */
} ia_decode_shape;

IA_API const char* ia_last_error(void);
IA_API int ia_version(void);

/*
 * Per-block summaries of a paged sequence batch: over the valid tokens of each
 * logical block of block_size tokens, counts, mean key k_bar, mean value
 * v_bar, elementwise k_max / k_min and the max token value-norm v_norm_max,
 * plus v_norm_all = max over blocks.  Replaces _build_prompt_blocks
 * (CBT/core.py:449-500) for paged pools.  Outputs are [batch, Hkv, nb_max, D]
 * (k_bar, v_bar, k_max, k_min), [batch, Hkv, nb_max] (v_norm_max),
 * [batch, Hkv] (v_norm_all) and [batch, nb_max] (counts, int32); any output
 * pointer except counts may be NULL to skip it.  Blocks at or past a
 * sequence's end get count 0, zero means and -inf/+inf/-inf extrema/norms.
 * seq_lens is a device array [batch].
 */
IA_API int ia_build_block_summaries(const ia_paged_kv* kv, const int32_t* seq_lens, int32_t batch,
                             int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t nb_max, void* k_bar, int32_t k_bar_dtype, void* v_bar,
                             int32_t v_bar_dtype, void* k_max, void* k_min,
                             int32_t bounds_dtype, float* v_norm_max, float* v_norm_all,
                             int32_t* counts, void* stream);

/*
 * Incremental form of ia_build_block_summaries for sequences that grew from
 * old_seq_lens[b] to seq_lens[b] tokens (device arrays; old <= new and
 * new - old <= max_new_tokens): only blocks [old / block_size,
 * ceil(new / block_size)) are recomputed (the partial block at the old end and
 * every block the new tokens reach) and v_norm_all is raised to their norms.
 * The result equals a full rebuild at seq_lens, bit for bit.  Outputs as for
 * ia_build_block_summaries, holding the summaries at old_seq_lens on entry.
 * The reference never refreshes its summaries (generated tokens stay an exact
 * suffix, CBT/core.py:1325-1339); this is the serving pool's maintenance step.
 */
IA_API int ia_update_block_summaries(const ia_paged_kv* kv, const int32_t* old_seq_lens,
                                     const int32_t* seq_lens, int32_t batch, int32_t n_kv_heads,
                                     int32_t head_dim, int32_t block_size, int32_t nb_max,
                                     int32_t max_new_tokens, void* k_bar, int32_t k_bar_dtype,
                                     void* v_bar, int32_t v_bar_dtype, void* k_max, void* k_min,
                                     int32_t bounds_dtype, float* v_norm_max, float* v_norm_all,
                                     int32_t* counts, void* stream);

/*
 * Append one token's K/V per sequence into the paged pool: k_new/v_new
 * [batch, Hkv, D] (pool dtype; rows contiguous, strides in elements) are written
 * at logical position seq_lens[b] through the block table, then seq_lens[b] is
 * incremented, all on the device (a captured decode step can replay it).  The
 * page that holds the position must already be mapped (bt_cols and n_pages
 * bound it; a position past them is skipped and its length left unchanged).
 * bf16 and f32 pools only.  New entry point: the reference appends through
 * transformers' KV cache (torch.cat / StaticCache index_copy).
 */
IA_API int ia_append_kv(const ia_paged_kv* kv, const void* k_new, const void* v_new, int64_t new_batch_stride,
                        int64_t new_head_stride, int32_t* seq_lens, int32_t batch, int32_t n_kv_heads,
                        int32_t head_dim, void* stream);

/*
 * The block keys a top-k rule scores, one row of head_dim contiguous elements per
 * block: row j of (b, h) at b * batch_stride + h * head_stride + j * head_dim
 * elements (16-byte aligned rows).
 *   IA_SCORE_MEAN_KEY: score = mean_g(q[b, h*G+g] . k_bar[b, h, j]) / sqrt(D), the
 *     group-mean representative score of CBG/methods/quest.py:101 with the block's
 *     mean key as representative (k_bar);
 *   IA_SCORE_QUEST: score = mean_g sum_d max(q_gd k_max_d, q_gd k_min_d), Quest's page
 *     bound (CBG/methods/quest.py:97-101; k_max, k_min).
 * The mean-key score has no "+ log(count)" term: every block but the last holds
 * block_size tokens, so the term is a constant that cannot change the order, and
 * the Quest rule the top-k configurations follow ranks pages by q.k alone.
 */
enum {
  IA_SCORE_MEAN_KEY = 0,
  IA_SCORE_QUEST = 1,
};
typedef struct ia_block_keys {
  int32_t score; /* IA_SCORE_MEAN_KEY or IA_SCORE_QUEST */
  int32_t dtype; /* IA_F32 or IA_BF16 (every key array) */
  const void* k_bar;
  const void* k_max;
  const void* k_min;
  int64_t batch_stride, head_stride;
} ia_block_keys;

/*
 * Top-k block selection.  Per (b, h) the result is the forced blocks (the first
 * forced_first and last forced_last valid blocks) plus the top k_eff of the others
 * by score (ia_block_keys), ties to the lower index, with k_eff = k - #forced when
 * forced_in_k else k (k_per_seq, a device array [batch], overrides k per sequence
 * when non-NULL).  idx[b, h, 0:n_sel[b,h]] receives the chosen block ids in
 * ascending order (idx row stride k_cap >= k_eff + #forced).  scores may be NULL;
 * otherwise it receives [batch, Hkv, nb_max] float32 (-inf past the end).
 * The selection rule is the group-mean + torch.topk of CBG/methods/quest.py:91-103;
 * the reference's condition-block path selects by an eps threshold instead
 * (_select_prompt_blocks_triton, CBT/core.py:701-744).
 */
IA_API size_t ia_select_topk_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t nb_max);
IA_API int ia_select_topk(const ia_decode_shape* shape, const void* q, const ia_block_keys* keys,
                   const int32_t* seq_lens, int32_t block_size, int32_t nb_max, int32_t k,
                   const int32_t* k_per_seq, int32_t forced_first, int32_t forced_last,
                   int32_t forced_in_k,
                   int32_t* idx, int32_t k_cap, int32_t* n_sel, float* scores, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Block mask [batch, n_kv_heads, nb] uint8 of a top-k selection: 1 for the blocks
 * idx[b, h, 0:n_sel[b, h]] (ids outside [0, nb) ignored), 0 elsewhere.  With
 * ia_fixed_mask_decode it gives the top-k finalize with representatives for the
 * unselected blocks (the external-mask semantics of fixed_mask_hybrid_attention,
 * CBG/real_attention_benchmark/fixed_mask.py:38-239, applied to a top-k
 * selection); no single reference function corresponds.
 */
IA_API int ia_topk_block_mask(const int32_t* idx, const int32_t* n_sel, int32_t k_cap, int32_t batch,
                              int32_t n_kv_heads, int32_t nb, uint8_t* mask, void* stream);

/*
 * Sparse paged decode (finalize attention over selected blocks).  For each
 * (b, q row) the softmax of q . K^T * scale over the valid tokens of the blocks
 * idx[b, h, 0:n_sel[b,h]] (block_size tokens each), applied to V; split-K with an
 * online-softmax merge (CBT/page_attention.py:206-255, CBT/legacy.py:765-794): one
 * flat grid of about one workgroup per CU, each (b, h) row split into items in
 * proportion to its 16-token subtiles.  out: [batch, n_q_heads, D] contiguous,
 * out_dtype IA_F32 or IA_BF16.  batch * n_kv_heads must not exceed 8192
 * (IA_ERR_UNSUPPORTED).  Replaces the selected-page stream of
 * _condition_block_finalize_attention_kernel for the top-k rule.
 */
IA_API size_t ia_paged_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group,
                                      int32_t head_dim, int32_t max_items);
IA_API int ia_sparse_paged_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                           const int32_t* seq_lens, int32_t block_size, const int32_t* idx,
                           int32_t k_cap, const int32_t* n_sel, float scale, void* out,
                           int32_t out_dtype, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * Dense paged decode: softmax(q . K^T * scale) V over every valid token
 * (seq_lens[b] tokens) of each sequence.  The dense fallback of
 * _sdpa_full_attention_forward (CBT/core.py:1158-1177) over a paged pool.
 */
IA_API int ia_paged_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                    const int32_t* seq_lens, int32_t max_seq_len, float scale, void* out,
                    int32_t out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-block summaries consumed by the condition (eps-threshold) rule: arrays
 * [batch, Hkv, nb, D] (k_bar, k_max, k_min, v_bar; contiguous), v_norm_max
 * [batch, Hkv, nb] and v_norm_all [batch, Hkv] float32, counts [batch, nb]
 * int32 (valid tokens per block; 0 = no block).  block_size = tokens per block.
 * This is the prefix dict of _build_prompt_blocks (CBT/core.py:449-500) with a
 * batch dimension.  bounds_packed = 1: the bounds are the reference's packed
 * k_bounds instead (CBT/core.py:490-499, CONDITION_BLOCK_TMA_BOUNDS=1): k_max points
 * to [batch, Hkv, nb, 2 D] whose element pair (k_max, k_min) of dimension e sits at
 * [2e, 2e + 1], and k_min is not read (the statistics read each lane's pairs with
 * the same two 16-byte loads as the separate rows).
 */
typedef struct ia_block_summaries {
  const void* k_bar;
  const void* k_max;
  const void* k_min;
  const void* v_bar;
  int32_t k_bar_dtype, bounds_dtype, v_bar_dtype; /* IA_F32 or IA_BF16 */
  const float* v_norm_max;
  const float* v_norm_all;
  const int32_t* counts;
  int32_t nb;
  int32_t block_size;
  int32_t bounds_packed; /* 0: k_max and k_min rows; 1: packed k_bounds at k_max */
} ia_block_summaries;

/*
 * The exact suffix (generated tokens kept outside the blocks, CBT/core.py:1316-
 * 1324): token t of batch entry b, kv head h at k + b*k_batch_stride +
 * h*k_head_stride + t*k_token_stride (elements, same dtype as the prompt K/V).
 * len is device memory (entry b, or entry 0 for all when len_stride == 0) so a
 * captured decode step can advance it (CBT/page_attention.py:256-259); cap bounds it.
 */
typedef struct ia_suffix_kv {
  const void* k;
  const void* v;
  int64_t k_batch_stride, k_head_stride, k_token_stride;
  int64_t v_batch_stride, v_head_stride, v_token_stride;
  const int32_t* len;
  int32_t len_stride;
  int32_t cap;
} ia_suffix_kv;

/*
 * Selection statistics of the condition rule: replaces
 * _run_condition_block_selection_stats / _condition_block_selection_stats_kernel
 * (CBT/core.py:573-698, :747-814) and, when globals != NULL, the reduce kernel
 * (CBT/core.py:817-847).  Outputs s, delta [batch, rows, nb], partial
 * [batch, 4, rows, ceil(nb/16)] = (z_m, z_l, c_m, c_l) per 16-block chunk,
 * globals [batch, 4, rows].
 */
IA_API int ia_condition_selection_stats(const ia_decode_shape* shape, const void* q,
                                        const ia_block_summaries* sm, int32_t term1_mass_exp,
                                        float* s, float* delta, float* partial, float* globals,
                                        void* stream);

/*
 * The eps threshold of the condition rule: replaces
 * _condition_block_selection_finalize_kernel (CBT/core.py:850-905).  selected
 * [batch, rows, nb] uint8 (the group decision broadcast to the group's rows),
 * z [batch, rows, nb] float32 (may be NULL).
 */
IA_API int ia_condition_select(const ia_decode_shape* shape, const ia_block_summaries* sm,
                               const float* s, const float* delta, const float* globals, float eps,
                               int32_t term1_mass_exp, uint8_t* selected, float* z, void* stream);

/*
 * Fused condition-block decode: statistics, routing, representatives of the
 * unselected blocks, the selected blocks' tokens and the exact suffix in one
 * online softmax.  Replaces _condition_block_decode_output_fused_triton
 * (CBT/core.py:1035-1155).  selected (optional) receives [batch, rows, nb].
 * out: [batch, n_q_heads, D].
 */
IA_API size_t ia_condition_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group,
                                          int32_t head_dim, int32_t nb, int32_t suffix_cap);
IA_API int ia_condition_decode(const ia_decode_shape* shape, const void* q,
                               const ia_block_summaries* sm, const ia_paged_kv* prompt,
                               const ia_suffix_kv* suffix, float eps, int32_t term1_mass_exp,
                               uint8_t* selected, float scale, void* out, int32_t out_dtype,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * ia_condition_decode in one launch.  Each (sequence, kv head) row is split into n
 * items, item i owning blocks i, i + n, i + 2n, ... (so neighbouring selected blocks
 * spread over the items); an item computes the statistics of its blocks, the row's items exchange their partials of the row statistics (tagged
 * words in the workspace, each wait bounded by the wait limit, a partial still
 * missing then computed by the waiting item itself), every item merges them in
 * item order, routes its blocks, forms the representative partial of its
 * unselected blocks and streams its selected blocks (the last item also the exact
 * suffix), and the last item of the row to finish merges the items' partials.
 * The selection equals ia_condition_decode's except for blocks whose condition is
 * within float rounding of eps (the row statistics are summed in another order);
 * the output agrees to float rounding.  Arguments as for ia_condition_decode; the
 * workspace (ia_condition_decode_fused_workspace_size bytes, sized by batch, heads,
 * group and head_dim only) must be zero-filled before its first use and then left
 * to the library: it carries per-row counts and epochs from call to call and may
 * serve calls of any prompt length and eps with that (batch, n_kv_heads, group,
 * head_dim).  Calls sharing a workspace must not overlap.  Returns
 * IA_ERR_UNSUPPORTED when ia_condition_decode_fused_items is 0 for the call.
 * Replaces _condition_block_decode_output_fused_triton (CBT/core.py:1035-1155).
 */
IA_API size_t ia_condition_decode_fused_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group,
                                                       int32_t head_dim);
/* Items per (sequence, kv head) of ia_condition_decode_fused on the current device
 * for this call shape (kv_dtype IA_BF16 or IA_F32 matching q; suffix_cap as in
 * ia_suffix_kv), or 0 when the call does not fit one launch: GQA groups above 4,
 * head_dim other than 64 or 128, or more rows than the device holds items of at
 * most 512 blocks at once.  No reference counterpart (a capability query). */
IA_API int32_t ia_condition_decode_fused_items(const ia_decode_shape* shape, const ia_block_summaries* sm,
                                               int32_t kv_dtype, int32_t suffix_cap);
IA_API int ia_condition_decode_fused(const ia_decode_shape* shape, const void* q,
                                     const ia_block_summaries* sm, const ia_paged_kv* prompt,
                                     const ia_suffix_kv* suffix, float eps, int32_t term1_mass_exp,
                                     uint8_t* selected, float scale, void* out, int32_t out_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * ia_fixed_mask_decode in one launch: the one-launch call of
 * ia_condition_decode_fused with the caller's mask as the selection (no statistics,
 * no hand-off between the items); each item's representatives are weighted against
 * their own largest logit.  The output agrees with ia_fixed_mask_decode's to float
 * rounding.  Workspace and fit as for ia_condition_decode_fused (k_max and k_min are
 * not read).  Replaces fixed_mask_hybrid_attention
 * (CBG/real_attention_benchmark/fixed_mask.py:250-348).
 */
IA_API int ia_fixed_mask_decode_fused(const ia_decode_shape* shape, const void* q,
                                      const ia_block_summaries* sm, const uint8_t* mask,
                                      const ia_paged_kv* prompt, const ia_suffix_kv* suffix, float scale,
                                      void* out, int32_t out_dtype, void* workspace,
                                      size_t workspace_bytes, void* stream);

/*
 * Hybrid decode with an external per-(batch, kv head) block mask [batch, Hkv, nb]
 * uint8: representatives recomputed as q.k_bar/sqrt(D) + log(count), q and k_bar
 * rounded to bfloat16 for bfloat16 caches.
 * Replaces fixed_mask_hybrid_attention (CBG/real_attention_benchmark/fixed_mask.py:
 * 250-348).  Workspace as for ia_condition_decode.
 */
IA_API int ia_fixed_mask_decode(const ia_decode_shape* shape, const void* q,
                                const ia_block_summaries* sm, const uint8_t* mask,
                                const ia_paged_kv* prompt, const ia_suffix_kv* suffix, float scale,
                                void* out, int32_t out_dtype, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * One top-k decode-attention layer call in one launch.  One flat grid of about one
 * workgroup per CU; each (sequence, kv head) row is split into items in proportion
 * to the blocks its rule selects.  Item i of a row scores its share of the row's
 * blocks (as ia_select_topk computes them, bit for bit), the row's items exchange
 * their score ranges, every item applies ia_select_topk's rule (forced blocks, k or
 * k_per_seq, ties to the lower index) to the whole row and streams its share of
 * the chosen blocks, and the last item of the row to finish merges the items'
 * split-K partials into the output.  The items of a row hand each other their
 * scores through the workspace as tagged entries, waiting for a partner's at most
 * the wait limit (ia_set_wait_limit); scores still missing then are computed by
 * the waiting item itself, so the result never depends on timing.  (When every row
 * has the same work and a row has at most two items, each item scores the whole
 * row itself instead, with the same arithmetic.  Launches with k_per_seq, the
 * variable-length batches, load the keys as whole rows and pass them through LDS to
 * the matrix-core operand layout, which streams faster where items differ in length;
 * the words reaching the products are the same.)  Equal to
 * ia_select_topk + ia_sparse_paged_decode, bit for bit.  idx/n_sel (optional,
 * together) receive the selection.  Requires nb_max <= 4096 and k_cap <= 512
 * (IA_ERR_UNSUPPORTED otherwise: use the two calls).  The workspace
 * (ia_sparse_topk_decode_workspace_size bytes) must be zero-filled before its first
 * use and then left to the library, and used with one set of (batch, n_kv_heads,
 * group, head_dim, nb_max, k_cap, block_size) (zero-fill it again for another): it
 * carries a per-row call count and finished-item count from call to call.  Its size
 * follows the device's resident workgroups (one split-K slot per workgroup): size
 * it with the device current on which the call runs.  Calls that share
 * a workspace must not overlap.  Replaces the selection +
 * finalize pair of one decode step, _select_prompt_blocks_triton +
 * _condition_block_decode_output_fused_triton (CBT/core.py:701-744, :1035-1155),
 * for the BASELINE's top-k rule.
 */
IA_API size_t ia_sparse_topk_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t group,
                                                   int32_t head_dim, int32_t nb_max, int32_t k_cap,
                                                   int32_t block_size);
IA_API int ia_sparse_topk_decode(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                                 const int32_t* seq_lens, const ia_block_keys* keys, int32_t block_size,
                                 int32_t nb_max, int32_t k, const int32_t* k_per_seq, int32_t forced_first,
                                 int32_t forced_last, int32_t forced_in_k, int32_t k_cap, float scale, void* out,
                                 int32_t out_dtype, int32_t* idx, int32_t* n_sel, void* workspace,
                                 size_t workspace_bytes, void* stream);

/*
 * ia_sparse_topk_decode on a scratch buffer the library holds (no workspace
 * argument): no counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * allocation): the call allocates nothing (no hipMalloc, hipFree or allocating
 * library routine).  The buffer is a static device array of
 * IA_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call of more
 * than 2048 (sequence, kv head) rows, or whose workspace (its rows' part at the
 * buffer's start counted as 2048 rows) would exceed the buffer, fails with
 * IA_ERR_WORKSPACE.
 * Every call on a GPU shares that GPU's buffer, which keeps state from call to
 * call (per-row counts and epochs; every published word carries its row's tag),
 * so calls of different shapes may follow each other in any order, also as graph
 * replays between eager calls.  The first call on a device runs a clear kernel of
 * the whole buffer on `stream` first (inside a graph being captured it becomes a
 * node of the graph, so every replay clears, and the next call outside the graph
 * clears again).  Calls that overlap on one GPU race.  Results equal
 * ia_sparse_topk_decode's, bit for bit.
 */
#define IA_NOALLOC_SCRATCH_BYTES (16u << 20)
IA_API int ia_sparse_topk_decode_noalloc(const ia_decode_shape* shape, const void* q, const ia_paged_kv* kv,
                                         const int32_t* seq_lens, const ia_block_keys* keys, int32_t block_size,
                                         int32_t nb_max, int32_t k, const int32_t* k_per_seq,
                                         int32_t forced_first, int32_t forced_last, int32_t forced_in_k,
                                         int32_t k_cap, float scale, void* out, int32_t out_dtype, int32_t* idx,
                                         int32_t* n_sel, void* stream);

/*
 * Bound of every wait of one workgroup on another inside the one-launch calls
 * (ia_sparse_topk_decode and its no-alloc form, ia_condition_decode_fused,
 * ia_fixed_mask_decode_fused), in ticks of the GPU's 100 MHz constant clock
 * (default 20,000 = 200 us, ~15x the longest prologue; a negative value restores
 * it).  Returns the previous bound.  Applies to calls issued after it on any
 * thread.  A wait that reaches the bound makes the waiting item compute the missing
 * block scores or statistics itself: the same results, later (a bound of 0 makes
 * every such item do so; the tests use it to exercise that path).  So when the
 * launch's workgroups are not all resident together (other work sharing the GPU),
 * a call costs at most about this bound more.  The merging item's reads of partials
 * whose items have finished (their stores already issued) wait at least 20 ms
 * whatever this bound.  No reference counterpart.
 */
IA_API int64_t ia_set_wait_limit(int64_t ticks);

/*
 * Diagnostic: the number of waits of the one-launch calls that reached their bound
 * on the current device since the process started or the last reset (reset != 0
 * zeroes the count after reading it).  Each was a hand-off computed by the waiting
 * item itself (same results), or a merge read that still missed after 20 ms (the
 * row's output is then NaN).  Reads device memory synchronously: not for a hot loop
 * or graph capture.  No reference counterpart.
 */
IA_API int64_t ia_wait_fallbacks(int32_t reset);

/* Most split-K items per (b, h) the two decode entry points use for the given
 * workload (the stride of the partials); size the decode workspace with it.
 * Tokens of ia_paged_decode past max_seq_len (rounded up to a 128-token tile) are
 * not read, whatever seq_lens holds. */
IA_API int32_t ia_sparse_max_items(int32_t batch, int32_t n_kv_heads, int32_t k_cap);
IA_API int32_t ia_dense_max_items(int32_t batch, int32_t n_kv_heads, int32_t max_seq_len);

#ifdef __cplusplus
}
#endif

#endif /* INTERATTN_AMD_H */
