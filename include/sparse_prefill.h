/*
 * C ABI of the MI355X (gfx950) sparse-prefill attention library
 * (exp3_amd/_C/libexp3_amd.so).
 *
 * The reference (Yuhang-dev/exp3) has no native FFI: its hot path is Python
 * functions over Triton kernels and PyTorch ops. Each entry point below replaces
 * one of those Python functions and cites it (paths relative to the reference
 * repository). The Python wrappers in exp3_amd/ keep the reference names,
 * argument meanings, dtypes and exceptions and call these through ctypes.
 *
 * Conventions
 *   - Device pointers only; every buffer is allocated by the caller. No entry
 *     point allocates, frees or synchronises; work is enqueued on `stream`
 *     (a hipStream_t, NULL = default stream).
 *   - Tensors in the reference's [batch, sequence, heads, dim] order are passed
 *     as a base pointer plus int64 strides in ELEMENTS (4 for [B,S,H,D], 3 for
 *     [B,S,H]); the innermost (dim) stride must be 1.
 *   - Score / mask / index tensors use [batch, query_block, key_block, head].
 *     Outputs documented as "contiguous" must be densely packed in that order.
 *   - bf16 tensors are raw 16-bit bf16 bit patterns; masks are uint8 (0 / 1).
 *   - block_size must be 128; head_dim 128 (the Qwen2.5-7B shape) or 256 (Qwen3.5
 *     full-attention layers, check_qwen35_math.py) for every entry point that
 *     takes one. q_heads must be a multiple of kv_heads.
 *   - Return 0 on success or a negative SPX_E* code; spx_last_error() then
 *     returns a thread-local message.
 */
#ifndef EXP3_AMD_SPARSE_PREFILL_H
#define EXP3_AMD_SPARSE_PREFILL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPX_OK 0
#define SPX_EINVAL (-1)       /* bad argument: shape, stride, null pointer     */
#define SPX_EUNSUPPORTED (-2) /* valid in the reference, not built here       */
#define SPX_ELAUNCH (-3)      /* HIP launch / runtime failure                 */

#define SPX_ABI_VERSION 8

/* int32 counters a work_queue argument of the attention entry points points to. */
#define SPX_WORK_QUEUE_INTS 16

/* Selector ids for spx_selector_scores (kernels.py:62). */
#define SPX_SELECTOR_MEAN_BALANCED 0
#define SPX_SELECTOR_CGF_MEAN 1
#define SPX_SELECTOR_DISPERSION_MEAN 2

const char* spx_last_error(void);
int spx_abi_version(void);

/* ------------------------------------------------------------- pooling */

/* bf16 block mean of K over the valid tokens of each 128-token block.
 * Replaces upstream/flashprefill_native_forward.py:420-442 (block_mean_k) and its
 * Triton kernel compute_mean_vector (:27-69).
 * mean_k: contiguous [B, NB, Hkv, D] bf16, NB = ceil(seq / 128). */
int spx_block_mean_k(const void* k, const int64_t* k_strides, int batch, int seq,
                     int kv_heads, int head_dim, int block_size, void* mean_k,
                     void* stream);

/* FP32 block descriptors: mean_k, mean_v, var_k (contiguous [B, NB, Hkv, D]),
 * sigma_v ([B, NB, Hkv]) and counts ([NB] int32).
 * Replaces kernels.py:22-46 (block_descriptors). */
int spx_block_descriptors(const void* k, const int64_t* k_strides, const void* v,
                          const int64_t* v_strides, int batch, int seq, int kv_heads,
                          int head_dim, int block_size, float* mean_k, float* mean_v,
                          float* var_k, float* sigma_v, int32_t* counts, void* stream);

/* One pass over K and V producing any subset of: bf16 mean K (as
 * spx_block_mean_k), the FP32 descriptors (as spx_block_descriptors) and the
 * attention tiles the attention entry points read. Null outputs are skipped;
 * key_tiles and value_tiles are produced together.
 * key_tiles:   [B, Hkv, NB, 128, D] bf16, the block's K rows;
 * value_tiles: [B, Hkv, NB, D, 128] bf16 (D = 128), V transposed per block with
 *              the key permutation documented in exp3_amd/csrc/common.h; for
 *              D = 256 the same storage holds four 32-key sub-blocks
 *              [256 dims][32 key slots] per block.
 * Rows / keys past seq are zero. In a key tile the 16-byte chunk c of row r is
 * stored at chunk position c ^ (r & 15) (c < D / 8); in a D = 128 value tile the
 * same rule holds per dim row, in a D = 256 sub-block chunk c (< 4) of dim row d
 * sits at c ^ ((d >> 2) & 3) (the attention kernels' LDS layouts).
 * Fuses kernels.py:22-46 with upstream/flashprefill_native_forward.py:420-442
 * (the descriptor stage of attention.py:80-86). */
int spx_block_pool(const void* k, const int64_t* k_strides, const void* v,
                   const int64_t* v_strides, int batch, int seq, int kv_heads,
                   int head_dim, int block_size, void* mean_k_bf16, float* mean_k,
                   float* mean_v, float* var_k, float* sigma_v, int32_t* counts,
                   void* key_tiles, void* value_tiles, void* stream);

/* ------------------------------------------------------------- routing */

/* Normalised V1 block scores, written to score (strided [B, NB, NB, Hq] fp32;
 * every entry is written, entries with key block > query block are 0).
 * Replaces upstream/flashprefill_native_forward.py:445-475 (v1_scores), i.e. the
 * Triton kernel compute_block_score (:89-175) followed by normalize_scores
 * (:410-417). mean_k is bf16 [B, NB, Hkv, D] with the given strides. */
int spx_v1_scores(const void* q, const int64_t* q_strides, const void* mean_k,
                  const int64_t* mean_k_strides, int batch, int seq, int q_heads,
                  int kv_heads, int head_dim, int block_size, float scale,
                  float* score, const int64_t* score_strides, void* stream);

/* V1 threshold + protected selection with ascending index lists.
 * keep = score >= fp32(max_j score * alpha) (or the min_budget branch), protected
 * = j < attention_sink | 0 <= t - j < window | t >= query_blocks - last_n_blocks_full,
 * active = (keep | protected) & j <= t.
 * indices: contiguous [B, QB, KB, H] int64 (active ids ascending, then KB);
 * counts: contiguous [B, QB, H] int32; mask: optional contiguous uint8 mask of the
 * active set (what kernels.py:163-176 mask_from_indices would give).
 * Replaces upstream/flashprefill_native_forward.py:357-407 (deal_output_score). */
int spx_deal_output_score(const float* score, const int64_t* score_strides, int batch,
                          int query_blocks, int key_blocks, int heads, int attention_sink,
                          int window, float alpha, int last_n_blocks_full, int min_budget,
                          int64_t* indices, int32_t* counts, uint8_t* mask, void* stream);

/* Threshold selection of the new selectors: alpha == 0 selects every causal block,
 * else routed = score > 0 & score >= fp32(alpha * max_j score), united with the
 * protected set and intersected with j <= t. mask: contiguous uint8 [B,QB,KB,H];
 * indices / counts optional (as spx_deal_output_score; kernels.py:154-160).
 * Replaces kernels.py:129-151 (protected_selection). */
int spx_protected_selection(const float* score, const int64_t* score_strides, int batch,
                            int query_blocks, int key_blocks, int heads, float alpha,
                            int sink_blocks, int window_blocks, int last_full_blocks,
                            uint8_t* mask, int64_t* indices, int32_t* counts, void* stream);

/* Fused V1 route: spx_v1_scores and spx_deal_output_score without the scores
 * passing through HBM, the selection reading the exact score values it writes
 * (two kernels on `stream`: the block products leave per-block partials in each
 * tile's own [KB, H] slab of `indices`, which the second overwrites with the
 * lists). score may be NULL (not stored); mask may be NULL. q_heads <= 256;
 * indices 8-byte aligned. Replaces attention.py:87-105 (_v1_selection's
 * selector + indices stages). */
int spx_v1_route(const void* q, const int64_t* q_strides, const void* mean_k,
                 const int64_t* mean_k_strides, int batch, int seq, int q_heads,
                 int kv_heads, int head_dim, int block_size, float scale, float alpha,
                 int attention_sink, int window, int last_n_blocks_full, float* score,
                 int64_t* indices, int32_t* counts, uint8_t* mask, void* stream);

/* kernels.py:154-160 (indices_from_mask). mask: contiguous uint8 [B,QB,KB,H]. */
int spx_indices_from_mask(const uint8_t* mask, int batch, int query_blocks, int key_blocks,
                          int heads, int64_t* indices, int32_t* counts, void* stream);

/* kernels.py:163-176 (mask_from_indices). indices contiguous int64, counts int32. */
int spx_mask_from_indices(const int64_t* indices, const int32_t* counts, int batch,
                          int query_blocks, int key_blocks, int heads, uint8_t* mask,
                          void* stream);

/* Balanced / CGF / dispersion block scores (selector = SPX_SELECTOR_*), written to
 * score (strided [B, NB, NB, Hq] fp32, every entry written).
 * mean_k, var_k: contiguous fp32 [B, NB, Hkv, D]; sigma_v [B, NB, Hkv];
 * counts [NB] int32. workspace: caller-allocated device memory of
 * spx_selector_workspace_bytes() bytes, 16-byte aligned (the bf16 hi/lo split of
 * mean_k and var_k, rewritten by every call; calls that overlap on one workspace
 * race). Replaces kernels.py:49-126 (selector_scores). */
int spx_selector_scores(const void* q, const int64_t* q_strides, const float* mean_k,
                        const float* var_k, const float* sigma_v, const int32_t* counts,
                        int batch, int seq, int q_heads, int kv_heads, int head_dim,
                        int block_size, int selector, float scale, void* workspace,
                        float* score, const int64_t* score_strides, void* stream);

/* Bytes of the spx_selector_scores workspace (B * Hkv * ceil(NB / 32) * D / 128 * 32 KB), or -1
 * for an unsupported shape. Helper of spx_selector_scores (no reference counterpart). */
int64_t spx_selector_workspace_bytes(int batch, int seq, int kv_heads, int head_dim);

/* spx_selector_scores without the workspace argument and without any allocation: the
 * split workspace is a file-scope device array of 8 MiB per GPU (held until the
 * process ends), so the shape must satisfy B * Hkv * ceil(NB / 32) * D / 128 <= 256, i.e.
 * spx_selector_workspace_bytes() <= 8 MiB (larger shapes return SPX_EUNSUPPORTED).
 * Results are identical to spx_selector_scores'. The stream must belong to the
 * current device. Calls that overlap on one GPU race on the shared array.
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops). */
int spx_selector_scores_noalloc(const void* q, const int64_t* q_strides, const float* mean_k,
                                const float* var_k, const float* sigma_v,
                                const int32_t* counts, int batch, int seq, int q_heads,
                                int kv_heads, int head_dim, int block_size, int selector,
                                float scale, float* score, const int64_t* score_strides,
                                void* stream);

/* ----------------------------------------------------------- attention */

/* Block-sparse causal flash attention over each (query tile, head)'s index list.
 * key_tiles / value_tiles come from spx_block_pool. indices: int64 [B, NB, NB, Hq] (strided),
 * counts: int32 [B, NB, Hq] (strided); indices == NULL selects every causal block
 * (dense causal attention). out: bf16 [B, S, Hq, D] (strided); lse: natural-log LSE
 * fp32 [B, S, Hq] (strided, may be NULL). List ids outside [0, NB) are skipped;
 * only the block equal to the query tile is masked (key > query). head_dim 128 or 256.
 * work_queue (optional, here and in the two fused variants below): a 4-byte aligned
 * device array of SPX_WORK_QUEUE_INTS int32, all 0 when the launch starts. With it
 * the head_dim 128 kernel runs a persistent grid (one workgroup per CU taking work
 * items from these counters: no workgroup launch gaps between items, and the fast
 * XCDs take more of the light last third of the tile pairs); at head_dim 256 the
 * last third of the tiles is taken from work_queue[0] the same way. The values it
 * is left holding are unspecified: zero it before the next use, and use one array
 * per launch in flight. NULL keeps one workgroup per item; the results are
 * identical either way.
 * Replaces upstream/flashprefill_native_forward.py:478-521 (exact_attention) and the
 * Triton kernel _flash_forward (:215-354). */
int spx_exact_attention(const void* q, const int64_t* q_strides, const void* key_tiles,
                        const void* value_tiles,
                        const int64_t* indices, const int64_t* index_strides,
                        const int32_t* counts, const int64_t* count_strides, int batch,
                        int seq, int q_heads, int kv_heads, int head_dim, int block_size,
                        float scale, void* out, const int64_t* out_strides, float* lse,
                        const int64_t* lse_strides, int32_t* work_queue,
                        void* stream);

/* Exact attention with the block-mean correction fused in: each row additionally
 * attends to the fp32 mean K / mean V (logit + ln n_j) of every full-history block
 * j < t that is not in its tile's list, inside the same online softmax, so the
 * result equals the logaddexp merge of the exact and mean paths.
 * mean_k, mean_v: contiguous fp32 [B, NB, Hkv, D]; block_counts: [NB] int32.
 * Replaces the exact + mean + merge stages of attention.py:253-305:
 * upstream exact_attention, kernels.py:179-230 (mean_tail) and kernels.py:312-325
 * (merge_exact_mean). */
int spx_sparse_attention_mean(const void* q, const int64_t* q_strides, const void* key_tiles,
                              const void* value_tiles,
                              const int64_t* indices, const int64_t* index_strides,
                              const int32_t* counts, const int64_t* count_strides,
                              const float* mean_k, const float* mean_v,
                              const int32_t* block_counts, int batch, int seq, int q_heads,
                              int kv_heads, int head_dim, int block_size, float scale,
                              void* out, const int64_t* out_strides, float* lse,
                              const int64_t* lse_strides, int32_t* work_queue,
                              void* stream);

/* Mean path alone: fp32 output and LSE of each row against the mean K / V of the
 * unselected full-history blocks of its tile (selection given as index lists,
 * e.g. from spx_indices_from_mask). out: fp32 [B, S, Hq, D] strided; lse strided.
 * Replaces kernels.py:179-230 (mean_tail). */
int spx_mean_tail(const void* q, const int64_t* q_strides, const int64_t* indices,
                  const int64_t* index_strides, const int32_t* counts,
                  const int64_t* count_strides, const float* mean_k, const float* mean_v,
                  const int32_t* block_counts, int batch, int seq, int q_heads, int kv_heads,
                  int head_dim, int block_size, float scale, float* out,
                  const int64_t* out_strides, float* lse, const int64_t* lse_strides,
                  void* stream);

/* logaddexp merge of an exact (bf16 output, fp32 LSE) and a mean (fp32 output,
 * fp32 LSE) path; writes bf16 output and fp32 total LSE (lse_out may be NULL).
 * Replaces kernels.py:312-325 (merge_exact_mean). */
int spx_merge_exact_mean(const void* exact_out, const int64_t* exact_strides,
                         const float* exact_lse, const int64_t* exact_lse_strides,
                         const float* mean_out, const int64_t* mean_strides,
                         const float* mean_lse, const int64_t* mean_lse_strides, int batch,
                         int seq, int heads, int head_dim, void* out,
                         const int64_t* out_strides, float* lse_out,
                         const int64_t* lse_out_strides, void* stream);

/* ---------------------------------------------------------- rescue tail */

/* Mean query of every query tile over its real rows: fp32 [B, NB, Hq, D]
 * (contiguous, caller-allocated). q: unit dim stride, 16-byte aligned base, batch /
 * sequence / head strides multiples of 8 elements (as for the other Q inputs).
 * Replaces the q_mean of kernels.py:274-276 (rescue_tail). */
int spx_tile_mean_query(const void* q, const int64_t* q_strides, int batch, int seq, int q_heads,
                        int head_dim, int block_size, float* qmean, void* stream);

/* Rescue token of every (query tile t, key block j < t, q head): the position p of
 * the block maximising qmean[t, h] . k[j, p] (dot products to fp32 accuracy: bf16
 * keys times the fp32 means split exactly into three bf16 parts, on MFMA; the first
 * position on ties). qmean (16-byte aligned) from spx_tile_mean_query; key_tiles from
 * spx_block_pool.
 * choice: uint8 [B, NB, NB, Hq] contiguous, 0 where j >= t.
 * Replaces kernels.py:277-283 (token_scores / argmax inside rescue_tail). */
int spx_rescue_choice(const float* qmean, const void* key_tiles, int batch, int seq, int q_heads,
                      int kv_heads, int head_dim, int block_size, uint8_t* choice, void* stream);

/* Rescue path alone: fp32 output and natural-log LSE of each row against one entry
 * per unselected full-history block of its tile (the block's rescue token: its key
 * and value, logit scale q.k) and, with remainder != 0, a second entry with the mean
 * K / V of the block's other 127 tokens (logit + ln 127). Selection as index lists;
 * mean_k / mean_v (fp32 [B, NB, Hkv, D], from spx_block_descriptors) are read only
 * with remainder. v: the layer's V [B, S, Hkv, D] bf16 (strided, 16-byte aligned
 * rows): the tokens' value rows. Replaces kernels.py:233-309 (rescue_tail). */
int spx_rescue_tail(const void* q, const int64_t* q_strides, const void* key_tiles,
                    const void* value_tiles, const int64_t* indices, const int64_t* index_strides,
                    const int32_t* counts, const int64_t* count_strides, const uint8_t* choice,
                    const void* v, const int64_t* v_strides,
                    const float* mean_k, const float* mean_v, int remainder, int batch, int seq,
                    int q_heads, int kv_heads, int head_dim, int block_size, float scale,
                    float* out, const int64_t* out_strides, float* lse,
                    const int64_t* lse_strides, void* stream);

/* Exact attention with the rescue path fused into the same online softmax (equal
 * to the logaddexp merge of the two); arguments as spx_rescue_tail. Replaces the exact + rescue + merge stages of
 * attention.py:306-331 (fp_v1_rescue / fp_v1_rescue_v2): upstream exact_attention,
 * kernels.py:233-309 (rescue_tail) and kernels.py:312-325 (merge_exact_mean). */
int spx_sparse_attention_rescue(const void* q, const int64_t* q_strides, const void* key_tiles,
                                const void* value_tiles, const int64_t* indices,
                                const int64_t* index_strides, const int32_t* counts,
                                const int64_t* count_strides, const uint8_t* choice,
                                const void* v, const int64_t* v_strides,
                                const float* mean_k, const float* mean_v, int remainder,
                                int batch, int seq, int q_heads, int kv_heads, int head_dim,
                                int block_size, float scale, void* out,
                                const int64_t* out_strides, float* lse,
                                const int64_t* lse_strides, int32_t* work_queue,
                                void* stream);

/* ----------------------------------------------------------- accounting */

/* Integer counters of kernels.py:328-407 (selection_accounting) from a contiguous
 * uint8 mask [B, NB, NB, H]: totals[0] = exact token pairs, [1] = selected block
 * entries, [2] = mean proxy entries, [3] = sum over selected entries of
 * ceil(rows / q_tile) (times ceil(128 / k_tile) gives the physical QK tiles;
 * q_tile <= 0 skips it). totals: 4 int64, overwritten. */
int spx_selection_accounting(const uint8_t* mask, int batch, int blocks, int heads, int seq,
                             int block_size, int q_tile, int64_t* totals, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXP3_AMD_SPARSE_PREFILL_H */
