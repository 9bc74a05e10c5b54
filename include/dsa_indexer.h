/*
 * dsa_indexer.h -- C ABI of the MI355X (gfx950) DeepSeek-Sparse-Attention indexer path:
 * paged fp8 K-cache gather/dequant, MQA indexer logits on fp8 MFMA, and the exact top-2048
 * select with its page-table transform.
 *
 * Conventions shared by every entry point:
 *   - all pointers are device pointers unless stated; sizes and strides are in elements of the
 *     pointed-to type unless the name ends in `_bytes`;
 *   - work is enqueued on `stream` and never synchronised; launch shapes depend only on the
 *     scalar arguments, so every call can be captured into a hipGraph;
 *   - no entry point allocates device memory: workspaces are passed in by the caller, sized by
 *     the matching *_workspace_bytes query, and cleared on device by the entry point itself;
 *   - return value: DSA_OK, or an error code with a message available from dsa_last_error()
 *     (thread-local, valid until the next call on the same thread).
 *
 * K-cache layout (the indexer's 132-byte/token paged layout): page p starts at
 * kv_cache + p * page_stride_bytes and holds 64 tokens as [64 x 128 fp8 e4m3fn][64 x fp32 scale].
 * A token slot id is page * 64 + offset.
 */
#ifndef DSA_INDEXER_H_
#define DSA_INDEXER_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  DSA_OK = 0,
  DSA_ERR_INVALID = 1,   /* an argument violates the documented contract */
  DSA_ERR_WORKSPACE = 2, /* the workspace passed in is smaller than required */
  DSA_ERR_LAUNCH = 3,    /* the HIP runtime rejected a launch */
};

#define DSA_PAGE_TOKENS 64
#define DSA_HEAD_DIM 128
#define DSA_TOPK 2048

/* Message describing the last error returned on this thread ("" after success). */
const char* dsa_last_error(void);

/* Number of compute units of the current device (used by the split policy of the top-k). */
int dsa_device_cu_count(int* n_cu);

/* ---------------------------------------------------------------------------------------------
 * Paged K-cache dequant, indexer layout (132 B/token).
 *   out[i, 0:128] = bf16_rne(f32(fp8[slot_i, :]) * scale[slot_i])
 * Replaces the role of sglang's dequantize_k_cache_paged for the indexer cache; its numerics
 * follow prefill/patches/dequant_k_cache.py.diff:30-36 (fp32 product of the fp8 value and its
 * scale, rounded once to bf16).  slots: int32 [n_tokens]; out: bf16 [n_tokens, >=128] with row
 * stride out_stride (elements).  page_stride_bytes % 16 == 0 and >= 64 * 132.
 */
int dsa_dequant_k_paged(const uint8_t* kv_cache, int64_t page_stride_bytes, const int32_t* slots,
                        int64_t n_tokens, uint16_t* out, int64_t out_stride, hipStream_t stream);

/* Same as dsa_dequant_k_paged, but gathers into contiguous fp8 + fp32 scale buffers without
 * dequantising (the layout the prefill logits path can consume): k8 [n_tokens, 128] u8,
 * scale [n_tokens] f32. */
int dsa_gather_k_paged(const uint8_t* kv_cache, int64_t page_stride_bytes, const int32_t* slots,
                       int64_t n_tokens, uint8_t* k8, float* scale, hipStream_t stream);

/* MLA 656-byte slot dequant (prefill/patches/dequant_k_cache.py.diff:16-42,51-69):
 * slot = [512 fp8][4 x fp32 group scales][64 bf16 rope];
 *   out[i, 0:512]   = bf16_rne(f32(fp8[src, j]) * scale[src, j / 128])
 *   out[i, 512:576] = rope[src]
 * cache: u8 [pool, >=656] with row stride cache_stride_bytes (% 16 == 0); slots int32 [n]
 * (a negative slot, a padded entry, gives a zero row); out bf16 [n, >=576] with row stride
 * out_stride (elements, % 8 == 0). */
int dsa_dequant_mla_paged(const uint8_t* cache, int64_t cache_stride_bytes, const int32_t* slots,
                          int64_t n_tokens, uint16_t* out, int64_t out_stride, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Indexer q quantisation (the step sglang runs before the paged logits; the per-token fp8
 * convention is hcu_ops/csrc/norm_quant.cu:13-14 applied per (row, head)):
 *   sq = absmax(q[r,h,:]) / 448;  q8[r,h,:] = fp8_rne(q * (448 / absmax));  w_eff[r,h] = w[r,h] * sq
 * (absmax == 0 gives q8 = 0 and w_eff = 0).  q_bf16 [rows, heads, 128] contiguous; w [rows, heads]
 * f32; q8 [rows, heads, 128] u8; w_eff [rows, heads] f32. */
int dsa_quant_q_fp8(const uint16_t* q_bf16, const float* w, int64_t rows, int heads, uint8_t* q8,
                    float* w_eff, hipStream_t stream);

/* Indexer K-cache writer: quantises k (bf16 [n_tokens, 128]) per token with absmax/448 and
 * stores fp8 + fp32 scale at slots[i] in the 132-B paged layout; a negative slot (a padded
 * entry) stores nothing. */
int dsa_store_k_cache(const uint16_t* k_bf16, int64_t n_tokens, const int32_t* slots,
                      uint8_t* kv_cache, int64_t page_stride_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Paged MQA indexer logits for decode (replaces hcu_ops _C.mqa_logits_hist,
 * hcu_ops/csrc/mqa_hist.cu:324-405, and lightop page_mqa_logits_sparse_mask[_grouped]):
 *   logits[r, t] = scale[t] * sum_h w[r, h] * relu(sum_d q8[r, h, d] * k8[t, d])   (t < len[r])
 *   mask[r, t/16] bit t%16 = t < len[r] && bits(logits[r, t]) != 0
 * len[r] = clamp(context_lens[r], 0, width).  Rows come in groups of `group_size` consecutive
 * rows that share the block table row of the group's first row (mqa_hist.cu:93-95,162).
 * q8 [B, heads, 128] u8 (fp8 e4m3fn), w [B, heads] f32, context_lens [B] i32,
 * block_table [B, bt_pages] i32 with row stride bt_stride, width == bt_pages * 64 (mqa_hist.cu:346),
 * logits [B, width] f32 with row stride logits_stride; entries t >= len[r] are not written.
 * mask [B, width / 16] i16 with row stride mask_stride: every word is written.
 * heads in {32, 64}; B % group_size == 0; rows_per_cta divides group_size and is in {1,2,3,4,8}.
 * target_ctas: number of CTAs the K pages are spread over, each CTA streaming a slice of one
 * request (<= 0: as many as are resident at once); the grid is target_ctas + B / rows_per_cta.
 * hist_ws (nullable, int32 [B * (2 * 4096 + 2)], 16-B aligned): the pass-1 workspace of a
 * following dsa_topk_transform_pre, in its layout [12-bit histograms rows*4096 | second block
 * rows*4096 | (positives, zeros) rows*2]; of the second block the top-k uses words 0..2 of each
 * row (its per-row counters).  fuse_pass1 = 1 (needs hist_lens, int32 [B], and
 * rows_per_cta <= 3; the reference's fused kHist path, mqa_hist.cu:135-138,219-304): pass 1
 * (12-bit key histogram + positive / zero counts of every row whose min(hist_lens[r], width) >
 * 2048) is built here, inside the logits kernel, and the second block is zeroed whole.
 * fuse_pass1 = 0: only the counters are zeroed, inside the logits kernel (no extra launch); the
 * top-k then selects with its sampled threshold. */
int dsa_mqa_logits_decode(const uint8_t* q8, const float* w, int heads, int64_t batch,
                          int group_size, const uint8_t* kv_cache, int64_t page_stride_bytes,
                          const int32_t* context_lens, const int32_t* block_table,
                          int64_t bt_stride, int64_t bt_pages, float* logits,
                          int64_t logits_stride, int16_t* mask, int64_t mask_stride,
                          int rows_per_cta, int target_ctas, const int32_t* hist_lens,
                          int32_t* hist_ws, int fuse_pass1, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Prefill MQA indexer logits (the role of the prefill indexer's fp8 logits kernel, sglang
 * `_mqa_logits`, not vendored): rows attend to keys of one paged request:
 *   logits[r, t] = scale[t] * sum_h w[r, h] * relu(q8[r, h, :] . k8[t, :])   for t < len[r]
 * where key t lives at slot block_table[t / 64] * 64 + t % 64 of kv_cache.  len [rows] i32
 * (causal: prefix + i + 1), clamped to width.  Entries t >= len[r] are not written.
 * q8 [rows, heads, 128] u8; w [rows, heads] f32; block_table [>= ceil(width / 64)] i32;
 * logits [rows, width] f32 with row stride logits_stride.  Runs the decode kernel above with the
 * rows as one group, 8 rows per CTA. */
int dsa_mqa_logits_prefill(const uint8_t* q8, const float* w, int heads, int64_t rows,
                           const uint8_t* kv_cache, int64_t page_stride_bytes,
                           const int32_t* block_table, int64_t bt_pages, const int32_t* lens,
                           float* logits, int64_t logits_stride, int64_t width,
                           hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Exact top-2048 + page-table transform over (sparse-mask) indexer logits (replaces hcu_ops
 * _C.sparse_mask_topk_transform[_split][_pre], hcu_ops/csrc/sparse_mask_topk.cu:896-1051, and
 * lightop fast_topk_transform_sparse_mask_fused).
 * For row r with len = min(lengths[r], width):
 *   len <= 2048: out[r, i] = i < len ? page_table[pr, i] : -1
 *   otherwise:   out[r, :] holds page_table[pr, t] for the 2048 tokens t < len with the largest
 *                keys, ties at the threshold going to the lower t (sparse_mask_topk.cu:1-7).
 * A token whose mask bit is clear counts as +0 and its score is never used (the storage may be
 * garbage); mask == NULL means every score below len is valid.  The key of a score x is
 * (bits(x) & 0x80000000) ? ~bits(x) : bits(x) | 0x80000000 (sparse_mask_topk.cu:40-43).
 * The page-table row pr of score row r is r when cu_seqlens_q == NULL (decode layout), else the
 * request b with cu_seqlens_q[b] <= r < cu_seqlens_q[b+1] (n_req + 1 entries; varlen prefill).
 * Order within a row (the reference single kernel's, sparse_mask_topk.cu:301-345): the tokens whose
 * key is above the threshold in ascending token order, then the ties taken, ascending; a function of
 * the scores alone, the same on every run and graph replay.
 * score f32 [rows, width] row stride score_stride; mask i16 [rows, ceil(width/16)] row stride
 * mask_stride; lengths i32 [rows]; page_table i32 with pt_cols entries per row (tokens at or past
 * pt_cols map to -1) and row stride pt_stride (0: every row reads the same page-table row, e.g.
 * the query rows of one prefill request); out i32 [rows, 2048].
 * max_splits: CTAs a row may be split over (1 = one CTA per row).  Workspace: split rows need a
 * candidate list of 4096 entries each, 5120 for scores wider than 81,920 tokens (0 bytes when no
 * row is split).
 */
size_t dsa_topk_workspace_bytes(int64_t rows, int64_t width, int max_splits, int n_cu);
/* CTAs per row the top-k splits [rows, width] scores over (1: one CTA per row); the role of the
 * reference's _topk_splits (hcu_ops/hcu_ops/__init__.py:61-66) with this build's split policy. */
int dsa_topk_split_count(int64_t rows, int64_t width, int max_splits, int n_cu);
int dsa_topk_transform(const float* score, int64_t score_stride, int64_t width,
                       const int16_t* mask, int64_t mask_stride, const int32_t* lengths,
                       int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                       const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                       void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream);

/* dsa_topk_transform without the workspace argument, for callers that cannot allocate device
 * memory (code under hipGraph capture with no allocator at hand, tight serving loops, harnesses
 * that forbid allocation).  No counterpart in the reference.  The split path's workspace is a
 * built-in device array of dsa_topk_noalloc_max_bytes() (12.0 MiB: up to 256 rows split, 204 rows
 * of scores wider than 81,920 tokens) per device,
 * held until the process ends; its address is looked up on the first call on each device.
 * Inputs needing a larger workspace (dsa_topk_workspace_bytes) are rejected with
 * DSA_ERR_WORKSPACE.  Every call on one device shares that device's array: calls that overlap on
 * one device (concurrent streams or threads) race; the split counters are cleared on device at
 * the start of every call.  Same results as dsa_topk_transform. */
size_t dsa_topk_noalloc_max_bytes(void);
int dsa_topk_transform_noalloc(const float* score, int64_t score_stride, int64_t width,
                               const int16_t* mask, int64_t mask_stride, const int32_t* lengths,
                               int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                               const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                               int32_t* out, hipStream_t stream);

/* dsa_topk_transform with pass 1 (histogram and counts) already built into hist_ws by
 * dsa_mqa_logits_decode(hist_lens = lengths) (replaces
 * _C.sparse_mask_topk_transform_split_pre, sparse_mask_topk.cu:986-1051).  hist_ws is the
 * int32 [rows * (2 * 4096 + 2)] buffer given to the logits call; pass1_done says whether that
 * call built pass 1 (fuse_pass1: selection against its exact threshold bin), else the row is
 * selected with the sampled threshold (the logits call zeroed the counters).
 * Its per-row counters are consumed, so a hist_ws serves one top-k call; `workspace` as above. */
int dsa_topk_transform_pre(const float* score, int64_t score_stride, int64_t width,
                           const int16_t* mask, int64_t mask_stride, const int32_t* lengths,
                           int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                           const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                           int32_t* hist_ws, int pass1_done, void* workspace, size_t workspace_bytes,
                           int32_t* out, hipStream_t stream);

/* dsa_topk_transform / dsa_topk_transform_pre (hist_ws nullable) with the page table given as
 * the block table it expands (an optional form with no counterpart in the reference, whose
 * sparse_mask_topk.cu:348,751,804-807 gather page_table_size_1[row][t]): token t of a row maps
 * to block_table[row][t / 64] * 64 + t % 64, the entry page_table_size_1 holds when it is the
 * expansion of the 64-token-page block table, and tokens t >= bt_pages * 64 map to -1.
 * block_table [rows or n_req, bt_pages] i32 with row stride bt_stride (0: one row for all).
 * For callers that hold the block table: the transform reads 4 B per 64 tokens instead of 4 B
 * per token.  Same results as dsa_topk_transform on the expanded table. */
int dsa_topk_transform_blocks(const float* score, int64_t score_stride, int64_t width,
                              const int16_t* mask, int64_t mask_stride, const int32_t* lengths,
                              int64_t rows, const int32_t* block_table, int64_t bt_stride, int64_t bt_pages,
                              const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                              int32_t* hist_ws, int pass1_done, void* workspace, size_t workspace_bytes,
                              int32_t* out, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Prefill indexer of one request (the role of sglang's prefill indexer under
 * SGLANG_NSA_MQA_LOGITS_MEMORY_BUDGET_GB, prefill/p_opt.sh:58, at the cached-prefix call site
 * prefill/README.md:56-61; its kernels, lightop _mqa_logits + adaptive_topk, are not vendored):
 * the query rows are scored in slabs of slab_rows rows -- dsa_mqa_logits_prefill into the
 * workspace's logits slab [slab_rows, width] f32, then dsa_topk_transform of the slab's rows,
 * every row reading the request's one page-table row `page_table` (pt_cols entries, token ->
 * slot) -- so no more than one slab of logits ever exists.
 *   out[r, :] = the top-2048 (ties to the lower token) of row r's logits over keys t < lens[r],
 *               as page_table[t], -1 padded when min(lens[r], width) < 2048.
 * q8 / w / kv_cache / block_table / lens as in dsa_mqa_logits_prefill; out int32 [rows, 2048].
 * dsa_prefill_slab_rows gives the slab size a byte budget of logits allows (a multiple of 8
 * rows when at least 8 fit, capped at max_slab_rows > 0 and at rows);
 * dsa_prefill_indexer_workspace_bytes the workspace (256-B aligned) the call needs. */
int64_t dsa_prefill_slab_rows(int64_t rows, int64_t width, int64_t max_slab_rows, int64_t memory_budget_bytes);
size_t dsa_prefill_indexer_workspace_bytes(int64_t rows, int64_t width, int64_t slab_rows, int max_splits,
                                           int n_cu);
int dsa_prefill_indexer(const uint8_t* q8, const float* w, int heads, int64_t rows, const uint8_t* kv_cache,
                        int64_t page_stride_bytes, const int32_t* block_table, int64_t bt_pages,
                        const int32_t* lens, int64_t width, const int32_t* page_table, int64_t pt_cols,
                        int64_t slab_rows, int max_splits, int n_cu, void* workspace, size_t workspace_bytes,
                        int32_t* out, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Diagnostic, no counterpart in the reference: the fp8 MFMA throughput the chip reaches, the
 * measured ceiling beside the published dense fp8 peak that the prefill logits are set against.
 * ctas CTAs of 256 threads each run `iters` rounds of 8 independent
 * v_mfma_f32_16x16x128_f8f6f4 (65,536 flop each) on operands read from `operands` (>= 16,384
 * int32 words of fp8 codes, 4 per word; pass random non-NaN codes); epilogue = VALU operations
 * each MFMA result takes, of the logits epilogue's kind (ReLU + FMA per element): 0, 4, 8 or 16
 * (1 = 8, the logits epilogue's count).
 * flop per launch = ctas * 4 * iters * 8 * 65536.  sink: float [ctas * 256] (keeps the work
 * live); clocks: uint64 [2] = shader-clock ticks and 100 MHz ticks of CTA 0's loop. */
int dsa_mfma_fp8_probe(const int32_t* operands, int64_t n_words, float* sink, uint64_t* clocks, int ctas, int iters,
                       int epilogue, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_INDEXER_H_ */
