// Prefill indexer of one request: the paged fp8 logits of the query rows in row slabs whose
// size is bounded by a memory budget, each slab's per-row exact top-2048 + page-table transform
// right behind its logits.  Host code over the C ABI's logits and top-k entry points; the slab
// logits buffer and the top-k workspace are the caller's, so nothing is allocated and the whole
// loop can be captured in a hipGraph.
//
// Role in the reference: sglang's prefill indexer scores the query rows of a chunk against the
// cached prefix plus the chunk under SGLANG_NSA_MQA_LOGITS_MEMORY_BUDGET_GB
// (prefill/p_opt.sh:58; the cached-prefix call site is prefill/README.md:56-61), with lightop
// _mqa_logits and adaptive_topk (not vendored).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int64_t kSlabAlign = 8;  // the logits kernel scores a request's rows in CTAs of 8

int64_t slab_rows_of(int64_t rows, int64_t width, int64_t max_slab_rows, int64_t budget_bytes) {
  const int64_t row_bytes = width * static_cast<int64_t>(sizeof(float));
  int64_t s = budget_bytes > 0 ? budget_bytes / row_bytes : rows;
  if (max_slab_rows > 0 && s > max_slab_rows) s = max_slab_rows;
  if (s >= kSlabAlign) s -= s % kSlabAlign;
  if (s > rows) s = rows;
  return s < 1 ? 1 : s;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int64_t dsa_prefill_slab_rows(int64_t rows, int64_t width, int64_t max_slab_rows,
                                         int64_t memory_budget_bytes) {
  if (rows <= 0 || width <= 0) return 0;
  return slab_rows_of(rows, width, max_slab_rows, memory_budget_bytes);
}

extern "C" size_t dsa_prefill_indexer_workspace_bytes(int64_t rows, int64_t width, int64_t slab_rows, int max_splits,
                                                      int n_cu) {
  if (rows <= 0 || width <= 0 || slab_rows <= 0) return 0;
  const int64_t s = slab_rows < rows ? slab_rows : rows;
  // the top-k of a slab may split rows only when the slab is the whole (short) input
  size_t topk = dsa_topk_workspace_bytes(s, width, max_splits, n_cu);
  const int64_t tail = rows % s;
  if (tail) {
    const size_t t = dsa_topk_workspace_bytes(tail, width, max_splits, n_cu);
    topk = t > topk ? t : topk;
  }
  return align256(static_cast<size_t>(s) * static_cast<size_t>(width) * sizeof(float)) + topk;
}

extern "C" int dsa_prefill_indexer(const uint8_t* q8, const float* w, int heads, int64_t rows,
                                   const uint8_t* kv_cache, int64_t page_stride_bytes, const int32_t* block_table,
                                   int64_t bt_pages, const int32_t* lens, int64_t width, const int32_t* page_table,
                                   int64_t pt_cols, int64_t slab_rows, int max_splits, int n_cu, void* workspace,
                                   size_t workspace_bytes, int32_t* out, hipStream_t stream) {
  DSA_REQUIRE(rows >= 0 && width > 0 && width <= 0x7FFFFFFF, "dsa_prefill_indexer: rows / width out of range");
  if (rows == 0) return ok();
  DSA_REQUIRE(slab_rows >= 1, "dsa_prefill_indexer: slab_rows must be >= 1");
  DSA_REQUIRE(q8 && w && kv_cache && block_table && lens && page_table && out,
              "dsa_prefill_indexer: null pointer");
  DSA_REQUIRE(pt_cols >= 0, "dsa_prefill_indexer: pt_cols must be >= 0");
  const int64_t s = slab_rows < rows ? slab_rows : rows;
  const size_t need = dsa_prefill_indexer_workspace_bytes(rows, width, s, max_splits, n_cu);
  DSA_REQUIRE(workspace != nullptr && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
              "dsa_prefill_indexer: workspace of %zu bytes (256-B aligned) is needed, got %zu", need,
              workspace_bytes);
  float* logits = static_cast<float*>(workspace);
  char* topk_ws = static_cast<char*>(workspace) + align256(static_cast<size_t>(s) * width * sizeof(float));
  const size_t topk_bytes = workspace_bytes - (topk_ws - static_cast<char*>(workspace));
  for (int64_t r0 = 0; r0 < rows; r0 += s) {
    const int64_t n = rows - r0 < s ? rows - r0 : s;
    int st = dsa_mqa_logits_prefill(q8 + r0 * heads * kHeadDim, w + r0 * heads, heads, n, kv_cache,
                                    page_stride_bytes, block_table, bt_pages, lens + r0, logits, width, width,
                                    stream);
    if (st != DSA_OK) return st;
    // every row of the request reads the same page-table row (row stride 0)
    st = dsa_topk_transform(logits, width, width, nullptr, 0, lens + r0, n, page_table, 0, pt_cols, nullptr, n,
                            max_splits, n_cu, topk_ws, topk_bytes, out + r0 * kTopK, stream);
    if (st != DSA_OK) return st;
  }
  return ok();
}
