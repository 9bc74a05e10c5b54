// PyTorch-ROCm bind of the C ABI (include/dsa_indexer.h) as the `_C` module of the hcu_ops
// package.  The function names, argument order and contract checks mirror the reference's
// pybind exports (hcu_ops/csrc/bind.cpp:3-10,36-44,46-81) so the Python surface above can stay
// a drop-in; outputs and workspaces come from the caching allocator on the input's device and
// all work goes to the current HIP stream, so every call can be captured in a hipGraph.
#include <ATen/hip/HIPContext.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/extension.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "dsa_indexer.h"

namespace {

constexpr int64_t kPage = DSA_PAGE_TOKENS;
constexpr int64_t kHeadDim = DSA_HEAD_DIM;
constexpr int64_t kTopK = DSA_TOPK;
constexpr int64_t kBins = 4096;

// PyTorch-ROCm tensors report device type "cuda": use the guard / stream that masquerade as it.
hipStream_t cur_stream() { return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

void check_status(int st) { TORCH_CHECK(st == DSA_OK, dsa_last_error()); }

int n_cu() {
  int n = 0;
  check_status(dsa_device_cu_count(&n));
  return n;
}

void check_kv(const torch::Tensor& kv_cache) {
  TORCH_CHECK(kv_cache.is_cuda() && kv_cache.scalar_type() == at::kByte && kv_cache.dim() == 4 &&
                  kv_cache.size(1) == kPage && kv_cache.size(2) == 1 && kv_cache.size(3) == kHeadDim + 4 &&
                  kv_cache.stride(1) == kHeadDim + 4 && kv_cache.stride(3) == 1 && kv_cache.stride(0) % 16 == 0,
              "kv_cache must be packed fp8+scale uint8 [blocks, 64, 1, 132]");
}

// ------------------------------------------------------------------------------------------------
// Logits (hcu_ops/csrc/mqa_hist.cu:324-405).  persistent_ctas keeps the reference's meaning, CTAs
// per request row-set (its grid is persistent_ctas * B / rows_per_cta CTAs): > 0 spreads the K
// pages over that many CTAs in total, the balanced grid giving each row-set a share by its page
// count; <= 0 (the reference's lightop default and its -1 policy) takes every CTA that is
// resident at once.  hist_lens: also return zws, the paired split top-k's workspace.  With
// fuse_pass1 (the default, the reference's contract) pass 1 is built inside the logits kernel:
// zws = [12-bit key histograms | zeros | (positives, zeros)] of the rows longer than 2048
// (mqa_hist.cu:278-304); fuse_pass1 = false zeroes only the split top-k's per-row counters in
// zws (the paired top-k then selects with its sampled threshold: no histogram is built).
std::vector<torch::Tensor> mqa_logits_hist(const torch::Tensor& q, const torch::Tensor& kv_cache,
                                           const torch::Tensor& weights, const torch::Tensor& context_lens,
                                           const torch::Tensor& block_table, int64_t max_context_len,
                                           int64_t group_size, int64_t persistent_ctas, int64_t rows_per_cta,
                                           const c10::optional<torch::Tensor>& hist_lens, bool fuse_pass1) {
  TORCH_CHECK(q.is_cuda() && q.scalar_type() == at::kFloat8_e4m3fn && q.dim() == 4 && q.size(1) == 1 &&
                  (q.size(2) == 32 || q.size(2) == 64) && q.size(3) == kHeadDim && q.is_contiguous(),
              "q must be contiguous fp8 e4m3fn [B, 1, H, 128] with H in {32, 64}");
  const int64_t B = q.size(0);
  const int64_t H = q.size(2);
  check_kv(kv_cache);
  TORCH_CHECK(weights.scalar_type() == at::kFloat && weights.dim() == 2 && weights.size(0) == B &&
                  weights.size(1) == H && weights.is_contiguous(),
              "weights must be contiguous float32 [B, H]");
  TORCH_CHECK(context_lens.scalar_type() == at::kInt && context_lens.dim() == 1 && context_lens.size(0) == B &&
                  context_lens.is_contiguous(),
              "context_lens must be contiguous int32 [B]");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && block_table.dim() == 2 && block_table.size(0) == B &&
                  block_table.stride(1) == 1,
              "block_table must be row-contiguous int32 [B, pages]");
  TORCH_CHECK(max_context_len > 0 && max_context_len == block_table.size(1) * kPage,
              "max_context_len must equal block_table capacity");
  TORCH_CHECK(group_size >= 1 && B > 0 && B % group_size == 0, "batch must be a positive multiple of group_size");
  const bool hist = hist_lens.has_value();
  if (hist) {
    TORCH_CHECK(hist_lens->scalar_type() == at::kInt && hist_lens->dim() == 1 && hist_lens->size(0) == B &&
                    hist_lens->is_contiguous(),
                "hist_lens must be contiguous int32 [B]");
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto logits = torch::empty({B, max_context_len}, q.options().dtype(at::kFloat));
  const int64_t mask_stride = (max_context_len + 15) / 16;
  auto mask = torch::empty({B, mask_stride}, q.options().dtype(at::kShort));
  auto zws = torch::empty({hist ? B * (2 * kBins + 2) : 0}, q.options().dtype(at::kInt));
  const int64_t pages = block_table.size(1);
  const int64_t R = rows_per_cta > 0 ? rows_per_cta : (group_size % 2 == 0 ? 2 : 1);
  TORCH_CHECK(!(hist && fuse_pass1) || R <= 3,
              "the fused pass-1 histogram needs rows_per_cta <= 3 (pass fuse_pass1=False for more)");
  const int64_t per_set = std::min<int64_t>(std::max<int64_t>(persistent_ctas, 0), 1 << 16);
  const int target = static_cast<int>(std::min<int64_t>(per_set * (B / std::max<int64_t>(R, 1)), 1 << 24));
  check_status(dsa_mqa_logits_decode(
      reinterpret_cast<const uint8_t*>(q.data_ptr()), weights.data_ptr<float>(), static_cast<int>(H), B,
      static_cast<int>(group_size), kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0), context_lens.data_ptr<int>(),
      block_table.data_ptr<int>(), block_table.stride(0), pages, logits.data_ptr<float>(), logits.stride(0),
      mask.data_ptr<int16_t>(), mask_stride, static_cast<int>(R), target,
      hist ? hist_lens->data_ptr<int>() : nullptr, hist ? zws.data_ptr<int>() : nullptr, hist && fuse_pass1 ? 1 : 0,
      cur_stream()));
  return {logits, mask, zws};
}

// ------------------------------------------------------------------------------------------------
// Top-k (hcu_ops/csrc/sparse_mask_topk.cu:846-1051).
void check_topk(const torch::Tensor& score, const c10::optional<torch::Tensor>& nonzero_mask,
                const torch::Tensor& lengths, const torch::Tensor& page_table_size_1, int64_t topk) {
  TORCH_CHECK(topk == kTopK, "sparse-mask TopK requires topk=2048");
  TORCH_CHECK(score.is_cuda() && score.scalar_type() == at::kFloat && score.dim() == 2 && score.stride(1) == 1,
              "score must be row-contiguous float32 [rows, width]");
  const int64_t rows = score.size(0);
  if (nonzero_mask.has_value()) {
    TORCH_CHECK(nonzero_mask->scalar_type() == at::kShort && nonzero_mask->dim() == 2 &&
                    nonzero_mask->stride(1) == 1 && nonzero_mask->size(0) == rows &&
                    nonzero_mask->size(1) == (score.size(1) + 15) / 16,
                "nonzero_mask must be row-contiguous int16 [rows, ceil(width/16)]");
  }
  TORCH_CHECK(lengths.scalar_type() == at::kInt && lengths.dim() == 1 && lengths.is_contiguous() &&
                  lengths.size(0) == rows,
              "lengths must be contiguous int32 [rows]");
  TORCH_CHECK(page_table_size_1.scalar_type() == at::kInt && page_table_size_1.dim() == 2 &&
                  page_table_size_1.stride(1) == 1,
              "page_table_size_1 must be row-contiguous int32 [*, *]");
}

torch::Tensor topk_impl(const torch::Tensor& score, const c10::optional<torch::Tensor>& nonzero_mask,
                        const torch::Tensor& lengths, const torch::Tensor& page_table_size_1,
                        const torch::Tensor& cu_seqlens_q, int64_t topk, int64_t max_splits,
                        const torch::Tensor* zws, bool pass1_done, const torch::Tensor* out = nullptr,
                        bool blocks = false) {
  check_topk(score, nonzero_mask, lengths, page_table_size_1, topk);
  const int64_t rows = score.size(0);
  const int64_t width = score.size(1);
  // Decode layout: one page-table row per score row; otherwise cu_seqlens_q maps rows to the
  // page-table rows of their requests (varlen prefill).
  const bool decode_layout = cu_seqlens_q.size(0) == rows + 1 && page_table_size_1.size(0) == rows;
  if (!decode_layout) {
    TORCH_CHECK(cu_seqlens_q.scalar_type() == at::kInt && cu_seqlens_q.dim() == 1 && cu_seqlens_q.is_contiguous() &&
                    cu_seqlens_q.size(0) == page_table_size_1.size(0) + 1,
                "varlen layout needs int32 cu_seqlens_q [requests + 1] with one page-table row per request");
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(score.device());
  torch::Tensor dst;
  if (out != nullptr) {
    TORCH_CHECK(out->is_cuda() && out->scalar_type() == at::kInt && out->dim() == 2 && out->size(0) == rows &&
                    out->size(1) == kTopK && out->is_contiguous(),
                "out must be a contiguous int32 [rows, 2048] tensor");
    dst = *out;
  } else {
    dst = torch::empty({rows, kTopK}, score.options().dtype(at::kInt));
  }
  if (rows == 0) return dst;
  const int cus = n_cu();
  const int splits = static_cast<int>(std::max<int64_t>(1, max_splits));
  const size_t ws_bytes = dsa_topk_workspace_bytes(rows, width, splits, cus);
  auto ws = torch::empty({static_cast<int64_t>(ws_bytes)}, score.options().dtype(at::kByte));
  const int16_t* mp = nonzero_mask.has_value() ? nonzero_mask->data_ptr<int16_t>() : nullptr;
  const int64_t ms = nonzero_mask.has_value() ? nonzero_mask->stride(0) : 0;
  const int32_t* cu = decode_layout ? nullptr : cu_seqlens_q.data_ptr<int>();
  const int64_t n_req = decode_layout ? rows : page_table_size_1.size(0);
  int st;
  if (zws != nullptr) {
    TORCH_CHECK(zws->scalar_type() == at::kInt && zws->is_contiguous() && zws->numel() == rows * (2 * kBins + 2),
                "zws must be the int32 [rows * (2 * 4096 + 2)] pass-1 workspace");
  }
  if (blocks) {
    st = dsa_topk_transform_blocks(score.data_ptr<float>(), score.stride(0), width, mp, ms, lengths.data_ptr<int>(),
                                   rows, page_table_size_1.data_ptr<int>(), page_table_size_1.stride(0),
                                   page_table_size_1.size(1), cu, n_req, splits, cus,
                                   zws != nullptr ? zws->data_ptr<int>() : nullptr, pass1_done ? 1 : 0,
                                   ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, dst.data_ptr<int>(), cur_stream());
  } else if (zws != nullptr) {
    st = dsa_topk_transform_pre(score.data_ptr<float>(), score.stride(0), width, mp, ms, lengths.data_ptr<int>(),
                                rows, page_table_size_1.data_ptr<int>(), page_table_size_1.stride(0),
                                page_table_size_1.size(1), cu, n_req,
                                splits, cus, zws->data_ptr<int>(), pass1_done ? 1 : 0,
                                ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
                                dst.data_ptr<int>(), cur_stream());
  } else {
    st = dsa_topk_transform(score.data_ptr<float>(), score.stride(0), width, mp, ms, lengths.data_ptr<int>(), rows,
                            page_table_size_1.data_ptr<int>(), page_table_size_1.stride(0), page_table_size_1.size(1),
                            cu, n_req, splits, cus,
                            ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, dst.data_ptr<int>(), cur_stream());
  }
  check_status(st);
  return dst;
}

torch::Tensor sparse_mask_topk_transform(const torch::Tensor& score, const torch::Tensor& nonzero_mask,
                                         const torch::Tensor& lengths, const torch::Tensor& page_table_size_1,
                                         const torch::Tensor& cu_seqlens_q, int64_t topk) {
  return topk_impl(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk, 1, nullptr, false);
}

torch::Tensor sparse_mask_topk_transform_split(const torch::Tensor& score, const torch::Tensor& nonzero_mask,
                                               const torch::Tensor& lengths, const torch::Tensor& page_table_size_1,
                                               const torch::Tensor& cu_seqlens_q, int64_t topk, int64_t max_splits) {
  return topk_impl(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk, max_splits, nullptr, false);
}

torch::Tensor sparse_mask_topk_transform_split_pre(const torch::Tensor& score, const torch::Tensor& nonzero_mask,
                                                   const torch::Tensor& lengths,
                                                   const torch::Tensor& page_table_size_1,
                                                   const torch::Tensor& cu_seqlens_q, int64_t topk,
                                                   int64_t max_splits, const torch::Tensor& zws,
                                                   bool pass1_done) {
  return topk_impl(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk, max_splits, &zws,
                   pass1_done);
}

// The same with the block table that page_table_size_1 expands (4 B per 64-token page): token t
// maps to block_table[row][t / 64] * 64 + t % 64.  nonzero_mask None: dense scores.  zws:
// optional pass-1 workspace of a paired logits call, as in sparse_mask_topk_transform_split_pre.
torch::Tensor sparse_mask_topk_transform_blocks(const torch::Tensor& score,
                                                const c10::optional<torch::Tensor>& nonzero_mask,
                                                const torch::Tensor& lengths, const torch::Tensor& block_table,
                                                const torch::Tensor& cu_seqlens_q, int64_t topk, int64_t max_splits,
                                                const c10::optional<torch::Tensor>& zws, bool pass1_done) {
  return topk_impl(score, nonzero_mask, lengths, block_table, cu_seqlens_q, topk, max_splits,
                   zws.has_value() ? &*zws : nullptr, pass1_done, nullptr, true);
}

// Dense-score top-k (no sparse mask: every score below the row length is valid), e.g. prefill.
torch::Tensor topk_transform(const torch::Tensor& score, const torch::Tensor& lengths,
                             const torch::Tensor& page_table_size_1, const torch::Tensor& cu_seqlens_q,
                             int64_t topk, int64_t max_splits, const c10::optional<torch::Tensor>& out) {
  return topk_impl(score, c10::nullopt, lengths, page_table_size_1, cu_seqlens_q, topk, max_splits, nullptr, false,
                   out.has_value() ? &*out : nullptr);
}

// ------------------------------------------------------------------------------------------------
// Dequant / gather / quant.
torch::Tensor dequant_k_paged(const torch::Tensor& kv_cache, const torch::Tensor& slots) {
  check_kv(kv_cache);
  TORCH_CHECK(slots.scalar_type() == at::kInt && slots.dim() == 1 && slots.is_contiguous(),
              "slots must be contiguous int32 [n]");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(kv_cache.device());
  const int64_t n = slots.size(0);
  auto out = torch::empty({n, kHeadDim}, kv_cache.options().dtype(at::kBFloat16));
  check_status(dsa_dequant_k_paged(kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0), slots.data_ptr<int>(), n,
                                   reinterpret_cast<uint16_t*>(out.data_ptr()), out.stride(0), cur_stream()));
  return out;
}

std::vector<torch::Tensor> gather_k_paged(const torch::Tensor& kv_cache, const torch::Tensor& slots) {
  check_kv(kv_cache);
  TORCH_CHECK(slots.scalar_type() == at::kInt && slots.dim() == 1 && slots.is_contiguous(),
              "slots must be contiguous int32 [n]");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(kv_cache.device());
  const int64_t n = slots.size(0);
  auto k8 = torch::empty({n, kHeadDim}, kv_cache.options().dtype(at::kFloat8_e4m3fn));
  auto sc = torch::empty({n}, kv_cache.options().dtype(at::kFloat));
  check_status(dsa_gather_k_paged(kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0), slots.data_ptr<int>(), n,
                                  reinterpret_cast<uint8_t*>(k8.data_ptr()), sc.data_ptr<float>(), cur_stream()));
  return {k8, sc};
}

// sglang dequantize_k_cache_paged for the 656-B MLA slot (dequant_k_cache.py.diff:51-69).
torch::Tensor dequantize_k_cache_paged(const torch::Tensor& quant_k_cache, const torch::Tensor& page_table_1_flattened,
                                       int64_t group_size) {
  TORCH_CHECK(group_size == 128, "only group_size=128 is supported");
  TORCH_CHECK(quant_k_cache.is_cuda() && quant_k_cache.size(-1) == 656 && quant_k_cache.stride(-1) == 1,
              "quant_k_cache must be [..., 656] with a contiguous last dim");
  auto qk = quant_k_cache.view({-1, 656});
  TORCH_CHECK(qk.element_size() == 1, "quant_k_cache must be a 1-byte dtype (fp8 / uint8)");
  TORCH_CHECK(page_table_1_flattened.scalar_type() == at::kInt && page_table_1_flattened.dim() == 1 &&
                  page_table_1_flattened.is_contiguous(),
              "page_table_1_flattened must be contiguous int32 [n]");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(quant_k_cache.device());
  const int64_t n = page_table_1_flattened.size(0);
  auto out = torch::empty({n, 1, 576}, quant_k_cache.options().dtype(at::kBFloat16));
  check_status(dsa_dequant_mla_paged(reinterpret_cast<const uint8_t*>(qk.data_ptr()), qk.stride(0),
                                     page_table_1_flattened.data_ptr<int>(), n,
                                     reinterpret_cast<uint16_t*>(out.data_ptr()), 576, cur_stream()));
  return out;
}

std::vector<torch::Tensor> quant_q_fp8(const torch::Tensor& q, const torch::Tensor& weights) {
  TORCH_CHECK(q.is_cuda() && q.scalar_type() == at::kBFloat16 && q.is_contiguous() && q.size(-1) == kHeadDim,
              "q must be contiguous bf16 [..., H, 128]");
  TORCH_CHECK(q.dim() >= 2, "q must have a head dimension");
  const int64_t H = q.size(-2);
  const int64_t rows = q.numel() / (H * kHeadDim);
  TORCH_CHECK(weights.scalar_type() == at::kFloat && weights.is_contiguous() && weights.numel() == rows * H,
              "weights must be contiguous float32 with rows * H elements");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto q8 = torch::empty(q.sizes(), q.options().dtype(at::kFloat8_e4m3fn));
  auto w_eff = torch::empty(weights.sizes(), weights.options());
  check_status(dsa_quant_q_fp8(reinterpret_cast<const uint16_t*>(q.data_ptr()), weights.data_ptr<float>(), rows,
                               static_cast<int>(H), reinterpret_cast<uint8_t*>(q8.data_ptr()), w_eff.data_ptr<float>(),
                               cur_stream()));
  return {q8, w_eff};
}

void store_k_cache(const torch::Tensor& k, const torch::Tensor& slots, torch::Tensor& kv_cache) {
  check_kv(kv_cache);
  TORCH_CHECK(k.is_cuda() && k.scalar_type() == at::kBFloat16 && k.dim() == 2 && k.size(1) == kHeadDim &&
                  k.is_contiguous(),
              "k must be contiguous bf16 [n, 128]");
  TORCH_CHECK(slots.scalar_type() == at::kInt && slots.dim() == 1 && slots.size(0) == k.size(0) &&
                  slots.is_contiguous(),
              "slots must be contiguous int32 [n]");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(k.device());
  check_status(dsa_store_k_cache(reinterpret_cast<const uint16_t*>(k.data_ptr()), k.size(0), slots.data_ptr<int>(),
                                 kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0), cur_stream()));
}

// Prefill logits over one request's paged K: logits [rows, width], rows attend to keys < lens[r].
torch::Tensor mqa_logits_prefill(const torch::Tensor& q, const torch::Tensor& weights, const torch::Tensor& kv_cache,
                                 const torch::Tensor& block_table, const torch::Tensor& lens, int64_t width) {
  TORCH_CHECK(q.is_cuda() && q.scalar_type() == at::kFloat8_e4m3fn && q.dim() == 3 &&
                  (q.size(1) == 32 || q.size(1) == 64) && q.size(2) == kHeadDim && q.is_contiguous(),
              "q must be contiguous fp8 e4m3fn [rows, H, 128] with H in {32, 64}");
  const int64_t rows = q.size(0);
  const int64_t H = q.size(1);
  check_kv(kv_cache);
  TORCH_CHECK(weights.scalar_type() == at::kFloat && weights.dim() == 2 && weights.size(0) == rows &&
                  weights.size(1) == H && weights.is_contiguous(),
              "weights must be contiguous float32 [rows, H]");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && block_table.dim() == 1 && block_table.is_contiguous(),
              "block_table must be contiguous int32 [pages]");
  TORCH_CHECK(lens.scalar_type() == at::kInt && lens.dim() == 1 && lens.size(0) == rows && lens.is_contiguous(),
              "lens must be contiguous int32 [rows]");
  TORCH_CHECK(width > 0 && width <= block_table.size(0) * kPage, "width must be within the block table capacity");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto logits = torch::empty({rows, width}, q.options().dtype(at::kFloat));
  check_status(dsa_mqa_logits_prefill(reinterpret_cast<const uint8_t*>(q.data_ptr()), weights.data_ptr<float>(),
                                      static_cast<int>(H), rows, kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0),
                                      block_table.data_ptr<int>(), block_table.size(0), lens.data_ptr<int>(),
                                      logits.data_ptr<float>(), logits.stride(0), width, cur_stream()));
  return logits;
}

// Prefill indexer of one request (dsa_prefill_indexer): logits in slabs of at most
// max_slab_rows rows and memory_budget_bytes of f32 logits, each slab's top-2048 behind it.
// page_table_1: int32 [>= width] token -> slot of the request (the remap of the output).
torch::Tensor prefill_indexer(const torch::Tensor& q, const torch::Tensor& weights, const torch::Tensor& kv_cache,
                              const torch::Tensor& block_table, const torch::Tensor& lens, int64_t width,
                              const torch::Tensor& page_table_1, int64_t memory_budget_bytes, int64_t max_slab_rows,
                              int64_t max_splits, const c10::optional<torch::Tensor>& out) {
  TORCH_CHECK(q.is_cuda() && q.scalar_type() == at::kFloat8_e4m3fn && q.dim() == 3 &&
                  (q.size(1) == 32 || q.size(1) == 64) && q.size(2) == kHeadDim && q.is_contiguous(),
              "q must be contiguous fp8 e4m3fn [rows, H, 128] with H in {32, 64}");
  const int64_t rows = q.size(0);
  const int64_t H = q.size(1);
  check_kv(kv_cache);
  TORCH_CHECK(weights.scalar_type() == at::kFloat && weights.dim() == 2 && weights.size(0) == rows &&
                  weights.size(1) == H && weights.is_contiguous(),
              "weights must be contiguous float32 [rows, H]");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && block_table.dim() == 1 && block_table.is_contiguous(),
              "block_table must be contiguous int32 [pages]");
  TORCH_CHECK(lens.scalar_type() == at::kInt && lens.dim() == 1 && lens.size(0) == rows && lens.is_contiguous(),
              "lens must be contiguous int32 [rows]");
  TORCH_CHECK(page_table_1.scalar_type() == at::kInt && page_table_1.dim() == 1 && page_table_1.is_contiguous(),
              "page_table_1 must be contiguous int32 [tokens]");
  TORCH_CHECK(width > 0 && width <= block_table.size(0) * kPage, "width must be within the block table capacity");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  torch::Tensor dst;
  if (out.has_value()) {
    TORCH_CHECK(out->is_cuda() && out->scalar_type() == at::kInt && out->dim() == 2 && out->size(0) == rows &&
                    out->size(1) == kTopK && out->is_contiguous(),
                "out must be a contiguous int32 [rows, 2048] tensor");
    dst = *out;
  } else {
    dst = torch::empty({rows, kTopK}, q.options().dtype(at::kInt));
  }
  if (rows == 0) return dst;
  const int cus = n_cu();
  const int splits = static_cast<int>(std::max<int64_t>(1, max_splits));
  const int64_t slab = dsa_prefill_slab_rows(rows, width, max_slab_rows, memory_budget_bytes);
  const size_t ws_bytes = dsa_prefill_indexer_workspace_bytes(rows, width, slab, splits, cus);
  auto ws = torch::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  check_status(dsa_prefill_indexer(reinterpret_cast<const uint8_t*>(q.data_ptr()), weights.data_ptr<float>(),
                                   static_cast<int>(H), rows, kv_cache.data_ptr<uint8_t>(), kv_cache.stride(0),
                                   block_table.data_ptr<int>(), block_table.size(0), lens.data_ptr<int>(), width,
                                   page_table_1.data_ptr<int>(), page_table_1.size(0), slab, splits, cus,
                                   ws.data_ptr(), ws_bytes, dst.data_ptr<int>(), cur_stream()));
  return dst;
}

int64_t topk_splits(int64_t rows, int64_t width, int64_t max_splits, int64_t cus) {
  return dsa_topk_split_count(rows, width, static_cast<int>(std::max<int64_t>(1, max_splits)),
                              static_cast<int>(cus > 0 ? cus : n_cu()));
}

int64_t prefill_slab_rows(int64_t rows, int64_t width, int64_t memory_budget_bytes, int64_t max_slab_rows) {
  return dsa_prefill_slab_rows(rows, width, max_slab_rows, memory_budget_bytes);
}

// fp8 MFMA throughput probe (a diagnostic): one launch on the current stream; returns the sink
// float [ctas * 256] and the clocks int64 [2] (shader-clock ticks, 100 MHz ticks of CTA 0).
std::vector<torch::Tensor> mfma_fp8_probe(const torch::Tensor& operands, int64_t ctas, int64_t iters, int64_t epilogue) {
  TORCH_CHECK(operands.is_cuda() && operands.scalar_type() == at::kInt && operands.is_contiguous(),
              "operands must be a contiguous int32 CUDA tensor");
  TORCH_CHECK(ctas >= 1 && ctas <= (1 << 20) && iters >= 1 && iters <= (1 << 24), "bad ctas / iters");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(operands.device());
  auto sink = torch::empty({ctas * 256}, operands.options().dtype(at::kFloat));
  auto clocks = torch::zeros({2}, operands.options().dtype(at::kLong));
  check_status(dsa_mfma_fp8_probe(operands.data_ptr<int>(), operands.numel(), sink.data_ptr<float>(),
                                  reinterpret_cast<uint64_t*>(clocks.data_ptr<int64_t>()), static_cast<int>(ctas),
                                  static_cast<int>(iters), static_cast<int>(epilogue), cur_stream()));
  return {sink, clocks};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("mqa_logits_hist", &mqa_logits_hist,
        "paged fp8 MQA indexer logits + 16-token nonzero mask -> {logits, mask, zws}; with hist_lens zws is the "
        "paired split top-k's workspace with pass 1 built (fuse_pass1, the default) or only its counters zeroed",
        py::arg("q"), py::arg("kv_cache"), py::arg("weights"), py::arg("context_lens"), py::arg("block_table"),
        py::arg("max_context_len"), py::arg("group_size"), py::arg("persistent_ctas"), py::arg("rows_per_cta"),
        py::arg("hist_lens"), py::arg("fuse_pass1") = true);
  m.def("sparse_mask_topk_transform", &sparse_mask_topk_transform,
        "Exact top-2048 + page-table transform over sparse-mask MQA logits (one CTA per row)");
  m.def("sparse_mask_topk_transform_split", &sparse_mask_topk_transform_split,
        "Same as sparse_mask_topk_transform; few rows are split over several CTAs");
  m.def("sparse_mask_topk_transform_split_pre", &sparse_mask_topk_transform_split_pre,
        "sparse_mask_topk_transform_split on mqa_logits_hist's pass-1 workspace (pass1_done: built there)",
        py::arg("score"), py::arg("nonzero_mask"), py::arg("lengths"), py::arg("page_table_size_1"),
        py::arg("cu_seqlens_q"), py::arg("topk"), py::arg("max_splits"), py::arg("zws"),
        py::arg("pass1_done") = true);
  m.def("sparse_mask_topk_transform_blocks", &sparse_mask_topk_transform_blocks,
        "sparse_mask_topk_transform_split[_pre] with the 64-token-page block table instead of page_table_size_1",
        py::arg("score"), py::arg("nonzero_mask"), py::arg("lengths"), py::arg("block_table"),
        py::arg("cu_seqlens_q"), py::arg("topk"), py::arg("max_splits"), py::arg("zws") = py::none(),
        py::arg("pass1_done") = false);
  m.def("topk_transform", &topk_transform, "Exact top-2048 + page-table transform over dense scores (into out if given)",
        py::arg("score"), py::arg("lengths"), py::arg("page_table_size_1"), py::arg("cu_seqlens_q"), py::arg("topk"),
        py::arg("max_splits"), py::arg("out") = py::none());
  m.def("dequant_k_paged", &dequant_k_paged, "indexer 132-B paged fp8 K -> bf16 [n, 128]");
  m.def("gather_k_paged", &gather_k_paged, "indexer 132-B paged fp8 K -> contiguous (fp8 [n, 128], f32 [n])");
  m.def("dequantize_k_cache_paged", &dequantize_k_cache_paged, "MLA 656-B paged fp8 slot -> bf16 [n, 1, 576]");
  m.def("quant_q_fp8", &quant_q_fp8, "per-(row, head) fp8 quant of bf16 q -> (q8, weights * scale)");
  m.def("store_k_cache", &store_k_cache, "per-token fp8 quant of bf16 k into the 132-B paged K cache");
  m.def("mqa_logits_prefill", &mqa_logits_prefill, "prefill fp8 MQA indexer logits over one request's paged K");
  m.def("prefill_indexer", &prefill_indexer,
        "prefill indexer of one request: logits in budget-bounded row slabs, each slab's top-2048 + page-table "
        "transform behind it -> int32 [rows, 2048]",
        py::arg("q"), py::arg("weights"), py::arg("kv_cache"), py::arg("block_table"), py::arg("lens"),
        py::arg("width"), py::arg("page_table_1"), py::arg("memory_budget_bytes"), py::arg("max_slab_rows"),
        py::arg("max_splits"), py::arg("out") = py::none());
  m.def("topk_splits", &topk_splits, "CTAs per row the split top-k uses for [rows, width] scores (1: one per row)",
        py::arg("rows"), py::arg("width"), py::arg("max_splits"), py::arg("n_cu") = 0);
  m.def("prefill_slab_rows", &prefill_slab_rows, "rows per logits slab of prefill_indexer for a byte budget");
  m.def("mfma_fp8_probe", &mfma_fp8_probe,
        "fp8 MFMA throughput probe: ctas x 4 waves x iters x 8 MFMA 16x16x128, `epilogue` VALU operations per "
        "MFMA (0, 4, 8, 16; 1 = 8) -> (sink, clocks)", py::arg("operands"), py::arg("ctas"), py::arg("iters"),
        py::arg("epilogue"));
}
