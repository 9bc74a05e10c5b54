// Per-vector fp8 quantisation for the indexer: q (per row and head) and the K-cache writer
// (per token, into the 132-B paged layout).  Convention (hcu_ops/csrc/norm_quant.cu:13-14,
// applied per 128-element vector): amax = max|x|, scale = amax / 448,
// q = fp8_rne(x * (448 / amax)), with amax == 0 giving q = 0 and scale = 0.
// 16 lanes own one 128-element vector (8 bf16 = 16 B each); a wave handles 4 vectors.
#include "dsa_common.h"

namespace dsa {
namespace {

using u32x2 = __attribute__((ext_vector_type(2))) uint32_t;

constexpr int kQThreads = 256;
constexpr int kVecPerCta = kQThreads / 16;

// quant_vec16 (dsa_common.h) with the two code words as one 8-B store.
__device__ __forceinline__ float quant_vec(const uint16_t* src, int sub, u32x2& packed, float& scale) {
  uint32_t lo, hi;
  const float amax = quant_vec16(src, sub, lo, hi, scale);
  packed = u32x2{lo, hi};
  return amax;
}

__global__ __launch_bounds__(kQThreads) void quant_q_kernel(const uint16_t* __restrict__ q, const float* __restrict__ w,
                                                            int64_t n_vec, uint8_t* __restrict__ q8,
                                                            float* __restrict__ w_eff) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kVecPerCta + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (v >= n_vec) return;  // whole 16-lane groups drop out together
  // the weight's load goes out beside q's (used only by lane 0 it was issued after q's round trip)
  const float wv = w[v];
  u32x2 packed;
  float scale;
  quant_vec(q + v * kHeadDim, sub, packed, scale);
  *reinterpret_cast<u32x2*>(q8 + v * kHeadDim + sub * 8) = packed;
  w_eff[v] = wv * scale;  // the 16 lanes store one value to one address
}

__global__ __launch_bounds__(kQThreads) void store_k_kernel(const uint16_t* __restrict__ k, int64_t n,
                                                            const int32_t* __restrict__ slots,
                                                            uint8_t* __restrict__ kv, int64_t page_stride) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kVecPerCta + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (t >= n) return;
  const int32_t slot = slots[t];
  if (slot < 0) return;  // padded entries are not stored
  u32x2 packed;
  float scale;
  quant_vec(k + t * kHeadDim, sub, packed, scale);
  uint8_t* page = kv + static_cast<int64_t>(slot >> 6) * page_stride;
  const int off = slot & (kPage - 1);
  *reinterpret_cast<u32x2*>(page + off * kHeadDim + sub * 8) = packed;
  if (sub == 0) *reinterpret_cast<float*>(page + kPageFp8Bytes + off * 4) = scale;
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_quant_q_fp8(const uint16_t* q_bf16, const float* w, int64_t rows, int heads, uint8_t* q8,
                               float* w_eff, hipStream_t stream) {
  DSA_REQUIRE(rows >= 0 && heads > 0, "dsa_quant_q_fp8: rows must be >= 0 and heads > 0");
  const int64_t n_vec = rows * heads;
  if (n_vec == 0) return ok();
  DSA_REQUIRE(q_bf16 && w && q8 && w_eff, "dsa_quant_q_fp8: null pointer");
  DSA_REQUIRE((reinterpret_cast<uintptr_t>(q_bf16) & 15u) == 0 && (reinterpret_cast<uintptr_t>(q8) & 7u) == 0,
              "dsa_quant_q_fp8: q must be 16-B aligned and q8 8-B aligned");
  const int64_t grid = (n_vec + kVecPerCta - 1) / kVecPerCta;
  DSA_REQUIRE(grid <= 0x7FFFFFFF, "dsa_quant_q_fp8: too many rows");
  hipLaunchKernelGGL(quant_q_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kQThreads), 0, stream, q_bf16, w, n_vec,
                     q8, w_eff);
  return check_launch("dsa_quant_q_fp8");
}

extern "C" int dsa_store_k_cache(const uint16_t* k_bf16, int64_t n_tokens, const int32_t* slots, uint8_t* kv_cache,
                                 int64_t page_stride_bytes, hipStream_t stream) {
  DSA_REQUIRE(n_tokens >= 0, "dsa_store_k_cache: n_tokens must be >= 0");
  if (n_tokens == 0) return ok();
  DSA_REQUIRE(k_bf16 && slots && kv_cache, "dsa_store_k_cache: null pointer");
  DSA_REQUIRE(page_stride_bytes >= kPageBytes && page_stride_bytes % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(kv_cache) & 15u) == 0 && (reinterpret_cast<uintptr_t>(k_bf16) & 15u) == 0,
              "dsa_store_k_cache: pages must be >= 8448 B and 16-B aligned; k must be 16-B aligned");
  const int64_t grid = (n_tokens + kVecPerCta - 1) / kVecPerCta;
  DSA_REQUIRE(grid <= 0x7FFFFFFF, "dsa_store_k_cache: too many tokens");
  hipLaunchKernelGGL(store_k_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kQThreads), 0, stream, k_bf16, n_tokens,
                     slots, kv_cache, page_stride_bytes);
  return check_launch("dsa_store_k_cache");
}
