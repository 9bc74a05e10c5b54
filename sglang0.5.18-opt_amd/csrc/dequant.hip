// Paged K-cache gather / dequant kernels (HBM-bound, 128-bit loads and stores).
//
//   dequant_k_kernel   indexer 132-B layout -> bf16 [n, 128]
//   gather_k_kernel    indexer 132-B layout -> contiguous fp8 [n, 128] + fp32 scale [n]
//   dequant_mla_kernel MLA 656-B slot -> bf16 [n, 576]
//
// Numerics (prefill/patches/dequant_k_cache.py.diff:30-36): f32(fp8) is exact, one fp32
// multiply by the token's (group's) scale, one round-to-nearest-even to bf16 (NaN -> 0x7FC0).
// fp8 -> f32 uses the gfx950 OCP e4m3 conversion instruction (two values per instruction);
// the bf16 rounding is done with integer ops so NaNs come out canonical as in c10.
#include "dsa_common.h"

namespace dsa {
namespace {

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

// 16 fp8 bytes * s -> 16 bf16 (8 words).
__device__ __forceinline__ void dequant16(const u32x4 q, float s, u32x4& lo, u32x4& hi) {
  uint32_t out[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int v = static_cast<int>(q[w]);
    const auto f01 = __builtin_amdgcn_cvt_pk_f32_fp8(v, false);
    const auto f23 = __builtin_amdgcn_cvt_pk_f32_fp8(v, true);
    out[2 * w] = bf16_rne_bits(f01[0] * s) | (bf16_rne_bits(f01[1] * s) << 16);
    out[2 * w + 1] = bf16_rne_bits(f23[0] * s) | (bf16_rne_bits(f23[1] * s) << 16);
  }
  lo = u32x4{out[0], out[1], out[2], out[3]};
  hi = u32x4{out[4], out[5], out[6], out[7]};
}

constexpr int kDqThreads = 256;
constexpr int kChunksPerTok = kHeadDim / 16;  // 8 x 16 B per token

// Thread t of the grid handles 16-byte chunk (t % 8) of token (t / 8).
__global__ __launch_bounds__(kDqThreads) void dequant_k_kernel(
    const uint8_t* __restrict__ kv, int64_t page_stride, const int32_t* __restrict__ slots,
    int64_t n, uint16_t* __restrict__ out, int64_t out_stride) {
  const int64_t total = n * kChunksPerTok;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; g < total;
       g += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t tok = g >> 3;
    const int c = static_cast<int>(g & 7);
    const int32_t slot = slots[tok];
    u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
    if (slot >= 0) {
      const uint8_t* page = kv + static_cast<int64_t>(slot >> 6) * page_stride;
      const int off = slot & (kPage - 1);
      const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(page + off * kHeadDim + c * 16));
      const float s = *reinterpret_cast<const float*>(page + kPageFp8Bytes + off * 4);
      dequant16(q, s, lo, hi);
    }
    u32x4* o = reinterpret_cast<u32x4*>(out + tok * out_stride + c * 16);
    o[0] = lo;
    o[1] = hi;
  }
}

__global__ __launch_bounds__(kDqThreads) void gather_k_kernel(
    const uint8_t* __restrict__ kv, int64_t page_stride, const int32_t* __restrict__ slots,
    int64_t n, uint8_t* __restrict__ k8, float* __restrict__ scale) {
  const int64_t total = n * kChunksPerTok;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; g < total;
       g += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t tok = g >> 3;
    const int c = static_cast<int>(g & 7);
    const int32_t slot = slots[tok];
    u32x4 q = {0u, 0u, 0u, 0u};
    float s = 0.0f;
    if (slot >= 0) {
      const uint8_t* page = kv + static_cast<int64_t>(slot >> 6) * page_stride;
      const int off = slot & (kPage - 1);
      q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(page + off * kHeadDim + c * 16));
      s = *reinterpret_cast<const float*>(page + kPageFp8Bytes + off * 4);
    }
    *reinterpret_cast<u32x4*>(k8 + tok * kHeadDim + c * 16) = q;
    if (c == 0) scale[tok] = s;
  }
}

// MLA slot: [512 fp8 | 4 x f32 | 64 x bf16] = 656 B.  40 work items per token: 32 dequant
// chunks of 16 fp8 (group = chunk / 8) and 8 rope chunks of 16 B.
constexpr int kMlaNope = 512;
constexpr int kMlaScaleOff = 512;
constexpr int kMlaRopeOff = 528;
constexpr int kMlaItems = 40;
constexpr int kMlaUnroll = 4;  // work items per thread per pass, their loads issued together

// I: the index type (uint32_t when n * 40 fits, else int64_t).  Each pass takes kMlaUnroll items
// a grid apart: their slot indices, then their slot bytes, are loaded before any is used, so a
// thread keeps kMlaUnroll 16-B loads in flight (one dependent slot -> bytes chain per pass).
template <typename I>
__global__ __launch_bounds__(kDqThreads) void dequant_mla_kernel(
    const uint8_t* __restrict__ cache, int64_t stride, const int32_t* __restrict__ slots,
    int64_t n, uint16_t* __restrict__ out, int64_t out_stride) {
  constexpr int U = kMlaUnroll;
  const I total = static_cast<I>(n * kMlaItems);
  const I step = static_cast<I>(gridDim.x) * kDqThreads;
  for (I g0 = static_cast<I>(blockIdx.x) * kDqThreads + threadIdx.x; g0 < total; g0 += step * U) {
    I tok[U];
    int c[U];
    int32_t slot[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const I g = g0 + u * step;
      const bool in = g < total;
      tok[u] = in ? g / kMlaItems : 0;
      c[u] = static_cast<int>(g - tok[u] * kMlaItems);
      slot[u] = in ? slots[tok[u]] : -1;
    }
    u32x4 v[U];
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = u32x4{0u, 0u, 0u, 0u};
      s[u] = 0.0f;
      if (slot[u] >= 0) {
        const uint8_t* src = cache + static_cast<int64_t>(slot[u]) * stride;
        const bool nope = c[u] < 32;
        v[u] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(src + (nope ? c[u] * 16 : kMlaRopeOff + (c[u] - 32) * 16)));
        if (nope) s[u] = *reinterpret_cast<const float*>(src + kMlaScaleOff + (c[u] >> 3) * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (g0 + u * step >= total) break;
      uint16_t* dst = out + static_cast<int64_t>(tok[u]) * out_stride;
      if (c[u] < 32) {
        u32x4 lo, hi;
        dequant16(v[u], s[u], lo, hi);
        u32x4* o = reinterpret_cast<u32x4*>(dst + c[u] * 16);
        o[0] = lo;
        o[1] = hi;
      } else {
        *reinterpret_cast<u32x4*>(dst + kMlaNope + (c[u] - 32) * 8) = v[u];
      }
    }
  }
}

int grid_for(int64_t work_items, int64_t cap = 8192) {
  // Enough CTAs to cover the 256 CUs several times; the kernels grid-stride over the rest.
  const int64_t want = (work_items + kDqThreads - 1) / kDqThreads;
  return static_cast<int>(want < cap ? (want > 0 ? want : 1) : cap);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_dequant_k_paged(const uint8_t* kv_cache, int64_t page_stride_bytes,
                                   const int32_t* slots, int64_t n_tokens, uint16_t* out,
                                   int64_t out_stride, hipStream_t stream) {
  DSA_REQUIRE(n_tokens >= 0, "dsa_dequant_k_paged: n_tokens must be >= 0");
  if (n_tokens == 0) return ok();
  DSA_REQUIRE(kv_cache && slots && out, "dsa_dequant_k_paged: null pointer");
  DSA_REQUIRE(page_stride_bytes >= kPageBytes && page_stride_bytes % 16 == 0 && aligned16(kv_cache),
              "dsa_dequant_k_paged: pages must be >= 8448 B, 16-B aligned (page_stride %% 16 == 0)");
  DSA_REQUIRE(out_stride >= kHeadDim && out_stride % 8 == 0 && aligned16(out),
              "dsa_dequant_k_paged: out must be 16-B aligned with out_stride %% 8 == 0 and >= 128");
  hipLaunchKernelGGL(dequant_k_kernel, dim3(grid_for(n_tokens * kChunksPerTok)), dim3(kDqThreads), 0,
                     stream, kv_cache, page_stride_bytes, slots, n_tokens, out, out_stride);
  return check_launch("dsa_dequant_k_paged");
}

extern "C" int dsa_gather_k_paged(const uint8_t* kv_cache, int64_t page_stride_bytes,
                                  const int32_t* slots, int64_t n_tokens, uint8_t* k8, float* scale,
                                  hipStream_t stream) {
  DSA_REQUIRE(n_tokens >= 0, "dsa_gather_k_paged: n_tokens must be >= 0");
  if (n_tokens == 0) return ok();
  DSA_REQUIRE(kv_cache && slots && k8 && scale, "dsa_gather_k_paged: null pointer");
  DSA_REQUIRE(page_stride_bytes >= kPageBytes && page_stride_bytes % 16 == 0 && aligned16(kv_cache),
              "dsa_gather_k_paged: pages must be >= 8448 B, 16-B aligned (page_stride %% 16 == 0)");
  DSA_REQUIRE(aligned16(k8) && (reinterpret_cast<uintptr_t>(scale) & 3u) == 0,
              "dsa_gather_k_paged: k8 must be 16-B aligned and scale 4-B aligned");
  hipLaunchKernelGGL(gather_k_kernel, dim3(grid_for(n_tokens * kChunksPerTok)), dim3(kDqThreads), 0,
                     stream, kv_cache, page_stride_bytes, slots, n_tokens, k8, scale);
  return check_launch("dsa_gather_k_paged");
}

extern "C" int dsa_dequant_mla_paged(const uint8_t* cache, int64_t cache_stride_bytes,
                                     const int32_t* slots, int64_t n_tokens, uint16_t* out,
                                     int64_t out_stride, hipStream_t stream) {
  DSA_REQUIRE(n_tokens >= 0, "dsa_dequant_mla_paged: n_tokens must be >= 0");
  if (n_tokens == 0) return ok();
  DSA_REQUIRE(cache && slots && out, "dsa_dequant_mla_paged: null pointer");
  DSA_REQUIRE(cache_stride_bytes >= 656 && cache_stride_bytes % 16 == 0 && aligned16(cache),
              "dsa_dequant_mla_paged: slots must be >= 656 B with a 16-B aligned stride");
  DSA_REQUIRE(out_stride >= 576 && out_stride % 8 == 0 && aligned16(out),
              "dsa_dequant_mla_paged: out must be 16-B aligned with out_stride %% 8 == 0 and >= 576");
  const int64_t items = n_tokens * kMlaItems;
  // up to 32768 CTAs (a thread's passes then stay few; measured 2% faster than 8192 at 393K tokens)
  const dim3 grid(grid_for((items + kMlaUnroll - 1) / kMlaUnroll, 32768));
  if (items + static_cast<int64_t>(grid.x) * kDqThreads * kMlaUnroll <= 0xFFFFFFFFll) {
    hipLaunchKernelGGL(dequant_mla_kernel<uint32_t>, grid, dim3(kDqThreads), 0, stream, cache, cache_stride_bytes,
                       slots, n_tokens, out, out_stride);
  } else {
    hipLaunchKernelGGL(dequant_mla_kernel<int64_t>, grid, dim3(kDqThreads), 0, stream, cache, cache_stride_bytes,
                       slots, n_tokens, out, out_stride);
  }
  return check_launch("dsa_dequant_mla_paged");
}
