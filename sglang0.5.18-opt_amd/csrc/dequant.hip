// Paged K-cache gather / dequant kernels (HBM-bound; loads and stores are 16 B a lane, and
// every store covers whole output lines).
//
//   dequant_k_kernel   indexer 132-B layout -> bf16 [n, 128] (8 lanes per token)
//   gather_k_kernel    indexer 132-B layout -> contiguous fp8 [n, 128] + fp32 scale [n]
//   dequant_mla_kernel MLA 656-B slot -> bf16 [n, 576] (a wave per token)
//
// Numerics (prefill/patches/dequant_k_cache.py.diff:30-36): f32(fp8) is exact, one fp32
// multiply by the token's (group's) scale, one round-to-nearest-even to bf16 (NaN -> 0x7FC0).
// fp8 -> f32 uses the gfx950 OCP e4m3 conversion instruction (two values per instruction);
// the bf16 rounding is done with integer ops so NaNs come out canonical as in c10.
#include "dsa_common.h"

namespace dsa {
namespace {

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;
using u32x2 = __attribute__((ext_vector_type(2))) uint32_t;

// 8 fp8 bytes * s -> 8 bf16 (4 words).
__device__ __forceinline__ u32x4 dequant8(const u32x2 q, float s) {
  const auto f01 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q[0]), false);
  const auto f23 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q[0]), true);
  const auto f45 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q[1]), false);
  const auto f67 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q[1]), true);
  return u32x4{bf16_rne_bits(f01[0] * s) | (bf16_rne_bits(f01[1] * s) << 16),
               bf16_rne_bits(f23[0] * s) | (bf16_rne_bits(f23[1] * s) << 16),
               bf16_rne_bits(f45[0] * s) | (bf16_rne_bits(f45[1] * s) << 16),
               bf16_rne_bits(f67[0] * s) | (bf16_rne_bits(f67[1] * s) << 16)};
}

template <bool kNt>
__device__ __forceinline__ void store16(uint16_t* p, const u32x4 v) {
  if constexpr (kNt) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
  else *reinterpret_cast<u32x4*>(p) = v;
}

template <bool kNt>
__device__ __forceinline__ void store4(uint16_t* p, uint32_t v) {
  if constexpr (kNt) __builtin_nontemporal_store(v, reinterpret_cast<uint32_t*>(p));
  else *reinterpret_cast<uint32_t*>(p) = v;
}

constexpr int kDqThreads = 256;
constexpr int kChunksPerTok = kHeadDim / 16;  // 8 x 16 B per token

// 8 lanes per token, 8 consecutive tokens (an octet) a wave: lane j of a token's 8 loads its
// fp8 bytes 16j .. 16j + 15 (one 16-B load; the token's 8 lanes read its 128-B row of the page,
// one cache line).  Lanes j and j ^ 4 then swap one 8-B half, so that each of the two 16-B
// stores a lane makes writes whole 128-B output lines: store 0 the first line of every row
// (bf16 0-63), store 1 the second.  Stores are nontemporal: whole-line streaming writes leave
// no dirty L2 lines for the end-of-kernel write-back, whatever the output size (73,728 tokens
// into a 19 MB output: 6.2 us with plain stores, 4.8 us nontemporal; interleaved half-line
// stores 7.4 us).  One octet a wave (more waves in flight measured faster than two octets a
// wave, 6.2 vs 7.0 us with plain stores).
constexpr int kKLanes = 8;
constexpr int kKTokPerWave = kWave / kKLanes;

__global__ __launch_bounds__(kDqThreads) void dequant_k_kernel(
    const uint8_t* __restrict__ kv, int64_t page_stride, const int32_t* __restrict__ slots,
    int64_t n, uint16_t* __restrict__ out, int64_t out_stride) {
  constexpr int kWavesPerCta = kDqThreads / kWave;
  const int lane = threadIdx.x & 63;
  const int sub = lane & (kKLanes - 1);
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * kWavesPerCta;
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWavesPerCta + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // lane j < 4 holds 8-B chunks 2j, 2j + 1 of the row (output line 0), lane 4 + i chunks
  // 8 + 2i, 9 + 2i (line 1); after the swap lane j < 4 stores chunks 2j and 8 + 2j, lane 4 + i
  // chunks 2i + 1 and 9 + 2i
  const bool lo = sub < 4;
  const int c0 = lo ? 2 * sub : 2 * (sub - 4) + 1;
  for (int64_t o = w0; o * kKTokPerWave < n; o += n_waves) {  // wave-uniform
    const int64_t tok = o * kKTokPerWave + lane / kKLanes;
    const int32_t sl = tok < n ? slots[tok] : -1;
    u32x4 q = {0u, 0u, 0u, 0u};
    float s = 0.0f;
    if (sl >= 0) {
      const uint8_t* page = kv + static_cast<int64_t>(sl >> 6) * page_stride;
      const int off = sl & (kPage - 1);
      q = *reinterpret_cast<const u32x4*>(page + off * kHeadDim + sub * 16);
      s = *reinterpret_cast<const float*>(page + kPageFp8Bytes + off * 4);
    }
    const uint32_t got0 = __shfl_xor(lo ? q[2] : q[0], 4);
    const uint32_t got1 = __shfl_xor(lo ? q[3] : q[1], 4);
    const u32x2 first = lo ? u32x2{q[0], q[1]} : u32x2{got0, got1};
    const u32x2 second = lo ? u32x2{got0, got1} : u32x2{q[2], q[3]};
    if (tok < n) {
      uint16_t* dst = out + tok * out_stride + c0 * 8;
      store16<true>(dst, dequant8(first, s));
      store16<true>(dst + 64, dequant8(second, s));
    }
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

// MLA slot: [512 fp8 | 4 x f32 | 64 x bf16] = 656 B -> bf16 [576].  One wave per token: lane i
// dequantises fp8 bytes 8i .. 8i + 7 (scale group i / 16) into output bytes 16i .. 16i + 15, and
// lanes 0-31 copy rope bytes 4i .. 4i + 3 behind them; the token's slot index is a scalar load,
// so every load and store of the wave covers one contiguous span of the slot or of the output
// row (one 1 KB store, one 128 B store).  A wave takes kMlaTok tokens a pass, n_waves apart,
// with every load of the pass issued before the first is used; the launch gives every wave one
// pass.  kNtOut: the rows are stored nontemporally (an output larger than the MALL).
constexpr int kMlaScaleOff = 512;
constexpr int kMlaRopeOff = 528;
constexpr int kMlaTok = 2;

template <bool kNtOut>
__global__ __launch_bounds__(kDqThreads) void dequant_mla_kernel(
    const uint8_t* __restrict__ cache, int64_t stride, const int32_t* __restrict__ slots,
    int64_t n, uint16_t* __restrict__ out, int64_t out_stride) {
  constexpr int U = kMlaTok;
  constexpr int kWavesPerCta = kDqThreads / kWave;
  const int lane = threadIdx.x & 63;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * kWavesPerCta;
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWavesPerCta + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int64_t t0 = w0; t0 < n; t0 += n_waves * U) {  // wave-uniform
    int32_t sl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u * n_waves;
      sl[u] = t < n ? slots[t] : -1;
    }
    u32x2 q[U];
    float s[U];
    uint32_t rp[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      q[u] = u32x2{0u, 0u};
      s[u] = 0.0f;
      rp[u] = 0u;
      if (sl[u] >= 0) {  // wave-uniform
        const uint8_t* src = cache + static_cast<int64_t>(sl[u]) * stride;
        q[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src + lane * 8));
        s[u] = *reinterpret_cast<const float*>(src + kMlaScaleOff + (lane >> 4) * 4);
        if (lane < 32) rp[u] = *reinterpret_cast<const uint32_t*>(src + kMlaRopeOff + lane * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u * n_waves;
      if (t >= n) break;
      uint16_t* dst = out + t * out_stride;
      store16<kNtOut>(dst + lane * 8, dequant8(q[u], s[u]));
      if (lane < 32) store4<kNtOut>(dst + 512 + lane * 2, rp[u]);
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
  const int64_t ctas = ((n_tokens + kKTokPerWave - 1) / kKTokPerWave + 3) / 4;  // an octet a wave
  hipLaunchKernelGGL(dequant_k_kernel, dim3(static_cast<uint32_t>(ctas < 0x7FFFFFFF ? ctas : 0x7FFFFFFF)),
                     dim3(kDqThreads), 0, stream, kv_cache, page_stride_bytes, slots, n_tokens, out, out_stride);
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
  // a wave per kMlaTok tokens, one pass each (measured on 392,832 tokens: 2 tokens a wave 123 us,
  // 4 127 us, 8 132 us; grids capped at 8192 CTAs with more passes a wave 134 us)
  const int64_t ctas = ((n_tokens + kMlaTok - 1) / kMlaTok + 3) / 4;
  const dim3 grid(static_cast<uint32_t>(ctas < 0x7FFFFFFF ? ctas : 0x7FFFFFFF));
  // nontemporal rows when the output exceeds the 256 MB MALL (392,832 tokens, 453 MB: 141 -> 123
  // us; 131,072 tokens, 151 MB: 40 us plain, 44 us nontemporal)
  if (n_tokens * out_stride * 2 > (256ll << 20)) {
    hipLaunchKernelGGL(dequant_mla_kernel<true>, grid, dim3(kDqThreads), 0, stream, cache, cache_stride_bytes, slots,
                       n_tokens, out, out_stride);
  } else {
    hipLaunchKernelGGL(dequant_mla_kernel<false>, grid, dim3(kDqThreads), 0, stream, cache, cache_stride_bytes, slots,
                       n_tokens, out, out_stride);
  }
  return check_launch("dsa_dequant_mla_paged");
}
