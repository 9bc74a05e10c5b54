// Paged MQA indexer logits for decode on gfx950 fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4).
//
//   logits[r, t] = scale[t] * sum_h w[r, h] * relu(q8[r, h, :] . k8[t, :])
//   mask[r, t/16] bit t%16 = t < len[r] && bits(logits[r, t]) != 0
//
// Semantics follow hcu_ops/csrc/mqa_hist.cu:96-273 (rows of a request group share the first
// row's block table, the K scale is applied after the weighted ReLU sum, mask bit = kept and
// nonzero); the work decomposition is this file's own:
//
//  * One MFMA computes a [16 heads x 16 tokens] tile with the whole 128-deep contraction.  The
//    A operand is q (heads), held in VGPRs for the life of the wave: lane l holds head
//    tile*16 + l%16, bytes (l/16)*32 .. +32.  The B operand is 16 tokens of a K page loaded
//    straight from HBM with the same byte mapping (2 x 16 B per lane, 2 KB contiguous per wave),
//    so the instruction's K ordering is the same permutation on both sides and cancels.
//  * Result lane l holds heads 4*(l/16)+i of token l%16: the epilogue is an in-lane
//    max/fma chain over H/4 values, a row-swap sum over lanes l^16 and l^32, and a lane select that leaves
//    lane l with token l of the page.  One 256 B logits store and one K-scale load per page.
//  * Balanced static grid: a row group is R rows of one request (one K page stream feeds all R
//    rows).  Every CTA reads the groups' lengths and gives group g ceil(pages_g * T / P) CTAs
//    (P = total pages, T = the target CTA count), so each CTA streams ~P / T consecutive pages of
//    a single group whatever the length mix; the grid (T + groups) depends only on shapes, so
//    the launch can be captured in a hipGraph.  The CTA's block-table slice is staged in LDS; its
//    4 waves take pages w, w+4, ... and keep the next two pages in flight while scoring one.
//  * Mask words of pages past a group's length are zeroed by CTA g (grid >= groups), so no
//    separate mask memset is launched.
//  * kHist: also the top-k pass-1 histogram (12-bit key[31:20] of the nonzero logits of rows
//    with min(hist_len, width) > 2048, plus positive / zero counts), as LDS counts flushed once
//    per CTA with one global atomic per nonzero bin; mqa_hist_init_kernel seeds the zero bin /
//    zero count with the row length (mqa_hist.cu:278-304) and every CTA subtracts its nonzero
//    tokens.
#include "dsa_common.h"

namespace dsa {
namespace {

using i32x8 = __attribute__((ext_vector_type(8))) int;
using f32x4 = __attribute__((ext_vector_type(4))) float;
using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

constexpr int kThreads = 256;
constexpr int kWavesPerCta = kThreads / kWave;
constexpr int kMaxCtaPages = 1024;  // host keeps P / T <= 1024 so the block-table slice fits LDS

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  // scale operands 0 select the unscaled v_mfma_f32_16x16x128_f8f6f4 (both operands fp8 e4m3)
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// 32 bytes at p (16-B aligned) as an MFMA operand.
__device__ __forceinline__ i32x8 load_frag(const uint8_t* p) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(p);
  const u32x4 b = *reinterpret_cast<const u32x4*>(p + 16);
  return i32x8{(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
}

struct PageRegs {
  i32x8 k[4];  // 4 sub-tiles of 16 tokens
  float scale; // scale of token lane_id() of the page
};

__device__ __forceinline__ void load_page(const uint8_t* __restrict__ kv, int64_t page_stride, int phys, int lane,
                                          PageRegs& pr) {
  const uint8_t* page = kv + static_cast<int64_t>(phys) * page_stride;
  const uint8_t* p = page + (lane & 15) * kHeadDim + (lane >> 4) * 32;
#pragma unroll
  for (int st = 0; st < 4; ++st) pr.k[st] = load_frag(p + st * 16 * kHeadDim);
  pr.scale = reinterpret_cast<const float*>(page + kPageFp8Bytes)[lane];
}

struct DecodeArgs {
  const uint8_t* q8;
  const float* w;
  const uint8_t* kv;
  int64_t page_stride;
  const int32_t* ctx;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_pages;
  int width;
  float* logits;
  int64_t logits_stride;
  int16_t* mask;
  int64_t mask_stride;
  int group;
  int R;
  int n_groups;  // batch / R
  int target;    // T: CTAs the pages are spread over
  const int32_t* hist_lens;
  int32_t* hist_ws;
  int64_t batch;
};

__device__ __forceinline__ int clamp_len(int l, int width) { return l < 0 ? 0 : (l > width ? width : l); }

// Pages of row group g: ceil(max over its R rows of len / 64).
__device__ __forceinline__ int group_pages(const DecodeArgs& a, int g) {
  int m = 0;
  for (int r = 0; r < a.R; ++r) m = max(m, clamp_len(a.ctx[g * a.R + r], a.width));
  return (m + kPage - 1) / kPage;
}

__device__ __forceinline__ int group_ctas(int pages, int total_pages, int target) {
  if (pages == 0) return 0;
  return static_cast<int>((static_cast<int64_t>(pages) * target + total_pages - 1) / total_pages);
}

// Block-wide (256 threads) sum and exclusive prefix.
__device__ __forceinline__ int block_excl(int x, int& total, int* s_w) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int inc = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) s_w[w] = inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int v = 0; v < kWavesPerCta; ++v) {
    before += v < w ? s_w[v] : 0;
    tot += s_w[v];
  }
  __syncthreads();
  total = tot;
  return before + inc - x;
}

template <int H, int R, bool kHist>
__global__ __launch_bounds__(kThreads) void mqa_logits_decode_kernel(const DecodeArgs a) {
  constexpr int HT = H / 16;  // head tiles
  extern __shared__ int s_hist[];  // kHist: [R][kBins]
  __shared__ int s_cnt[2 * R];
  __shared__ int s_w[kWavesPerCta];
  __shared__ int s_assign[3];  // group, index within the group's CTAs, the group's CTA count
  __shared__ int s_bt[kMaxCtaPages];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cta = blockIdx.x;

  // ---- work assignment (identical in every CTA) ----
  const int per_t = (a.n_groups + kThreads - 1) / kThreads;
  const int g_lo = min(tid * per_t, a.n_groups);
  const int g_hi = min(g_lo + per_t, a.n_groups);
  int my_pages = 0;
  for (int g = g_lo; g < g_hi; ++g) my_pages += group_pages(a, g);
  int total_pages;
  block_excl(my_pages, total_pages, s_w);
  if (tid == 0) s_assign[0] = -1;
  int my_ctas = 0;
  for (int g = g_lo; g < g_hi; ++g) my_ctas += group_ctas(group_pages(a, g), total_pages, a.target);
  int total_ctas;
  int c0 = block_excl(my_ctas, total_ctas, s_w);
  if (cta >= c0 && cta < c0 + my_ctas) {
    for (int g = g_lo; g < g_hi; ++g) {
      const int n = group_ctas(group_pages(a, g), total_pages, a.target);
      if (cta < c0 + n) {
        s_assign[0] = g;
        s_assign[1] = cta - c0;
        s_assign[2] = n;
        break;
      }
      c0 += n;
    }
  }

  // ---- mask words past group `cta`'s pages (grid >= groups, so every group has an owner) ----
  if (cta < a.n_groups) {
    const int p0 = group_pages(a, cta);
    const int words = (a.bt_pages - p0) * 4;
    for (int r = 0; r < R; ++r) {
      int16_t* m = a.mask + static_cast<int64_t>(cta * R + r) * a.mask_stride + p0 * 4;
      for (int i = tid; i < words; i += kThreads) m[i] = 0;
    }
  }
  __syncthreads();
  const int grp = s_assign[0];
  if (grp < 0) return;  // uniform: no pages for this CTA
  const int j = s_assign[1];
  const int nj = s_assign[2];

  const int row0 = grp * R;
  const int group_row = (row0 / a.group) * a.group;
  int len[R];
  int hlim[R];
  int max_len = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    len[r] = clamp_len(a.ctx[row0 + r], a.width);
    max_len = max(max_len, len[r]);
    hlim[r] = 0;
    if constexpr (kHist) {
      int h = a.hist_lens[row0 + r];
      h = h < a.width ? h : a.width;
      hlim[r] = h > kTopK ? h : 0;
    }
  }
  const int pages = (max_len + kPage - 1) / kPage;
  const int p_begin = static_cast<int>(static_cast<int64_t>(pages) * j / nj);
  const int p_end = static_cast<int>(static_cast<int64_t>(pages) * (j + 1) / nj);
  const int n_local = p_end - p_begin;  // <= kMaxCtaPages by the host's choice of target

  const int32_t* btr = a.bt + static_cast<int64_t>(group_row) * a.bt_stride + p_begin;
  for (int i = tid; i < n_local; i += kThreads) s_bt[i] = btr[i];
  if constexpr (kHist) {
    for (int i = tid; i < R * kBins; i += kThreads) s_hist[i] = 0;
    if (tid < 2 * R) s_cnt[tid] = 0;
  }
  __syncthreads();

  // q / w fragments (see header comment for the lane mapping).
  i32x8 qf[R][HT];
  float wf[R][HT * 4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t* qr = a.q8 + static_cast<int64_t>(row0 + r) * H * kHeadDim + (lane & 15) * kHeadDim + (lane >> 4) * 32;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) qf[r][ht] = load_frag(qr + ht * 16 * kHeadDim);
    const float* wr = a.w + static_cast<int64_t>(row0 + r) * H + 4 * (lane >> 4);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
      for (int i = 0; i < 4; ++i) wf[r][ht * 4 + i] = wr[ht * 16 + i];
    }
  }

  int nz[R], pos[R];
#pragma unroll
  for (int r = 0; r < R; ++r) nz[r] = pos[r] = 0;

  // Scores one page held in registers: MFMA tiles, weighted ReLU head sum, mask / logits stores
  // and the fused pass-1 histogram.
  auto score_page = [&](int i, const PageRegs& cur) {
    float val[R];
#pragma unroll
    for (int r = 0; r < R; ++r) val[r] = 0.0f;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        f32x4 acc[HT];
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma_fp8(qf[r][ht], cur.k[st], f32x4{0.f, 0.f, 0.f, 0.f});
        float s = 0.0f;
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
          for (int e = 0; e < 4; ++e) s += relu_bits(acc[ht][e]) * wf[r][ht * 4 + e];
        }
        s = sum_lanes_16_32(s);
        val[r] = (lane >> 4) == st ? s : val[r];
      }
    }
    const int p = p_begin + i;
    const int token = p * kPage + lane;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = val[r] * cur.scale;
      const bool live = token < len[r];
      const bool keep = live && __float_as_uint(v) != 0u;
      const uint64_t bits = __ballot(keep);
      const int64_t row = row0 + r;
      if (lane < 4) a.mask[row * a.mask_stride + p * 4 + lane] = static_cast<int16_t>((bits >> (16 * lane)) & 0xFFFFu);
      if (live) a.logits[row * a.logits_stride + token] = v;
      if constexpr (kHist) {
        if (keep && token < hlim[r]) {
          const uint32_t key = float_key(v);
          atomicAdd(&s_hist[r * kBins + static_cast<int>(key >> 20)], 1);
          ++nz[r];
          pos[r] += key > kZeroKey;
        }
      }
    }
  };

  // Pages w, w+4, ... with two pages in flight while one is scored.  The loop is unrolled over
  // three register sets so that no set is copied (a copy would wait for its loads), and the
  // prefetches are unconditional -- past the end they re-read the wave's last page, an L2 hit --
  // so the in-order load counter only ever waits for the page being scored.
  constexpr int kStepP = kWavesPerCta;
  int i = wave;
  if (i < n_local) {
    const int last = wave + (n_local - 1 - wave) / kStepP * kStepP;
    auto page_of = [&](int k) { return s_bt[k < last ? k : last]; };
    PageRegs pa, pb, pc;
    load_page(a.kv, a.page_stride, page_of(i), lane, pa);
    load_page(a.kv, a.page_stride, page_of(i + kStepP), lane, pb);
    while (true) {
      load_page(a.kv, a.page_stride, page_of(i + 2 * kStepP), lane, pc);
      score_page(i, pa);
      i += kStepP;
      if (i >= n_local) break;
      load_page(a.kv, a.page_stride, page_of(i + 2 * kStepP), lane, pa);
      score_page(i, pb);
      i += kStepP;
      if (i >= n_local) break;
      load_page(a.kv, a.page_stride, page_of(i + 2 * kStepP), lane, pb);
      score_page(i, pc);
      i += kStepP;
      if (i >= n_local) break;
    }
  }

  if constexpr (kHist) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = wave_sum(nz[r]);
      const int q = wave_sum(pos[r]);
      if (lane == 0 && n) {
        atomicAdd(&s_cnt[2 * r], n);
        atomicAdd(&s_cnt[2 * r + 1], q);
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (hlim[r] == 0) continue;
      int32_t* gh = a.hist_ws + static_cast<int64_t>(row0 + r) * kBins;
      int32_t* gcnt = a.hist_ws + 2 * a.batch * kBins + 2 * static_cast<int64_t>(row0 + r);
      for (int b = tid; b < kBins; b += kThreads) {
        const int c = s_hist[r * kBins + b];
        if (c) atomicAdd(&gh[b], c);
      }
      if (tid == 0) {
        const int n = s_cnt[2 * r];
        const int q = s_cnt[2 * r + 1];
        if (n) {
          atomicSub(&gh[kZeroBin], n);
          atomicSub(&gcnt[1], n);
        }
        if (q) atomicAdd(&gcnt[0], q);
      }
    }
  }
}

// Seeds the top-k pass-1 workspace: every token below min(hist_len, width) counts as a zero
// until the logits kernel subtracts its nonzero ones.  Rows with <= 2048 tokens stay empty.
// Of the second histogram block of the layout ([ghist1 | ghist2 | cnt], the reference's
// workspace size) only words 0..2 of each row are used -- as the split top-k's per-row counters
// -- and zeroed.
__global__ __launch_bounds__(256) void mqa_hist_init_kernel(const int32_t* __restrict__ hist_lens, int width,
                                                            int64_t batch, int32_t* __restrict__ ws) {
  const int64_t row = blockIdx.x;
  int h = hist_lens[row];
  h = h < width ? h : width;
  const int zeros = h > kTopK ? h : 0;
  int4* g1 = reinterpret_cast<int4*>(ws + row * kBins);
  for (int i = threadIdx.x; i < kBins / 4; i += 256) g1[i] = make_int4(i == kZeroBin / 4 ? zeros : 0, 0, 0, 0);
  if (threadIdx.x == 0) {
    int32_t* c = ws + 2 * batch * kBins + 2 * row;
    c[0] = 0;
    c[1] = zeros;
  }
  if (threadIdx.x < 3) ws[(batch + row) * kBins + threadIdx.x] = 0;
}

template <int H, int R, bool kHist>
void launch_one(const DecodeArgs& a, uint32_t grid, hipStream_t stream) {
  const size_t lds = kHist ? static_cast<size_t>(R) * kBins * sizeof(int) : 0;
  hipLaunchKernelGGL((mqa_logits_decode_kernel<H, R, kHist>), dim3(grid), dim3(kThreads), lds, stream, a);
}

template <int H, bool kHist>
void launch_r(const DecodeArgs& a, int R, uint32_t grid, hipStream_t stream) {
  switch (R) {
    case 1: launch_one<H, 1, kHist>(a, grid, stream); break;
    case 2: launch_one<H, 2, kHist>(a, grid, stream); break;
    case 3: launch_one<H, 3, kHist>(a, grid, stream); break;
    default:
      if constexpr (!kHist) launch_one<H, 4, false>(a, grid, stream);
      break;
  }
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_mqa_logits_decode(const uint8_t* q8, const float* w, int heads, int64_t batch, int group_size,
                                     const uint8_t* kv_cache, int64_t page_stride_bytes,
                                     const int32_t* context_lens, const int32_t* block_table, int64_t bt_stride,
                                     int64_t bt_pages, float* logits, int64_t logits_stride, int16_t* mask,
                                     int64_t mask_stride, int rows_per_cta, int target_ctas,
                                     const int32_t* hist_lens, int32_t* hist_ws, hipStream_t stream) {
  DSA_REQUIRE(heads == 32 || heads == 64, "dsa_mqa_logits_decode: heads must be 32 or 64 (got %d)", heads);
  DSA_REQUIRE(batch >= 0 && group_size >= 1, "dsa_mqa_logits_decode: batch must be >= 0 and group_size >= 1");
  DSA_REQUIRE(batch % group_size == 0, "dsa_mqa_logits_decode: batch must be a multiple of group_size");
  if (rows_per_cta <= 0) rows_per_cta = group_size % 2 == 0 ? 2 : 1;
  DSA_REQUIRE(rows_per_cta >= 1 && rows_per_cta <= 4 && group_size % rows_per_cta == 0,
              "dsa_mqa_logits_decode: rows_per_cta must be in 1..4 and divide group_size");
  DSA_REQUIRE(bt_pages > 0 && bt_pages * kPage <= 0x7FFFFFFF,
              "dsa_mqa_logits_decode: block table capacity must be positive and below 2^31 tokens");
  if (batch == 0) return ok();
  DSA_REQUIRE(q8 && w && kv_cache && context_lens && block_table && logits && mask,
              "dsa_mqa_logits_decode: null pointer");
  DSA_REQUIRE(page_stride_bytes >= kPageBytes && page_stride_bytes % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(kv_cache) & 15u) == 0,
              "dsa_mqa_logits_decode: kv_cache pages must be >= 8448 B with a 16-B aligned stride");
  DSA_REQUIRE((reinterpret_cast<uintptr_t>(q8) & 15u) == 0, "dsa_mqa_logits_decode: q8 must be 16-B aligned");
  const int64_t width = bt_pages * kPage;
  DSA_REQUIRE(bt_stride >= bt_pages && logits_stride >= width && mask_stride >= width / 16,
              "dsa_mqa_logits_decode: strides smaller than the block table capacity");
  DSA_REQUIRE((hist_lens == nullptr) == (hist_ws == nullptr),
              "dsa_mqa_logits_decode: hist_lens and hist_ws go together");
  const bool hist = hist_ws != nullptr;  // 32-bit LDS counters: no limit on tokens per CTA
  DSA_REQUIRE(!hist || rows_per_cta <= 3,
              "dsa_mqa_logits_decode: the fused histogram needs rows_per_cta <= 3 (16 KB of LDS per row)");
  const int64_t n_groups = batch / rows_per_cta;
  DSA_REQUIRE(n_groups <= 0x3FFFFFFF, "dsa_mqa_logits_decode: batch too large");
  if (target_ctas <= 0) {
    // Two CTAs fit a CU; the per-group rounding adds up to one CTA per group, so aim below the
    // resident count by the group count to finish in one round of CTAs.
    int n_cu = 0;
    const int st = dsa_device_cu_count(&n_cu);
    if (st != DSA_OK) return st;
    const int64_t slots = 2 * static_cast<int64_t>(n_cu);
    target_ctas = static_cast<int>(slots - n_groups > n_cu ? slots - n_groups : n_cu);
  }
  // Keep every CTA's page slice within the LDS block-table stage: P / T <= kMaxCtaPages.
  const int64_t max_pages = n_groups * bt_pages;
  int64_t target = target_ctas;
  if (target * kMaxCtaPages < max_pages) target = (max_pages + kMaxCtaPages - 1) / kMaxCtaPages;
  const int64_t grid = target + n_groups;
  DSA_REQUIRE(grid <= 0x7FFFFFFF, "dsa_mqa_logits_decode: grid too large");

  DecodeArgs a;
  a.q8 = q8;
  a.w = w;
  a.kv = kv_cache;
  a.page_stride = page_stride_bytes;
  a.ctx = context_lens;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.bt_pages = static_cast<int>(bt_pages);
  a.width = static_cast<int>(width);
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.mask = mask;
  a.mask_stride = mask_stride;
  a.group = group_size;
  a.R = rows_per_cta;
  a.n_groups = static_cast<int>(n_groups);
  a.target = static_cast<int>(target);
  a.hist_lens = hist_lens;
  a.hist_ws = hist_ws;
  a.batch = batch;

  if (hist) {
    hipLaunchKernelGGL(mqa_hist_init_kernel, dim3(static_cast<uint32_t>(batch)), dim3(256), 0, stream, hist_lens,
                       a.width, batch, hist_ws);
  }
  const uint32_t g = static_cast<uint32_t>(grid);
  if (heads == 64) {
    if (hist) launch_r<64, true>(a, rows_per_cta, g, stream);
    else launch_r<64, false>(a, rows_per_cta, g, stream);
  } else {
    if (hist) launch_r<32, true>(a, rows_per_cta, g, stream);
    else launch_r<32, false>(a, rows_per_cta, g, stream);
  }
  return check_launch("dsa_mqa_logits_decode");
}
