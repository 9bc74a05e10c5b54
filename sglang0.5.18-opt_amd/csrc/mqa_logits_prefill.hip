// Prefill MQA indexer logits on gfx950 fp8 MFMA:
//   logits[r, t] = scale[t] * sum_h w[r, h] * relu(q8[r, h, :] . k8[t, :]),  t < len[r]
// with key t read from the paged 132-B K cache through the request's block table.
//
// This is a dense GEMM [rows*H x 128] . [128 x keys] with a ReLU-weighted head reduction in
// the epilogue.  Work decomposition:
//  * a CTA (4 waves) owns 8 consecutive query rows; each wave holds 2 rows x H heads of q as
//    MFMA A fragments in VGPRs (lane l: head tile*16 + l%16, bytes (l/16)*32 .. +32);
//  * the CTA streams the request's K pages (64 keys = 8 KB fp8 + 256 B scales) through a
//    double-buffered LDS tile; rows are padded to 144 B so the 16 lanes reading 16 different
//    keys at one byte offset fall into different banks;
//  * per page and row: 4 key sub-tiles x H/16 MFMAs (v_mfma_f32_16x16x128_f8f6f4), then the
//    epilogue of the decode kernel (max/fma over the lane's heads, one reduce-scatter of the four
//    sub-tiles over the 16-lane rows) leaves lane l with key l of the page: one 256 B store per
//    page and row;
//  * causal skipping: a wave skips a page for a row once the page starts at or past len[row];
//    the CTA stops after the last page any of its rows needs.
#include "dsa_common.h"

namespace dsa {
namespace {

using i32x8 = __attribute__((ext_vector_type(8))) int;
using f32x4 = __attribute__((ext_vector_type(4))) float;
using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 2;
constexpr int kRowsPerCta = 4 * kRowsPerWave;
constexpr int kLdsRow = kHeadDim + 16;        // padded key row in LDS
constexpr int kLdsPage = kPage * kLdsRow;     // 9216 B

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ i32x8 frag_from(const u32x4& a, const u32x4& b) {
  return i32x8{(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
}

struct PrefillArgs {
  const uint8_t* q8;
  const float* w;
  const uint8_t* kv;
  int64_t page_stride;
  const int32_t* bt;
  int bt_pages;
  const int32_t* lens;
  int rows;
  int width;
  float* logits;
  int64_t logits_stride;
};

template <int H>
__global__ __launch_bounds__(kThreads, 2) void mqa_logits_prefill_kernel(const PrefillArgs a) {
  constexpr int HT = H / 16;
  __shared__ __attribute__((aligned(16))) uint8_t s_k[2][kLdsPage];
  __shared__ float s_scale[2][kPage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row_base = blockIdx.x * kRowsPerCta;

  // Lengths of the CTA's rows (uniform reads); rows past the end have length 0.
  int cta_max = 0;
  int len[kRowsPerWave] = {};
#pragma unroll
  for (int i = 0; i < kRowsPerCta; ++i) {
    const int row = row_base + i;
    int l = row < a.rows ? a.lens[row] : 0;
    l = l < 0 ? 0 : (l > a.width ? a.width : l);
    cta_max = l > cta_max ? l : cta_max;
    if (i / kRowsPerWave == wave) len[i % kRowsPerWave] = l;
  }
  const int n_pages = (cta_max + kPage - 1) / kPage;
  if (n_pages == 0) return;

  // q / w fragments of this wave's rows.
  i32x8 qf[kRowsPerWave][HT];
  float wf[kRowsPerWave][HT * 4];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    const int row = min(row_base + wave * kRowsPerWave + r, a.rows - 1);
    const uint8_t* qr = a.q8 + static_cast<int64_t>(row) * H * kHeadDim + (lane & 15) * kHeadDim + (lane >> 4) * 32;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(qr + ht * 16 * kHeadDim);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(qr + ht * 16 * kHeadDim + 16);
      qf[r][ht] = frag_from(lo, hi);
    }
    const float* wr = a.w + static_cast<int64_t>(row) * H + 4 * (lane >> 4);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
      for (int i = 0; i < 4; ++i) wf[r][ht * 4 + i] = wr[ht * 16 + i];
    }
  }

  // Stage loader: thread t moves 32 B of key t/4 (chunk t%4) and, for t < 64, one scale.
  const int ld_tok = tid >> 2;
  const int ld_chunk = tid & 3;
  auto gload = [&](int p, u32x4& x0, u32x4& x1, float& sc) {
    const uint8_t* page = a.kv + static_cast<int64_t>(a.bt[p]) * a.page_stride;
    const uint8_t* src = page + ld_tok * kHeadDim + ld_chunk * 32;
    x0 = *reinterpret_cast<const u32x4*>(src);
    x1 = *reinterpret_cast<const u32x4*>(src + 16);
    sc = tid < kPage ? reinterpret_cast<const float*>(page + kPageFp8Bytes)[tid] : 0.0f;
  };
  auto lstore = [&](int buf, const u32x4& x0, const u32x4& x1, float sc) {
    uint8_t* dst = &s_k[buf][ld_tok * kLdsRow + ld_chunk * 32];
    *reinterpret_cast<u32x4*>(dst) = x0;
    *reinterpret_cast<u32x4*>(dst + 16) = x1;
    if (tid < kPage) s_scale[buf][tid] = sc;
  };

  {
    u32x4 x0, x1;
    float sc;
    gload(0, x0, x1, sc);
    lstore(0, x0, x1, sc);
  }
  __syncthreads();

  const int frag_off = (lane & 15) * kLdsRow + (lane >> 4) * 32;
  for (int p = 0; p < n_pages; ++p) {
    const int buf = p & 1;
    const bool more = p + 1 < n_pages;
    u32x4 x0, x1;
    float sc;
    if (more) gload(p + 1, x0, x1, sc);

    const int tok0 = p * kPage;
    bool act[kRowsPerWave];
    bool any = false;
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
      act[r] = tok0 < len[r];
      any |= act[r];
    }
    if (any) {
      float part[kRowsPerWave][4];  // this lane's heads' share of keys st * 16 + lane % 16
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) {
#pragma unroll
        for (int st = 0; st < 4; ++st) part[r][st] = 0.0f;
      }
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint8_t* src = &s_k[buf][st * 16 * kLdsRow + frag_off];
        const i32x8 kf = frag_from(*reinterpret_cast<const u32x4*>(src), *reinterpret_cast<const u32x4*>(src + 16));
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
          if (!act[r]) continue;
          f32x4 acc[HT];
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma_fp8(qf[r][ht], kf, f32x4{0.f, 0.f, 0.f, 0.f});
          float s = 0.0f;
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s += relu_bits(acc[ht][i]) * wf[r][ht * 4 + i];
          }
          part[r][st] = s;
        }
      }
      const float scale = s_scale[buf][lane];
      const int token = tok0 + lane;
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) {
        const int row = row_base + wave * kRowsPerWave + r;
        const float val = reduce_scatter_rows(part[r]);  // key `token` of the page
        if (act[r] && token < len[r]) a.logits[static_cast<int64_t>(row) * a.logits_stride + token] = val * scale;
      }
    }
    if (more) lstore(buf ^ 1, x0, x1, sc);
    __syncthreads();
  }
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_mqa_logits_prefill(const uint8_t* q8, const float* w, int heads, int64_t rows,
                                      const uint8_t* kv_cache, int64_t page_stride_bytes, const int32_t* block_table,
                                      int64_t bt_pages, const int32_t* lens, float* logits, int64_t logits_stride,
                                      int64_t width, hipStream_t stream) {
  DSA_REQUIRE(heads == 32 || heads == 64, "dsa_mqa_logits_prefill: heads must be 32 or 64 (got %d)", heads);
  DSA_REQUIRE(rows >= 0 && rows <= 0x7FFFFFFF, "dsa_mqa_logits_prefill: rows out of range");
  if (rows == 0) return ok();
  DSA_REQUIRE(q8 && w && kv_cache && block_table && lens && logits, "dsa_mqa_logits_prefill: null pointer");
  DSA_REQUIRE(bt_pages > 0 && width > 0 && width <= bt_pages * kPage && width <= 0x7FFFFFFF,
              "dsa_mqa_logits_prefill: width must be positive and within the block table capacity");
  DSA_REQUIRE(logits_stride >= width, "dsa_mqa_logits_prefill: logits_stride < width");
  DSA_REQUIRE(page_stride_bytes >= kPageBytes && page_stride_bytes % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(kv_cache) & 15u) == 0 && (reinterpret_cast<uintptr_t>(q8) & 15u) == 0,
              "dsa_mqa_logits_prefill: kv_cache pages (stride >= 8448, %% 16) and q8 must be 16-B aligned");
  PrefillArgs a;
  a.q8 = q8;
  a.w = w;
  a.kv = kv_cache;
  a.page_stride = page_stride_bytes;
  a.bt = block_table;
  a.bt_pages = static_cast<int>(bt_pages);
  a.lens = lens;
  a.rows = static_cast<int>(rows);
  a.width = static_cast<int>(width);
  a.logits = logits;
  a.logits_stride = logits_stride;
  const uint32_t grid = static_cast<uint32_t>((rows + kRowsPerCta - 1) / kRowsPerCta);
  if (heads == 64) hipLaunchKernelGGL(mqa_logits_prefill_kernel<64>, dim3(grid), dim3(kThreads), 0, stream, a);
  else hipLaunchKernelGGL(mqa_logits_prefill_kernel<32>, dim3(grid), dim3(kThreads), 0, stream, a);
  return check_launch("dsa_mqa_logits_prefill");
}
