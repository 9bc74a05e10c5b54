// Paged MQA indexer logits for decode and prefill on gfx950 fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4).
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
//    tile*16 + l%16, bytes (l/16)*32 .. +32.  The B operand is 16 tokens of a K page with the
//    same byte mapping, so the instruction's K ordering is the same permutation on both sides
//    and cancels.
//  * Result lane l holds heads 4*(l/16)+i of token l%16: the epilogue is an in-lane
//    max/fma chain over H/4 values; the four sub-tiles' partial sums then go through one
//    reduce-scatter over the 16-lane rows (row swaps) that leaves lane l with token l of the
//    page.  One 256 B logits store per page and row.
//  * K pages go HBM -> LDS by DMA (global_load_lds_dwordx4: no VGPR staging, so register
//    pressure does not limit the loads in flight).  A CTA runs S page streams; a stream's R
//    waves (one per row of the group) share each page through an LDS slot, and while a page is
//    scored the stream's next page lands in the other slot.  The 16-B chunks of a token are
//    XOR-swizzled in the slot so that the MFMA-layout ds_read_b128s are conflict-free.  A
//    stream's waves meet at one bare s_barrier per page, after each waited for its own share
//    of the DMA (explicit vmcnt); a page's stores are issued at the next step, before its DMA,
//    so that wait never covers them.  S, the slot count and the CTA's block-table slice are
//    chosen per (R, histogram) for LDS / register fit (Shape).
//  * Balanced static grid: a row group is R rows of one request.  Every CTA reads the groups'
//    lengths and gives group g ceil(pages_g * T / P) CTAs (P = total pages, T = the target CTA
//    count), so each CTA streams ~P / T consecutive pages of a single group whatever the length
//    mix; the grid (T + groups) depends only on shapes, so the launch can be captured in a
//    hipGraph, and T is chosen so that every CTA is resident at once.
//  * Mask words past a group's pages are zeroed by the group's own CTAs (a share each, 8-B
//    stores), so no separate mask memset is launched; a group with no pages still gets a CTA.
//  * Prefill is the same kernel with a request's query rows as one group in CTAs of 8 rows:
//    8 waves share one page stream, so a K page is read from HBM once per 8 query rows and
//    ds_read once per wave; no mask is written (mask == nullptr).
//  * kHist: also the top-k pass-1 histogram (12-bit key[31:20] of the nonzero logits of rows
//    with min(hist_len, width) > 2048, plus positive / zero counts), as 16-bit LDS counts (two
//    bins a word; a CTA's tokens per row stay below 2^16) flushed once per CTA with one global
//    atomic per nonzero bin; mqa_hist_init_kernel seeds the zero bin / zero count with the row
//    length (mqa_hist.cu:278-304) and every CTA subtracts its nonzero tokens.
#include "dsa_common.h"

namespace dsa {
namespace {

using i32x8 = __attribute__((ext_vector_type(8))) int;
using f32x4 = __attribute__((ext_vector_type(4))) float;
using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

constexpr int kLdsBytes = 163840;  // LDS per CU
constexpr int kMaxWavesCu = 16;    // waves per CU the register budget (<= 128 VGPRs) allows

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

// LDS chunk (16 B units) of token t's K bytes [16 p, 16 p + 16) within a page slot: rows of
// 8 chunks, chunk p of token t stored at position p ^ ((t >> 1) & 7), so the 16 lanes of one
// ds_read_b128 (16 consecutive tokens, the same p) hit 16 distinct 16-B bank groups.
__device__ __forceinline__ int swz(int t, int p) { return t * 8 + (p ^ ((t >> 1) & 7)); }

// DMA of one page (8448 B) into an LDS slot by the R waves of a stream, global -> LDS with no
// register staging.  Block j (j = r, r + R, ...; 1 KB = tokens 8j .. 8j + 7): lane i fills slot
// chunk 64 j + i with the global chunk that belongs there; the last wave also copies the 64
// token scales behind the K bytes.
template <int R>
__device__ __forceinline__ void dma_page(const uint8_t* page, uint8_t* slot, int r, int lane) {
#pragma unroll
  for (int j = r; j < 8; j += R) {
    const uint32_t c = j * 64 + lane;
    const uint32_t t = c >> 3;
    const uint32_t p = (c & 7) ^ ((t >> 1) & 7);
    // unsigned 32-bit lane offsets: a wave-uniform page pointer then serves as the scalar base
    __builtin_amdgcn_global_load_lds(page + (t * kHeadDim + p * 16), slot + j * 1024, 16, 0, 0);
  }
  if (r == R - 1)
    __builtin_amdgcn_global_load_lds(page + static_cast<uint32_t>(kPageFp8Bytes + lane * 4), slot + kPageFp8Bytes, 4,
                                     0, 0);
}

// 32 bytes (chunks p0, p0 + 1) of token t from a slot, as an MFMA operand.
__device__ __forceinline__ i32x8 lds_frag(const uint8_t* slot, int t, int p0) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(slot + swz(t, p0) * 16);
  const u32x4 b = *reinterpret_cast<const u32x4*>(slot + swz(t, p0 + 1) * 16);
  return i32x8{(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
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
  int32_t* hist_ws;   // kHist: the fused pass-1 workspace
  int32_t* zero_ws;   // non-null: the paired top-k's workspace, whose counters are zeroed here
  int64_t batch;
  int nt_logits;      // logits stored nontemporally (a logits block larger than the L2s hold)
  int slice_pages;    // > 0: slice-major assignment (assign_slices) with slices of this many pages
};

__device__ __forceinline__ int clamp_len(int l, int width) { return l < 0 ? 0 : (l > width ? width : l); }

// Pages of row group g: ceil(max over its R rows of len / 64).
__device__ __forceinline__ int group_pages(const DecodeArgs& a, int g) {
  int m = 0;
  for (int r = 0; r < a.R; ++r) m = max(m, clamp_len(a.ctx[g * a.R + r], a.width));
  return (m + kPage - 1) / kPage;
}

// A group with no pages still gets one CTA: it zeroes the group's mask rows.
__device__ __forceinline__ int group_ctas(int pages, int total_pages, int target) {
  if (pages == 0) return 1;
  return static_cast<int>((static_cast<int64_t>(pages) * target + total_pages - 1) / total_pages);
}

// Work assignment, identical in every CTA: s_assign = {group (-1: none), index among the group's
// CTAs, their count}; group g gets ceil(pages_g * T / P) CTAs.  Ends before a barrier (the caller's).
template <int NT>
__device__ void assign_cta(const DecodeArgs& a, int (&s_w)[2][NT / kWave], int* s_assign) {
  const int tid = threadIdx.x;
  const int cta = blockIdx.x;
  // Thread tid owns groups [g_lo, g_hi); their page counts are read once and kept (up to kGpt
  // a thread, else re-read).
  constexpr int kGpt = 4;
  const int per_t = (a.n_groups + NT - 1) / NT;
  const int g_lo = min(tid * per_t, a.n_groups);
  const int g_hi = min(g_lo + per_t, a.n_groups);
  const bool cached = per_t <= kGpt;  // block-uniform
  int gp[kGpt];
  int my_pages = 0;
  if (cached) {
#pragma unroll
    for (int i = 0; i < kGpt; ++i) {
      gp[i] = g_lo + i < g_hi ? group_pages(a, g_lo + i) : 0;
      my_pages += gp[i];
    }
  } else {
    for (int g = g_lo; g < g_hi; ++g) my_pages += group_pages(a, g);
  }
  int total_pages;
  block_excl_sum<NT>(my_pages, total_pages, s_w[0]);
  if (tid == 0) s_assign[0] = -1;
  int my_ctas = 0;
  if (cached) {
#pragma unroll
    for (int i = 0; i < kGpt; ++i) my_ctas += g_lo + i < g_hi ? group_ctas(gp[i], total_pages, a.target) : 0;
  } else {
    for (int g = g_lo; g < g_hi; ++g) my_ctas += group_ctas(group_pages(a, g), total_pages, a.target);
  }
  int total_ctas;
  int c0 = block_excl_sum<NT>(my_ctas, total_ctas, s_w[1]);
  if (cta >= c0 && cta < c0 + my_ctas) {
    for (int i = 0; g_lo + i < g_hi; ++i) {
      int p;
      if (cached) {
        p = gp[0];
#pragma unroll
        for (int j = 1; j < kGpt; ++j) p = i == j ? gp[j] : p;
      } else {
        p = group_pages(a, g_lo + i);
      }
      const int n = group_ctas(p, total_pages, a.target);
      if (cta < c0 + n) {
        s_assign[0] = g_lo + i;
        s_assign[1] = cta - c0;
        s_assign[2] = n;
        break;
      }
      c0 += n;
    }
  }
}

// Slice-major assignment (the prefill launches): the K pages of every group are cut into slices of
// SL = a.slice_pages pages, and CTA c takes the c-th (slice, group) pair in slice-then-group
// order, so the CTAs resident at one time -- consecutive blockIdx, spread over the 8 XCDs by
// blockIdx % 8 -- work on the same slice of K for different row groups: each XCD's L2 then holds
// one slice (SL * 8448 B) that all of its CTAs read, where the group-major balanced grid has every
// XCD's resident CTAs spread over the whole K range (a prefill's 10-20 MB of K misses the L2s).
// s_assign = {group (-1: none), slice, the group's pages}.  Ends before a barrier (the caller's).
constexpr int kMaxSlices = 64;  // slices a group may have (the host sizes SL for it)

template <int NT>
__device__ void assign_slices(const DecodeArgs& a, int (&s_w)[2][NT / kWave], int* s_nsl, int* s_assign) {
  const int tid = threadIdx.x;
  const int cta = blockIdx.x;
  const int SL = a.slice_pages;
  // s_nsl[n] = groups with n slices
  for (int i = tid; i <= kMaxSlices; i += NT) s_nsl[i] = 0;
  if (tid == 0) s_assign[0] = -1;
  __syncthreads();
  for (int g = tid; g < a.n_groups; g += NT) {
    const int ns = (group_pages(a, g) + SL - 1) / SL;
    atomicAdd(&s_nsl[ns < kMaxSlices ? ns : kMaxSlices], 1);
  }
  __syncthreads();
  // this CTA's slice j: pairs of slice j are the groups with more than j slices
  int j = 0, before = 0, in_j = 0;
  for (; j < kMaxSlices; ++j) {
    in_j = 0;
    for (int n = j + 1; n <= kMaxSlices; ++n) in_j += s_nsl[n];
    if (cta < before + in_j) break;
    before += in_j;
  }
  if (j == kMaxSlices) return;  // block-uniform: no pair left for this CTA
  const int rank = cta - before;  // the rank-th group (in group order) with more than j slices
  int seen = 0;
  for (int g0 = 0; g0 < a.n_groups; g0 += NT) {  // block-uniform
    const int g = g0 + tid;
    int pages = 0;
    bool has = false;
    if (g < a.n_groups) {
      pages = group_pages(a, g);
      has = (pages + SL - 1) / SL > j;
    }
    int total;
    const int pre = block_excl_sum<NT>(has ? 1 : 0, total, s_w[(g0 / NT) & 1]);
    if (has && seen + pre == rank) {
      s_assign[0] = g;
      s_assign[1] = j;
      s_assign[2] = pages;
    }
    seen += total;
    if (seen > rank) break;  // block-uniform
  }
}

// The same for up to 64 groups, computed by every wave on its own (lane g holds group g): no
// LDS and no barrier before the CTA's first block-table read.  Returns {group (-1: none), index
// within the group's CTAs, their count}, wave-uniform.
__device__ __forceinline__ int3 assign_cta_wave(const DecodeArgs& a) {
  const int lane = threadIdx.x & 63;
  const int cta = blockIdx.x;
  const bool in = lane < a.n_groups;
  const int pages = in ? group_pages(a, lane) : 0;
  const int incl_p = wave_prefix_sum(pages);
  const int total = __builtin_amdgcn_readlane(incl_p, 63);
  const int ctas = in ? group_ctas(pages, total, a.target) : 0;
  const int incl = wave_prefix_sum(ctas);
  const int c0 = incl - ctas;
  const uint64_t m = __ballot(in && cta >= c0 && cta < incl);
  if (m == 0) return make_int3(-1, 0, 0);
  const int l = static_cast<int>(__builtin_ctzll(m));
  return make_int3(l, cta - __builtin_amdgcn_readlane(c0, l), __builtin_amdgcn_readlane(ctas, l));
}

// Launch shape per (rows per CTA R, fused histogram): S page streams per CTA with NS LDS slots
// each, and the block-table slice a CTA stages (the host keeps P / T within it; it also bounds a
// row's tokens per CTA below 2^16 for the 16-bit histogram counters).  Measured on the 64-request
// MTP decode: one stream per CTA (eight CTAs per CU) without the histogram; with it, the 8 KB
// per row of counters is amortised over two streams (R = 2) or four (R = 1).  One-row CTAs run
// two streams (half the CTAs to dispatch for the same pages in flight: 32 x 16K decode 16.1 ->
// 15.7 us, 1 x 4K 6.4 -> 6.3 us; two-row CTAs measured 0.5 us slower with two).
template <int R, bool kHist>
struct Shape {
  static constexpr int S = kHist ? (R == 1 ? 4 : (R == 2 ? 2 : 1)) : (R == 1 ? 2 : 1);
  static constexpr int NS = 2;
  static constexpr int kMaxPages = S == 1 ? 255 : (S == 2 ? 511 : 1023);
  static constexpr int kLds = S * NS * kPageBytes + (kHist ? R * kBins * 2 : 0) + kMaxPages * 4 + 512;
  static constexpr int kByLds = kLdsBytes / kLds;
  static constexpr int kByWaves = kMaxWavesCu / (R * S) > 0 ? kMaxWavesCu / (R * S) : 1;
  static constexpr int kCtasPerCu = kByLds < kByWaves ? kByLds : kByWaves;
  static constexpr int kThreads = R * S * kWave;
  static constexpr int kWavesPerSimd = (kCtasPerCu * R * S + 3) / 4;
};

// VMEM ops of wave r's share of a page DMA (blocks r, r + R, ... of 8; the last wave adds the
// scales).
template <int R>
__device__ __forceinline__ int dma_ops(int r) { return (8 - r + R - 1) / R + (r == R - 1 ? 1 : 0); }

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..15 (gfx9 encoding; expcnt / lgkmcnt not waited).
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F79); break;
  }
}

// kMask = false: a.mask is null (prefill), known at compile time, so the page loop carries no
// mask state.
template <int H, int R, bool kHist, bool kMask>
__global__ __launch_bounds__((Shape<R, kHist>::kThreads)) __attribute__((amdgpu_waves_per_eu(
    Shape<R, kHist>::kWavesPerSimd))) void mqa_logits_decode_kernel(const DecodeArgs a) {
  constexpr int HT = H / 16;  // head tiles
  using Sh = Shape<R, kHist>;
  constexpr int S = Sh::S;
  constexpr int NS = Sh::NS;
  static_assert(NS == 2 || NS == 3, "2 or 3 page slots per stream");
  constexpr int NT = Sh::kThreads;
  __shared__ __attribute__((aligned(16))) uint8_t s_slot0[S][kPageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t s_slot1[S][kPageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t s_slot2[NS > 2 ? S : 1][NS > 2 ? kPageBytes : 16];
  __shared__ uint32_t s_hist[kHist ? R * kBins / 2 : 1];  // 16-bit counters, two bins per word
  __shared__ int s_cnt[2 * R];
  __shared__ int s_w[2][NT / kWave];
  __shared__ int s_assign[3];  // group, index within the group's CTAs, the group's CTA count
  __shared__ int s_nsl[kMask ? 1 : kMaxSlices + 1];  // slice-major assignment (prefill, no mask)
  __shared__ int s_bt[Sh::kMaxPages];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: row pointers become scalar
  const int cta = blockIdx.x;

  int grp, jc, nj;
  int slice_begin = -1, slice_pages = 0;  // slice-major: the CTA's first page, its group's pages
  if (!kMask && a.slice_pages > 0) {  // block-uniform
    if constexpr (!kMask) {
      assign_slices<NT>(a, s_w, s_nsl, s_assign);
      __syncthreads();
      grp = s_assign[0];
      jc = s_assign[1];
      nj = 1;
      slice_begin = jc * a.slice_pages;
      slice_pages = s_assign[2];
    }
  } else if (a.n_groups <= kWave) {  // block-uniform
    const int3 as = assign_cta_wave(a);
    grp = uniform(as.x);
    jc = uniform(as.y);
    nj = uniform(as.z);
  } else {
    assign_cta<NT>(a, s_w, s_assign);
    __syncthreads();
    grp = s_assign[0];
    jc = s_assign[1];
    nj = s_assign[2];
  }

  // The paired top-k's per-row counters (words 0..2 of each row of the workspace's second
  // block [histograms rows*4096 | counters rows*4096 | counts rows*2]), a row per CTA; issued
  // after the CTA's page stream, so that no DMA wait covers these stores.
  auto zero_share = [&]() {
    if (a.zero_ws == nullptr) return;
    for (int64_t rr = cta; rr < a.batch; rr += gridDim.x)
      if (tid < 3) a.zero_ws[(a.batch + rr) * kBins + tid] = 0;
  };
  if (grp < 0) {  // uniform: no pages for this CTA
    zero_share();
    return;
  }

  // wave = row r of the group x stream s: stream s takes the CTA's pages s, s + S, ...; its R
  // waves share each page through an LDS slot, one row each.
  const int r = wave / S;
  const int s = wave % S;
  const int row0 = grp * R;
  const int row = row0 + r;
  const int group_row = (row0 / a.group) * a.group;
  int max_len = 0;
#pragma unroll
  for (int q = 0; q < R; ++q) max_len = max(max_len, clamp_len(a.ctx[row0 + q], a.width));
  const int len = clamp_len(a.ctx[row], a.width);
  int hlim = 0;
  if constexpr (kHist) {
    int h = a.hist_lens[row];
    h = h < a.width ? h : a.width;
    hlim = h > kTopK ? h : 0;
  }
  const int pages = (max_len + kPage - 1) / kPage;
  const int p_begin = slice_begin >= 0 ? slice_begin : static_cast<int>(static_cast<int64_t>(pages) * jc / nj);
  const int p_end = slice_begin >= 0 ? min(slice_begin + a.slice_pages, slice_pages)
                                     : static_cast<int>(static_cast<int64_t>(pages) * (jc + 1) / nj);
  const int n_local = p_end - p_begin;  // <= Sh::kMaxPages by the host's choice of target
  const int32_t* btr = a.bt + static_cast<int64_t>(group_row) * a.bt_stride + p_begin;

  // The block-table entries of the stream's first two pages, read together and waited for
  // here: the second page's DMA then needs no wait (one later would also wait for the first
  // page, every VMEM operation before it counting).  Then the first page of every stream.
  int bt_first = 0, bt_second = 0;
  if (s < n_local) bt_first = btr[s];
  if (S + s < n_local) bt_second = btr[S + s];
  wait_vmcnt(0);
  if (s < n_local) dma_page<R>(a.kv + static_cast<int64_t>(bt_first) * a.page_stride, s_slot0[s], r, lane);

  // q / w fragments of this wave's row: lane l holds head ht*16 + l%16, bytes (l/16)*32 .. +32,
  // and the weights of heads ht*16 + 4*(l/16) + e, the rows of the MFMA result it holds.
  i32x8 qf[HT];
  float wf[HT * 4];
  {
    const uint8_t* qr = a.q8 + static_cast<int64_t>(row) * H * kHeadDim + (lane & 15) * kHeadDim + (lane >> 4) * 32;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) qf[ht] = load_frag(qr + ht * 16 * kHeadDim);
    const float* wr = a.w + static_cast<int64_t>(row) * H + 4 * (lane >> 4);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
      for (int e = 0; e < 4; ++e) wf[ht * 4 + e] = wr[ht * 16 + e];
    }
  }

  // The CTA's block-table slice straight into LDS (no register round trip, so nothing here
  // waits for the loads above), then the second page of every stream: while the first pages
  // are in flight, the memory system already has the next ones.  Step 0 waits for everything
  // but that second page, and its barrier publishes s_bt and the zeroed counters; no barrier
  // is needed here.
  for (int b = wave * kWave; b < n_local; b += NT)
    if (b + lane < n_local) __builtin_amdgcn_global_load_lds(btr + b + lane, &s_bt[b], 4, 0, 0);
  if (S + s < n_local) dma_page<R>(a.kv + static_cast<int64_t>(bt_second) * a.page_stride, s_slot1[s], r, lane);
  if constexpr (kHist) {
    for (int i = tid; i < R * kBins / 2; i += NT) s_hist[i] = 0;
    if (tid < 2 * R) s_cnt[tid] = 0;
  }
  // Mask words of the group's rows past its pages (no CTA scores them) are zeroed by the
  // group's CTAs, a share each: one 8-B store per page and row when the layout allows it.
  // Issued after the page stream, so that no DMA wait covers these stores.
  auto zero_mask_tail = [&]() {
    const int tail = a.bt_pages - pages;
    const int units = R * tail;
    const int u0 = static_cast<int>(static_cast<int64_t>(units) * jc / nj);
    const int u1 = static_cast<int>(static_cast<int64_t>(units) * (jc + 1) / nj);
    const bool wide = (reinterpret_cast<uintptr_t>(a.mask) & 7u) == 0 && (a.mask_stride & 3) == 0;
    for (int u = kMask && a.mask != nullptr ? u0 + tid : u1; u < u1; u += NT) {
      const int rr = u / tail;
      int16_t* m = a.mask + static_cast<int64_t>(row0 + rr) * a.mask_stride + (pages + u - rr * tail) * 4;
      if (wide) {
        *reinterpret_cast<uint64_t*>(m) = 0;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) m[e] = 0;
      }
    }
  };

  int nz = 0, pos = 0;
  const int n_steps = (n_local + S - 1) / S;  // block-uniform
  const int t_lo = lane & 15;
  const int p0 = (lane >> 4) * 2;

  // Results of a scored page are written at the start of the next step, before that step's DMA
  // is issued: the wait at the top of a step then finds the stores older than the DMA, and the
  // LDS histogram atomics never have a DMA in flight to wait for.
  int pend_p = -1;  // page of the held results (wave-uniform), -1: none
  float pend_v = 0.0f;
  uint64_t pend_bits = 0;
  // the row's logits / mask rows as scalar bases, the token as an unsigned 32-bit lane offset:
  // each store is the scalar-base form, no 64-bit address arithmetic per lane
  float* const lrow = a.logits + static_cast<int64_t>(row) * a.logits_stride;
  int16_t* const mrow = a.mask + static_cast<int64_t>(row) * a.mask_stride;
  auto flush = [&]() {
    if (pend_p < 0) return;
    const int token = pend_p * kPage + lane;
    if (kMask && a.mask != nullptr && lane < 4)
      *reinterpret_cast<int16_t*>(reinterpret_cast<char*>(mrow) + static_cast<uint32_t>((pend_p * 4 + lane) * 2)) =
          static_cast<int16_t>((pend_bits >> (16 * lane)) & 0xFFFFu);
    if (token < len) {
      const uint32_t off = static_cast<uint32_t>(token * 4);
      // the nontemporal form as asm: a builtin hint on one branch would be merged with the
      // plain store of the other
      if (a.nt_logits) asm volatile("global_store_dword %0, %1, %2 nt" ::"v"(off), "v"(pend_v), "s"(lrow) : "memory");
      else *reinterpret_cast<float*>(reinterpret_cast<char*>(lrow) + off) = pend_v;
    }
    if constexpr (kHist) {
      if (((pend_bits >> lane) & 1u) && token < hlim) {
        const uint32_t key = float_key(pend_v);
        atomicAdd(&s_hist[r * (kBins / 2) + static_cast<int>(key >> 21)], 1u << ((key >> 16) & 16u));
        ++nz;
        pos += key > kZeroKey;
      }
    }
    pend_p = -1;
  };

  // One step: page i of this stream is in `cur`; page i + (NS - 1) S is sent to `nxt`.
  const int n_dma = dma_ops<R>(r);
  auto step = [&](int k, uint8_t* cur, uint8_t* nxt) {
    const int i = k * S + s;  // this stream's page (local index)
    // this wave's share of page i has landed: the only VMEM ops issued after it are the DMAs of
    // the pages still ahead of it (page i + S at step 0, or always with NS = 3, if it exists).
    // The barrier publishes every wave's share and retires the readers of `nxt` from the
    // previous step.
    if ((NS > 2 || k == 0) && i + S < n_local) wait_vmcnt(n_dma);
    else wait_vmcnt(0);
    // a bare s_barrier: __syncthreads' release fence would wait for every LDS DMA in flight
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS histogram updates are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    flush();
    if (i + (NS - 1) * S < n_local && (NS > 2 || k > 0)) {  // NS = 2: page S + s came with the prologue
      // the entry is the same in every lane: as a scalar, the page address is scalar arithmetic
      // and the DMA takes it as its scalar base (no 64-bit per-lane address math)
      const int pg = __builtin_amdgcn_readfirstlane(s_bt[i + (NS - 1) * S]);
      dma_page<R>(a.kv + static_cast<int64_t>(pg) * a.page_stride, nxt, r, lane);
    }
    if (i >= n_local) return;  // stream-uniform (the stream still takes part in the barriers)
    const float scale = reinterpret_cast<const float*>(cur + kPageFp8Bytes)[lane];
    float part[4];  // this lane's heads' share of tokens st * 16 + lane % 16
    // One-row CTAs read the page's four K fragments from LDS before the first MFMA, instead of
    // each right before its MFMAs (32 x 16K logits 15.1 -> 14.8 us, 128 x 16K 47.0 -> 46.5 us); with
    // more rows a CTA the extra registers cost occupancy that the prefill kernel needs (1797 ->
    // 1816-1846 us per slab), and the MTP batch is unchanged.
    constexpr int kPf = R == 1 ? 4 : 1;
    i32x8 kfs[kPf];
    if constexpr (kPf == 4) {
#pragma unroll
      for (int st = 0; st < 4; ++st) kfs[st] = lds_frag(cur, st * 16 + t_lo, p0);
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      i32x8 kf;
      if constexpr (kPf == 4) kf = kfs[st];
      else kf = lds_frag(cur, st * 16 + t_lo, p0);
      f32x4 acc[HT];
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma_fp8(qf[ht], kf, f32x4{0.f, 0.f, 0.f, 0.f});
      float sum = 0.0f;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += relu_bits(acc[ht][e]) * wf[ht * 4 + e];
      }
      part[st] = sum;
    }
    const float val = reduce_scatter_rows(part);  // token `lane` of the page
    const int p = p_begin + i;
    const float v = val * scale;
    pend_p = p;
    pend_v = v;
    pend_bits = ((kMask && a.mask != nullptr) || kHist) ? __ballot(p * kPage + lane < len && __float_as_uint(v) != 0u) : 0;
  };
  // the two slots of a stream are distinct LDS objects, so the compiler can tell that the
  // reads of one do not wait for the DMA into the other
  if constexpr (NS == 2) {
    for (int k = 0; k < n_steps; k += 2) {
      step(k, s_slot0[s], s_slot1[s]);
      if (k + 1 < n_steps) step(k + 1, s_slot1[s], s_slot0[s]);
    }
  } else {
    for (int k = 0; k < n_steps; k += 3) {
      step(k, s_slot0[s], s_slot2[s]);
      if (k + 1 < n_steps) step(k + 1, s_slot1[s], s_slot0[s]);
      if (k + 2 < n_steps) step(k + 2, s_slot2[s], s_slot1[s]);
    }
  }
  flush();
  zero_mask_tail();
  zero_share();

  if constexpr (kHist) {
    const int n = wave_sum(nz);
    const int q = wave_sum(pos);
    if (lane == 0 && n) {
      atomicAdd(&s_cnt[2 * r], n);
      atomicAdd(&s_cnt[2 * r + 1], q);
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      int h = a.hist_lens[row0 + rr];
      h = h < a.width ? h : a.width;
      if (h <= kTopK) continue;  // block-uniform
      int32_t* gh = a.hist_ws + static_cast<int64_t>(row0 + rr) * kBins;
      int32_t* gcnt = a.hist_ws + 2 * a.batch * kBins + 2 * static_cast<int64_t>(row0 + rr);
      for (int wd = tid; wd < kBins / 2; wd += NT) {
        const uint32_t c = s_hist[rr * (kBins / 2) + wd];
        if (c & 0xFFFFu) atomicAdd(&gh[2 * wd], static_cast<int>(c & 0xFFFFu));
        if (c >> 16) atomicAdd(&gh[2 * wd + 1], static_cast<int>(c >> 16));
      }
      if (tid == 0) {
        const int n = s_cnt[2 * rr];
        const int q = s_cnt[2 * rr + 1];
        if (n) {
          atomicSub(&gh[kZeroBin], n);
          atomicSub(&gcnt[1], n);
        }
        if (q) atomicAdd(&gcnt[0], q);
      }
    }
  }
}

// Seeds the top-k pass-1 workspace (mqa_hist.cu:278-304): every token below
// min(hist_len, width) counts as a zero until the logits kernel subtracts its nonzero ones; rows
// with <= 2048 tokens stay empty.  The second histogram block of the layout ([ghist1 | ghist2 |
// cnt], the reference's workspace) is zeroed whole, as the reference leaves it; of it the split
// top-k uses words 0..2 of each row as its per-row counters.
__global__ __launch_bounds__(256) void mqa_hist_init_kernel(const int32_t* __restrict__ hist_lens, int width,
                                                            int64_t batch, int32_t* __restrict__ ws) {
  const int64_t row = blockIdx.x;
  int h = hist_lens[row];
  h = h < width ? h : width;
  const int zeros = h > kTopK ? h : 0;
  int4* g1 = reinterpret_cast<int4*>(ws + row * kBins);
  int4* g2 = reinterpret_cast<int4*>(ws + (batch + row) * kBins);
  for (int i = threadIdx.x; i < kBins / 4; i += 256) {
    g1[i] = make_int4(i == kZeroBin / 4 ? zeros : 0, 0, 0, 0);
    g2[i] = make_int4(0, 0, 0, 0);
  }
  if (threadIdx.x == 0) {
    int32_t* c = ws + 2 * batch * kBins + 2 * row;
    c[0] = 0;
    c[1] = zeros;
  }
}

template <int H, int R, bool kHist>
void launch_one(const DecodeArgs& a, uint32_t grid, hipStream_t stream) {
  if constexpr (R == 8) {  // eight rows a CTA: the prefill shape, which writes no mask
    if (a.mask == nullptr) {
      hipLaunchKernelGGL((mqa_logits_decode_kernel<H, R, kHist, false>), dim3(grid), dim3(Shape<R, kHist>::kThreads),
                         0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((mqa_logits_decode_kernel<H, R, kHist, true>), dim3(grid), dim3(Shape<R, kHist>::kThreads), 0,
                     stream, a);
}

template <int H, bool kHist>
void launch_r(const DecodeArgs& a, int R, uint32_t grid, hipStream_t stream) {
  switch (R) {
    case 1: launch_one<H, 1, kHist>(a, grid, stream); break;
    case 2: launch_one<H, 2, kHist>(a, grid, stream); break;
    case 3: launch_one<H, 3, kHist>(a, grid, stream); break;
    case 4:
      if constexpr (!kHist) launch_one<H, 4, false>(a, grid, stream);
      break;
    default:
      if constexpr (!kHist) launch_one<H, 8, false>(a, grid, stream);
      break;
  }
}

// (CTAs per CU, pages per CTA) of a launch shape, on the host.
void shape_host(int R, bool hist, int& ctas_per_cu, int& max_pages) {
  switch (hist ? R + 16 : R) {
    case 1: ctas_per_cu = Shape<1, false>::kCtasPerCu; max_pages = Shape<1, false>::kMaxPages; break;
    case 2: ctas_per_cu = Shape<2, false>::kCtasPerCu; max_pages = Shape<2, false>::kMaxPages; break;
    case 3: ctas_per_cu = Shape<3, false>::kCtasPerCu; max_pages = Shape<3, false>::kMaxPages; break;
    case 4: ctas_per_cu = Shape<4, false>::kCtasPerCu; max_pages = Shape<4, false>::kMaxPages; break;
    case 8: ctas_per_cu = Shape<8, false>::kCtasPerCu; max_pages = Shape<8, false>::kMaxPages; break;
    case 17: ctas_per_cu = Shape<1, true>::kCtasPerCu; max_pages = Shape<1, true>::kMaxPages; break;
    case 18: ctas_per_cu = Shape<2, true>::kCtasPerCu; max_pages = Shape<2, true>::kMaxPages; break;
    default: ctas_per_cu = Shape<3, true>::kCtasPerCu; max_pages = Shape<3, true>::kMaxPages; break;
  }
}

// Enqueues the kernel for a.batch rows in groups of R (a.group rows share a block-table row;
// a.width caps the lengths).  a's pointers, strides and sizes are set and checked by the caller.
int enqueue(DecodeArgs a, int heads, int R, int target_ctas, bool hist, const int32_t* hist_lens, int32_t* hist_ws,
            hipStream_t stream, const char* who, bool slice_major = false) {
  const int64_t n_groups = a.batch / R;
  DSA_REQUIRE(n_groups <= 0x3FFFFFFF, "%s: too many rows", who);
  int ctas_per_cu = 1, max_cta_pages = 1;
  shape_host(R, hist, ctas_per_cu, max_cta_pages);
  a.slice_pages = 0;
  const int64_t width_pages = (a.width + kPage - 1) / kPage;
  // (the maskless eight-row instantiation is the one that carries the slice-major assignment)
  if (slice_major && R == 8 && a.mask == nullptr && width_pages <= static_cast<int64_t>(kMaxSlices) * max_cta_pages) {
    // slices as long as the block-table stage allows (the balanced grid's slice length at these
    // shapes), a CTA per (slice, group) pair the widest group could need
    const int64_t n_sl = (width_pages + max_cta_pages - 1) / max_cta_pages;
    const int64_t grid = n_groups * n_sl;
    DSA_REQUIRE(grid <= 0x7FFFFFFF, "%s: grid too large", who);
    a.R = R;
    a.n_groups = static_cast<int>(n_groups);
    a.slice_pages = static_cast<int>((width_pages + n_sl - 1) / n_sl);
    a.nt_logits = a.batch * static_cast<int64_t>(a.width) * 4 > (16ll << 20) ? 1 : 0;
    a.target = 0;
    a.hist_lens = nullptr;
    a.hist_ws = nullptr;
    a.zero_ws = nullptr;
    const uint32_t g = static_cast<uint32_t>(grid);
    if (heads == 64) launch_r<64, false>(a, R, g, stream);
    else launch_r<32, false>(a, R, g, stream);
    return check_launch(who);
  }
  if (target_ctas <= 0) {
    // All CTAs resident at once: the per-group rounding adds up to one CTA per group, so aim
    // below the resident count by the group count.
    int n_cu = 0;
    const int st = dsa_device_cu_count(&n_cu);
    if (st != DSA_OK) return st;
    const int64_t slots = ctas_per_cu * static_cast<int64_t>(n_cu);
    int64_t t = slots - n_groups > slots / 2 ? slots - n_groups : slots / 2;
    // no more CTAs than the block tables hold pages: past one page a CTA, the extra CTAs only add
    // dispatch (one row of 4096 tokens, 64 pages: 1023 CTAs 5.7 us, 64-128 CTAs 4.0-4.3 us)
    const int64_t bt_total = n_groups * ((a.width + kPage - 1) / kPage);
    if (t > bt_total) t = bt_total > 0 ? bt_total : 1;
    target_ctas = static_cast<int>(t);
  }
  // Keep every CTA's page slice within the LDS block-table stage: P / T <= max_pages.
  const int64_t max_pages = n_groups * ((a.width + kPage - 1) / kPage);
  DSA_REQUIRE(max_pages <= 0x7FFFFFFF, "%s: the groups' pages (%lld) must fit in 32 bits", who,
              static_cast<long long>(max_pages));
  int64_t target = target_ctas;
  if (target * max_cta_pages < max_pages) target = (max_pages + max_cta_pages - 1) / max_cta_pages;
  const int64_t grid = target + n_groups;
  DSA_REQUIRE(grid <= 0x7FFFFFFF, "%s: grid too large", who);
  a.R = R;
  a.n_groups = static_cast<int>(n_groups);
  // A logits block beyond half the chip's 32 MB of L2 streams out with nontemporal stores: the
  // block does not stay cached for the top-k anyway, and the launch then ends without a large
  // dirty-line writeback (measured on the 64-request MTP batch, 33.6 MB: logits launch 56.5 ->
  // 54.3 us, logits + top-k 83.4 -> 79.4 us; a 2 MB block keeps its cached stores).
  a.nt_logits = a.batch * static_cast<int64_t>(a.width) * 4 > (16ll << 20) ? 1 : 0;
  a.target = static_cast<int>(target);
  a.hist_lens = hist ? hist_lens : nullptr;
  a.hist_ws = hist ? hist_ws : nullptr;
  a.zero_ws = hist ? nullptr : hist_ws;
  if (hist) {
    hipLaunchKernelGGL(mqa_hist_init_kernel, dim3(static_cast<uint32_t>(a.batch)), dim3(256), 0, stream, hist_lens,
                       a.width, a.batch, hist_ws);
  }
  const uint32_t g = static_cast<uint32_t>(grid);
  if (heads == 64) {
    if (hist) launch_r<64, true>(a, R, g, stream);
    else launch_r<64, false>(a, R, g, stream);
  } else {
    if (hist) launch_r<32, true>(a, R, g, stream);
    else launch_r<32, false>(a, R, g, stream);
  }
  return check_launch(who);
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_mqa_logits_decode(const uint8_t* q8, const float* w, int heads, int64_t batch, int group_size,
                                     const uint8_t* kv_cache, int64_t page_stride_bytes,
                                     const int32_t* context_lens, const int32_t* block_table, int64_t bt_stride,
                                     int64_t bt_pages, float* logits, int64_t logits_stride, int16_t* mask,
                                     int64_t mask_stride, int rows_per_cta, int target_ctas,
                                     const int32_t* hist_lens, int32_t* hist_ws, int fuse_pass1,
                                     hipStream_t stream) {
  DSA_REQUIRE(heads == 32 || heads == 64, "dsa_mqa_logits_decode: heads must be 32 or 64 (got %d)", heads);
  DSA_REQUIRE(batch >= 0 && group_size >= 1, "dsa_mqa_logits_decode: batch must be >= 0 and group_size >= 1");
  DSA_REQUIRE(batch % group_size == 0, "dsa_mqa_logits_decode: batch must be a multiple of group_size");
  if (rows_per_cta <= 0) rows_per_cta = group_size % 2 == 0 ? 2 : 1;
  DSA_REQUIRE((rows_per_cta >= 1 && rows_per_cta <= 4 || rows_per_cta == 8) && group_size % rows_per_cta == 0,
              "dsa_mqa_logits_decode: rows_per_cta must be 1, 2, 3, 4 or 8 and divide group_size");
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
  DSA_REQUIRE(!fuse_pass1 || (hist_lens != nullptr && hist_ws != nullptr),
              "dsa_mqa_logits_decode: fuse_pass1 needs hist_lens and hist_ws");
  DSA_REQUIRE(hist_ws == nullptr || (reinterpret_cast<uintptr_t>(hist_ws) & 15u) == 0,
              "dsa_mqa_logits_decode: hist_ws must be 16-B aligned");
  const bool hist = fuse_pass1 != 0;
  DSA_REQUIRE(!hist || rows_per_cta <= 3,
              "dsa_mqa_logits_decode: the fused histogram needs rows_per_cta <= 3 (8 KB of LDS per row)");

  DecodeArgs a{};
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
  a.batch = batch;
  return enqueue(a, heads, rows_per_cta, target_ctas, hist, hist_lens, hist_ws, stream, "dsa_mqa_logits_decode");
}

// Prefill: the rows of one request are one group sharing the request's block table, scored by
// the same kernel in CTAs of 8 rows (8 waves on one LDS page stream: each K page read from HBM
// once per 8 query rows); a row count that is not a multiple of 8 ends in groups of 4 and of
// 1-3 rows, each its own launch.  No mask is written.
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
  int64_t done = 0;
  for (const int R : {8, 4, 2, 1}) {
    const int64_t n = (rows - done) / R * R;
    if (n == 0) continue;
    DecodeArgs a{};
    a.q8 = q8 + done * heads * kHeadDim;
    a.w = w + done * heads;
    a.kv = kv_cache;
    a.page_stride = page_stride_bytes;
    a.ctx = lens + done;
    a.bt = block_table;
    a.bt_stride = bt_pages;
    a.bt_pages = static_cast<int>(bt_pages);
    a.width = static_cast<int>(width);
    a.logits = logits + done * logits_stride;
    a.logits_stride = logits_stride;
    a.mask = nullptr;
    a.mask_stride = 0;
    a.group = static_cast<int>(n);
    a.batch = n;
    const int st = enqueue(a, heads, R, 0, false, nullptr, nullptr, stream, "dsa_mqa_logits_prefill", true);
    if (st != DSA_OK) return st;
    done += n;
  }
  return ok();
}
