// Exact top-2048 + page-table transform over (sparse-mask) indexer logits, gfx950.
//
// Contract (hcu_ops/csrc/sparse_mask_topk.cu:1-22,141-349): per row, the 2048 tokens t < len
// with the largest keys, ties at the threshold to the lower t; masked-out tokens are +0;
// rows with len <= 2048 copy page_table[0:len] and pad with -1.  Only the set is the contract.
//
// Algorithm (this file's own; radix digits 12/12/8 of the 32-bit key):
//   pass 1   LDS histogram of key[31:20] over the nonzero tokens, positive / zero counts.
//            positives <= 2048 <= positives + zeros: the threshold is +0 (sparse fast path).
//   pass 2   one ordered compaction over the row: tokens whose digit is above the threshold
//            bin t1 go straight to the output (list A); tokens in bin t1 go to an LDS candidate
//            list C (key, token) in token order.
//   resolve  key[19:8] and key[7:0] histograms over C in LDS give the exact threshold key and
//            the number of threshold ties to take; C is emitted in token order, so the ties that
//            win are the lowest-index ones.
//   overflow if C does not fit in LDS the two digit passes and the emission re-read the row.
// So a row is read twice (once if pass 1 comes from the logits kernel) instead of four times.
// Split variant (few rows): S CTAs per row share pass 1 through global atomics, compact their
// slice into per-slice global lists, and one CTA per row merges the lists (slices are
// contiguous token ranges, so slice order is token order) and resolves C.
// Every loop bound is block-uniform; no host synchronisation; launch shapes depend only on
// (rows, width, splits), so the whole path can be captured in a hipGraph.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kTk = 1024;              // threads per CTA
constexpr int kTkWaves = kTk / kWave;  // 16
constexpr int kStep = kTk * 4;         // tokens per block step (4 per thread)
constexpr int kCapC = 8192;            // LDS candidate capacity (single / merge kernels)
constexpr int kCapSlice = 4096;        // per-slice candidate capacity in the split workspace
constexpr int kMaxSplit = 64;

struct RowSrc {
  const float* vals;
  const int16_t* mask;  // nullable: all scores below len valid
  int len;
};

// Keys of tokens [i0, i0 + 4) (i0 % 4 == 0) and the bitmask of those below r.len.
template <bool kVec>
__device__ __forceinline__ uint32_t load_keys4(const RowSrc& r, int i0, uint32_t (&k)[4]) {
  const int safe = i0 < r.len ? i0 : 0;
  float v[4];
  if constexpr (kVec) {
    const float4 f = *reinterpret_cast<const float4*>(r.vals + safe);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = safe + j;
      v[j] = r.vals[t < r.len ? t : r.len - 1];
    }
  }
  uint32_t m = 0xFu;
  if (r.mask != nullptr) m = (static_cast<uint32_t>(static_cast<uint16_t>(r.mask[safe >> 4])) >> (safe & 15)) & 0xFu;
#pragma unroll
  for (int j = 0; j < 4; ++j) k[j] = ((m >> j) & 1u) ? float_key(v[j]) : kZeroKey;
  const int rem = r.len - i0;
  const int nv = rem <= 0 ? 0 : (rem < 4 ? rem : 4);
  return (1u << nv) - 1u;
}

// Block-exclusive prefix of two per-thread counts (each in [0, 4]) in thread order.
// s_scan: int2[2][kTkWaves], double-buffered by `parity`, so one barrier per call suffices.
__device__ __forceinline__ void block_prefix2(int ca, int cb, int& pa, int& pb, int& ta, int& tb, int2* s_scan,
                                              int parity) {
  int wa, wb;
  const int xa = wave_prefix_small(ca, wa);
  const int xb = wave_prefix_small(cb, wb);
  const int w = threadIdx.x >> 6;
  int2* buf = s_scan + parity * kTkWaves;
  if (lane_id() == 0) buf[w] = make_int2(wa, wb);
  __syncthreads();
  int ba = 0, bb = 0, sa = 0, sb = 0;
#pragma unroll
  for (int v = 0; v < kTkWaves; ++v) {
    const int2 t = buf[v];
    ba += v < w ? t.x : 0;
    bb += v < w ? t.y : 0;
    sa += t.x;
    sb += t.y;
  }
  pa = ba + xa;
  pb = bb + xb;
  ta = sa;
  tb = sb;
}

__device__ __forceinline__ int block_sum(int x, int* s_red) {
  x = wave_sum(x);
  if (lane_id() == 0) s_red[threadIdx.x >> 6] = x;
  __syncthreads();
  int s = 0;
#pragma unroll
  for (int v = 0; v < kTkWaves; ++v) s += s_red[v];
  __syncthreads();
  return s;
}

// Finds bin t with suffix(t) >= need > suffix(t + 1); s_res = {t, suffix(t + 1)}.
// Requires sum(hist) >= need >= 1.  Ends with a barrier.
template <int NB>
__device__ void find_threshold(const int* hist, int need, int* s_wtot, int* s_res) {
  constexpr int BPT = NB >= kTk ? NB / kTk : 1;
  constexpr int ACTIVE = NB / BPT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  int h[BPT];
  int s = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    h[j] = tid < ACTIVE ? hist[tid * BPT + j] : 0;
    s += h[j];
  }
  int x = s;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_down(x, o);
    if (lane + o < kWave) x += y;
  }
  if (lane == 0) s_wtot[w] = x;
  __syncthreads();
  int after = 0;
  for (int v = w + 1; v < kTkWaves; ++v) after += s_wtot[v];
  const int suf = x + after;
  const int suf_next = suf - s;
  if (tid < ACTIVE && suf >= need && suf_next < need) {
    int acc = suf_next;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      if (acc + h[j] >= need) {
        s_res[0] = tid * BPT + j;
        s_res[1] = acc;
        break;
      }
      acc += h[j];
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void zero_lds(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += kTk) p[i] = 0;
}

// Output write guarded to the row's 2048 entries (inputs that break the contract -- e.g. a
// pass-1 histogram built for other lengths -- give wrong rows, never stray writes).
__device__ __forceinline__ void put(int32_t* dst, int i, int32_t v) {
  if (static_cast<unsigned>(i) < static_cast<unsigned>(kTopK)) dst[i] = v;
}

// Page-table entry of token t (-1 past the row's entries).
struct PtRow {
  const int32_t* p;
  int cols;
  __device__ __forceinline__ int32_t operator[](int t) const { return t < cols ? p[t] : -1; }
};

// Page-table row of score row `row`: the row itself (decode layout) or its request.
__device__ __forceinline__ int pt_row_of(int row, const int32_t* cu, int n_req) {
  if (cu == nullptr) return row;
  int lo = 0, hi = n_req - 1;  // last b with cu[b] <= row
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// LDS of the single / merge kernels.
struct TopkLds {
  int hist[kBins];
  uint32_t ckey[kCapC];
  int cidx[kCapC];
  int2 scan[2 * kTkWaves];
  int wtot[kTkWaves];
  int red[kTkWaves];
  int res[2];
};

// Pass 1 over [begin, end): LDS histogram of key[31:20] of nonzero tokens (zeros are added to
// the zero bin once); returns positives / zeros of the range (block-uniform).
template <bool kVec>
__device__ void pass_hist(const RowSrc& r, int begin, int end, int* hist, int* s_red, int& pos, int& zeros) {
  RowSrc rr = r;
  rr.len = end;
  int zc = 0, pc = 0;
  for (int base = begin; base < end; base += kStep) {
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(rr, base + static_cast<int>(threadIdx.x) * 4, k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if ((valid >> j) & 1u) {
        if (k[j] == kZeroKey) {
          ++zc;
        } else {
          pc += k[j] > kZeroKey;
          atomicAdd(&hist[k[j] >> 20], 1);
        }
      }
    }
  }
  pos = block_sum(pc, s_red);
  zeros = block_sum(zc, s_red);
}

// Ordered emission over [begin, end) of the row for a fixed threshold key `thr`:
//  cond(key) selects the tokens that may be above the threshold (all of them, or digit == t1);
//  keys > thr go to dst[gt_base + rank], keys == thr with tie rank < remaining go to
//  dst[tie_base + rank].  gt_off / tie_off: ranks already used by earlier ranges.
template <bool kVec, typename Cond>
__device__ void emit_range(const RowSrc& r, int begin, int end, Cond cond, uint32_t thr, int gt_base, int tie_base,
                           int remaining, int gt_off, int tie_off, const PtRow& pt, int32_t* dst, int2* s_scan) {
  RowSrc rr = r;
  rr.len = end;
  int gt_pos = gt_off, tie_pos = tie_off;
  int parity = 0;
  for (int base = begin; base < end; base += kStep) {
    const int i0 = base + static_cast<int>(threadIdx.x) * 4;
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(rr, i0, k);
    int ng = 0, ne = 0;
    bool g[4], e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool v = ((valid >> j) & 1u) && cond(k[j]);
      g[j] = v && k[j] > thr;
      e[j] = v && k[j] == thr;
      ng += g[j];
      ne += e[j];
    }
    int pg, pe, tg, te;
    block_prefix2(ng, ne, pg, pe, tg, te, s_scan, parity);
    parity ^= 1;
    pg += gt_pos;
    pe += tie_pos;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (g[j]) put(dst, gt_base + pg, pt[i0 + j]);
      if (e[j] && pe < remaining) put(dst, tie_base + pe, pt[i0 + j]);
      pg += g[j];
      pe += e[j];
    }
    gt_pos += tg;
    tie_pos += te;
  }
}

// Resolves the exact threshold among the LDS candidates C (all with digit t1, in token order)
// and emits them.  above1 = tokens already emitted (digit > t1); need1 = 2048 - above1.
__device__ void resolve_lds(TopkLds& L, int n_c, uint32_t t1, int above1, const PtRow& pt, int32_t* dst) {
  const int need1 = kTopK - above1;
  zero_lds(L.hist, kBins);
  __syncthreads();
  for (int e = threadIdx.x; e < n_c; e += kTk) atomicAdd(&L.hist[(L.ckey[e] >> 8) & 0xFFFu], 1);
  __syncthreads();
  find_threshold<kBins>(L.hist, need1, L.wtot, L.res);
  const uint32_t prefix24 = (t1 << 12) | static_cast<uint32_t>(L.res[0]);
  const int need2 = need1 - L.res[1];
  zero_lds(L.hist, 256);
  __syncthreads();
  for (int e = threadIdx.x; e < n_c; e += kTk) {
    const uint32_t key = L.ckey[e];
    if ((key >> 8) == prefix24) atomicAdd(&L.hist[key & 0xFFu], 1);
  }
  __syncthreads();
  find_threshold<256>(L.hist, need2, L.wtot, L.res);
  const uint32_t thr = (prefix24 << 8) | static_cast<uint32_t>(L.res[0]);
  const int remaining = need2 - L.res[1];
  const int tie_base = kTopK - remaining;
  int gt_pos = 0, tie_pos = 0, parity = 0;
  for (int base = 0; base < n_c; base += kTk) {
    const int e = base + static_cast<int>(threadIdx.x);
    const uint32_t key = e < n_c ? L.ckey[e] : 0u;
    const bool g = e < n_c && key > thr;
    const bool q = e < n_c && key == thr;
    int pg, pe, tg, te;
    block_prefix2(g, q, pg, pe, tg, te, L.scan, parity);
    parity ^= 1;
    pg += gt_pos;
    pe += tie_pos;
    if (g) put(dst, above1 + pg, pt[L.cidx[e]]);
    if (q && pe < remaining) put(dst, tie_base + pe, pt[L.cidx[e]]);
    gt_pos += tg;
    tie_pos += te;
  }
}

// Threshold resolution by re-reading the row (candidates did not fit): digit passes over the
// tokens of bin t1, then the ordered emission of those above / at the threshold.
template <bool kVec>
__device__ void resolve_rescan(TopkLds& L, const RowSrc& r, uint32_t t1, int above1, const PtRow& pt,
                               int32_t* dst) {
  const int need1 = kTopK - above1;
  zero_lds(L.hist, kBins);
  __syncthreads();
  for (int base = 0; base < r.len; base += kStep) {
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(r, base + static_cast<int>(threadIdx.x) * 4, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((valid >> j) & 1u) && (k[j] >> 20) == t1) atomicAdd(&L.hist[(k[j] >> 8) & 0xFFFu], 1);
  }
  __syncthreads();
  find_threshold<kBins>(L.hist, need1, L.wtot, L.res);
  const uint32_t prefix24 = (t1 << 12) | static_cast<uint32_t>(L.res[0]);
  const int need2 = need1 - L.res[1];
  zero_lds(L.hist, 256);
  __syncthreads();
  for (int base = 0; base < r.len; base += kStep) {
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(r, base + static_cast<int>(threadIdx.x) * 4, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((valid >> j) & 1u) && (k[j] >> 8) == prefix24) atomicAdd(&L.hist[k[j] & 0xFFu], 1);
  }
  __syncthreads();
  find_threshold<256>(L.hist, need2, L.wtot, L.res);
  const uint32_t thr = (prefix24 << 8) | static_cast<uint32_t>(L.res[0]);
  const int remaining = need2 - L.res[1];
  emit_range<kVec>(
      r, 0, r.len, [t1](uint32_t k) { return (k >> 20) == t1; }, thr, above1, kTopK - remaining, remaining, 0, 0, pt,
      dst, L.scan);
}

struct TopkArgs {
  const float* score;
  int64_t score_stride;
  int width;
  const int16_t* mask;
  int64_t mask_stride;
  const int32_t* lengths;
  int rows;
  const int32_t* pt;
  int64_t pt_stride;
  int pt_cols;  // entries per page-table row; tokens past it map to -1
  const int32_t* cu;
  int n_req;
  int32_t* out;
  // split / pre workspace
  int S;
  int32_t* ghist;   // [rows][kBins]          (pass 1)
  int32_t* gcnt;    // [rows][2] = (positives, zeros)
  int32_t* cnt_ac;  // [rows][S][2] = (|A_s|, |C_s|)
  int32_t* list_a;  // [rows][S][kTopK]
  int32_t* list_c;  // [rows][S][kCapSlice][2] = (key, token)
};

__device__ __forceinline__ RowSrc row_src(const TopkArgs& a, int row, int len) {
  RowSrc r;
  r.vals = a.score + static_cast<int64_t>(row) * a.score_stride;
  r.mask = a.mask ? a.mask + static_cast<int64_t>(row) * a.mask_stride : nullptr;
  r.len = len;
  return r;
}

__device__ __forceinline__ int row_len(const TopkArgs& a, int row) {
  const int l = a.lengths[row];
  return l < 0 ? 0 : (l < a.width ? l : a.width);
}

__device__ __forceinline__ PtRow pt_row(const TopkArgs& a, int row) {
  PtRow p;
  p.p = a.pt + static_cast<int64_t>(pt_row_of(row, a.cu, a.n_req)) * a.pt_stride;
  p.cols = a.pt_cols;
  return p;
}

__device__ __forceinline__ void copy_short_row(const PtRow& pt, int32_t* dst, int len) {
  for (int i = threadIdx.x; i < kTopK; i += kTk) dst[i] = i < len ? pt[i] : -1;
}

// One CTA per row.  kPre: pass 1 (histogram + counts) comes from a.ghist / a.gcnt.
template <bool kVec, bool kPre>
__global__ __launch_bounds__(kTk) void topk_single_kernel(const TopkArgs a) {
  __shared__ TopkLds L;
  const int row = blockIdx.x;
  const int len = row_len(a, row);
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  if (len <= kTopK) {
    copy_short_row(pt, dst, len);
    return;
  }
  const RowSrc r = row_src(a, row, len);

  int pos, zeros;
  if constexpr (kPre) {
    const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
    for (int i = threadIdx.x; i < kBins; i += kTk) L.hist[i] = gh[i];
    pos = a.gcnt[2 * row];
    zeros = a.gcnt[2 * row + 1];
    __syncthreads();
  } else {
    zero_lds(L.hist, kBins);
    __syncthreads();
    pass_hist<kVec>(r, 0, len, L.hist, L.red, pos, zeros);
    if (threadIdx.x == 0 && zeros) L.hist[kZeroBin] += zeros;
    __syncthreads();
  }

  if (pos <= kTopK && pos + zeros >= kTopK) {
    // Threshold is +0: every positive token plus the lowest-index zeros.
    const int remaining = kTopK - pos;
    emit_range<kVec>(
        r, 0, len, [](uint32_t) { return true; }, kZeroKey, 0, pos, remaining, 0, 0, pt, dst, L.scan);
    return;
  }
  find_threshold<kBins>(L.hist, kTopK, L.wtot, L.res);
  const uint32_t t1 = static_cast<uint32_t>(L.res[0]);
  const int above1 = L.res[1];

  // Pass 2: list A straight to the output, list C into LDS, both in token order.
  int a_pos = 0, c_pos = 0, parity = 0;
  for (int base = 0; base < len; base += kStep) {
    const int i0 = base + static_cast<int>(threadIdx.x) * 4;
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(r, i0, k);
    int na = 0, nc = 0;
    bool fa[4], fc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool v = (valid >> j) & 1u;
      fa[j] = v && (k[j] >> 20) > t1;
      fc[j] = v && (k[j] >> 20) == t1;
      na += fa[j];
      nc += fc[j];
    }
    int pa, pc, ta, tc;
    block_prefix2(na, nc, pa, pc, ta, tc, L.scan, parity);
    parity ^= 1;
    pa += a_pos;
    pc += c_pos;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (fa[j]) put(dst, pa, pt[i0 + j]);
      if (fc[j] && pc < kCapC) {
        L.ckey[pc] = k[j];
        L.cidx[pc] = i0 + j;
      }
      pa += fa[j];
      pc += fc[j];
    }
    a_pos += ta;
    c_pos += tc;
  }
  __syncthreads();
  if (c_pos <= kCapC) resolve_lds(L, c_pos, t1, above1, pt, dst);
  else resolve_rescan<kVec>(L, r, t1, above1, pt, dst);
}

// ---------------------------------------------------------------------------------------------
// Split variant.  Slices are whole kStep blocks; CTAs are slice-major (blockIdx = s * rows + row)
// so the live slices of consecutive rows spread over the XCDs.
__device__ __forceinline__ int slice_len(int len, int S) {
  const int per = (len + S - 1) / S;
  return (per + kStep - 1) / kStep * kStep;
}

__global__ __launch_bounds__(256) void topk_zero_kernel(int32_t* __restrict__ ghist, int32_t* __restrict__ gcnt) {
  const int row = blockIdx.x;
  int4* g = reinterpret_cast<int4*>(ghist + static_cast<int64_t>(row) * kBins);
  for (int i = threadIdx.x; i < kBins / 4; i += 256) g[i] = make_int4(0, 0, 0, 0);
  if (threadIdx.x < 2) gcnt[2 * row + threadIdx.x] = 0;
}

template <bool kVec>
__global__ __launch_bounds__(kTk) void topk_split_hist_kernel(const TopkArgs a) {
  __shared__ int hist[kBins];
  __shared__ int red[kTkWaves];
  const int row = blockIdx.x % a.rows;
  const int s = blockIdx.x / a.rows;
  const int len = row_len(a, row);
  if (len <= kTopK) return;
  const int sl = slice_len(len, a.S);
  const int begin = s * sl;
  if (begin >= len) return;
  const int end = min(begin + sl, len);
  zero_lds(hist, kBins);
  __syncthreads();
  int pos, zeros;
  pass_hist<kVec>(row_src(a, row, len), begin, end, hist, red, pos, zeros);
  int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
  for (int i = threadIdx.x; i < kBins; i += kTk) {
    const int c = hist[i] + (i == kZeroBin ? zeros : 0);
    if (c) atomicAdd(&gh[i], c);
  }
  if (threadIdx.x == 0) {
    if (pos) atomicAdd(&a.gcnt[2 * row], pos);
    if (zeros) atomicAdd(&a.gcnt[2 * row + 1], zeros);
  }
}

// Per slice: ordered compaction into list A (certain) and list C (threshold candidates).
template <bool kVec>
__global__ __launch_bounds__(kTk) void topk_split_compact_kernel(const TopkArgs a) {
  __shared__ int hist[kBins];
  __shared__ int2 scan[2 * kTkWaves];
  __shared__ int wtot[kTkWaves];
  __shared__ int res[2];
  const int row = blockIdx.x % a.rows;
  const int s = blockIdx.x / a.rows;
  const int len = row_len(a, row);
  if (len <= kTopK) return;
  const int sl = slice_len(len, a.S);
  const int begin = s * sl;
  if (begin >= len) return;
  const int end = min(begin + sl, len);
  const int pos = a.gcnt[2 * row];
  const int zeros = a.gcnt[2 * row + 1];
  const bool fast = pos <= kTopK && pos + zeros >= kTopK;
  uint32_t t1 = 0;
  int cap_c = kCapSlice;
  if (fast) {
    cap_c = min(kCapSlice, kTopK - pos);  // only the first `remaining` zeros can be selected
  } else {
    const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
    for (int i = threadIdx.x; i < kBins; i += kTk) hist[i] = gh[i];
    __syncthreads();
    find_threshold<kBins>(hist, kTopK, wtot, res);
    t1 = static_cast<uint32_t>(res[0]);
  }
  const int64_t slot = static_cast<int64_t>(row) * a.S + s;
  int32_t* la = a.list_a + slot * kTopK;
  int32_t* lc = a.list_c + slot * kCapSlice * 2;
  RowSrc r = row_src(a, row, end);
  int a_pos = 0, c_pos = 0, parity = 0;
  for (int base = begin; base < end; base += kStep) {
    const int i0 = base + static_cast<int>(threadIdx.x) * 4;
    uint32_t k[4];
    const uint32_t valid = load_keys4<kVec>(r, i0, k);
    int na = 0, nc = 0;
    bool fa[4], fc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool v = (valid >> j) & 1u;
      fa[j] = v && (fast ? k[j] > kZeroKey : (k[j] >> 20) > t1);
      fc[j] = v && (fast ? k[j] == kZeroKey : (k[j] >> 20) == t1);
      na += fa[j];
      nc += fc[j];
    }
    int pa, pc, ta, tc;
    block_prefix2(na, nc, pa, pc, ta, tc, scan, parity);
    parity ^= 1;
    pa += a_pos;
    pc += c_pos;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (fa[j] && pa < kTopK) la[pa] = i0 + j;
      if (fc[j] && pc < cap_c) {
        lc[2 * pc] = static_cast<int>(k[j]);
        lc[2 * pc + 1] = i0 + j;
      }
      pa += fa[j];
      pc += fc[j];
    }
    a_pos += ta;
    c_pos += tc;
  }
  if (threadIdx.x == 0) {
    a.cnt_ac[2 * slot] = a_pos;
    a.cnt_ac[2 * slot + 1] = c_pos;
  }
}

// One CTA per row: merges the slices' lists, resolves the threshold, writes the output.
template <bool kVec>
__global__ __launch_bounds__(kTk) void topk_split_finish_kernel(const TopkArgs a) {
  __shared__ TopkLds L;
  __shared__ int s_pre[2 * kMaxSplit + 2];
  const int row = blockIdx.x;
  const int len = row_len(a, row);
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  if (len <= kTopK) {
    copy_short_row(pt, dst, len);
    return;
  }
  const int sl = slice_len(len, a.S);
  const int n_sl = (len + sl - 1) / sl;
  const int pos = a.gcnt[2 * row];
  const int zeros = a.gcnt[2 * row + 1];
  const bool fast = pos <= kTopK && pos + zeros >= kTopK;
  const int32_t* cnt = a.cnt_ac + static_cast<int64_t>(row) * a.S * 2;
  if (threadIdx.x == 0) {
    // Exclusive prefixes of |A_s| and |C_s| over slices; overflow flag at the end.
    int pa = 0, pc = 0, over = 0;
    for (int s = 0; s < n_sl; ++s) {
      s_pre[2 * s] = pa;
      s_pre[2 * s + 1] = pc;
      pa += cnt[2 * s];
      const int c = cnt[2 * s + 1];
      over |= !fast && c > kCapSlice;
      pc += c;
    }
    s_pre[2 * n_sl] = pa;
    s_pre[2 * n_sl + 1] = over || (!fast && pc > kCapC) ? -1 : pc;
  }
  __syncthreads();
  const int n_a = s_pre[2 * n_sl];
  const int n_c = s_pre[2 * n_sl + 1];

  // List A (already in token order per slice) -> output positions [0, n_a).
  for (int s = 0; s < n_sl; ++s) {
    const int32_t* la = a.list_a + (static_cast<int64_t>(row) * a.S + s) * kTopK;
    const int m = min(cnt[2 * s], kTopK);
    const int off = s_pre[2 * s];
    for (int i = threadIdx.x; i < m; i += kTk) put(dst, off + i, pt[la[i]]);
  }
  if (fast) {
    // Ties are zeros: the first (2048 - pos) of the slices' zero lists, in slice order.
    const int remaining = kTopK - pos;
    for (int s = 0; s < n_sl; ++s) {
      const int32_t* lc = a.list_c + (static_cast<int64_t>(row) * a.S + s) * kCapSlice * 2;
      const int off = s_pre[2 * s + 1];
      const int m = min(cnt[2 * s + 1], kCapSlice);
      for (int i = threadIdx.x; i < m; i += kTk)
        if (off + i < remaining) put(dst, pos + off + i, pt[lc[2 * i + 1]]);
    }
    return;
  }
  // Non-fast: t1 from the global histogram (same as the compact kernels computed).
  const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
  for (int i = threadIdx.x; i < kBins; i += kTk) L.hist[i] = gh[i];
  __syncthreads();
  find_threshold<kBins>(L.hist, kTopK, L.wtot, L.res);
  const uint32_t t1 = static_cast<uint32_t>(L.res[0]);
  const int above1 = L.res[1];
  if (n_c >= 0) {
    for (int s = 0; s < n_sl; ++s) {
      const int32_t* lc = a.list_c + (static_cast<int64_t>(row) * a.S + s) * kCapSlice * 2;
      const int off = s_pre[2 * s + 1];
      const int m = cnt[2 * s + 1];
      for (int i = threadIdx.x; i < m; i += kTk) {
        L.ckey[off + i] = static_cast<uint32_t>(lc[2 * i]);
        L.cidx[off + i] = lc[2 * i + 1];
      }
    }
    __syncthreads();
    resolve_lds(L, n_c, t1, above1, pt, dst);
  } else {
    resolve_rescan<kVec>(L, row_src(a, row, len), t1, above1, pt, dst);
  }
}

int split_count(int64_t rows, int64_t width, int max_splits, int n_cu) {
  if (rows <= 0) return 1;
  int64_t s = (width + 2 * kStep - 1) / (2 * kStep);  // >= 8192 tokens per slice
  s = s < 1 ? 1 : s;
  const int64_t by_cu = n_cu / rows;
  s = s < by_cu ? s : by_cu;
  const int64_t cap = max_splits < kMaxSplit ? max_splits : kMaxSplit;
  s = s < cap ? s : cap;
  return static_cast<int>(s < 1 ? 1 : s);
}

struct WsLayout {
  size_t ghist, gcnt, cnt_ac, list_a, list_c, total;
};

WsLayout ws_layout(int64_t rows, int S) {
  WsLayout l;
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.ghist = take(sizeof(int32_t) * rows * kBins);
  l.gcnt = take(sizeof(int32_t) * rows * 2);
  l.cnt_ac = take(sizeof(int32_t) * rows * S * 2);
  l.list_a = take(sizeof(int32_t) * rows * S * kTopK);
  l.list_c = take(sizeof(int32_t) * rows * S * kCapSlice * 2);
  l.total = off;
  return l;
}

int topk_common(const float* score, int64_t score_stride, int64_t width, const int16_t* mask, int64_t mask_stride,
                const int32_t* lengths, int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu, const int32_t* pre_hist,
                void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream, const char* who) {
  DSA_REQUIRE(rows >= 0 && rows <= 0x7FFFFFFF, "%s: rows out of range", who);
  DSA_REQUIRE(width >= 0 && width <= 0x7FFFFFFF, "%s: width out of range", who);
  if (rows == 0) return ok();
  DSA_REQUIRE(score && lengths && page_table && out, "%s: null pointer", who);
  DSA_REQUIRE(score_stride >= width, "%s: score_stride < width", who);
  DSA_REQUIRE(mask == nullptr || mask_stride >= (width + 15) / 16, "%s: mask_stride < ceil(width / 16)", who);
  DSA_REQUIRE(cu_seqlens_q == nullptr || n_req >= 1, "%s: cu_seqlens_q needs n_req >= 1", who);
  DSA_REQUIRE(max_splits >= 1, "%s: max_splits must be >= 1", who);
  DSA_REQUIRE(pt_cols >= 0 && pt_stride >= pt_cols, "%s: page-table row stride < its entries per row", who);
  const bool vec = width % 4 == 0 && score_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(score) & 15u) == 0;

  TopkArgs a;
  a.score = score;
  a.score_stride = score_stride;
  a.width = static_cast<int>(width);
  a.mask = mask;
  a.mask_stride = mask_stride;
  a.lengths = lengths;
  a.rows = static_cast<int>(rows);
  a.pt = page_table;
  a.pt_stride = pt_stride;
  a.pt_cols = static_cast<int>(pt_cols < width ? pt_cols : width);
  a.cu = cu_seqlens_q;
  a.n_req = static_cast<int>(n_req);
  a.out = out;
  const int S = split_count(rows, width, max_splits, n_cu);
  a.S = S;
  a.ghist = a.gcnt = a.cnt_ac = a.list_a = a.list_c = nullptr;
  const dim3 grid_rows(static_cast<uint32_t>(rows));

  if (pre_hist != nullptr) {
    a.ghist = const_cast<int32_t*>(pre_hist);
    a.gcnt = const_cast<int32_t*>(pre_hist) + 2 * rows * kBins;
  }
  if (S <= 1) {
    if (pre_hist) {
      if (vec) hipLaunchKernelGGL((topk_single_kernel<true, true>), grid_rows, dim3(kTk), 0, stream, a);
      else hipLaunchKernelGGL((topk_single_kernel<false, true>), grid_rows, dim3(kTk), 0, stream, a);
    } else {
      if (vec) hipLaunchKernelGGL((topk_single_kernel<true, false>), grid_rows, dim3(kTk), 0, stream, a);
      else hipLaunchKernelGGL((topk_single_kernel<false, false>), grid_rows, dim3(kTk), 0, stream, a);
    }
    return check_launch(who);
  }
  const WsLayout l = ws_layout(rows, S);
  DSA_REQUIRE(workspace != nullptr && workspace_bytes >= l.total,
              "%s: workspace of %zu bytes is smaller than the %zu required", who, workspace_bytes, l.total);
  DSA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "%s: workspace must be 16-B aligned", who);
  char* ws = static_cast<char*>(workspace);
  if (!pre_hist) {
    a.ghist = reinterpret_cast<int32_t*>(ws + l.ghist);
    a.gcnt = reinterpret_cast<int32_t*>(ws + l.gcnt);
  }
  a.cnt_ac = reinterpret_cast<int32_t*>(ws + l.cnt_ac);
  a.list_a = reinterpret_cast<int32_t*>(ws + l.list_a);
  a.list_c = reinterpret_cast<int32_t*>(ws + l.list_c);
  const dim3 grid_split(static_cast<uint32_t>(rows * S));
  if (!pre_hist) {
    hipLaunchKernelGGL(topk_zero_kernel, grid_rows, dim3(256), 0, stream, a.ghist, a.gcnt);
    if (vec) hipLaunchKernelGGL((topk_split_hist_kernel<true>), grid_split, dim3(kTk), 0, stream, a);
    else hipLaunchKernelGGL((topk_split_hist_kernel<false>), grid_split, dim3(kTk), 0, stream, a);
  }
  if (vec) {
    hipLaunchKernelGGL((topk_split_compact_kernel<true>), grid_split, dim3(kTk), 0, stream, a);
    hipLaunchKernelGGL((topk_split_finish_kernel<true>), grid_rows, dim3(kTk), 0, stream, a);
  } else {
    hipLaunchKernelGGL((topk_split_compact_kernel<false>), grid_split, dim3(kTk), 0, stream, a);
    hipLaunchKernelGGL((topk_split_finish_kernel<false>), grid_rows, dim3(kTk), 0, stream, a);
  }
  return check_launch(who);
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_topk_workspace_bytes(int64_t rows, int64_t width, int max_splits, int n_cu) {
  const int S = split_count(rows, width, max_splits < 1 ? 1 : max_splits, n_cu);
  if (S <= 1 || rows <= 0) return 0;
  return ws_layout(rows, S).total;
}

extern "C" int dsa_topk_transform(const float* score, int64_t score_stride, int64_t width, const int16_t* mask,
                                  int64_t mask_stride, const int32_t* lengths, int64_t rows,
                                  const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                                  const int32_t* cu_seqlens_q,
                                  int64_t n_req, int max_splits, int n_cu, void* workspace, size_t workspace_bytes,
                                  int32_t* out, hipStream_t stream) {
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, nullptr, workspace, workspace_bytes, out, stream,
                     "dsa_topk_transform");
}

extern "C" int dsa_topk_transform_pre(const float* score, int64_t score_stride, int64_t width, const int16_t* mask,
                                      int64_t mask_stride, const int32_t* lengths, int64_t rows,
                                      const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                                      const int32_t* cu_seqlens_q,
                                      int64_t n_req, int max_splits, int n_cu, const int32_t* hist_ws,
                                      void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream) {
  DSA_REQUIRE(hist_ws != nullptr, "dsa_topk_transform_pre: hist_ws is null");
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, hist_ws, workspace, workspace_bytes, out, stream,
                     "dsa_topk_transform_pre");
}
