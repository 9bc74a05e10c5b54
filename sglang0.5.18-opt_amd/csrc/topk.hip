// Exact top-2048 + page-table transform over (sparse-mask) indexer logits, gfx950.
//
// Contract (hcu_ops/csrc/sparse_mask_topk.cu:1-22,141-349): per row, the 2048 tokens t < len
// with the largest keys, ties at the threshold to the lower t; masked-out tokens are +0;
// rows with len <= 2048 copy page_table[0:len] and pad with -1.  Only the set is the contract
// (the order within a row is unspecified here, as it differs between the reference's variants).
//
// Algorithm (this file's own; radix digits 12/12/8 of the 32-bit key):
//   pass 1   histogram of key[31:20] over the nonzero tokens plus positive / zero counts (or
//            taken from the logits kernel).  positives <= 2048 <= positives + zeros means the
//            threshold is +0 (sparse fast path).  Otherwise the threshold digit t1 follows.
//   collect  one unordered pass over the row: tokens above bin t1 (or positive, fast path) are
//            written straight to the output, tokens in bin t1 become candidates (key, token);
//            positions come from wave-aggregated LDS atomics, so the streaming loop has no
//            barriers and keeps several loads in flight per lane.
//   resolve  the candidates (in LDS) go through the three digit passes to the exact threshold
//            key and the number `remaining` of threshold ties to take.  If there are more ties
//            than that, a second radix select over ~token among the ties keeps the lowest
//            indices.  Fast path: the first `remaining` zeros come from an ordered scan of the
//            row's prefix, which stops as soon as enough were found.
//   overflow candidates that do not fit in LDS are resolved by re-reading the row.
// Few rows: S CTAs per row run pass 1 (global histogram) and the collection of one slice each;
// one CTA per row then merges the slices' candidates and resolves.  Many rows: one CTA per row
// does everything.  No host synchronisation; launch shapes depend only on (rows, width,
// splits), so the whole path can be captured in a hipGraph.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kTk = 1024;       // threads of the single / finish CTAs
constexpr int kTs = 256;        // threads of the split pass-1 / collect CTAs
constexpr int kCapC = 8192;     // candidates a row can resolve in LDS
constexpr int kCapSlice = 4096; // candidates one collect CTA stages (and stores per slice)
constexpr int kMaxSplit = 64;
constexpr int kUnroll = 4;      // float4 groups in flight per lane

struct RowSrc {
  const float* vals;
  const int16_t* mask;  // nullable: all scores below len valid
  int len;
};

// Keys of tokens [i0, i0 + 4) (i0 % 4 == 0) and the bitmask of those below r.len.  Past the
// end the loads are redirected to token 0, so they stay inside the row.
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

template <int NT>
__device__ __forceinline__ int block_sum(int x, int* s_red) {
  constexpr int W = NT / kWave;
  x = wave_sum(x);
  if (lane_id() == 0) s_red[threadIdx.x >> 6] = x;
  __syncthreads();
  int s = 0;
#pragma unroll
  for (int v = 0; v < W; ++v) s += s_red[v];
  __syncthreads();
  return s;
}

// Block-exclusive prefix (thread order) of a per-thread count in [0, 7]; one barrier, with the
// wave totals double-buffered by `parity` so back-to-back calls do not race.
template <int NT>
__device__ __forceinline__ int block_prefix(int c, int& total, int* s_scan, int parity) {
  constexpr int W = NT / kWave;
  int wt;
  const int x = wave_prefix_small(c, wt);
  const int w = threadIdx.x >> 6;
  int* buf = s_scan + parity * W;
  if (lane_id() == 0) buf[w] = wt;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int v = 0; v < W; ++v) {
    before += v < w ? buf[v] : 0;
    tot += buf[v];
  }
  total = tot;
  return before + x;
}

// Finds bin t with suffix(t) >= need > suffix(t + 1); s_res = {t, suffix(t + 1)} ({0, 0} if the
// histogram holds fewer than `need`, which consistent inputs never do).  Ends with a barrier.
template <int NB, int NT>
__device__ void find_threshold(const int* hist, int need, int* s_wtot, int* s_res) {
  constexpr int W = NT / kWave;
  constexpr int BPT = NB >= NT ? NB / NT : 1;
  constexpr int ACTIVE = NB / BPT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  if (tid == 0) {
    s_res[0] = 0;
    s_res[1] = 0;
  }
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
#pragma unroll
  for (int v = 0; v < W; ++v) after += v > w ? s_wtot[v] : 0;
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

template <int NT>
__device__ __forceinline__ void zero_lds(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += NT) p[i] = 0;
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

// Threshold facts of a row from its pass-1 histogram: fast path, digit t1, tokens above t1.
struct Meta {
  bool fast;
  uint32_t t1;
  int above1;
  int pos;
};

template <int NT>
__device__ Meta row_meta(const int* hist_lds, int pos, int zeros, int* s_wtot, int* s_res) {
  Meta m;
  m.pos = pos;
  m.fast = pos <= kTopK && pos + zeros >= kTopK;
  m.t1 = 0;
  m.above1 = pos;
  if (!m.fast) {
    find_threshold<kBins, NT>(hist_lds, kTopK, s_wtot, s_res);
    m.t1 = static_cast<uint32_t>(s_res[0]);
    m.above1 = s_res[1];
  }
  return m;
}

// Pass 1 over [begin, end) of the row into an LDS histogram (zeros counted, not binned);
// returns the range's positive / zero counts (block-uniform).
template <bool kVec, int NT>
__device__ void pass_hist(const RowSrc& r, int begin, int end, int* hist, int* s_red, int& pos, int& zeros) {
  RowSrc rr = r;
  rr.len = end;
  int zc = 0, pc = 0;
  for (int b = begin + static_cast<int>(threadIdx.x) * 4; b < end; b += NT * 4 * kUnroll) {
    uint32_t k[kUnroll][4];
    uint32_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = load_keys4<kVec>(rr, b + u * NT * 4, k[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if ((v[u] >> j) & 1u) {
          if (k[u][j] == kZeroKey) {
            ++zc;
          } else {
            pc += k[u][j] > kZeroKey;
            atomicAdd(&hist[k[u][j] >> 20], 1);
          }
        }
      }
    }
  }
  pos = block_sum<NT>(pc, s_red);
  zeros = block_sum<NT>(zc, s_red);
}

// Candidate staging of a CTA: certain tokens (A) and threshold-bin candidates (C).
struct Stage {
  int* a;         // token indices, capacity cap_a
  uint32_t* ck;   // candidate keys, capacity cap_c
  int* ci;        // candidate tokens
  int* n_a;       // LDS counters
  int* n_c;
  int cap_a;
  int cap_c;
};

// One batch of kUnroll float4 groups per lane: loads first, use later.
struct Batch {
  uint32_t k[kUnroll][4];
  uint32_t v[kUnroll];
};

template <bool kVec, int NT>
__device__ __forceinline__ void load_batch(const RowSrc& rr, int b, Batch& x) {
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) x.v[u] = load_keys4<kVec>(rr, b + u * NT * 4, x.k[u]);
}

// A = keys above bin t1 (fast path: positive keys), C = keys in bin t1 (none on the fast
// path); wave-aggregated LDS atomics give the staging positions.
template <int NT>
__device__ __forceinline__ void process_batch(int b, const Batch& x, const Meta& m, const Stage& st) {
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    int na = 0, nc = 0;
    bool fa[4], fc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = (x.v[u] >> j) & 1u;
      const uint32_t d = x.k[u][j] >> 20;
      fa[j] = valid && (m.fast ? x.k[u][j] > kZeroKey : d > m.t1);
      fc[j] = valid && !m.fast && d == m.t1;
      na += fa[j];
      nc += fc[j];
    }
    int ta, tc;
    int pa = wave_prefix_small(na, ta);
    int pc = wave_prefix_small(nc, tc);
    if (ta | tc) {  // wave-uniform
      int base_a = 0, base_c = 0;
      if (lane_id() == 0) {
        if (ta) base_a = atomicAdd(st.n_a, ta);
        if (tc) base_c = atomicAdd(st.n_c, tc);
      }
      base_a = __shfl(base_a, 0);
      base_c = __shfl(base_c, 0);
      const int i0 = b + u * NT * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (fa[j]) {
          const int idx = base_a + pa++;
          if (idx < st.cap_a) st.a[idx] = i0 + j;
        }
        if (fc[j]) {
          const int idx = base_c + pc++;
          if (idx < st.cap_c) {
            st.ck[idx] = x.k[u][j];
            st.ci[idx] = i0 + j;
          }
        }
      }
    }
  }
}

// Unordered collection over [begin, end) (lane offsets added here).  `first`, if given, holds
// the already-loaded first batch (issued before the threshold was known, to overlap its latency).
template <bool kVec, int NT>
__device__ void collect(const RowSrc& r, int begin, int end, const Meta& m, const Stage& st, const Batch* first) {
  RowSrc rr = r;
  rr.len = end;
  int b = begin + static_cast<int>(threadIdx.x) * 4;
  if (first != nullptr) {
    process_batch<NT>(b, *first, m, st);
    b += NT * 4 * kUnroll;
  }
  for (; b < end; b += NT * 4 * kUnroll) {
    Batch x;
    load_batch<kVec, NT>(rr, b, x);
    process_batch<NT>(b, x, m, st);
  }
}

// Radix select over LDS members: the key `thr` such that `need` members have key >= thr and the
// number of members with key > thr (returned in above).  key_of(e) / member(e) index 0..n-1.
// d1_known >= 0: every member's key[31:20] is d1_known (the first digit pass is skipped).
template <int NT, typename KeyOf, typename Member>
__device__ uint32_t radix_select(int n, int need, KeyOf key_of, Member member, int* hist, int* s_wtot, int* s_res,
                                 int& above, int d1_known = -1) {
  uint32_t d1;
  int ab = 0;
  int need2 = need;
  if (d1_known >= 0) {
    d1 = static_cast<uint32_t>(d1_known);
  } else {
    zero_lds<NT>(hist, kBins);
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += NT)
      if (member(e)) atomicAdd(&hist[key_of(e) >> 20], 1);
    __syncthreads();
    find_threshold<kBins, NT>(hist, need, s_wtot, s_res);
    d1 = static_cast<uint32_t>(s_res[0]);
    ab = s_res[1];
    need2 = need - s_res[1];
  }
  zero_lds<NT>(hist, kBins);
  __syncthreads();
  for (int e = threadIdx.x; e < n; e += NT) {
    if (!member(e)) continue;
    const uint32_t k = key_of(e);
    if ((k >> 20) == d1) atomicAdd(&hist[(k >> 8) & 0xFFFu], 1);
  }
  __syncthreads();
  find_threshold<kBins, NT>(hist, need2, s_wtot, s_res);
  const uint32_t p24 = (d1 << 12) | static_cast<uint32_t>(s_res[0]);
  ab += s_res[1];
  const int need3 = need2 - s_res[1];
  zero_lds<NT>(hist, 256);
  __syncthreads();
  for (int e = threadIdx.x; e < n; e += NT) {
    if (!member(e)) continue;
    const uint32_t k = key_of(e);
    if ((k >> 8) == p24) atomicAdd(&hist[k & 0xFFu], 1);
  }
  __syncthreads();
  find_threshold<256, NT>(hist, need3, s_wtot, s_res);
  above = ab + s_res[1];
  return (p24 << 8) | static_cast<uint32_t>(s_res[0]);
}

struct ResolveLds {
  int hist[kBins];
  uint32_t ck[kCapC];
  int ci[kCapC];
  int scan[2 * (kTk / kWave)];
  int wtot[kTk / kWave];
  int red[kTk / kWave];
  int res[2];
  int misc[4];
};

// Resolves the LDS candidates (all in bin t1, unordered) of a row whose above1 tokens above
// bin t1 are already in dst[0, above1).
__device__ void resolve_lds(ResolveLds& L, int n_c, uint32_t t1, int above1, const PtRow& pt, int32_t* dst) {
  const int need1 = kTopK - above1;
  int gt;
  const uint32_t thr = radix_select<kTk>(
      n_c, need1, [&](int e) { return L.ck[e]; }, [](int) { return true; }, L.hist, L.wtot, L.res, gt,
      static_cast<int>(t1));
  const int remaining = need1 - gt;
  const int tie_base = kTopK - remaining;
  // ties at thr: all of them, unless there are more than `remaining` -- then the lowest tokens,
  // found by a radix select over ~token among the ties.
  int n_eq = 0;
  for (int e = threadIdx.x; e < n_c; e += kTk) n_eq += L.ck[e] == thr;
  n_eq = block_sum<kTk>(n_eq, L.red);
  uint32_t idx_thr = 0;  // ties kept: ~token >= idx_thr
  if (n_eq > remaining) {
    int unused;
    idx_thr = radix_select<kTk>(
        n_c, remaining, [&](int e) { return ~static_cast<uint32_t>(L.ci[e]); },
        [&](int e) { return L.ck[e] == thr; }, L.hist, L.wtot, L.res, unused);
  }
  int gt_pos = 0, tie_pos = 0, parity = 0;
  for (int base = 0; base < n_c; base += kTk) {
    const int e = base + static_cast<int>(threadIdx.x);
    const uint32_t key = e < n_c ? L.ck[e] : 0u;
    const bool g = e < n_c && key > thr;
    const bool q = e < n_c && key == thr && ~static_cast<uint32_t>(L.ci[e]) >= idx_thr;
    int tg, tq;
    const int pg = block_prefix<kTk>(g, tg, L.scan, parity);
    parity ^= 1;
    const int pq = block_prefix<kTk>(q, tq, L.scan, parity);
    parity ^= 1;
    if (g) put(dst, above1 + gt_pos + pg, pt[L.ci[e]]);
    if (q) put(dst, tie_base + tie_pos + pq, pt[L.ci[e]]);
    gt_pos += tg;
    tie_pos += tq;
  }
}

// Ordered scan of the row for the first `remaining` tokens with key == thr that pass `cond`
// (fast path: the zeros; rescan: the ties), written to dst[base + rank]; stops once enough
// were found unless gt is set.  gt: also write the keys > thr that pass cond to
// dst[gt_base + rank] (rescan only; then the whole row is scanned).
template <bool kVec, typename Cond>
__device__ void ordered_scan(const RowSrc& r, Cond cond, uint32_t thr, bool gt, int gt_base, int base, int remaining,
                             const PtRow& pt, int32_t* dst, int* s_scan) {
  int taken = 0, gt_pos = 0, parity = 0;
  for (int b0 = 0; b0 < r.len && (gt || taken < remaining); b0 += kTk * 4) {
    const int i0 = b0 + static_cast<int>(threadIdx.x) * 4;
    uint32_t k[4];
    const uint32_t v = load_keys4<kVec>(r, i0, k);
    int ne = 0, ng = 0;
    bool e[4], g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool c = ((v >> j) & 1u) && cond(k[j]);
      e[j] = c && k[j] == thr;
      g[j] = gt && c && k[j] > thr;
      ne += e[j];
      ng += g[j];
    }
    int te, tg;
    int pe = block_prefix<kTk>(ne, te, s_scan, parity);
    parity ^= 1;
    int pg = block_prefix<kTk>(ng, tg, s_scan, parity);
    parity ^= 1;
    pe += taken;
    pg += gt_pos;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (e[j] && pe < remaining) put(dst, base + pe, pt[i0 + j]);
      if (g[j]) put(dst, gt_base + pg, pt[i0 + j]);
      pe += e[j];
      pg += g[j];
    }
    taken += te;
    gt_pos += tg;
  }
}

// Threshold resolution by re-reading the row (candidates did not fit in LDS): digit passes over
// the tokens of bin t1, then an ordered emission of those above / at the threshold.
template <bool kVec>
__device__ void resolve_rescan(ResolveLds& L, const RowSrc& r, uint32_t t1, int above1, const PtRow& pt,
                               int32_t* dst) {
  const int need1 = kTopK - above1;
  zero_lds<kTk>(L.hist, kBins);
  __syncthreads();
  for (int b = static_cast<int>(threadIdx.x) * 4; b < r.len; b += kTk * 4) {
    uint32_t k[4];
    const uint32_t v = load_keys4<kVec>(r, b, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((v >> j) & 1u) && (k[j] >> 20) == t1) atomicAdd(&L.hist[(k[j] >> 8) & 0xFFFu], 1);
  }
  __syncthreads();
  find_threshold<kBins, kTk>(L.hist, need1, L.wtot, L.res);
  const uint32_t prefix24 = (t1 << 12) | static_cast<uint32_t>(L.res[0]);
  const int need2 = need1 - L.res[1];
  zero_lds<kTk>(L.hist, 256);
  __syncthreads();
  for (int b = static_cast<int>(threadIdx.x) * 4; b < r.len; b += kTk * 4) {
    uint32_t k[4];
    const uint32_t v = load_keys4<kVec>(r, b, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((v >> j) & 1u) && (k[j] >> 8) == prefix24) atomicAdd(&L.hist[k[j] & 0xFFu], 1);
  }
  __syncthreads();
  find_threshold<256, kTk>(L.hist, need2, L.wtot, L.res);
  const uint32_t thr = (prefix24 << 8) | static_cast<uint32_t>(L.res[0]);
  const int remaining = need2 - L.res[1];
  ordered_scan<kVec>(
      r, [t1](uint32_t k) { return (k >> 20) == t1; }, thr, true, above1, kTopK - remaining, remaining, pt, dst,
      L.scan);
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
  int S;
  int32_t* ghist;   // [rows][kBins]  pass-1 histogram
  int32_t* gcnt;    // [rows][2] = (positives, zeros)
  int32_t* ctr;     // per row: output positions used by the collect CTAs (row stride ctr_stride)
  int64_t ctr_stride;
  int32_t* c_cnt;   // [rows][S] candidates found per slice
  int32_t* c_list;  // [rows][S][kCapSlice][2] = (key, token)
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

template <int NT>
__device__ __forceinline__ void copy_short_row(const PtRow& pt, int32_t* dst, int len) {
  for (int i = threadIdx.x; i < kTopK; i += NT) dst[i] = i < len ? pt[i] : -1;
}

// ---------------------------------------------------------------------------------------------
// One CTA per row.  kPre: pass 1 (histogram + counts) comes from a.ghist / a.gcnt.
template <bool kVec, bool kPre>
__global__ __launch_bounds__(kTk) void topk_single_kernel(const TopkArgs a) {
  __shared__ ResolveLds L;
  __shared__ int s_a[kTopK];
  const int row = blockIdx.x;
  const int len = row_len(a, row);
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  if (len <= kTopK) {
    copy_short_row<kTk>(pt, dst, len);
    return;
  }
  const RowSrc r = row_src(a, row, len);
  int pos, zeros;
  Batch first;
  if constexpr (kPre) {
    load_batch<kVec, kTk>(r, static_cast<int>(threadIdx.x) * 4, first);  // overlaps the pass-1 loads
    const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
    for (int i = threadIdx.x; i < kBins; i += kTk) L.hist[i] = gh[i];
    pos = a.gcnt[2 * row];
    zeros = a.gcnt[2 * row + 1];
    __syncthreads();
  } else {
    zero_lds<kTk>(L.hist, kBins);
    __syncthreads();
    pass_hist<kVec, kTk>(r, 0, len, L.hist, L.red, pos, zeros);
    if (threadIdx.x == 0 && zeros) L.hist[kZeroBin] += zeros;
    __syncthreads();
  }
  const Meta m = row_meta<kTk>(L.hist, pos, zeros, L.wtot, L.res);
  if (threadIdx.x == 0) L.misc[0] = L.misc[1] = 0;
  __syncthreads();
  Stage st{s_a, L.ck, L.ci, &L.misc[0], &L.misc[1], kTopK, kCapC};
  collect<kVec, kTk>(r, 0, len, m, st, kPre ? &first : nullptr);
  __syncthreads();
  const int n_a = min(L.misc[0], kTopK);
  const int n_c = L.misc[1];
  for (int i = threadIdx.x; i < n_a; i += kTk) put(dst, i, pt[s_a[i]]);
  if (m.fast) {
    ordered_scan<kVec>(
        r, [](uint32_t) { return true; }, kZeroKey, false, 0, m.pos, kTopK - m.pos, pt, dst, L.scan);
  } else if (n_c <= kCapC) {
    resolve_lds(L, n_c, m.t1, m.above1, pt, dst);
  } else {
    resolve_rescan<kVec>(L, r, m.t1, m.above1, pt, dst);
  }
}

// ---------------------------------------------------------------------------------------------
// Split variant.  Slices are multiples of 1024 tokens; CTAs are slice-major (blockIdx = s *
// rows + row), so the slices of consecutive rows spread over the XCDs.
__device__ __forceinline__ int slice_len(int len, int S) {
  const int per = (len + S - 1) / S;
  return (per + 1023) / 1024 * 1024;
}

// Zeroes the pass-1 histogram, counts and output counters of the split path.
__global__ __launch_bounds__(256) void topk_zero_kernel(int32_t* __restrict__ ghist, int32_t* __restrict__ gcnt,
                                                        int32_t* __restrict__ ctr, int64_t ctr_stride) {
  const int row = blockIdx.x;
  int4* g = reinterpret_cast<int4*>(ghist + static_cast<int64_t>(row) * kBins);
  for (int i = threadIdx.x; i < kBins / 4; i += 256) g[i] = make_int4(0, 0, 0, 0);
  if (threadIdx.x < 2) gcnt[2 * row + threadIdx.x] = 0;
  if (threadIdx.x == 2) ctr[row * ctr_stride] = 0;
}

template <bool kVec>
__global__ __launch_bounds__(kTs) void topk_split_hist_kernel(const TopkArgs a) {
  __shared__ int hist[kBins];
  __shared__ int red[kTs / kWave];
  const int row = blockIdx.x % a.rows;
  const int s = blockIdx.x / a.rows;
  const int len = row_len(a, row);
  if (len <= kTopK) return;
  const int sl = slice_len(len, a.S);
  const int begin = s * sl;
  if (begin >= len) return;
  const int end = min(begin + sl, len);
  zero_lds<kTs>(hist, kBins);
  __syncthreads();
  int pos, zeros;
  pass_hist<kVec, kTs>(row_src(a, row, len), begin, end, hist, red, pos, zeros);
  int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
  for (int i = threadIdx.x; i < kBins; i += kTs) {
    const int c = hist[i] + (i == kZeroBin ? zeros : 0);
    if (c) atomicAdd(&gh[i], c);
  }
  if (threadIdx.x == 0) {
    if (pos) atomicAdd(&a.gcnt[2 * row], pos);
    if (zeros) atomicAdd(&a.gcnt[2 * row + 1], zeros);
  }
}

// Per slice: unordered collection; A goes straight to the output through one global atomic
// per CTA, C is stored in the slice's candidate list.
template <bool kVec>
__global__ __launch_bounds__(kTs) void topk_split_collect_kernel(const TopkArgs a) {
  __shared__ int hist[kBins];
  __shared__ int s_a[kTopK];
  __shared__ uint32_t s_ck[kCapSlice];
  __shared__ int s_ci[kCapSlice];
  __shared__ int s_wtot[kTs / kWave];
  __shared__ int s_res[2];
  __shared__ int s_n[3];
  const int row = blockIdx.x % a.rows;
  const int s = blockIdx.x / a.rows;
  const int len = row_len(a, row);
  if (len <= kTopK) return;
  const int sl = slice_len(len, a.S);
  const int begin = s * sl;
  if (begin >= len) return;
  const int end = min(begin + sl, len);
  RowSrc r = row_src(a, row, end);
  Batch first;
  load_batch<kVec, kTs>(r, begin + static_cast<int>(threadIdx.x) * 4, first);  // overlaps the pass-1 loads
  const int pos = a.gcnt[2 * row];
  const int zeros = a.gcnt[2 * row + 1];
  const bool fast = pos <= kTopK && pos + zeros >= kTopK;
  if (!fast) {
    const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
    for (int i = threadIdx.x; i < kBins; i += kTs) hist[i] = gh[i];
  }
  if (threadIdx.x == 0) s_n[0] = s_n[1] = 0;
  __syncthreads();
  const Meta m = row_meta<kTs>(hist, pos, zeros, s_wtot, s_res);
  Stage st{s_a, s_ck, s_ci, &s_n[0], &s_n[1], kTopK, kCapSlice};
  collect<kVec, kTs>(r, begin, end, m, st, &first);
  __syncthreads();
  const int n_a = min(s_n[0], kTopK);
  const int n_c = s_n[1];
  if (threadIdx.x == 0) {
    s_n[2] = n_a ? atomicAdd(a.ctr + row * a.ctr_stride, n_a) : 0;
    a.c_cnt[static_cast<int64_t>(row) * a.S + s] = n_c;
  }
  __syncthreads();
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  const int base = s_n[2];
  for (int i = threadIdx.x; i < n_a; i += kTs) put(dst, base + i, pt[s_a[i]]);
  int32_t* lc = a.c_list + (static_cast<int64_t>(row) * a.S + s) * kCapSlice * 2;
  const int m_c = min(n_c, kCapSlice);
  for (int i = threadIdx.x; i < m_c; i += kTs) {
    lc[2 * i] = static_cast<int>(s_ck[i]);
    lc[2 * i + 1] = s_ci[i];
  }
}

// One CTA per row: merges the slices' candidates and resolves the threshold (or, on the fast
// path, takes the lowest-index zeros).
template <bool kVec>
__global__ __launch_bounds__(kTk) void topk_split_finish_kernel(const TopkArgs a) {
  __shared__ ResolveLds L;
  __shared__ int s_off[kMaxSplit + 1];
  const int row = blockIdx.x;
  const int len = row_len(a, row);
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  if (len <= kTopK) {
    copy_short_row<kTk>(pt, dst, len);
    return;
  }
  const RowSrc r = row_src(a, row, len);
  const int pos = a.gcnt[2 * row];
  const int zeros = a.gcnt[2 * row + 1];
  if (pos <= kTopK && pos + zeros >= kTopK) {
    ordered_scan<kVec>(
        r, [](uint32_t) { return true; }, kZeroKey, false, 0, pos, kTopK - pos, pt, dst, L.scan);
    return;
  }
  const int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
  for (int i = threadIdx.x; i < kBins; i += kTk) L.hist[i] = gh[i];
  __syncthreads();
  const Meta m = row_meta<kTk>(L.hist, pos, zeros, L.wtot, L.res);
  const int sl = slice_len(len, a.S);
  const int n_sl = (len + sl - 1) / sl;
  if (threadIdx.x == 0) {
    int off = 0;
    bool over = false;
    for (int s = 0; s < n_sl; ++s) {
      const int c = a.c_cnt[static_cast<int64_t>(row) * a.S + s];
      s_off[s] = off;
      over |= c > kCapSlice;
      off += c;
    }
    s_off[n_sl] = over || off > kCapC ? -1 : off;
  }
  __syncthreads();
  const int n_c = s_off[n_sl];
  if (n_c < 0) {
    resolve_rescan<kVec>(L, r, m.t1, m.above1, pt, dst);
    return;
  }
  for (int s = 0; s < n_sl; ++s) {
    const int32_t* lc = a.c_list + (static_cast<int64_t>(row) * a.S + s) * kCapSlice * 2;
    const int off = s_off[s];
    const int cnt = (s + 1 < n_sl ? s_off[s + 1] : n_c) - off;
    for (int i = threadIdx.x; i < cnt; i += kTk) {
      L.ck[off + i] = static_cast<uint32_t>(lc[2 * i]);
      L.ci[off + i] = lc[2 * i + 1];
    }
  }
  __syncthreads();
  resolve_lds(L, n_c, m.t1, m.above1, pt, dst);
}

int split_count(int64_t rows, int64_t width, int max_splits, int n_cu) {
  if (rows <= 0) return 1;
  int64_t s = (width + 4095) / 4096;  // >= 4096 tokens per slice
  s = s < 1 ? 1 : s;
  const int64_t by_cu = (2 * static_cast<int64_t>(n_cu)) / rows;
  s = s < by_cu ? s : by_cu;
  const int64_t cap = max_splits < kMaxSplit ? max_splits : kMaxSplit;
  s = s < cap ? s : cap;
  return static_cast<int>(s < 1 ? 1 : s);
}

struct WsLayout {
  size_t ghist, gcnt, ctr, c_cnt, c_list, total;
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
  l.ctr = take(sizeof(int32_t) * rows);
  l.c_cnt = take(sizeof(int32_t) * rows * S);
  l.c_list = take(sizeof(int32_t) * rows * S * kCapSlice * 2);
  l.total = off;
  return l;
}

int topk_common(const float* score, int64_t score_stride, int64_t width, const int16_t* mask, int64_t mask_stride,
                const int32_t* lengths, int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu, int32_t* pre_hist,
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
  a.ghist = a.gcnt = a.ctr = a.c_cnt = a.c_list = nullptr;
  a.ctr_stride = 1;
  const dim3 grid_rows(static_cast<uint32_t>(rows));

  if (pre_hist != nullptr) {
    // [ghist1 rows*4096 | ghist2 rows*4096 | cnt rows*2]; word 0 of each ghist2 row is the row's
    // output counter (zeroed by the logits call that built pass 1).
    a.ghist = pre_hist;
    a.ctr = pre_hist + rows * kBins;
    a.ctr_stride = kBins;
    a.gcnt = pre_hist + 2 * rows * kBins;
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
    a.ctr = reinterpret_cast<int32_t*>(ws + l.ctr);
  }
  a.c_cnt = reinterpret_cast<int32_t*>(ws + l.c_cnt);
  a.c_list = reinterpret_cast<int32_t*>(ws + l.c_list);
  const dim3 grid_split(static_cast<uint32_t>(rows * S));
  if (!pre_hist) {
    hipLaunchKernelGGL(topk_zero_kernel, grid_rows, dim3(256), 0, stream, a.ghist, a.gcnt, a.ctr, a.ctr_stride);
    if (vec) hipLaunchKernelGGL((topk_split_hist_kernel<true>), grid_split, dim3(kTs), 0, stream, a);
    else hipLaunchKernelGGL((topk_split_hist_kernel<false>), grid_split, dim3(kTs), 0, stream, a);
  }
  if (vec) {
    hipLaunchKernelGGL((topk_split_collect_kernel<true>), grid_split, dim3(kTs), 0, stream, a);
    hipLaunchKernelGGL((topk_split_finish_kernel<true>), grid_rows, dim3(kTk), 0, stream, a);
  } else {
    hipLaunchKernelGGL((topk_split_collect_kernel<false>), grid_split, dim3(kTs), 0, stream, a);
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
                                  const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                                  void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream) {
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, nullptr, workspace, workspace_bytes, out, stream,
                     "dsa_topk_transform");
}

extern "C" int dsa_topk_transform_pre(const float* score, int64_t score_stride, int64_t width, const int16_t* mask,
                                      int64_t mask_stride, const int32_t* lengths, int64_t rows,
                                      const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                                      const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                                      int32_t* hist_ws, void* workspace, size_t workspace_bytes, int32_t* out,
                                      hipStream_t stream) {
  DSA_REQUIRE(hist_ws != nullptr, "dsa_topk_transform_pre: hist_ws is null");
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, hist_ws, workspace, workspace_bytes, out, stream,
                     "dsa_topk_transform_pre");
}
