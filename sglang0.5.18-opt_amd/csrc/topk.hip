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
// Few rows: S CTAs per row collect one slice each (taking pass 1 from the logits kernel, or
// from a split pass-1 kernel), publish their A tokens and candidates through per-row global
// counters, and the last CTA of the row to finish (device-scope atomic) resolves the threshold.
// Many rows: one CTA per row does everything.  No host synchronisation; launch shapes depend
// only on (rows, width, splits), so the whole path can be captured in a hipGraph.
#include "dsa_common.h"

namespace dsa {
namespace {

constexpr int kTk = 1024;   // threads of the one-CTA-per-row kernel
constexpr int kTs = 512;    // threads of the split collect / resolve CTAs
constexpr int kCapC = 8192; // candidates the one-CTA-per-row kernel resolves in LDS
constexpr int kCapS = 4096; // candidates of a row the split kernel resolves in LDS
constexpr int kMaxSplit = 64;
constexpr int kUnroll = 4;  // float4 groups per lane in one batch (two batches in flight)

struct RowSrc {
  const float* vals;
  const int16_t* mask;  // never null: without a mask it points at the scores and mask_or = 0xFFFF
  uint32_t mask_or;
  int len;
};

// Raw scores of tokens [i0, i0 + 4) (i0 % 4 == 0) and the mask word holding their bits, loaded
// but not yet used, so that a batch of them stays in flight.  Past the end the loads are
// redirected to token 0, so they stay inside the row.
struct Quad {
  float v[4];
  uint16_t mw;
};

template <bool kVec>
__device__ __forceinline__ void load_quad(const RowSrc& r, int i0, Quad& q) {
  const int safe = i0 < r.len ? i0 : 0;
  if constexpr (kVec) {
    const float4 f = *reinterpret_cast<const float4*>(r.vals + safe);
    q.v[0] = f.x;
    q.v[1] = f.y;
    q.v[2] = f.z;
    q.v[3] = f.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = safe + j;
      q.v[j] = r.vals[t < r.len ? t : r.len - 1];
    }
  }
  q.mw = static_cast<uint16_t>(r.mask[safe >> 4]);  // unconditional: a dummy word without a mask
}

// Keys of a loaded quad (masked-out tokens are +0) and the bitmask of its tokens below r.len.
__device__ __forceinline__ uint32_t quad_keys(const RowSrc& r, int i0, const Quad& q, uint32_t (&k)[4]) {
  const int safe = i0 < r.len ? i0 : 0;
  const uint32_t m = ((q.mw | r.mask_or) >> (safe & 15)) & 0xFu;
#pragma unroll
  for (int j = 0; j < 4; ++j) k[j] = ((m >> j) & 1u) ? float_key(q.v[j]) : kZeroKey;
  const int rem = r.len - i0;
  const int nv = rem <= 0 ? 0 : (rem < 4 ? rem : 4);
  return (1u << nv) - 1u;
}

template <bool kVec>
__device__ __forceinline__ uint32_t load_keys4(const RowSrc& r, int i0, uint32_t (&k)[4]) {
  Quad q;
  load_quad<kVec>(r, i0, q);
  return quad_keys(r, i0, q, k);
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

// Finds bin t with suffix(t) >= need > suffix(t + 1) of a histogram held in registers (thread
// tid owns bins tid * BPT .. tid * BPT + BPT - 1); s_res = {t, suffix(t + 1), count of t} ({0, 0,
// 0} if the histogram holds fewer than `need`, which consistent inputs never do).  Ends with a
// barrier.
template <int NT, int BPT>
__device__ void find_threshold_regs(const int (&h)[BPT], int need, int* s_wtot, int* s_res) {
  constexpr int W = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  if (tid == 0) {
    s_res[0] = 0;
    s_res[1] = 0;
    s_res[2] = 0;
  }
  int s = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) s += h[j];
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
  if (suf >= need && suf_next < need) {
    int acc = suf_next;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      if (acc + h[j] >= need) {
        s_res[0] = tid * BPT + j;
        s_res[1] = acc;
        s_res[2] = h[j];
        break;
      }
      acc += h[j];
    }
  }
  __syncthreads();
}

// The same over an LDS histogram of NB bins.
template <int NB, int NT>
__device__ void find_threshold(const int* hist, int need, int* s_wtot, int* s_res) {
  constexpr int BPT = NB >= NT ? NB / NT : 1;
  constexpr int ACTIVE = NB / BPT;
  int h[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) h[j] = static_cast<int>(threadIdx.x) < ACTIVE ? hist[threadIdx.x * BPT + j] : 0;
  find_threshold_regs<NT, BPT>(h, need, s_wtot, s_res);
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

// Page-table entry of token t (-1 outside the row's entries).
struct PtRow {
  const int32_t* p;
  int cols;
  __device__ __forceinline__ int32_t operator[](int t) const {
    return static_cast<unsigned>(t) < static_cast<unsigned>(cols) ? p[t] : -1;
  }
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

// One batch: kUnroll quads per lane, NT * 4 tokens apart.
struct Batch {
  Quad q[kUnroll];
};

template <bool kVec, int NT>
__device__ __forceinline__ void load_batch(const RowSrc& rr, int b, Batch& x) {
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) load_quad<kVec>(rr, b + u * NT * 4, x.q[u]);
}

// Streams n_batches batches from lane offset b with two in flight: x0 / x1 hold the first two on
// entry (issued by the caller, possibly before other work), and each is reloaded right after
// fn(b, batch) used it -- no register copies, so the in-order load counter only ever waits for
// the batch being used.
template <bool kVec, int NT, typename Fn>
__device__ __forceinline__ void stream_batches(const RowSrc& rr, int b, int n_batches, Batch& x0, Batch& x1, Fn fn) {
  constexpr int kStep = NT * 4 * kUnroll;
  for (int i = 0; i < n_batches; i += 2) {
    fn(b, x0);
    if (i + 2 < n_batches) load_batch<kVec, NT>(rr, b + 2 * kStep, x0);
    if (i + 1 >= n_batches) break;
    fn(b + kStep, x1);
    if (i + 3 < n_batches) load_batch<kVec, NT>(rr, b + 3 * kStep, x1);
    b += 2 * kStep;
  }
}

// Pass 1 over [begin, end) (end > begin) of the row into the LDS histogram `hist` (zeroed here;
// zeros counted, not binned); returns the range's positive / zero counts (block-uniform).
template <bool kVec, int NT>
__device__ void pass_hist(const RowSrc& r, int begin, int end, int* hist, int* s_red, int& pos, int& zeros) {
  constexpr int kStep = NT * 4 * kUnroll;
  RowSrc rr = r;
  rr.len = end;
  const int b0 = begin + static_cast<int>(threadIdx.x) * 4;
  Batch x0, x1;
  load_batch<kVec, NT>(rr, b0, x0);
  load_batch<kVec, NT>(rr, b0 + kStep, x1);
  zero_lds<NT>(hist, kBins);  // while the first batches are in flight
  __syncthreads();
  int zc = 0, pc = 0;
  stream_batches<kVec, NT>(rr, b0, (end - begin + kStep - 1) / kStep, x0, x1, [&](int b, const Batch& x) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      uint32_t k[4];
      const uint32_t v = quad_keys(rr, b + u * NT * 4, x.q[u], k);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if ((v >> j) & 1u) {
          if (k[j] == kZeroKey) {
            ++zc;
          } else {
            pc += k[j] > kZeroKey;
            atomicAdd(&hist[k[j] >> 20], 1);
          }
        }
      }
    }
  });
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

// A = keys above bin t1 (fast path: positive keys), C = keys in bin t1 (none on the fast
// path).  A lane flags its (at most 16) hits of the batch in two bitmasks; one wave prefix per
// list and one wave-aggregated LDS atomic per list and batch give every hit its staging slot.
template <int NT>
__device__ __forceinline__ void process_batch(const RowSrc& rr, int b, const Batch& x, const Meta& m,
                                              const Stage& st) {
  static_assert(kUnroll * 4 <= 16, "hit masks hold 16 keys");
  uint32_t k[kUnroll][4];
  uint32_t fa = 0, fc = 0;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t v = quad_keys(rr, b + u * NT * 4, x.q[u], k[u]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = (v >> j) & 1u;
      const uint32_t d = k[u][j] >> 20;
      fa |= static_cast<uint32_t>(valid && (m.fast ? k[u][j] > kZeroKey : d > m.t1)) << (u * 4 + j);
      fc |= static_cast<uint32_t>(valid && !m.fast && d == m.t1) << (u * 4 + j);
    }
  }
  int ta, tc;
  int pa = wave_prefix_5(__popc(fa), ta);
  int pc = wave_prefix_5(__popc(fc), tc);
  if ((ta | tc) == 0) return;  // wave-uniform
  int base_a = 0, base_c = 0;
  if (lane_id() == 0) {
    if (ta) base_a = atomicAdd(st.n_a, ta);
    if (tc) base_c = atomicAdd(st.n_c, tc);
  }
  pa += uniform(base_a);
  pc += uniform(base_c);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = u * 4 + j;
      const int t = b + u * NT * 4 + j;
      if ((fa >> e) & 1u) {
        if (pa < st.cap_a) st.a[pa] = t;
        ++pa;
      }
      if ((fc >> e) & 1u) {
        if (pc < st.cap_c) {
          st.ck[pc] = k[u][j];
          st.ci[pc] = t;
        }
        ++pc;
      }
    }
  }
}

// Unordered collection of n_batches batches from lane offset b (x0 / x1: the first two, already
// issued).  Loads past rr.len are redirected inside the row and masked off.
template <bool kVec, int NT>
__device__ void collect(const RowSrc& rr, int b, int n_batches, const Meta& m, const Stage& st, Batch& x0,
                        Batch& x1) {
  stream_batches<kVec, NT>(rr, b, n_batches, x0, x1,
                           [&](int bb, const Batch& x) { process_batch<NT>(rr, bb, x, m, st); });
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

template <int NT, int CAP>
struct ResolveLds {
  int hist[kBins];
  uint32_t ck[CAP];
  int ci[CAP];
  int scan[2 * (NT / kWave)];
  int wtot[NT / kWave];
  int red[NT / kWave];
  int res[3];
  int misc[4];
};

// Resolves the LDS candidates (all in bin t1, unordered) of a row whose above1 tokens above
// bin t1 are already in dst[0, above1): digit passes over key[19:8] and key[7:0], then the
// ties at the threshold key, lowest tokens first.  The general path of resolve_lds.
template <int NT, int CAP>
__device__ void resolve_lds_radix(ResolveLds<NT, CAP>& L, int n_c, uint32_t t1, int above1, const PtRow& pt,
                                  int32_t* dst) {
  const int need1 = kTopK - above1;
  int gt;
  const uint32_t thr = radix_select<NT>(
      n_c, need1, [&](int e) { return L.ck[e]; }, [](int) { return true; }, L.hist, L.wtot, L.res, gt,
      static_cast<int>(t1));
  const int remaining = need1 - gt;
  const int tie_base = kTopK - remaining;
  // ties at thr: all of them, unless there are more than `remaining` -- then the lowest tokens,
  // found by a radix select over ~token among the ties.
  int n_eq = 0;
  for (int e = threadIdx.x; e < n_c; e += NT) n_eq += L.ck[e] == thr;
  n_eq = block_sum<NT>(n_eq, L.red);
  uint32_t idx_thr = 0;  // ties kept: ~token >= idx_thr
  if (n_eq > remaining) {
    int unused;
    idx_thr = radix_select<NT>(
        n_c, remaining, [&](int e) { return ~static_cast<uint32_t>(L.ci[e]); },
        [&](int e) { return L.ck[e] == thr; }, L.hist, L.wtot, L.res, unused);
  }
  int gt_pos = 0, tie_pos = 0, parity = 0;
  for (int base = 0; base < n_c; base += NT) {
    const int e = base + static_cast<int>(threadIdx.x);
    const uint32_t key = e < n_c ? L.ck[e] : 0u;
    const bool g = e < n_c && key > thr;
    const bool q = e < n_c && key == thr && ~static_cast<uint32_t>(L.ci[e]) >= idx_thr;
    int tg, tq;
    const int pg = block_prefix<NT>(g, tg, L.scan, parity);
    parity ^= 1;
    const int pq = block_prefix<NT>(q, tq, L.scan, parity);
    parity ^= 1;
    if (g) put(dst, above1 + gt_pos + pg, pt[L.ci[e]]);
    if (q) put(dst, tie_base + tie_pos + pq, pt[L.ci[e]]);
    gt_pos += tg;
    tie_pos += tq;
  }
}

// Resolves the LDS candidates (all in bin t1, unordered, n_c of them) of a row whose above1
// tokens above bin t1 are already in dst[0, above1).  One digit pass over key[19:8] splits them
// into certain ones (digit above the threshold digit d2, emitted at once) and the members of
// digit d2, which are few for any spread of values: each member's exact rank in (key desc,
// token asc) order decides it.  More members than threads (heavy ties) take the radix path.
template <int NT, int CAP>
__device__ void resolve_lds(ResolveLds<NT, CAP>& L, int n_c, uint32_t t1, int above1, const PtRow& pt, int32_t* dst) {
  const int need1 = kTopK - above1;
  zero_lds<NT>(L.hist, kBins);
  if (threadIdx.x == 0) L.misc[0] = L.misc[1] = 0;
  __syncthreads();
  for (int e = threadIdx.x; e < n_c; e += NT) atomicAdd(&L.hist[(L.ck[e] >> 8) & 0xFFFu], 1);
  __syncthreads();
  find_threshold<kBins, NT>(L.hist, need1, L.wtot, L.res);
  const uint32_t d2 = static_cast<uint32_t>(L.res[0]);
  const int above2 = L.res[1];
  const int n2 = L.res[2];
  if (n2 > NT) {  // block-uniform
    resolve_lds_radix(L, n_c, t1, above1, pt, dst);
    return;
  }
  const int need2 = need1 - above2;  // members to take
  // the histogram is consumed: its first 2 * NT words hold the members' keys and tokens
  uint32_t* mk = reinterpret_cast<uint32_t*>(L.hist);
  int* mt = L.hist + NT;
  for (int e = threadIdx.x; e < n_c; e += NT) {
    const uint32_t k = L.ck[e];
    const uint32_t d = (k >> 8) & 0xFFFu;
    if (d > d2) {
      put(dst, above1 + atomicAdd(&L.misc[0], 1), pt[L.ci[e]]);
    } else if (d == d2) {
      const int q = atomicAdd(&L.misc[1], 1);
      if (q < NT) {
        mk[q] = k;
        mt[q] = L.ci[e];
      }
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < n2) {
    const uint32_t k = mk[t];
    const int tok = mt[t];
    int rank = 0;
    for (int j = 0; j < n2; ++j) {
      const uint32_t kj = mk[j];
      rank += kj > k || (kj == k && mt[j] < tok);
    }
    if (rank < need2) put(dst, kTopK - need2 + rank, pt[tok]);
  }
}

// Ordered scan of the row for the first `remaining` tokens with key == thr that pass `cond`
// (fast path: the zeros; rescan: the ties), written to dst[base + rank]; stops once enough
// were found unless gt is set.  gt: also write the keys > thr that pass cond to
// dst[gt_base + rank] (rescan only; then the whole row is scanned).
template <bool kVec, int NT, typename Cond>
__device__ void ordered_scan(const RowSrc& r, Cond cond, uint32_t thr, bool gt, int gt_base, int base, int remaining,
                             const PtRow& pt, int32_t* dst, int* s_scan) {
  int taken = 0, gt_pos = 0, parity = 0;
  for (int b0 = 0; b0 < r.len && (gt || taken < remaining); b0 += NT * 4) {
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
    int pe = block_prefix<NT>(ne, te, s_scan, parity);
    parity ^= 1;
    int pg = block_prefix<NT>(ng, tg, s_scan, parity);
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
template <bool kVec, int NT, int CAP>
__device__ void resolve_rescan(ResolveLds<NT, CAP>& L, const RowSrc& r, uint32_t t1, int above1, const PtRow& pt,
                               int32_t* dst) {
  const int need1 = kTopK - above1;
  zero_lds<NT>(L.hist, kBins);
  __syncthreads();
  for (int b = static_cast<int>(threadIdx.x) * 4; b < r.len; b += NT * 4) {
    uint32_t k[4];
    const uint32_t v = load_keys4<kVec>(r, b, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((v >> j) & 1u) && (k[j] >> 20) == t1) atomicAdd(&L.hist[(k[j] >> 8) & 0xFFFu], 1);
  }
  __syncthreads();
  find_threshold<kBins, NT>(L.hist, need1, L.wtot, L.res);
  const uint32_t prefix24 = (t1 << 12) | static_cast<uint32_t>(L.res[0]);
  const int need2 = need1 - L.res[1];
  zero_lds<NT>(L.hist, 256);
  __syncthreads();
  for (int b = static_cast<int>(threadIdx.x) * 4; b < r.len; b += NT * 4) {
    uint32_t k[4];
    const uint32_t v = load_keys4<kVec>(r, b, k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((v >> j) & 1u) && (k[j] >> 8) == prefix24) atomicAdd(&L.hist[k[j] & 0xFFu], 1);
  }
  __syncthreads();
  find_threshold<256, NT>(L.hist, need2, L.wtot, L.res);
  const uint32_t thr = (prefix24 << 8) | static_cast<uint32_t>(L.res[0]);
  const int remaining = need2 - L.res[1];
  ordered_scan<kVec, NT>(
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
  int S;             // slices per row of the split pass-1 kernel
  int T;             // CTAs the balanced split kernel spreads the rows' tokens over
  int32_t* ghist;    // [rows][kBins]  pass-1 histogram
  int32_t* gcnt;     // [rows][2] = (positives, zeros)
  int32_t* ctr;      // per row (stride ctr_stride): [0] output slots taken, [1] candidates
                     // published, [2] slice CTAs finished -- zero before the split kernel
  int64_t ctr_stride;
  uint32_t* c_keys;  // [rows][kCapS] candidate keys published by the slice CTAs
  int32_t* c_tok;    // [rows][kCapS] their tokens
};

__device__ __forceinline__ RowSrc row_src(const TopkArgs& a, int row, int len) {
  RowSrc r;
  r.vals = a.score + static_cast<int64_t>(row) * a.score_stride;
  // without a mask, a dummy in-row address (word t/16 lies inside the row's first t floats)
  r.mask = a.mask ? a.mask + static_cast<int64_t>(row) * a.mask_stride : reinterpret_cast<const int16_t*>(r.vals);
  r.mask_or = a.mask ? 0u : 0xFFFFu;
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
  __shared__ ResolveLds<kTk, kCapC> L;
  __shared__ int s_a[kTopK];
  constexpr int kStep = kTk * 4 * kUnroll;
  const int row = blockIdx.x;
  const int len = row_len(a, row);
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  if (len <= kTopK) {
    copy_short_row<kTk>(pt, dst, len);
    return;
  }
  const RowSrc r = row_src(a, row, len);
  const int b0 = static_cast<int>(threadIdx.x) * 4;
  const int n_batches = (len + kStep - 1) / kStep;
  Batch x0, x1;
  Meta m;
  if constexpr (kPre) {
    // pass-1 slots (4 bins per thread) first, then the first two batches, so that waiting for
    // the histogram does not wait for the batches
    const int4 h4 = reinterpret_cast<const int4*>(a.ghist + static_cast<int64_t>(row) * kBins)[threadIdx.x];
    const int pos = a.gcnt[2 * row];
    const int zeros = a.gcnt[2 * row + 1];
    load_batch<kVec, kTk>(r, b0, x0);
    load_batch<kVec, kTk>(r, b0 + kStep, x1);
    m.pos = pos;
    m.fast = pos <= kTopK && pos + zeros >= kTopK;
    m.t1 = 0;
    m.above1 = pos;
    if (threadIdx.x == 0) L.misc[0] = L.misc[1] = 0;
    if (!m.fast) {
      const int h[4] = {h4.x, h4.y, h4.z, h4.w};
      find_threshold_regs<kTk, 4>(h, kTopK, L.wtot, L.res);
      m.t1 = static_cast<uint32_t>(L.res[0]);
      m.above1 = L.res[1];
    } else {
      __syncthreads();
    }
  } else {
    int pos, zeros;
    pass_hist<kVec, kTk>(r, 0, len, L.hist, L.red, pos, zeros);
    if (threadIdx.x == 0 && zeros) L.hist[kZeroBin] += zeros;
    load_batch<kVec, kTk>(r, b0, x0);
    load_batch<kVec, kTk>(r, b0 + kStep, x1);
    __syncthreads();
    m = row_meta<kTk>(L.hist, pos, zeros, L.wtot, L.res);
    if (threadIdx.x == 0) L.misc[0] = L.misc[1] = 0;
    __syncthreads();
  }
  Stage st{s_a, L.ck, L.ci, &L.misc[0], &L.misc[1], kTopK, kCapC};
  collect<kVec, kTk>(r, b0, n_batches, m, st, x0, x1);
  __syncthreads();
  const int n_a = min(L.misc[0], kTopK);
  const int n_c = L.misc[1];
  for (int i = threadIdx.x; i < n_a; i += kTk) put(dst, i, pt[s_a[i]]);
  if (m.fast) {
    ordered_scan<kVec, kTk>(
        r, [](uint32_t) { return true; }, kZeroKey, false, 0, m.pos, kTopK - m.pos, pt, dst, L.scan);
  } else if (n_c <= kCapC) {
    resolve_lds(L, n_c, m.t1, m.above1, pt, dst);
  } else {
    resolve_rescan<kVec>(L, r, m.t1, m.above1, pt, dst);
  }
}

// ---------------------------------------------------------------------------------------------
// Split variant.  CTAs cover balanced slices of the rows (split_assign).
// Zeroes the pass-1 histogram, counts and per-row counters of the split path.
__global__ __launch_bounds__(256) void topk_zero_kernel(int32_t* __restrict__ ghist, int32_t* __restrict__ gcnt,
                                                        int32_t* __restrict__ ctr, int64_t ctr_stride) {
  const int row = blockIdx.x;
  int4* g = reinterpret_cast<int4*>(ghist + static_cast<int64_t>(row) * kBins);
  for (int i = threadIdx.x; i < kBins / 4; i += 256) g[i] = make_int4(0, 0, 0, 0);
  if (threadIdx.x < 2) gcnt[2 * row + threadIdx.x] = 0;
  if (threadIdx.x < 3) ctr[row * ctr_stride + threadIdx.x] = 0;
}

struct SplitLds {
  union {
    struct {
      int a[kTopK];
      uint32_t ck[kCapS];
      int ci[kCapS];
    } col;                          // collection staging of this CTA's slice
    ResolveLds<kTs, kCapS> res;     // the row's resolution (last CTA only)
  } u;
  int wtot[kTs / kWave];
  int res[3];
  int n[6];
  long long lsum[kTs / kWave];
  int slot[3];
};

struct HistLds {
  int hist[kBins];
  int red[kTs / kWave];
  int wtot[kTs / kWave];
  long long lsum[kTs / kWave];
  int slot[3];
};

// Balanced split: row r gets c_r = ceil(len_r * T / L) CTAs (L = the summed lengths of the rows
// longer than 2048; a row of <= 2048 tokens gets one CTA, which copies it), in row order, so
// that every CTA streams about L / T tokens whatever the length mix; the sum is <= T + rows, the
// grid.  Needs rows <= kTs.  s_slot = {row (-1: none), index among the row's CTAs, c_r}.
template <typename Lds>
__device__ void split_assign(const TopkArgs& a, int T, Lds& L) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int len = tid < a.rows ? row_len(a, tid) : 0;
  long long big = len > kTopK ? len : 0;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) big += __shfl_xor(big, o);
  if (lane == 0) L.lsum[w] = big;
  if (tid == 0) L.slot[0] = -1;
  __syncthreads();
  long long total = 0;
#pragma unroll
  for (int v = 0; v < kTs / kWave; ++v) total += L.lsum[v];
  int c = 0;
  if (tid < a.rows) c = len > kTopK ? static_cast<int>((static_cast<long long>(len) * T + total - 1) / total) : 1;
  int inc = c;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) L.wtot[w] = inc;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int v = 0; v < kTs / kWave; ++v) before += v < w ? L.wtot[v] : 0;
  const int first = before + inc - c;
  const int cta = blockIdx.x;
  if (cta >= first && cta < first + c) {
    L.slot[0] = tid;
    L.slot[1] = cta - first;
    L.slot[2] = c;
  }
  __syncthreads();
}

// Slice of a row (by split_assign) this CTA covers: [begin, end) of len tokens, n_sl slices in
// the row; false when the CTA has none.  Slices are whole 256-token blocks.
__device__ __forceinline__ bool split_slice(int len, int c, int j, int& begin, int& end, int& n_sl) {
  const int sl = ((len + c - 1) / c + 255) / 256 * 256;
  begin = j * sl;
  end = min(begin + sl, len);
  n_sl = (len + sl - 1) / sl;
  return begin < len;
}

// Pass 1 of one balanced slice (the split kernel's slices) into the row's global histogram and
// positive / zero counts, which start at zero.
template <bool kVec>
__global__ __launch_bounds__(kTs) void topk_split_hist_kernel(const TopkArgs a) {
  __shared__ HistLds L;
  split_assign(a, a.T, L);
  const int row = L.slot[0];
  if (row < 0) return;  // block-uniform
  const int len = row_len(a, row);
  if (len <= kTopK) return;
  int begin, end, n_sl;
  if (!split_slice(len, L.slot[2], L.slot[1], begin, end, n_sl)) return;
  int pos, zeros;
  pass_hist<kVec, kTs>(row_src(a, row, len), begin, end, L.hist, L.red, pos, zeros);
  int32_t* gh = a.ghist + static_cast<int64_t>(row) * kBins;
  for (int i = threadIdx.x; i < kBins; i += kTs) {
    const int c = L.hist[i] + (i == kZeroBin ? zeros : 0);
    if (c) atomicAdd(&gh[i], c);
  }
  if (threadIdx.x == 0) {
    if (pos) atomicAdd(&a.gcnt[2 * row], pos);
    if (zeros) atomicAdd(&a.gcnt[2 * row + 1], zeros);
  }
}

// Per slice (balanced over the rows by split_assign): pass-1 threshold (from the row's
// histogram), unordered collection, then the A
// tokens go straight to the output and the candidates to the row's published list, both at
// positions from the row's global counters.  The CTA that finishes the row's last slice
// resolves the threshold over the published candidates (or re-reads the row if they exceed
// kCapS; fast path: takes the lowest-index zeros).
template <bool kVec>
__global__ __launch_bounds__(kTs) void topk_split_kernel(const TopkArgs a) {
  __shared__ SplitLds L;
  constexpr int kStep = kTs * 4 * kUnroll;
  const int tid = threadIdx.x;
  split_assign(a, a.T, L);
  const int row = L.slot[0];
  if (row < 0) return;  // block-uniform
  const int len = row_len(a, row);
  if (len <= kTopK) {
    copy_short_row<kTs>(pt_row(a, row), a.out + static_cast<int64_t>(row) * kTopK, len);
    return;
  }
  int begin, end, n_sl;
  if (!split_slice(len, L.slot[2], L.slot[1], begin, end, n_sl)) return;

  // pass-1 slots (8 bins per thread) and counts first, then the first two batches
  const int4* gh4 = reinterpret_cast<const int4*>(a.ghist + static_cast<int64_t>(row) * kBins);
  const int4 g0 = gh4[2 * tid];
  const int4 g1 = gh4[2 * tid + 1];
  const int pos = a.gcnt[2 * row];
  const int zeros = a.gcnt[2 * row + 1];
  RowSrc rr = row_src(a, row, end);
  const int b0 = begin + tid * 4;
  Batch x0, x1;
  load_batch<kVec, kTs>(rr, b0, x0);
  load_batch<kVec, kTs>(rr, b0 + kStep, x1);

  Meta m;
  m.pos = pos;
  m.fast = pos <= kTopK && pos + zeros >= kTopK;
  m.t1 = 0;
  m.above1 = pos;
  int cnt_t1 = 0;
  if (tid == 0) L.n[0] = L.n[1] = 0;
  if (!m.fast) {
    const int h[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    find_threshold_regs<kTs, 8>(h, kTopK, L.wtot, L.res);
    m.t1 = static_cast<uint32_t>(L.res[0]);
    m.above1 = L.res[1];
    cnt_t1 = L.res[2];
  } else {
    __syncthreads();
  }
  // every CTA of the row takes the same decision: candidates are published only if the whole
  // bin t1 of the row fits the resolver's LDS
  const bool publish = !m.fast && cnt_t1 <= kCapS;
  Stage st{L.u.col.a, L.u.col.ck, L.u.col.ci, &L.n[0], &L.n[1], kTopK, publish ? kCapS : 0};
  collect<kVec, kTs>(rr, b0, (end - begin + kStep - 1) / kStep, m, st, x0, x1);
  __syncthreads();

  const int n_a = min(L.n[0], kTopK);
  const int n_c = min(L.n[1], kCapS);
  int32_t* ctr = a.ctr + static_cast<int64_t>(row) * a.ctr_stride;
  if (tid == 0) {
    L.n[2] = n_a ? atomicAdd(&ctr[0], n_a) : 0;
    L.n[3] = publish && n_c ? atomicAdd(&ctr[1], n_c) : 0;
  }
  __syncthreads();
  const PtRow pt = pt_row(a, row);
  int32_t* dst = a.out + static_cast<int64_t>(row) * kTopK;
  const int base_a = L.n[2];
  for (int i = tid; i < n_a; i += kTs) put(dst, base_a + i, pt[L.u.col.a[i]]);
  uint32_t* lk = a.c_keys + static_cast<int64_t>(row) * kCapS;
  int32_t* lt = a.c_tok + static_cast<int64_t>(row) * kCapS;
  if (publish) {
    const int base_c = L.n[3];
    for (int i = tid; i < n_c; i += kTs) {
      const int j = base_c + i;
      if (j < kCapS) {
        __hip_atomic_store(&lk[j], L.u.col.ck[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&lt[j], L.u.col.ci[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // Candidates travel between CTAs (and XCDs) through device-coherent (agent-scope) stores and
  // loads.  Every wave waits for its stores to complete before the barrier, so the row
  // counter's increment below comes after all of this CTA's candidates; the CTA that makes the
  // last increment reads them back with device-coherent loads.  No L2 write-back / invalidate
  // fence is needed (a __threadfence per wave costs tens of microseconds here).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) L.n[4] = atomicAdd(&ctr[2], 1) == n_sl - 1;
  __syncthreads();
  if (!L.n[4]) return;

  const RowSrc r = row_src(a, row, len);
  if (m.fast) {
    ordered_scan<kVec, kTs>(
        r, [](uint32_t) { return true; }, kZeroKey, false, 0, m.pos, kTopK - m.pos, pt, dst, L.u.res.scan);
    return;
  }
  if (!publish) {
    resolve_rescan<kVec>(L.u.res, r, m.t1, m.above1, pt, dst);
    return;
  }
  const int n_tot = cnt_t1;  // every CTA published its share of bin t1 (cnt_t1 <= kCapS)
  for (int i = tid; i < n_tot; i += kTs) {
    L.u.res.ck[i] = __hip_atomic_load(&lk[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.u.res.ci[i] = __hip_atomic_load(&lt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  resolve_lds(L.u.res, n_tot, m.t1, m.above1, pt, dst);
}

// Slices per row of the split path (1: one CTA per row).  At most ~3 split CTAs fit a CU.
int split_count(int64_t rows, int64_t width, int max_splits, int n_cu) {
  if (rows <= 0 || rows > kTs) return 1;  // the balanced split assigns one row per thread
  int64_t s = (width + 8191) / 8192;  // splitting rows of <= 8192 tokens does not pay
  s = s < 1 ? 1 : s;
  const int64_t by_cu = (3 * static_cast<int64_t>(n_cu)) / rows;
  s = s < by_cu ? s : by_cu;
  const int64_t cap = max_splits < kMaxSplit ? max_splits : kMaxSplit;
  s = s < cap ? s : cap;
  return static_cast<int>(s < 1 ? 1 : s);
}

// CTAs the balanced split kernel spreads the rows' tokens over (its grid adds one per row):
// rows * S, capped so that the grid stays within ~3 resident CTAs per CU.
int split_target(int64_t rows, int S, int n_cu) {
  const int64_t fit = 3 * static_cast<int64_t>(n_cu) - rows;
  int64_t t = rows * S;
  t = t < fit ? t : fit;
  return static_cast<int>(t < rows ? rows : t);
}

struct WsLayout {
  size_t ghist, gcnt, ctr, c_keys, c_tok, total;
};

WsLayout ws_layout(int64_t rows) {
  WsLayout l;
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.ghist = take(sizeof(int32_t) * rows * kBins);
  l.gcnt = take(sizeof(int32_t) * rows * 2);
  l.ctr = take(sizeof(int32_t) * rows * 4);
  l.c_keys = take(sizeof(uint32_t) * rows * kCapS);
  l.c_tok = take(sizeof(int32_t) * rows * kCapS);
  l.total = off;
  return l;
}

int topk_common(const float* score, int64_t score_stride, int64_t width, const int16_t* mask, int64_t mask_stride,
                const int32_t* lengths, int64_t rows, const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu, int32_t* pre_hist,
                bool pass1_done, void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream,
                const char* who) {
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
  a.T = 0;
  a.ghist = a.gcnt = a.ctr = a.c_tok = nullptr;
  a.c_keys = nullptr;
  a.ctr_stride = 1;
  const dim3 grid_rows(static_cast<uint32_t>(rows));

  if (pre_hist != nullptr) {
    // [ghist1 rows*4096 | ghist2 rows*4096 | cnt rows*2]; words 0..2 of each ghist2 row are the
    // row's split counters (zeroed by the logits call that built pass 1).
    a.ghist = pre_hist;
    a.ctr = pre_hist + rows * kBins;
    a.ctr_stride = kBins;
    a.gcnt = pre_hist + 2 * rows * kBins;
  }
  if (S <= 1) {
    if (pre_hist && pass1_done) {
      if (vec) hipLaunchKernelGGL((topk_single_kernel<true, true>), grid_rows, dim3(kTk), 0, stream, a);
      else hipLaunchKernelGGL((topk_single_kernel<false, true>), grid_rows, dim3(kTk), 0, stream, a);
    } else {
      if (vec) hipLaunchKernelGGL((topk_single_kernel<true, false>), grid_rows, dim3(kTk), 0, stream, a);
      else hipLaunchKernelGGL((topk_single_kernel<false, false>), grid_rows, dim3(kTk), 0, stream, a);
    }
    return check_launch(who);
  }
  const WsLayout l = ws_layout(rows);
  DSA_REQUIRE(workspace != nullptr && workspace_bytes >= l.total,
              "%s: workspace of %zu bytes is smaller than the %zu required", who, workspace_bytes, l.total);
  DSA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "%s: workspace must be 16-B aligned", who);
  char* ws = static_cast<char*>(workspace);
  if (!pre_hist) {
    a.ghist = reinterpret_cast<int32_t*>(ws + l.ghist);
    a.gcnt = reinterpret_cast<int32_t*>(ws + l.gcnt);
    a.ctr = reinterpret_cast<int32_t*>(ws + l.ctr);
    a.ctr_stride = 4;
  }
  a.c_keys = reinterpret_cast<uint32_t*>(ws + l.c_keys);
  a.c_tok = reinterpret_cast<int32_t*>(ws + l.c_tok);
  a.T = split_target(rows, S, n_cu);
  const dim3 grid_bal(static_cast<uint32_t>(a.T + rows));
  if (!pre_hist) hipLaunchKernelGGL(topk_zero_kernel, grid_rows, dim3(256), 0, stream, a.ghist, a.gcnt, a.ctr, a.ctr_stride);
  if (!pass1_done) {
    if (vec) hipLaunchKernelGGL((topk_split_hist_kernel<true>), grid_bal, dim3(kTs), 0, stream, a);
    else hipLaunchKernelGGL((topk_split_hist_kernel<false>), grid_bal, dim3(kTs), 0, stream, a);
  }
  if (vec) hipLaunchKernelGGL((topk_split_kernel<true>), grid_bal, dim3(kTs), 0, stream, a);
  else hipLaunchKernelGGL((topk_split_kernel<false>), grid_bal, dim3(kTs), 0, stream, a);
  return check_launch(who);
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_topk_workspace_bytes(int64_t rows, int64_t width, int max_splits, int n_cu) {
  const int S = split_count(rows, width, max_splits < 1 ? 1 : max_splits, n_cu);
  if (S <= 1 || rows <= 0) return 0;
  return ws_layout(rows).total;
}

extern "C" int dsa_topk_transform(const float* score, int64_t score_stride, int64_t width, const int16_t* mask,
                                  int64_t mask_stride, const int32_t* lengths, int64_t rows,
                                  const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                                  const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                                  void* workspace, size_t workspace_bytes, int32_t* out, hipStream_t stream) {
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, nullptr, false, workspace, workspace_bytes, out, stream,
                     "dsa_topk_transform");
}

extern "C" int dsa_topk_transform_pre(const float* score, int64_t score_stride, int64_t width, const int16_t* mask,
                                      int64_t mask_stride, const int32_t* lengths, int64_t rows,
                                      const int32_t* page_table, int64_t pt_stride, int64_t pt_cols,
                                      const int32_t* cu_seqlens_q, int64_t n_req, int max_splits, int n_cu,
                                      int32_t* hist_ws, int pass1_done, void* workspace, size_t workspace_bytes,
                                      int32_t* out, hipStream_t stream) {
  DSA_REQUIRE(hist_ws != nullptr, "dsa_topk_transform_pre: hist_ws is null");
  return topk_common(score, score_stride, width, mask, mask_stride, lengths, rows, page_table, pt_stride, pt_cols,
                     cu_seqlens_q, n_req, max_splits, n_cu, hist_ws, pass1_done != 0, workspace, workspace_bytes, out,
                     stream, "dsa_topk_transform_pre");
}
