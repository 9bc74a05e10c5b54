/*
 * Sequential C restatement of the reference's single-CTA exact top-2048 select
 * (hcu_ops/csrc/sparse_mask_topk.cu:141-349) -- oracle / test infrastructure only.
 *
 * Per row (len = min(lengths[r], width)):
 *   len <= 2048            dst[i] = i < len ? pt[i] : -1                          (:166-169)
 *   pass 1                 12-bit histogram of key[31:20] of nonzero tokens, positive and
 *                          zero counts; zeros go to the zero bin                    (:199-227)
 *   pos <= 2048 <= pos+zero threshold key = +0, remaining = 2048 - pos              (:231-234)
 *   otherwise              t1 = find_threshold(hist, 2048), 12-bit histogram of key[19:8]
 *                          inside t1, t2, then an 8-bit histogram of key[7:0] inside the
 *                          24-bit prefix, t3; thr = prefix24 << 8 | t3               (:236-298)
 *   pass 4                 ascending t: key > thr -> next slot; key == thr -> tie slot while
 *                          fewer than `remaining` ties were taken                   (:301-348)
 * The output order is therefore [all keys > thr ascending t][ties ascending t], the order of
 * the reference's single kernel.
 */
#include <stdint.h>
#include <string.h>

#define TOPK 2048
#define ZERO_KEY 0x80000000u

static uint32_t float_key(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static uint32_t token_key(const float* s, const int16_t* m, int t) {
  if (m != NULL && !(((uint16_t)m[t >> 4] >> (t & 15)) & 1u)) return ZERO_KEY;
  return float_key(s[t]);
}

/* bin t with suffix(t) >= need > suffix(t + 1); *above = suffix(t + 1)  (:96-138) */
static int find_threshold(const int* hist, int nb, int need, int* above) {
  int suf = 0;
  for (int b = nb - 1; b >= 0; --b) {
    if (suf + hist[b] >= need) {
      *above = suf;
      return b;
    }
    suf += hist[b];
  }
  *above = suf;
  return 0; /* unreachable when sum(hist) >= need */
}

/* Page-table entry of token t: -1 past the row's pt_cols entries (a table narrower than the
 * row; the reference requires >= len entries, this build maps the rest to -1). */
static int32_t pt_at(const int32_t* pt, int pt_cols, int t) { return t < pt_cols ? pt[t] : -1; }

void topk_radix_row(const float* score, const int16_t* mask, int len, const int32_t* pt, int pt_cols, int32_t* dst) {
  static int hist[4096];
  if (len <= TOPK) {
    for (int i = 0; i < TOPK; ++i) dst[i] = i < len ? pt_at(pt, pt_cols, i) : -1;
    return;
  }
  memset(hist, 0, sizeof(hist));
  int pos = 0, zeros = 0;
  for (int t = 0; t < len; ++t) {
    const uint32_t key = token_key(score, mask, t);
    if (key == ZERO_KEY) {
      ++zeros;
    } else {
      pos += key > ZERO_KEY;
      ++hist[key >> 20];
    }
  }
  hist[ZERO_KEY >> 20] += zeros;
  uint32_t thr;
  int remaining;
  if (pos <= TOPK && pos + zeros >= TOPK) {
    thr = ZERO_KEY;
    remaining = TOPK - pos;
  } else {
    int above;
    const uint32_t t1 = (uint32_t)find_threshold(hist, 4096, TOPK, &above);
    const int need1 = TOPK - above;
    memset(hist, 0, sizeof(hist));
    if (t1 == (ZERO_KEY >> 20)) hist[(ZERO_KEY >> 8) & 0xFFFu] += zeros;
    for (int t = 0; t < len; ++t) {
      const uint32_t key = token_key(score, mask, t);
      if ((key >> 20) == t1 && key != ZERO_KEY) ++hist[(key >> 8) & 0xFFFu];
    }
    const uint32_t t2 = (uint32_t)find_threshold(hist, 4096, need1, &above);
    const uint32_t prefix24 = (t1 << 12) | t2;
    const int need2 = need1 - above;
    memset(hist, 0, 256 * sizeof(int));
    if (prefix24 == (ZERO_KEY >> 8)) hist[ZERO_KEY & 0xFFu] += zeros;
    for (int t = 0; t < len; ++t) {
      const uint32_t key = token_key(score, mask, t);
      if ((key >> 8) == prefix24 && key != ZERO_KEY) ++hist[key & 0xFFu];
    }
    const uint32_t t3 = (uint32_t)find_threshold(hist, 256, need2, &above);
    thr = (prefix24 << 8) | t3;
    remaining = need2 - above;
  }
  const int tie_base = TOPK - remaining;
  int a = 0, ties = 0;
  for (int t = 0; t < len; ++t) {
    const uint32_t key = token_key(score, mask, t);
    if (key > thr) dst[a++] = pt_at(pt, pt_cols, t);
    else if (key == thr && ties < remaining) dst[tie_base + ties++] = pt_at(pt, pt_cols, t);
  }
}

/* Batched entry: rows of score [rows, score_stride], mask [rows, mask_stride] (nullable),
 * page-table row pr = r (cu == NULL) or the request b with cu[b] <= r < cu[b + 1], pt_cols
 * entries per page-table row. */
void topk_radix(const float* score, int64_t score_stride, int width, const int16_t* mask, int64_t mask_stride,
                const int32_t* lengths, int rows, const int32_t* pt, int64_t pt_stride, int pt_cols, const int32_t* cu,
                int n_req, int32_t* out) {
  for (int r = 0; r < rows; ++r) {
    int pr = r;
    if (cu != NULL) {
      pr = 0;
      while (pr + 1 < n_req && cu[pr + 1] <= r) ++pr;
    }
    int len = lengths[r];
    len = len < 0 ? 0 : (len < width ? len : width);
    topk_radix_row(score + (int64_t)r * score_stride, mask ? mask + (int64_t)r * mask_stride : NULL, len,
                   pt + (int64_t)pr * pt_stride, pt_cols, out + (int64_t)r * TOPK);
  }
}
