// Shared constants, device helpers and host-side status plumbing of the gfx950 DSA indexer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "../../include/dsa_indexer.h"

namespace dsa {

constexpr int kWave = 64;
constexpr int kPage = DSA_PAGE_TOKENS;          // tokens per K-cache page
constexpr int kHeadDim = DSA_HEAD_DIM;          // fp8 bytes per K token / q head
constexpr int kTokBytes = kHeadDim + 4;         // fp8 row + fp32 scale
constexpr int kPageFp8Bytes = kPage * kHeadDim; // scales start here inside a page
constexpr int kPageBytes = kPage * kTokBytes;   // 8448
constexpr int kTopK = DSA_TOPK;
constexpr int kBins = 4096;                     // 12-bit radix digit
constexpr uint32_t kZeroKey = 0x80000000u;      // key of +0.0 (and of masked-out tokens)
constexpr int kZeroBin = static_cast<int>(kZeroKey >> 20);
constexpr int kHistWsPerRow = 2 * kBins + 2;    // [ghist1 | ghist2 | (positives, zeros)]
// Word 3 of a raw buffer descriptor on gfx9-family chips (gfx950): 32-bit data format, no
// swizzle; with stride 0 a load whose byte offset is at or past num_records returns 0.
constexpr int kBufferDword3 = 0x00020000;

// ------------------------------------------------------------------------------------------
// Order-preserving float -> uint32 key (sparse_mask_topk.cu:40-43): larger float, larger key;
// -0.0 sorts just below +0.0.
__device__ __forceinline__ uint32_t float_key(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// fp32 -> bf16, round to nearest even, NaN -> 0x7FC0 (the c10::BFloat16 conversion).
__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (f != f) ? 0x7FC0u : r;
}

// fp32 -> OCP fp8 e4m3fn (bias 7, max 448, no infinities), round to nearest even, not
// saturating: |x| > 464 (which rounds past 448; 464 itself ties to the even 448), infinities and
// NaN give 0x7F | sign -- the behaviour of torch's float -> float8_e4m3fn cast.  Written from
// the format definition with no select or branch (a converted select becomes a branch per
// value, and many conversions in a row then spill): on a = |x| clamped to [2^-6, inf), the
// normal code (3 mantissa bits kept, RNE on the other 20; >= 0x7F past 448, capped there) plus
// the subnormal code of min(a, 2^-6) (RNE on the grid of 2^-9: 8 at 2^-6) minus 8.
__device__ __forceinline__ uint32_t fp8_e4m3_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t lo = min(a, 0x3C800000u);
  const uint32_t hi = max(a, 0x3C800000u);
  const uint32_t sub = static_cast<uint32_t>(rintf(__uint_as_float(lo) * 512.0f));
  const uint32_t nrm = min(((hi + 0x7FFFFu + ((hi >> 20) & 1u)) >> 20) - (120u << 3), 0x7Fu);
  return (nrm + sub - 8u) | sign;
}

// Factors of the per-vector fp8 quantisation (hcu_ops/csrc/norm_quant.cu:13-14): for
// amax = max|x| over the vector, the codes are fp8_e4m3_rne(x * inv) with inv = 448 / amax
// (0 when amax == 0) and the dequantisation scale is amax / 448.
__device__ __forceinline__ void quant_factors(float amax, float& inv, float& scale) {
  inv = amax == 0.0f ? 0.0f : 448.0f / amax;
  scale = amax / 448.0f;
}

// One 128-element bf16 vector quantised by 16 lanes (lane `sub` holds elements 8 sub .. 8 sub + 7;
// the 16 lanes are 16 consecutive lanes of the wave, aligned to 16): the vector's amax (all 16
// lanes agree), its dequantisation scale and this lane's 8 fp8 codes packed in two words.
__device__ __forceinline__ float quant_vec16(const uint16_t* src, int sub, uint32_t& lo, uint32_t& hi, float& scale) {
  const uint4 raw = *reinterpret_cast<const uint4*>(src + sub * 8);
  const uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(r[i] << 16);
    x[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
  // max over the 16 lanes (one DPP row) without LDS: lane ^ 1, lane ^ 2 (quad_perm), then the
  // row's half mirror (lane i <-> 7 - i within 8) and mirror (i <-> 15 - i)
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x4E, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x141, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x140, 0xF, 0xF, false)));
  float inv;
  quant_factors(amax, inv, scale);
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = fp8_e4m3_rne(x[i] * inv);
  lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  return amax;
}

// ------------------------------------------------------------------------------------------
// Wave helpers (wave64).
__device__ __forceinline__ int lane_id() { return static_cast<int>(__lane_id()); }

// Number of set bits of `mask` in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Inclusive suffix sum over the wave (lane l: sum of lanes l..63).  Within each 16-lane row a
// Hillis-Steele scan on DPP row shifts (row_shl n: lane l reads lane l + n of its row, 0 past
// the row's end), then the totals of the rows above, read from their first lanes.
__device__ __forceinline__ int wave_suffix_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x101, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x102, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x108, 0xF, 0xF, true);
  const int r1 = __builtin_amdgcn_readlane(x, 16);
  const int r2 = __builtin_amdgcn_readlane(x, 32);
  const int r3 = __builtin_amdgcn_readlane(x, 48);
  const int row = lane_id() >> 4;
  return x + (row < 1 ? r1 : 0) + (row < 2 ? r2 : 0) + (row < 3 ? r3 : 0);
}

// Inclusive prefix sum over the wave (lane l: sum of lanes 0..l), the mirror of wave_suffix_sum
// (row_shr n: lane l reads lane l - n of its row, 0 before the row's start).
__device__ __forceinline__ int wave_prefix_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane_id() >> 4;
  return x + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

// Exclusive prefix (lane order) and wave total of per-lane counts in [0, 7]: three ballots.
__device__ __forceinline__ int wave_prefix_small(int c, int& total) {
  const uint64_t b0 = __ballot(c & 1);
  const uint64_t b1 = __ballot(c & 2);
  const uint64_t b2 = __ballot(c & 4);
  total = __popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2);
  return lanes_below(b0) + 2 * lanes_below(b1) + 4 * lanes_below(b2);
}

// The same for per-lane counts in [0, 31]: five ballots.
__device__ __forceinline__ int wave_prefix_5(int c, int& total) {
  int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const uint64_t b = __ballot(c & (1 << k));
    total += __popcll(b) << k;
    before += lanes_below(b) << k;
  }
  return before;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Block-wide (NT threads) exclusive prefix (thread order) and total of a per-thread count; one
// barrier; s_w (NT / 64 words) must not be reused before the next barrier.
template <int NT>
__device__ __forceinline__ int block_excl_sum(int x, int& total, int* s_w) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int inc = wave_prefix_sum(x);
  if (lane == 63) s_w[w] = inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int v = 0; v < NT / kWave; ++v) {
    before += v < w ? s_w[v] : 0;
    tot += s_w[v];
  }
  total = tot;
  return before + inc - x;
}

// Slot of this lane among the active lanes of its wave with `pred` set, from one atomic add of
// their count on *ctr (LDS or global) by the lowest of them.  Lanes without pred get a value
// they must not use.  Replaces one same-address atomic per lane, which the LDS serialises.
__device__ __forceinline__ int wave_slot(bool pred, int* ctr) {
  const uint64_t m = __ballot(pred);
  int base = 0;
  if (m != 0) {  // wave-uniform
    const int leader = static_cast<int>(__builtin_ctzll(m));
    if (lane_id() == leader) base = atomicAdd(ctr, static_cast<int>(__popcll(m)));
    base = __builtin_amdgcn_readlane(base, leader);
  }
  return base + lanes_below(m);
}

// The first of c (0 .. 31) consecutive slots for this lane, the lanes' slots in lane order after
// one atomic add of the wave's total on *ctr (LDS or global) by lane 0.  Every lane of the wave
// must call it.
__device__ __forceinline__ int wave_slot_n(int c, int* ctr) {
  int total;
  const int before = wave_prefix_5(c, total);
  int base = 0;
  if (total != 0 && lane_id() == 0) base = atomicAdd(ctr, total);
  return uniform(base) + before;
}

// max(x, +0) as one integer max on the float bits: negative floats (and -0.0) are negative
// integers, so they become +0; other values, NaNs included, pass unchanged.  fmaxf would add a
// NaN-quieting max per element.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// Reduce-scatter of four per-lane values over the four 16-lane rows of the wave: lane l ends
// with sum over the rows g of v[l / 16] from lane (l % 16) + 16 g, i.e. row g keeps entry g
// summed over all rows.  Two row-pair exchanges (v_permlane16_swap, each moving a register's odd
// rows against another's even rows) halve the entries, one half exchange (v_permlane32_swap)
// halves them again: 3 swaps and 3 adds instead of 4 x (2 swaps + 2 adds) and a select per
// entry.  The additions associate as ((row 0 + row 1) + (row 2 + row 3)), the order of
// sum_lanes_16_32, so the results are the same bits.
__device__ __forceinline__ float reduce_scatter_rows(const float (&v)[4]) {
  const auto p01 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[0]), __float_as_uint(v[1]), false, false);
  const auto p23 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[2]), __float_as_uint(v[3]), false, false);
  const float a = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);  // entry g & 1, rows g, g ^ 1
  const float b = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);  // entry 2 + (g & 1)
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// x + x[lane ^ 16] and then + x[lane ^ 32], in every lane, with the gfx950 row-swap VALU ops
// (v_permlane16_swap / v_permlane32_swap) instead of LDS-routed shuffles.  Swapping a register
// with itself leaves lane l of the two results holding x[l] and x[l ^ 16] (resp. ^ 32), in an
// order that makes the sum identical in all lanes of a pair.
__device__ __forceinline__ float sum_lanes_16_32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace dsa

// ------------------------------------------------------------------------------------------
// Host-side status plumbing (defined in status.cpp).
namespace dsa {
int fail(int code, const char* fmt, ...);
int ok();
int check_launch(const char* what);
}  // namespace dsa

#define DSA_REQUIRE(cond, ...)                                      \
  do {                                                              \
    if (!(cond)) return ::dsa::fail(DSA_ERR_INVALID, __VA_ARGS__);  \
  } while (0)
