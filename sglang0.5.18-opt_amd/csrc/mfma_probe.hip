// fp8 MFMA throughput probe (gfx950): the measured ceiling the prefill logits kernel is set against,
// beside the published dense fp8 peak.
//
// Every wave keeps eight independent v_mfma_f32_16x16x128_f8f6f4 accumulator chains busy on
// operands read once from a caller buffer of fp8 codes (random codes give the data-dependent
// power and clock behaviour of real operands; all-zero operands run faster than real ones).  With
// NV > 0 each MFMA result instead goes through NV VALU operations of the logits kernel's kind
// (ReLU as an integer max on the float bits, then an FMA by a head weight into a running sum; NV =
// 8 is the logits epilogue's count per MFMA: four result elements, two operations each), so the
// NV = 4, 8, 16 figures trace what each VALU operation per MFMA costs the fp8 MFMA rate.  Thread
// 0 of CTA 0 reads the shader clock (s_memtime) and the 100 MHz reference clock (s_memrealtime)
// around its loop, which gives the clock the chip ran at.
#include "dsa_common.h"

namespace dsa {
namespace {

using i32x8 = __attribute__((ext_vector_type(8))) int;
using f32x4 = __attribute__((ext_vector_type(4))) float;

constexpr int kProbeThreads = 256;
constexpr int kProbeWords = 16384;  // operand words read by the probe (64 KiB)
constexpr int kChains = 8;

template <int NV>
__global__ __launch_bounds__(kProbeThreads) void mfma_probe_kernel(const int32_t* __restrict__ src,
                                                                   float* __restrict__ sink,
                                                                   uint64_t* __restrict__ clocks, int iters) {
  static_assert(NV == 0 || NV == 4 || NV == 8 || NV == 16, "VALU operations per MFMA");
  const int lane = threadIdx.x & 63;
  i32x8 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[j][e] = src[(lane * 64 + j * 8 + e) & (kProbeWords - 1)];
      b[j][e] = src[(lane * 64 + 32 + j * 8 + e) & (kProbeWords - 1)];
    }
  const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
  uint64_t t0 = 0, r0 = 0;
  if (timer) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  f32x4 acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  const float w = 0.37f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kChains; ++j) {
      const i32x8& bb = b[(j >> 2) + 2 * (it & 1)];
      if constexpr (NV == 0) {
        acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j & 3], bb, acc[j], 0, 0, 0, 0, 0, 0);
      } else {
        const f32x4 r = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j & 3], bb, f32x4{0.f, 0.f, 0.f, 0.f},
                                                                         0, 0, 0, 0, 0, 0);
        constexpr int NE = NV >= 8 ? 4 : NV / 2;  // result elements taken through ReLU + FMA
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          s[e & 1] = fmaf(relu_bits(r[e]), w, s[e & 1]);
          if constexpr (NV == 16) s[2 + (e & 1)] = fmaf(relu_bits(-r[e]), w, s[2 + (e & 1)]);
        }
      }
    }
  }
  if (timer) {
    clocks[0] = __builtin_amdgcn_s_memtime() - t0;
    clocks[1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
  float t = s[0] + s[1] + s[2] + s[3];
#pragma unroll
  for (int j = 0; j < kChains; ++j) t += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = t;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_mfma_fp8_probe(const int32_t* operands, int64_t n_words, float* sink, uint64_t* clocks,
                                  int ctas, int iters, int epilogue, hipStream_t stream) {
  using namespace dsa;
  DSA_REQUIRE(operands && sink && clocks, "dsa_mfma_fp8_probe: null pointer");
  DSA_REQUIRE(n_words >= kProbeWords, "dsa_mfma_fp8_probe: needs %d operand words, got %lld", kProbeWords,
              static_cast<long long>(n_words));
  DSA_REQUIRE(ctas >= 1 && ctas <= (1 << 20) && iters >= 1, "dsa_mfma_fp8_probe: bad ctas %d / iters %d", ctas,
              iters);
  const int nv = epilogue == 1 ? 8 : epilogue;  // 1: the logits epilogue's 8
  DSA_REQUIRE(nv == 0 || nv == 4 || nv == 8 || nv == 16,
              "dsa_mfma_fp8_probe: epilogue must be 0, 1, 4, 8 or 16 VALU operations per MFMA (got %d)", epilogue);
  const dim3 g(ctas), b(kProbeThreads);
  switch (nv) {
    case 0: hipLaunchKernelGGL(mfma_probe_kernel<0>, g, b, 0, stream, operands, sink, clocks, iters); break;
    case 4: hipLaunchKernelGGL(mfma_probe_kernel<4>, g, b, 0, stream, operands, sink, clocks, iters); break;
    case 8: hipLaunchKernelGGL(mfma_probe_kernel<8>, g, b, 0, stream, operands, sink, clocks, iters); break;
    default: hipLaunchKernelGGL(mfma_probe_kernel<16>, g, b, 0, stream, operands, sink, clocks, iters); break;
  }
  return check_launch("dsa_mfma_fp8_probe");
}
