// Practical MFMA ceiling probe: a measurement aid for benchmarks, not part of
// the attention path. Back-to-back 32x32x16 MFMAs (bf16 or fp16) on every CU,
// one wave per SIMD, four independent accumulator chains per wave, with new
// operand bits every 32 MFMAs (a linear congruential step on one A and one B
// register, exponent bits held in a normal range), so the matrix unit draws
// the power of real data rather than of constant operands. Timing it beside
// the attention kernels on the same board gives the MFMA rate the board's
// power limit allows when the matrix unit does nothing else.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace dmad {
namespace {

template <bool F16>
__global__ __launch_bounds__(256, 1) void mfma_probe_kernel(float* sink, int rounds) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  f32x16_t acc[4] = {};
  u32x4_t a[8], b[8];
  const unsigned t = threadIdx.x;
  // sign and mantissa bits vary; the exponent stays near 1.0 (bf16: 2^-3..2^0, fp16: 2^-2..2^-1)
  const unsigned keep = F16 ? 0x83FF83FFu : 0x80FF80FFu;
  const unsigned base = F16 ? 0x34003400u : 0x3E003E00u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned h = (t * 2654435761u) ^ (j * 40503u + e * 977u);
      a[j][e] = (h & keep) | base;
      b[j][e] = ((h * 1664525u + 1013904223u) & keep) | base;
    }
  }
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
      for (int m = 0; m < 32; ++m) {
        const u32x4_t x = a[m & 7], y = b[(m + 3) & 7];
        if constexpr (F16)
          acc[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, x),
                                                              __builtin_bit_cast(f16x8_t, y), acc[m & 3], 0, 0, 0);
        else
          acc[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, x),
                                                               __builtin_bit_cast(bf16x8_t, y), acc[m & 3], 0, 0, 0);
        if (m == 16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[jj][e] = ((a[jj][e] * 1664525u + 1013904223u) & keep) | base;
            b[jj][e] = ((b[jj][e] * 22695477u + 1u) & keep) | base;
          }
        }
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[j][i];
  sink[(int64_t)blockIdx.x * 256 + t] = s;
}

}  // namespace
}  // namespace dmad

namespace dmad {
hipError_t launch_mfma_probe(bool f16, int blocks, int rounds, float* sink, hipStream_t s) {
  if (f16)
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, sink, rounds);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, sink, rounds);
  return hipGetLastError();
}
}  // namespace dmad
