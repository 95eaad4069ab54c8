// Instantiates attn_fwd32_kernel (64-, 128- and 256-wide heads) for one element type: compiled once per type
// with -DDMAD_T=<0 bf16 | 1 f16> and MFMAs in VGPR form, so that the
// accumulators and score tiles take the VGPRs and Q, Qd the AGPRs.
#include "launch.h"

#ifndef DMAD_T
#error "DMAD_T must be defined"
#endif

namespace dmad {

#if DMAD_T == 0
using Elt = __bf16;
#else
using Elt = _Float16;
#endif

static_assert(Fwd32Cfg<kFwdJvp>::BM == kMagiBlockM && Fwd32Cfg<kFwdJvp, 64>::BM == kMagiBlockM, "block-sparse tasks are 128-query tiles");

template <typename T, int MODE, int D>
static hipError_t fwd32_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd32_kernel<T, MODE, false, D>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int MODE, int D>
static hipError_t fwd32_magi_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd32_kernel<T, MODE, true, D>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t fwd32x2_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd32_x2_kernel<T>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int D>
static FwdLaunchFn fwd32_magi_mode(int mode) {
  switch (mode) {
    case kFwdJvp: return &fwd32_magi_launch<Elt, kFwdJvp, D>;
    case kFwdJvpQOnly: return &fwd32_magi_launch<Elt, kFwdJvpQOnly, D>;
    default: return nullptr;
  }
}

template <int D>
static FwdLaunchFn fwd32_mode(int mode) {
  switch (mode) {
    case kFwdPlain: return &fwd32_launch<Elt, kFwdPlain, D>;
    case kFwdJvp: return &fwd32_launch<Elt, kFwdJvp, D>;
    case kFwdJvpQOnly: return &fwd32_launch<Elt, kFwdJvpQOnly, D>;
    default: return nullptr;
  }
}

template <>
FwdLaunchFn fwd32_magi_select<Elt>(int mode, int d) {
  return d == 64    ? fwd32_magi_mode<64>(mode)
         : d == 128 ? fwd32_magi_mode<128>(mode)
         : d == 256 ? fwd32_magi_mode<256>(mode)
                    : nullptr;
}

template <>
FwdLaunchFn fwd32x2_select<Elt>(int mode, int d) {
  return fwd32x2_supported(mode, d, d) ? &fwd32x2_launch<Elt> : nullptr;
}

template <>
FwdLaunchFn fwd32_select<Elt>(int mode, int d) {
  return d == 64 ? fwd32_mode<64>(mode) : d == 128 ? fwd32_mode<128>(mode) : d == 256 ? fwd32_mode<256>(mode) : nullptr;
}

}  // namespace dmad
