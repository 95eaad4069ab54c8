// Instantiates attn_fwd32_kernel for one element type: compiled once per type
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

static_assert(Fwd32Cfg<kFwdJvp>::BM == kMagiBlockM, "block-sparse tasks are 128-query tiles");

template <typename T, int MODE>
static hipError_t fwd32_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd32_kernel<T, MODE>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int MODE>
static hipError_t fwd32_magi_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd32_kernel<T, MODE, true>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <>
FwdLaunchFn fwd32_magi_select<Elt>(int mode) {
  switch (mode) {
    case kFwdJvp: return &fwd32_magi_launch<Elt, kFwdJvp>;
    case kFwdJvpQOnly: return &fwd32_magi_launch<Elt, kFwdJvpQOnly>;
    default: return nullptr;
  }
}

template <>
FwdLaunchFn fwd32_select<Elt>(int mode) {
  switch (mode) {
    case kFwdPlain: return &fwd32_launch<Elt, kFwdPlain>;
    case kFwdJvp: return &fwd32_launch<Elt, kFwdJvp>;
    case kFwdJvpQOnly: return &fwd32_launch<Elt, kFwdJvpQOnly>;
    default: return nullptr;
  }
}

}  // namespace dmad
