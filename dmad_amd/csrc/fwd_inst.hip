// Instantiates the forward kernels for one (element type, Dqk) pair:
// compiled once per pair with -DDMAD_T=<0 bf16 | 1 f16> -DDMAD_D=<Dqk> and
// MFMAs in VGPR form (their results feed the softmax's VALU work directly,
// with no copies out of AGPRs).
#include "launch.h"

#ifndef DMAD_T
#error "DMAD_T must be defined"
#endif
#ifndef DMAD_D
#error "DMAD_D must be defined"
#endif

namespace dmad {

#if DMAD_T == 0
using Elt = __bf16;
#else
using Elt = _Float16;
#endif

static_assert(FwdSimpleCfg<DMAD_D, 16, kFwdJvp>::BM == kMagiBlockM, "block-sparse tasks are 128-query tiles");

static_assert(fwd_simple_dvc(kFwdJvp, 256) * fwd_generic_chunks(kFwdJvp, 256, 256, true) == 256,
              "the launcher's grid matches the kernel's V halves");

template <typename T, int DQK, int DV, int MODE>
static hipError_t fwd_launch(const FwdParams& p, int grid, hipStream_t s) {
  constexpr GenericFwd kind = generic_fwd_kind<DQK, DV, MODE>();  // launch.h
  if constexpr (kind == GenericFwd::kStream)
    hipLaunchKernelGGL((attn_fwd_stream_kernel<T, DQK, DV, MODE>), dim3(grid), dim3(512), 0, s, p);
  else if constexpr (kind == GenericFwd::kTiled)
    hipLaunchKernelGGL((attn_fwd_kernel<T, DQK, DV, MODE>), dim3(grid), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((attn_fwd_simple_kernel<T, DQK, DV, MODE>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int DQK, int DV>
static FwdLaunchFn fwd_mode(int mode) {
  switch (mode) {
    case kFwdPlain: return &fwd_launch<T, DQK, DV, kFwdPlain>;
    case kFwdJvp: return &fwd_launch<T, DQK, DV, kFwdJvp>;
    case kFwdJvpQOnly: return &fwd_launch<T, DQK, DV, kFwdJvpQOnly>;
    default: return nullptr;
  }
}

template <typename T, int DQK, int DV, int MODE>
static hipError_t fwd_magi_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd_simple_kernel<T, DQK, DV, MODE, true>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int DQK, int DV>
static FwdLaunchFn fwd_magi_mode(int mode) {
  switch (mode) {
    case kFwdJvp: return &fwd_magi_launch<T, DQK, DV, kFwdJvp>;
    case kFwdJvpQOnly: return &fwd_magi_launch<T, DQK, DV, kFwdJvpQOnly>;
    default: return nullptr;
  }
}

template <>
FwdLaunchFn fwd_magi_select<Elt, DMAD_D>(int dv, int mode) {
  switch (dv) {
    case 16: return fwd_magi_mode<Elt, DMAD_D, 16>(mode);
    case 32: return fwd_magi_mode<Elt, DMAD_D, 32>(mode);
    case 64:
      if constexpr (fwd32_supported(DMAD_D, 64)) return fwd32_magi_select<Elt>(mode, 64);
      else return fwd_magi_mode<Elt, DMAD_D, 64>(mode);
    case 128:
      if constexpr (fwd32_supported(DMAD_D, 128)) return fwd32_magi_select<Elt>(mode, 128);
      else return fwd_magi_mode<Elt, DMAD_D, 128>(mode);
    case 256:
      if constexpr (fwd32_wide_supported(DMAD_D, 256)) return fwd32_magi_select<Elt>(mode, 256);
      else return fwd_magi_mode<Elt, DMAD_D, 256>(mode);
    default: return nullptr;
  }
}

template <>
FwdLaunchFn fwd_select<Elt, DMAD_D>(int dv, int mode) {
  switch (dv) {
    case 16: return fwd_mode<Elt, DMAD_D, 16>(mode);
    case 32: return fwd_mode<Elt, DMAD_D, 32>(mode);
    case 64:
      if constexpr (fwd32_supported(DMAD_D, 64)) return fwd32_select<Elt>(mode, 64);
      else return fwd_mode<Elt, DMAD_D, 64>(mode);
    case 128:
      if constexpr (fwd32_supported(DMAD_D, 128)) return fwd32_select<Elt>(mode, 128);
      else return fwd_mode<Elt, DMAD_D, 128>(mode);
    case 256:
      if constexpr (fwd32_wide_supported(DMAD_D, 256)) return fwd32_select<Elt>(mode, 256);
      else return fwd_mode<Elt, DMAD_D, 256>(mode);
    default: return nullptr;
  }
}

}  // namespace dmad
