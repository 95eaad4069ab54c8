// Instantiates the full-derivative passes for 128-wide heads (attn_bwd_full.h)
// for one element type (-DDMAD_T=<0 bf16 | 1 f16>). Compiled with MFMAs in VGPR
// form: the score tiles feed the VALU without AGPR->VGPR copies, while the
// stationary rows and the accumulators stay in AGPRs.
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

template <typename T>
static hipError_t kv_full_launch(const BwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kv_full_kernel<T, 128>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, bool TG>
static hipError_t dq_full_launch(const DqParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_dq_full_kernel<T, 128, TG>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <>
BwdLaunchFn kv_full_select<Elt>() {
  return &kv_full_launch<Elt>;
}

// Stored-score backward (launch.h): the full-derivative key pass writing dS,
// dSd and the query pass over them here; the dO-only pair in bwd_kv_inst.hip.
template <typename T>
static hipError_t kv_full_sc_launch(const BwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kv_full_kernel<T, 128, true>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}
template <typename T>
static hipError_t dq_sc2_launch(const DqParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_dq_sc_kernel<T, 2>), dim3(grid), dim3(DqScCfg<2>::NW * 64), 0, s, p);
  return hipGetLastError();
}
template <>
BwdLaunchFn kv_sc_select<Elt>(bool full) {
  return full ? &kv_full_sc_launch<Elt> : kv_sc_dout_only<Elt>();
}
template <>
DqLaunchFn dq_sc_select<Elt>(bool full) {
  return full ? &dq_sc2_launch<Elt> : dq_sc_dout_only<Elt>();
}

template <>
DqLaunchFn dq_full_select<Elt>(bool tangent_grads) {
  return tangent_grads ? &dq_full_launch<Elt, true> : &dq_full_launch<Elt, false>;
}

}  // namespace dmad
