// Instantiates the dO-only dK/dV pass for 64- and 128-wide heads (attn_bwd_kv_tr_kernel)
// for one element type (-DDMAD_T=<0 bf16 | 1 f16>). This unit is compiled with
// MFMAs in VGPR form, so the score tiles feed the softmax without AGPR->VGPR
// copies; the dK, dV accumulators are kept in AGPRs by the kernel itself.
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

template <typename T, int D>
static hipError_t kv_tr_launch(const BwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kv_tr_kernel<T, D>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <>
BwdLaunchFn kv_tr_select<Elt, 64>() {
  return &kv_tr_launch<Elt, 64>;
}
template <>
BwdLaunchFn kv_tr_select<Elt, 128>() {
  return &kv_tr_launch<Elt, 128>;
}

// dO-only half of the stored-score backward: the key pass writing dS and the
// query pass reading it back (the full-derivative half is in bwd_full_inst.hip)
template <typename T>
static hipError_t kv_sc_launch(const BwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kv_tr_kernel<T, 128, kScStore>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}
// the full derivative's tangent key pass on the dSd its key pass stored
template <typename T>
static hipError_t kv_ld_launch(const BwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kv_tr_kernel<T, 128, kScLoad>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}
template <typename T>
static hipError_t dq_sc1_launch(const DqParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_dq_sc_kernel<T, 1>), dim3(grid), dim3(DqScCfg<1>::NW * 64), 0, s, p);
  return hipGetLastError();
}
template <>
BwdLaunchFn kv_sc_dout_only<Elt>() {
  return &kv_sc_launch<Elt>;
}
template <>
DqLaunchFn dq_sc_dout_only<Elt>() {
  return &dq_sc1_launch<Elt>;
}
template <>
BwdLaunchFn kv_sc_tangent<Elt>() {
  return &kv_ld_launch<Elt>;
}

}  // namespace dmad
