// Instantiates the dO-only dQ pass for 64-, 128- and 256-wide heads
// (attn_bwd_dq_tr_kernel) for one element type (-DDMAD_T=<0 bf16 | 1 f16>). This
// unit is compiled with MFMAs in VGPR form: at D = 128 the kernel then fits 256
// VGPRs with no AGPRs, the score tiles need no AGPR->VGPR copies before the
// softmax, and two workgroups share a CU (64 KiB of LDS each); D = 256 keeps Q
// and dO in AGPRs, one workgroup per CU.
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
static hipError_t dq_tr_launch(const DqParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_dq_tr_kernel<T, D>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <>
DqLaunchFn dq_tr_select<Elt, 64>() {
  return &dq_tr_launch<Elt, 64>;
}
template <>
DqLaunchFn dq_tr_select<Elt, 128>() {
  return &dq_tr_launch<Elt, 128>;
}
template <>
DqLaunchFn dq_tr_select<Elt, 256>() {
  return &dq_tr_launch<Elt, 256>;
}

}  // namespace dmad
