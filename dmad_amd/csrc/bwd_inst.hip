// Instantiates the backward kernels for one (element type, head dim) pair:
// compiled once per pair with -DDMAD_T=<0 bf16 | 1 f16> -DDMAD_D=<D> and
// MFMAs in VGPR form (the score tiles feed P, dS on the VALU with no copies out
// of AGPRs).
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

// The launch choice below is the one launch.h names (kv_dout_only_name, dq_dout_only_name);
// it mirrors dout_only_kv_bmq<D>().
// (the dO-only passes for 64- and 128-wide heads, attn_bwd_kv_tr_kernel and
// attn_bwd_dq_tr_kernel, are compiled in bwd_kv_inst.hip and bwd_dq_inst.hip
// and selected in bwd_select / dq_select)
template <typename T, int D, int MODE>
static hipError_t bwd_launch(const BwdParams& p, int grid, hipStream_t s) {
  if constexpr (MODE == kBwdDoutOnly && kv_dout_only_pipe<D>())
    hipLaunchKernelGGL((attn_bwd_kv_pipe_kernel<T, D>), dim3(grid), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((attn_bwd_kernel<T, D, MODE>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int D, int MODE>
static hipError_t dq_launch(const DqParams& p, int grid, hipStream_t s) {
  if constexpr (MODE == kBwdDoutOnly && dq_dout_only_pipe<D>())
    hipLaunchKernelGGL((attn_bwd_dq_pipe_kernel<T, D>), dim3(grid), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, MODE>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <>
DqLaunchFn dq_select<Elt, DMAD_D>(int mode) {
  if (mode == kBwdDoutOnly) {
    if constexpr (dq_dout_only_rows<DMAD_D>()) return dq_tr_select<Elt, DMAD_D>();  // bwd_dq_inst.hip
    else return &dq_launch<Elt, DMAD_D, kBwdDoutOnly>;
  }
#if DMAD_D <= 128
  if (mode == kBwdFull) return &dq_launch<Elt, DMAD_D, kBwdFull>;
#endif
  return nullptr;
}

template <>
BwdLaunchFn bwd_select<Elt, DMAD_D>(int mode) {
  if (mode == kBwdDoutOnly) {
    if constexpr (kv_dout_only_rows<DMAD_D>()) return kv_tr_select<Elt, DMAD_D>();  // bwd_kv_inst.hip
    else return &bwd_launch<Elt, DMAD_D, kBwdDoutOnly>;
  }
#if DMAD_D <= 128
  if (mode == kBwdFull) return &bwd_launch<Elt, DMAD_D, kBwdFull>;
#endif
  return nullptr;
}

}  // namespace dmad
