// Launcher table shared by the per-(dtype, head-dim) instantiation units and
// the C ABI. Each unit is one compilation of fwd_inst.hip / bwd_inst.hip with
// DMAD_T and DMAD_D set, so the kernels build in parallel.
#pragma once
#include <hip/hip_runtime.h>
#include "attn_fwd.h"

namespace dmad {

typedef hipError_t (*FwdLaunchFn)(const FwdParams&, int grid, hipStream_t);

// Launcher for attn_fwd_kernel<T, DQK, DV, MODE>, or nullptr if (DV, MODE) is unsupported.
template <typename T, int DQK>
FwdLaunchFn fwd_select(int dv, int mode);

hipError_t launch_transpose_pad(const TransposeParams& p, int BH, hipStream_t s);

}  // namespace dmad
