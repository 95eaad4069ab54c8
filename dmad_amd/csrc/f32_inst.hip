// Instantiates the fp32 kernels (attn_f32.h) for one Q/K head dim: compiled
// once per head dim with -DDMAD_D=<Dqk>.
#include "launch.h"

#ifndef DMAD_D
#error "DMAD_D must be defined"
#endif

namespace dmad {

// the launcher's grid matches the kernel's query tile and column chunks
template <int DV, int MODE, bool MAGI>
constexpr bool f32_grid_matches() {
  using C = F32FwdCfg<DMAD_D, DV, MODE, MAGI>;
  return C::NCH == f32_fwd_chunks(MODE, DMAD_D, DV) && C::BM == f32_fwd_bm(MODE, DMAD_D) &&
         C::TASK_ROWS == kMagiBlockM;
}
static_assert(f32_grid_matches<256, kFwdJvp, false>() && f32_grid_matches<256, kFwdJvp, true>() &&
                  f32_grid_matches<128, kFwdJvp, false>() && f32_grid_matches<64, kFwdJvp, true>() &&
                  f32_grid_matches<256, kFwdJvpQOnly, false>() && f32_grid_matches<256, kFwdJvpQOnly, true>() &&
                  f32_grid_matches<256, kFwdPlain, false>() && f32_grid_matches<128, kFwdPlain, false>(),
              "the launcher's grid matches the kernel's query tile and column chunks");

template <int DQK, int DV, int MODE, bool MAGI>
static hipError_t f32_fwd_launch(const FwdParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attn_f32_fwd_kernel<DQK, DV, MODE, MAGI>), dim3(grid),
                     dim3(F32FwdCfg<DQK, DV, MODE, MAGI>::NT), 0, s, p);
  return hipGetLastError();
}

template <int DQK, int DV>
static FwdLaunchFn f32_fwd_mode(int mode, bool magi) {
  if (magi) {
    switch (mode) {
      case kFwdJvp: return &f32_fwd_launch<DQK, DV, kFwdJvp, true>;
      case kFwdJvpQOnly: return &f32_fwd_launch<DQK, DV, kFwdJvpQOnly, true>;
      default: return nullptr;
    }
  }
  switch (mode) {
    case kFwdPlain: return &f32_fwd_launch<DQK, DV, kFwdPlain, false>;
    case kFwdJvp: return &f32_fwd_launch<DQK, DV, kFwdJvp, false>;
    case kFwdJvpQOnly: return &f32_fwd_launch<DQK, DV, kFwdJvpQOnly, false>;
    default: return nullptr;
  }
}

template <>
FwdLaunchFn f32_fwd_select<DMAD_D>(int dv, int mode, bool magi) {
  switch (dv) {
    case 16: return f32_fwd_mode<DMAD_D, 16>(mode, magi);
    case 32: return f32_fwd_mode<DMAD_D, 32>(mode, magi);
    case 64: return f32_fwd_mode<DMAD_D, 64>(mode, magi);
    case 128: return f32_fwd_mode<DMAD_D, 128>(mode, magi);
    case 256: return f32_fwd_mode<DMAD_D, 256>(mode, magi);
    default: return nullptr;
  }
}

template <int D>
static hipError_t f32_prep_launch(const F32PrepParams& p, hipStream_t s) {
  const int64_t rows = (int64_t)p.BH * p.LQP;
  hipLaunchKernelGGL((attn_f32_bwd_prep_kernel<D>), dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int D>
static hipError_t f32_kv_launch(const BwdParams& p, const float* lse2, const float* dd, hipStream_t s) {
  using C = F32KvCfg<D>;
  const int grid = (p.Lk + C::BK - 1) / C::BK * p.B * p.H;
  hipLaunchKernelGGL((attn_f32_bwd_kv_kernel<D>), dim3(grid), dim3(C::NT), 0, s, p, lse2, dd);
  return hipGetLastError();
}

template <int D>
static hipError_t f32_dq_launch(const DqParams& p, const float* lse2, const float* dd, hipStream_t s) {
  using C = F32DqCfg<D>;
  const int grid = (p.Lq + C::BM - 1) / C::BM * p.B * p.H;
  hipLaunchKernelGGL((attn_f32_bwd_dq_kernel<D>), dim3(grid), dim3(C::NT), 0, s, p, lse2, dd);
  return hipGetLastError();
}

template <>
F32BwdFns f32_bwd_select<DMAD_D>() {
  return F32BwdFns{&f32_prep_launch<DMAD_D>, &f32_kv_launch<DMAD_D>, &f32_dq_launch<DMAD_D>};
}

}  // namespace dmad
