// Layout kernels around the attention passes (HBM-bound, O(L*D) work).
#include "launch.h"
#include "attn_bwd.h"

namespace dmad {

// One 64 (l) x 64 (d) tile per workgroup through LDS: reads are coalesced
// along d, writes along l.
__global__ __launch_bounds__(256) void transpose_pad_kernel(TransposeParams p) {
  __shared__ uint16_t tile[64][66];
  const int nlt = (p.LP + 63) >> 6;
  const int bh = blockIdx.x / nlt;
  const int l0 = (blockIdx.x - bh * nlt) * 64, d0 = blockIdx.y * 64;
  const int b = bh / p.H, h = bh - b * p.H;
  const uint16_t* x = (const uint16_t*)p.x + b * p.sb + h * p.sh;
  uint16_t* y = (uint16_t*)p.y + (int64_t)bh * p.DP * p.LP;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = tid + 256 * i;
    const int ll = idx >> 6, dd = idx & 63;
    const int l = l0 + ll, d = d0 + dd;
    tile[ll][dd] = (l < p.L && d < p.D) ? x[(int64_t)l * p.sl + d] : (uint16_t)0;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = tid + 256 * i;
    const int dd = idx >> 6, ll = idx & 63;
    const int l = l0 + ll, d = d0 + dd;
    if (d < p.DP && l < p.LP) y[(int64_t)d * p.LP + l] = tile[ll][dd];
  }
}

hipError_t launch_transpose_pad(const TransposeParams& p, int BH, hipStream_t s) {
  if (p.LP == 0 || BH == 0) return hipSuccess;
  dim3 grid(((p.LP + 63) / 64) * BH, (p.DP + 63) / 64, 1);
  hipLaunchKernelGGL(transpose_pad_kernel, grid, dim3(256), 0, s, p);
  return hipGetLastError();
}


// ---------------------------------------------------------------- backward helpers

template <typename T>
__device__ __forceinline__ float dot8(const uint16_t* a, const uint16_t* b) {
  const i32x4_t x = *(const i32x4_t*)a, y = *(const i32x4_t*)b;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = (uint32_t)x[i], w = (uint32_t)y[i];
    s = fmaf(Elem<T>::to_f32((uint16_t)(u & 0xffff)), Elem<T>::to_f32((uint16_t)(w & 0xffff)), s);
    s = fmaf(Elem<T>::to_f32((uint16_t)(u >> 16)), Elem<T>::to_f32((uint16_t)(w >> 16)), s);
  }
  return s;
}

template <typename T>
__global__ __launch_bounds__(256) void bwd_prep_kernel(PrepParams p) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)p.BH * p.LQP) return;
  const int bh = (int)(gid / p.LQP), q = (int)(gid - (int64_t)bh * p.LQP);
  const int b = bh / p.H, h = bh - b * p.H;
  float lse2 = __builtin_inff(), d_o = 0.f, d_to = 0.f, rho = 0.f, mu = 0.f;
  if (q < p.Lq) {
    const uint16_t* o = (const uint16_t*)p.o + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_sl;
    const uint16_t* dd = (const uint16_t*)p.dout + b * p.do_sb + h * p.do_sh + (int64_t)q * p.do_sl;
    const bool full = p.dto != nullptr;
    const uint16_t* to = full ? (const uint16_t*)p.to + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_sl : nullptr;
    const uint16_t* dt = full ? (const uint16_t*)p.dto + b * p.do_sb + h * p.do_sh + (int64_t)q * p.do_sl : nullptr;
    for (int d = 0; d < p.D; d += 8) {
      d_o += dot8<T>(dd + d, o + d);
      if (full) {
        d_to += dot8<T>(dt + d, to + d);
        rho += dot8<T>(dt + d, o + d);
      }
    }
    lse2 = p.lse[(int64_t)bh * p.Lq + q] * 1.4426950408889634f;
    if (full) mu = p.mu[(int64_t)bh * p.Lq + q];
  }
  if (p.stats_a) {
    float* s = p.stats_a + ((int64_t)bh * (p.LQP / p.BA) + q / p.BA) * 2 * p.BA + q % p.BA;
    s[0] = lse2;
    s[p.BA] = d_o;
  }
  if (p.stats_b) {
    float* s = p.stats_b + ((int64_t)bh * (p.LQP / 32) + q / 32) * 4 * 32 + q % 32;
    s[0] = lse2;
    s[32] = d_o + d_to - mu * rho;
    s[64] = mu;
    s[96] = rho;
  }
  if (p.stats_bt) {
    float* s = p.stats_bt + ((int64_t)bh * (p.LQP / p.BA) + q / p.BA) * 2 * p.BA + q % p.BA;
    s[0] = lse2;
    s[p.BA] = rho;
  }
}

static int64_t blocks_for(int64_t n) { return (n + 255) / 256; }

hipError_t launch_bwd_prep(const PrepParams& p, int dtype, hipStream_t s) {
  const int64_t nb = blocks_for((int64_t)p.BH * p.LQP);
  if (nb == 0) return hipSuccess;
  if (dtype == 0) hipLaunchKernelGGL(bwd_prep_kernel<__bf16>, dim3((unsigned)nb), dim3(256), 0, s, p);
  else hipLaunchKernelGGL(bwd_prep_kernel<_Float16>, dim3((unsigned)nb), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace dmad
