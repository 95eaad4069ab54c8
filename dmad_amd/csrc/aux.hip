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

// D/8 consecutive lanes share one query row, each lane reading 16 bytes of O,
// dO (and Od, dOd): every load instruction reads whole rows, and the per-row
// dot products finish with a butterfly over those lanes.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_prep_kernel(PrepParams p) {
  constexpr int LPR = D / 8;        // lanes per row
  constexpr int RPB = 256 / LPR;    // rows per workgroup
  const int sub = threadIdx.x % LPR;
  const int64_t gid = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const bool live = gid < (int64_t)p.BH * p.LQP;
  const int bh = live ? (int)(gid / p.LQP) : 0, q = live ? (int)(gid - (int64_t)bh * p.LQP) : p.Lq;
  const int b = bh / p.H, h = bh - b * p.H;
  const bool full = p.dto != nullptr;
  float d_o = 0.f, d_to = 0.f, rho = 0.f;
  if (q < p.Lq) {
    const int d = 8 * sub;
    const uint16_t* o = (const uint16_t*)p.o + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_sl + d;
    const uint16_t* dd = (const uint16_t*)p.dout + b * p.do_sb + h * p.do_sh + (int64_t)q * p.do_sl + d;
    d_o = dot8<T>(dd, o);
    if (full) {
      const uint16_t* to = (const uint16_t*)p.to + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_sl + d;
      const uint16_t* dt = (const uint16_t*)p.dto + b * p.do_sb + h * p.do_sh + (int64_t)q * p.do_sl + d;
      d_to = dot8<T>(dt, to);
      rho = dot8<T>(dt, o);
    }
  }
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) {
    d_o += __shfl_xor(d_o, m);
    if (full) {
      d_to += __shfl_xor(d_to, m);
      rho += __shfl_xor(rho, m);
    }
  }
  if (!live || sub != 0) return;
  float lse2 = __builtin_inff(), mu = 0.f;
  if (q < p.Lq) {
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

template <typename T>
static hipError_t launch_prep_t(const PrepParams& p, hipStream_t s) {
  const int64_t rows = (int64_t)p.BH * p.LQP;
  auto go = [&](auto kern, int lpr) {
    const int64_t nb = (rows * lpr + 255) / 256;
    hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(256), 0, s, p);
  };
  switch (p.D) {
    case 16: go(bwd_prep_kernel<T, 16>, 2); break;
    case 32: go(bwd_prep_kernel<T, 32>, 4); break;
    case 64: go(bwd_prep_kernel<T, 64>, 8); break;
    case 128: go(bwd_prep_kernel<T, 128>, 16); break;
    case 256: go(bwd_prep_kernel<T, 256>, 32); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_prep(const PrepParams& p, int dtype, hipStream_t s) {
  if ((int64_t)p.BH * p.LQP == 0) return hipSuccess;
  return dtype == 0 ? launch_prep_t<__bf16>(p, s) : launch_prep_t<_Float16>(p, s);
}

}  // namespace dmad
