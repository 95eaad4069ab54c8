// Layout kernels around the attention passes (HBM-bound, O(L*D) work).
#include "launch.h"

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
  dim3 grid(((p.LP + 63) / 64) * BH, (p.DP + 63) / 64, 1);
  hipLaunchKernelGGL(transpose_pad_kernel, grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace dmad
