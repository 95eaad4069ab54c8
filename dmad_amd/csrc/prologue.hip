// Fused attention-input prologue for gfx950: RMSNorm over the model dim and
// interleaved RoPE, for a Linear output and (optionally) its tangent, in one
// HBM pass.
//
// Per token row y (C = H*D values) and tangent ty, restating the reference's
// composition (WanRMSNorm._forward under torch.func.jvp,
// train/wan/rcm/networks/wan2pt1_jvp.py:207-216, then apply_rope_with_tangent,
// train/wan/rcm/utils/rope.py:56-70, 106-114):
//   r  = rsqrt(mean(y^2) + eps),  r' = -0.5 r^3 mean(2 y ty)        (float32)
//   q  = T(T(y r) * w),           q' = T(T(ty r + y r') * w)        (T = input type)
//   rotation of each pair (x[2i], x[2i+1]) of a head by angle freqs[l, i]:
//   x[2i] c - x[2i+1] s,  x[2i+1] c + x[2i] s   in float32, rounded to T
// with the same rounding points as the reference (the two products and the
// sum of the rotation are rounded separately: no fused multiply-add there).
//
// One wave per row: lane l owns the 16-byte chunks l, l+64, l+128, ... of the
// row, so every load and store instruction moves whole 1 KiB row segments.
// Chunk c sits at position c mod (D/8) inside its head. When D/8 divides 64
// (D = 8, 16, 32, 64, 128, 256, 512) that position is the same for all of a
// lane's chunks, so the sine and cosine of its 4 angles are computed once per
// row; where 4 or more lanes share a position (D <= 128) each of them computes
// one of the 4 and takes the others by cross-lane reads (sincosf takes its
// full range reduction at RoPE's large angles: 4-5% of the kernel at the 14B
// shape). For other head dims (D = 24, 40, 96, ...) the angles are recomputed
// per chunk. HBM-bound: per row 2C (or 4C with the tangent) bytes
// in and out, the weight and angles from cache.
#include "launch.h"

namespace dmad {

// NORM = false (no weight): the rotation alone, RoPE-with-tangent of
// train/wan/rcm/utils/rope.py:106-114 on its own.
template <typename T, int MAXC, bool JVP, bool ROPE, bool NORM>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(PrologueParams p) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // wave-uniform
  const int nch = p.C >> 3;   // 16-byte chunks per row
  const char* yrow = (const char*)p.y + row * p.y_stride * 2;
  const char* tyrow = JVP ? (const char*)p.ty + row * p.y_stride * 2 : nullptr;

  i32x4_t yv[MAXC], tv[MAXC];
  float s2 = 0.f, sd = 0.f;
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      // streamed once: non-temporal loads and stores keep them from churning the caches
      yv[j] = __builtin_nontemporal_load((const i32x4_t*)(yrow + c * 16));
      if constexpr (JVP) tv[j] = __builtin_nontemporal_load((const i32x4_t*)(tyrow + c * 16));
      if constexpr (!NORM) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t wy = (uint32_t)yv[j][e >> 1];
        const float a = Elem<T>::to_f32((uint16_t)((e & 1) ? (wy >> 16) : (wy & 0xffff)));
        s2 = fmaf(a, a, s2);
        if constexpr (JVP) {
          const uint32_t wt = (uint32_t)tv[j][e >> 1];
          const float b = Elem<T>::to_f32((uint16_t)((e & 1) ? (wt >> 16) : (wt & 0xffff)));
          sd = fmaf(a, b, sd);
        }
      }
    }
  }
  float r = 1.f, rd = 0.f;
  if constexpr (NORM) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      s2 += __shfl_xor(s2, m);
      if constexpr (JVP) sd += __shfl_xor(sd, m);
    }
    const float mean = s2 * p.inv_c;
    r = 1.0f / __builtin_sqrtf(mean + p.eps);
    rd = -0.5f * (r * r * r) * (2.0f * sd * p.inv_c);
  }

  // rotation angles of the 4 pairs of chunk c: i = 4 (c mod D/8) + k
  float cs[4], sn[4];
  const int cpd = p.D >> 3;                  // chunks per head
  const bool same_pos = (64 % cpd) == 0;     // every chunk of a lane at one in-head position
  const float* frow = nullptr;
  auto angles = [&](int c) {
    const float* f = frow + 4 * (c % cpd);
#pragma unroll
    for (int k = 0; k < 4; ++k) sincosf(f[k], &sn[k], &cs[k]);
  };
  if constexpr (ROPE) {
    frow = p.freqs + (int64_t)(row % p.L) * (p.D >> 1);
    if (same_pos && cpd <= 16) {
      // the 64 / cpd >= 4 lanes at one in-head position share its 4 angles:
      // lane computes angle (lane / cpd) % 4 and takes the others from the
      // lanes p + cpd k that computed them (same values, a quarter of the work)
      const int pos = lane % cpd, own = (lane / cpd) & 3;
      float s0, c0;
      sincosf(frow[4 * pos + own], &s0, &c0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sn[k] = __shfl(s0, pos + cpd * k);
        cs[k] = __shfl(c0, pos + cpd * k);
      }
    } else {
      angles(lane);
    }
  }

  char* orow = (char*)p.out + row * p.o_stride * 2;
  char* torow = JVP ? (char*)p.tout + row * p.o_stride * 2 : nullptr;
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) continue;
    i32x4_t wv = {};
    if constexpr (NORM) wv = *(const i32x4_t*)((const char*)p.w + c * 16);
    float q[8], tq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sh = (e & 1) ? 16 : 0;
      const float a = Elem<T>::to_f32((uint16_t)(((uint32_t)yv[j][e >> 1] >> sh) & 0xffff));
      float b = 0.f;
      if constexpr (JVP) b = Elem<T>::to_f32((uint16_t)(((uint32_t)tv[j][e >> 1] >> sh) & 0xffff));
      if constexpr (NORM) {
        const float w = Elem<T>::to_f32((uint16_t)(((uint32_t)wv[e >> 1] >> sh) & 0xffff));
        q[e] = Elem<T>::round(Elem<T>::round(__fmul_rn(a, r)) * w);
        if constexpr (JVP) tq[e] = Elem<T>::round(Elem<T>::round(__fadd_rn(__fmul_rn(b, r), __fmul_rn(a, rd))) * w);
      } else {
        q[e] = a;
        tq[e] = b;
      }
    }
    if constexpr (ROPE) {
      if (j > 0 && !same_pos) angles(c);  // wave-uniform branch
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float xe = q[2 * k], xo = q[2 * k + 1];
        q[2 * k] = __fadd_rn(__fmul_rn(xe, cs[k]), -__fmul_rn(xo, sn[k]));
        q[2 * k + 1] = __fadd_rn(__fmul_rn(xo, cs[k]), __fmul_rn(xe, sn[k]));
        if constexpr (JVP) {
          const float te = tq[2 * k], to = tq[2 * k + 1];
          tq[2 * k] = __fadd_rn(__fmul_rn(te, cs[k]), -__fmul_rn(to, sn[k]));
          tq[2 * k + 1] = __fadd_rn(__fmul_rn(to, cs[k]), __fmul_rn(te, sn[k]));
        }
      }
    }
    i32x4_t ov, tov;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ov[k] = (int)Elem<T>::pack2(q[2 * k], q[2 * k + 1]);
      if constexpr (JVP) tov[k] = (int)Elem<T>::pack2(tq[2 * k], tq[2 * k + 1]);
    }
    __builtin_nontemporal_store(ov, (i32x4_t*)(orow + c * 16));
    if constexpr (JVP) __builtin_nontemporal_store(tov, (i32x4_t*)(torow + c * 16));
  }
}

template <typename T, bool JVP, bool ROPE, bool NORM>
static hipError_t prologue_launch_t(const PrologueParams& p, hipStream_t s) {
  const unsigned grid = (unsigned)((p.rows + 3) / 4);
  if (p.C <= 64 * 8 * 4)
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, 4, JVP, ROPE, NORM>), dim3(grid), dim3(256), 0, s, p);
  else if (p.C <= 64 * 8 * 10)  // Wan2.1-14B, C = 5120: 126 VGPRs, four waves per SIMD
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, 10, JVP, ROPE, NORM>), dim3(grid), dim3(256), 0, s, p);
  else if (p.C <= 64 * 8 * 12)
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, 12, JVP, ROPE, NORM>), dim3(grid), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, kPrologueMaxChunks, JVP, ROPE, NORM>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, bool NORM>
static hipError_t prologue_launch_n(const PrologueParams& p, hipStream_t s) {
  const bool jvp = p.ty != nullptr, rope = p.freqs != nullptr;
  if (jvp && rope) return prologue_launch_t<T, true, true, NORM>(p, s);
  if (jvp) return prologue_launch_t<T, true, false, NORM>(p, s);
  if (rope) return prologue_launch_t<T, false, true, NORM>(p, s);
  return prologue_launch_t<T, false, false, NORM>(p, s);
}

template <typename T>
static hipError_t prologue_launch_d(const PrologueParams& p, hipStream_t s) {
  return p.w != nullptr ? prologue_launch_n<T, true>(p, s) : prologue_launch_n<T, false>(p, s);
}

hipError_t launch_rmsnorm_rope(const PrologueParams& p, int dtype, hipStream_t s) {
  if (p.rows == 0) return hipSuccess;
  return dtype == 0 ? prologue_launch_d<__bf16>(p, s) : prologue_launch_d<_Float16>(p, s);
}

}  // namespace dmad
