// dQ (and, for the full derivative, the Qd contribution) of the attention
// backward, as a query-stationary pass: no atomics, every dQ element is
// written once by the workgroup that owns its query row.
//
//   dO-only (mode A):  dS = P*(dO V^T - D),             dQ = s dS K
//   full    (mode B):  dS, dSd as in attn_bwd.h,         dQ = s(dS K + dSd Kd)
// with P = exp2(s*log2(e) * Q K^T - lse2) recomputed from the saved LSE.
//
// Layout mirrors the forward kernel: one workgroup = 4 waves = 128 query rows
// of one head; lane l of a wave owns query l%32, whose Q and dO (and Qd, dOd)
// slices stay in registers as B operands of S^T = K Q^T and dP^T = V dO^T.
// K, V (and Kd, Vd) rows and K^T (and Kd^T, from a transposed copy) stream
// through a double-buffered LDS ring. dS^T leaves the score C tile in
// B-operand layout (K rows are read in perm32 order), and dQ^T = K^T dS^T
// accumulates in registers with lane <-> query, so the per-row statistics are
// per-lane scalars.
#pragma once
#include <type_traits>

#include "attn_fwd.h"
#include "common.h"

namespace dmad {

struct DqParams {
  const void* q;
  const void* tq;
  const void* dout;
  const void* dto;
  const void* k;
  const void* tk;
  const void* v;
  const void* tv;
  const void* kT;   // K^T  [BH][DP][LKP]
  const void* tkT;  // Kd^T [BH][DP][LKP] (mode B)
  const float* stats;  // per-row statistics in the layout of the key-stationary kernel
  void* dq;
  void* dtq;  // dQd (full derivative with tangent gradients, 128-wide heads)
  int64_t q_sb, q_sh, q_sl;     // shared by Q, Qd
  int64_t do_sb, do_sh, do_sl;  // shared by dO, dOd
  int64_t k_sb, k_sh, k_sl;     // shared by K, Kd
  int64_t v_sb, v_sh, v_sl;     // shared by V, Vd
  int64_t dq_sb, dq_sh, dq_sl;
  int B, H, Lq, Lk, LQP, LKP;
  int stat_tile;  // query tile of the statistics layout
  float scale, scale_log2;
  int xcd_order;  // work items contiguous per XCD (common.h)
  // attn_bwd_dq_sc_kernel: the score gradients a STORE key pass wrote (ScLayout
  // in attn_bwd.h) for (b, h) slices bh0 .. bh0 + grid / query blocks - 1, slice
  // bh - bh0 at sc + (bh - bh0) sc_slice, with sc_nkb key blocks of 32
  const void* sc;
  int64_t sc_slice;
  int sc_nkb;
  int bh0;
};

template <int D, int MODE>
struct DqCfg {
  static constexpr int NW = 4;
  static constexpr int BM = 32 * NW;
  static constexpr int DP = D < 32 ? 32 : D;
  static constexpr bool FULL = MODE == 1;
  static constexpr int BN = (FULL || D > 128) ? 32 : 64;
  static constexpr int NB = BN / 32;
  static constexpr int KS = D / 16;
  static constexpr int DB = DP / 32;
  static constexpr int CK = D / 8;   // chunks per K / V row
  static constexpr int CT = BN / 8;  // chunks per K^T row
  static constexpr int NROW = FULL ? 4 : 2;  // K, V [, Kd, Vd]
  static constexpr int NTR = FULL ? 2 : 1;   // K^T [, Kd^T]
  static constexpr int ROW_BYTES = BN * D * 2;
  static constexpr int TR_BYTES = DP * BN * 2;
  static constexpr int OFF_TR = NROW * ROW_BYTES;
  static constexpr int STAGE = NROW * ROW_BYTES + NTR * TR_BYTES;
  static constexpr int NRI = BN * CK / 64;
  static constexpr int NTI = DP * CT / 64;
  static constexpr int RPW = (NRI + NW - 1) / NW;
  static constexpr int TPW = (NTI + NW - 1) / NW;
  static constexpr int NSTAT = FULL ? 4 : 2;
};

template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(DqParams p) {
  using C = DqCfg<D, MODE>;
  constexpr int BN = C::BN, NB = C::NB, KS = C::KS, DB = C::DB, CK = C::CK, CT = C::CT;
  constexpr bool FULL = C::FULL;
  __shared__ __attribute__((aligned(1024))) char smem[2 * C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;

  // ---- per-lane query operands and statistics
  const int qrow = qt * C::BM + wave * 32 + col;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
  i32x4_t qr[KS], dor[KS], tqr[KS], dtor[KS];
  {
    const uint32_t qo = (uint32_t)((int64_t)qrow * p.q_sl * 2) + half * 16;
    const uint32_t oo = (uint32_t)((int64_t)qrow * p.do_sl * 2) + half * 16;
    __amdgpu_buffer_rsrc_t rtq = rq, rdto = rdo;
    if constexpr (FULL) {
      rtq = make_rsrc((const char*)p.tq + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
      rdto = make_rsrc((const char*)p.dto + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qr[s] = buf_load16(rq, qo + s * 32);
      dor[s] = buf_load16(rdo, oo + s * 32);
      if constexpr (FULL) {
        tqr[s] = buf_load16(rtq, qo + s * 32);
        dtor[s] = buf_load16(rdto, oo + s * 32);
      }
    }
  }
  float lse2 = __builtin_inff(), dlt = 0.f, mu = 0.f, rho = 0.f;
  if (qrow < p.LQP) {
    const float* st = p.stats + ((int64_t)bh * (p.LQP / p.stat_tile) + qrow / p.stat_tile) * C::NSTAT * p.stat_tile +
                      qrow % p.stat_tile;
    lse2 = st[0];
    dlt = st[p.stat_tile];
    if constexpr (FULL) {
      mu = st[2 * p.stat_tile];
      rho = st[3 * p.stat_tile];
    }
  }

  // ---- key-side resources and per-lane DMA offsets
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const uint32_t kt_bytes = (uint32_t)((int64_t)C::DP * p.LKP * 2);
  const __amdgpu_buffer_rsrc_t rrow[4] = {
      make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes),
      make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes),
      make_rsrc((const char*)(FULL ? p.tk : p.k) + (b * p.k_sb + h * p.k_sh) * 2, k_bytes),
      make_rsrc((const char*)(FULL ? p.tv : p.v) + (b * p.v_sb + h * p.v_sh) * 2, v_bytes)};
  const __amdgpu_buffer_rsrc_t rtr[2] = {
      make_rsrc((const char*)p.kT + (int64_t)bh * kt_bytes, kt_bytes),
      make_rsrc((const char*)(FULL ? p.tkT : p.kT) + (int64_t)bh * kt_bytes, kt_bytes)};
  const int64_t row_sl[4] = {p.k_sl, p.v_sl, p.k_sl, p.v_sl};
  uint32_t roff_k[C::RPW], roff_v[C::RPW], toff[C::TPW];
#pragma unroll
  for (int j = 0; j < C::RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CK, phys = pch % CK;
    const int logical = phys ^ swz<CK>(perm32(row & 31) & 15);
    roff_k[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
    roff_v[j] = (uint32_t)((int64_t)row * p.v_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < C::TPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CT, phys = pch % CT;
    const int logical = phys ^ swz<CT>(d & 15);
    toff[j] = (uint32_t)(d * p.LKP * 2) + logical * 16;
  }

  auto issue_tile = [&](int kt, int stage) {
    char* st = smem + stage * C::STAGE;
#pragma unroll
    for (int t = 0; t < C::NROW; ++t) {
      const uint32_t rs = (uint32_t)((int64_t)kt * BN * row_sl[t] * 2);
#pragma unroll
      for (int j = 0; j < C::RPW; ++j) {
        const int i = wave + j * C::NW;
        if (i < C::NRI) buf_load16_lds(rrow[t], st + t * C::ROW_BYTES + i * 1024, (t & 1) ? roff_v[j] : roff_k[j], rs);
      }
    }
#pragma unroll
    for (int t = 0; t < C::NTR; ++t) {
#pragma unroll
      for (int j = 0; j < C::TPW; ++j) {
        const int i = wave + j * C::NW;
        if (i < C::NTI) buf_load16_lds(rtr[t], st + C::OFF_TR + t * C::TR_BYTES + i * 1024, toff[j], (uint32_t)kt * BN * 2);
      }
    }
  };

  const int rswz = swz<CK>(col & 15), tswz = swz<CT>(col & 15);
  const int rrow_off = perm32(col) * CK * 16;
  const int trow_off = col * CT * 16;

  f32x16_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[d][v] = 0.f;
  }

  const int ntiles = (p.Lk + BN - 1) / BN;
  issue_tile(0, 0);
  for (int kt = 0; kt < ntiles; ++kt) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < ntiles) issue_tile(kt + 1, (kt + 1) & 1);
    const char* st = smem + (kt & 1) * C::STAGE;

    // ---- S^T, dP^T (and Sd^T, dPd^T) for BN keys x 32 queries
    f32x16_t sacc[NB], dpacc[NB], tsacc[NB], dpdacc[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        sacc[kb][v] = 0.f;
        dpacc[kb][v] = 0.f;
        tsacc[kb][v] = 0.f;
        dpdacc[kb][v] = 0.f;
      }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
        const int off = kb * 32 * CK * 16 + rrow_off + (((2 * s + half) ^ rswz) << 4);
        const i32x4_t ak = *(const i32x4_t*)(st + off);
        const i32x4_t av = *(const i32x4_t*)(st + C::ROW_BYTES + off);
        sacc[kb] = mfma32(ak, qr[s], sacc[kb], T());
        dpacc[kb] = mfma32(av, dor[s], dpacc[kb], T());
        if constexpr (FULL) {
          const i32x4_t atk = *(const i32x4_t*)(st + 2 * C::ROW_BYTES + off);
          const i32x4_t atv = *(const i32x4_t*)(st + 3 * C::ROW_BYTES + off);
          tsacc[kb] = mfma32(ak, tqr[s], tsacc[kb], T());
          tsacc[kb] = mfma32(atk, qr[s], tsacc[kb], T());
          dpacc[kb] = mfma32(atv, dtor[s], dpacc[kb], T());
          dpdacc[kb] = mfma32(av, dtor[s], dpdacc[kb], T());
        }
      }
    }

    // ---- the last tile may hold keys >= Lk: their scores -> -inf (P = 0)
    if ((kt + 1) * BN > p.Lk) {
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          if (kt * BN + kb * 32 + 16 * (v >> 3) + 8 * half + (v & 7) >= p.Lk) sacc[kb][v] = -__builtin_inff();
        }
      }
    }

    // ---- dS (and dSd); value v of block kb is key kt*BN + kb*32 + 16t + 8*half + e (v = 8t + e)
    i32x4_t dsb[NB][2], tdsb[NB][2];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float dsv[8], tdsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int v = 8 * t + e;
          const float pe = fast_exp2(fmaf(sacc[kb][v], p.scale_log2, -lse2));
          if constexpr (!FULL) {
            dsv[e] = pe * (dpacc[kb][v] - dlt);
          } else {
            const float sd = tsacc[kb][v] * p.scale;
            const float dpd = dpdacc[kb][v];
            const float dp = dpacc[kb][v] + dpd * (sd - mu) - sd * rho;
            dsv[e] = pe * (dp - dlt);
            tdsv[e] = pe * (dpd - rho);
          }
        }
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          dsb[kb][t][e2] = (int)Elem<T>::pack2(dsv[2 * e2], dsv[2 * e2 + 1]);
          if constexpr (FULL) tdsb[kb][t][e2] = (int)Elem<T>::pack2(tdsv[2 * e2], tdsv[2 * e2 + 1]);
        }
      }
    }

    // ---- dQ^T += K^T dS^T (+ Kd^T dSd^T)
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ch = ((kb * 4 + 2 * t + half) ^ tswz) << 4;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const int off = C::OFF_TR + d * 32 * CT * 16 + trow_off + ch;
          const i32x4_t akt = *(const i32x4_t*)(st + off);
          acc[d] = mfma32(akt, dsb[kb][t], acc[d], T());
          if constexpr (FULL) {
            const i32x4_t atkt = *(const i32x4_t*)(st + C::TR_BYTES + off);
            acc[d] = mfma32(atkt, tdsb[kb][t], acc[d], T());
          }
        }
      }
    }
  }

  // ---- dQ = s (dQ^T)^T
  if (qrow < p.Lq) {
    char* dqp = (char*)p.dq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)qrow * p.dq_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int dc = d * 32 + 8 * j + 4 * half;
        if (D >= 32 || dc < D) {
          u32x2_t w = {Elem<T>::pack2(acc[d][4 * j] * p.scale, acc[d][4 * j + 1] * p.scale),
                       Elem<T>::pack2(acc[d][4 * j + 2] * p.scale, acc[d][4 * j + 3] * p.scale)};
          *(u32x2_t*)(dqp + dc * 2) = w;
        }
      }
    }
  }
}

// 16-query-per-wave variant of the dO-only dQ pass (8 waves, 2 per SIMD,
// 16x16x32 MFMAs), pipelined like the forward kernel:
//   step i: MFMA dQ^T += K^T dS^T of tile i-1 || VALU P, dS of tile i;
//           then MFMA S^T, dP^T of tile i+1.
template <int D>
struct DqPipeCfg {
  static constexpr int NW = 8;
  static constexpr int QW = 16;
  static constexpr int BM = QW * NW;
  static constexpr int BN = 32;
  static constexpr int KS = D / 32;
  static constexpr int DB = D / 16;
  static constexpr int CK = D / 8;   // chunks per K / V row
  static constexpr int CT = BN / 8;  // chunks per K^T row
  static constexpr int KT_ROWS = D < 32 ? 32 : D;  // rows per head of the K^T workspace
  static constexpr int ROW_BYTES = BN * D * 2;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_V = ROW_BYTES;
  static constexpr int OFF_KT = 2 * ROW_BYTES;
  static constexpr int STAGE = 3 * ROW_BYTES;
  static constexpr int NSTAGE = 4;
  static constexpr bool FITS = D >= 32 && NSTAGE * STAGE <= 160 * 1024;
  static constexpr int NRI = BN * CK / 64;
  static constexpr int NTI = D * CT / 64;
  static constexpr int RPW = (NRI + NW - 1) / NW;
  static constexpr int TPW = (NTI + NW - 1) / NW;
};

template <typename T, int D>
__global__ __launch_bounds__(512) void attn_bwd_dq_pipe_kernel(DqParams p) {
  using C = DqPipeCfg<D>;
  constexpr int BN = C::BN, KS = C::KS, DB = C::DB, CK = C::CK, CT = C::CT, NST = C::NSTAGE;
  __shared__ __attribute__((aligned(1024))) char smem[NST * C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;

  // ---- per-lane query operands and statistics
  const int qrow = qt * C::BM + wave * C::QW + col;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
  i32x4_t qr[KS], dor[KS];
  {
    const uint32_t qo = (uint32_t)((int64_t)qrow * p.q_sl * 2) + grp * 16;
    const uint32_t oo = (uint32_t)((int64_t)qrow * p.do_sl * 2) + grp * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qr[s] = buf_load16(rq, qo + s * 64);
      dor[s] = buf_load16(rdo, oo + s * 64);
    }
  }
  float lse2 = __builtin_inff(), dlt = 0.f;
  if (qrow < p.LQP) {
    const float* st = p.stats + ((int64_t)bh * (p.LQP / p.stat_tile) + qrow / p.stat_tile) * 2 * p.stat_tile +
                      qrow % p.stat_tile;
    lse2 = st[0];
    dlt = st[p.stat_tile];
  }

  // ---- key-side resources and per-lane DMA offsets
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const uint32_t kt_bytes = (uint32_t)((int64_t)C::KT_ROWS * p.LKP * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  const __amdgpu_buffer_rsrc_t rkt = make_rsrc((const char*)p.kT + (int64_t)bh * kt_bytes, kt_bytes);
  uint32_t roff_k[C::RPW], roff_v[C::RPW], toff[C::TPW];
#pragma unroll
  for (int j = 0; j < C::RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CK, phys = pch % CK;
    const int logical = phys ^ kswz16<CK>(row);
    roff_k[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
    roff_v[j] = (uint32_t)((int64_t)row * p.v_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < C::TPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CT, phys = pch % CT;
    const int logical = phys ^ swz<CT>(d & 15);
    toff[j] = (uint32_t)(d * p.LKP * 2) + logical * 16;
  }
  const uint32_t k_step = (uint32_t)((int64_t)BN * p.k_sl * 2);
  const uint32_t v_step = (uint32_t)((int64_t)BN * p.v_sl * 2);

  auto stage_ptr = [&](int kt) -> const char* { return smem + (kt & (NST - 1)) * C::STAGE; };
  auto issue_tile = [&](int kt) {
    char* st = smem + (kt & (NST - 1)) * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::RPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NRI) {
        buf_load16_lds(rk, st + C::OFF_K + i * 1024, roff_k[j], (uint32_t)kt * k_step);
        buf_load16_lds(rv, st + C::OFF_V + i * 1024, roff_v[j], (uint32_t)kt * v_step);
      }
    }
#pragma unroll
    for (int j = 0; j < C::TPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NTI) buf_load16_lds(rkt, st + C::OFF_KT + i * 1024, toff[j], (uint32_t)kt * BN * 2);
    }
  };

  int krow_off[2], kswzv[2];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int R = key_of_row16(sb, col);
    krow_off[sb] = R * CK * 16;
    kswzv[sb] = kswz16<CK>(R);
  }
  const int trow_off = col * CT * 16 + ((grp ^ swz<CT>(col)) << 4);

  f32x4_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[d][v] = 0.f;
  }
  const int ntiles = (p.Lk + BN - 1) / BN;

  // S^T, dP^T of one 32-key tile
  f32x4_t sc[2], dpc[2];
  auto scores = [&](const char* st) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int off = krow_off[sb] + (((4 * s + grp) ^ kswzv[sb]) << 4);
        const i32x4_t ak = *(const i32x4_t*)(st + C::OFF_K + off);
        const i32x4_t av = *(const i32x4_t*)(st + C::OFF_V + off);
        if (s == 0) {
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
          sc[sb] = mfma16(ak, qr[0], z, T());
          dpc[sb] = mfma16(av, dor[0], z, T());
        } else {
          sc[sb] = mfma16(ak, qr[s], sc[sb], T());
          dpc[sb] = mfma16(av, dor[s], dpc[sb], T());
        }
      }
    }
  };
  // dS of one tile, packed as the B operand (keys 8*grp + e)
  auto dscore = [&](int kt, auto TAIL, i32x4_t& dsk) {
    float dsv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sb = e >> 2, v = e & 3;
      float pe = fast_exp2(fmaf(sc[sb][v], p.scale_log2, -lse2));
      if constexpr (decltype(TAIL)::value) {
        if (kt * BN + 8 * grp + 4 * sb + v >= p.Lk) pe = 0.f;
      }
      dsv[e] = pe * (dpc[sb][v] - dlt);
    }
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) dsk[e2] = (int)Elem<T>::pack2(dsv[2 * e2], dsv[2 * e2 + 1]);
  };
  auto dq_update = [&](const char* st, const i32x4_t& dsk) {
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const i32x4_t akt = *(const i32x4_t*)(st + C::OFF_KT + d * 16 * CT * 16 + trow_off);
      acc[d] = mfma16(akt, dsk, acc[d], T());
    }
  };

  issue_tile(0);
  if (ntiles > 1) issue_tile(1);
  if (ntiles > 2) issue_tile(2);
  wait_vmem();
  __syncthreads();
  i32x4_t dsk;
  scores(stage_ptr(0));
  if (ntiles == 1) {
    dscore(0, std::true_type(), dsk);
  } else {
    dscore(0, std::false_type(), dsk);
    scores(stage_ptr(1));
  }
  int i = 1;
  for (; i + 1 < ntiles; ++i) {
    wait_vmem();
    __syncthreads();
    if (i + 2 < ntiles) issue_tile(i + 2);
    i32x4_t dsn;
    dq_update(stage_ptr(i - 1), dsk);
    dscore(i, std::false_type(), dsn);
    scores(stage_ptr(i + 1));
    dsk = dsn;
  }
  if (ntiles > 1) {
    i32x4_t dsn;
    dq_update(stage_ptr(i - 1), dsk);
    dscore(i, std::true_type(), dsn);
    dsk = dsn;
  }
  dq_update(stage_ptr(ntiles - 1), dsk);

  // ---- dQ = s (dQ^T)^T: lane (query col, group g) holds d = 16*dblk + 4g + v
  if (qrow < p.Lq) {
    char* dqp = (char*)p.dq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)qrow * p.dq_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int dc = d * 16 + 4 * grp;
      u32x2_t w = {Elem<T>::pack2(acc[d][0] * p.scale, acc[d][1] * p.scale),
                   Elem<T>::pack2(acc[d][2] * p.scale, acc[d][3] * p.scale)};
      *(u32x2_t*)(dqp + dc * 2) = w;
    }
  }
}

// dO-only dQ pass reading K^T straight from the row-major K tile with
// lds_read_tr16: 4 waves x 32 queries (lane <-> query, so the statistics are
// per-lane scalars), 32-key steps through a four-stage ring of K, V row tiles.
// Step j (after one barrier) is a fixed MFMA stream:
//   S^T = K Q^T, dP^T = V dO^T of tile j+1 (P, dS of tile j on the VALU), then
//   dQ^T += K^T dS^T of tile j (tile j+3 requested meanwhile).
// Keys at or beyond Lk read K = V = 0; their (finite) dS meets a zero K^T
// column, so no key mask is needed. Padded queries carry lse = +inf (P = 0).
template <int D>
struct DqTrCfg {
  static constexpr int NW = 4;
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 32;
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BN * ROWB;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_V = ROW_BYTES;
  static constexpr int STAGE = 2 * ROW_BYTES;
  static constexpr int NSTAGE = 4;
  static constexpr int NRI = BN * CR / 64;
  static constexpr int RPW = NRI / NW;
  static constexpr bool FITS = (D == 128 || D == 64 || D == 256) && NRI % NW == 0 && NSTAGE * STAGE <= 160 * 1024;
  static constexpr int LOADS = 2 * RPW;
};

// D = 256: 512-byte K, V rows (32 KiB stages, one workgroup per CU), Q and dO
// held in AGPRs (the dQ accumulators and score tiles take the VGPRs), one
// K-slice offset kept (slice s at sx ^ 32 s).
// D = 64 fits three waves per SIMD (168 VGPRs, 32 KiB of LDS per workgroup):
// the third wave hides more of the 6 VALU instructions per MFMA (1% faster at
// B=4, H=32, L=16384 than two waves at 172 VGPRs, with bitwise equal dQ).
template <typename T, int D>
__global__ __launch_bounds__(256, D == 64 ? 3 : 1) void attn_bwd_dq_tr_kernel(DqParams p) {
  using C = DqTrCfg<D>;
  constexpr int BN = C::BN, KS = C::KS, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  static_assert(C::FITS, "configuration does not fit");
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;
  const int ntiles = (p.Lk + BN - 1) / BN;

  // ---- this lane's query: Q, dO rows (B operands) and statistics
  const int query = qt * C::BM + wave * 32 + col;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
  i32x4_t qreg[KS], doreg[KS];
  {
    const uint32_t qo = (uint32_t)((int64_t)query * p.q_sl * 2) + half * 16;
    const uint32_t oo = (uint32_t)((int64_t)query * p.do_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qreg[s] = buf_load16(rq, qo + s * 32);
      doreg[s] = buf_load16(rdo, oo + s * 32);
    }
  }
  if constexpr (D == 256) {
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+a"(qreg[s]), "+a"(doreg[s]));
  }
  float lse2 = __builtin_inff(), dlt = 0.f;
  if (query < p.LQP) {
    const float* st = p.stats + ((int64_t)bh * (p.LQP / p.stat_tile) + query / p.stat_tile) * 2 * p.stat_tile +
                      query % p.stat_tile;
    lse2 = st[0];
    dlt = st[p.stat_tile];
  }

  // ---- key-side resources and per-lane DMA offsets
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  constexpr int RPW = C::RPW;
  uint32_t roff_k[RPW], roff_v[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ trswz<CR>(row & 15);
    roff_k[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
    roff_v[j] = (uint32_t)((int64_t)row * p.v_sl * 2) + logical * 16;
  }
  const uint32_t k_step = (uint32_t)((int64_t)BN * p.k_sl * 2);
  const uint32_t v_step = (uint32_t)((int64_t)BN * p.v_sl * 2);

  auto stage = [&](auto kk) -> lds_char_t* {
    constexpr int k = decltype(kk)::value & 3;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else if constexpr (k == 2) return (lds_char_t*)stg2;
    else return (lds_char_t*)stg3;
  };
  // request li (0 <= li < C::LOADS) of tile kt into stage st; tiles at or beyond
  // the end read zeros or in-range rows into a stage nobody reads again
  auto issue_load = [&](lds_char_t* st, int kt, int li) {
    const int jj = li >> 1, i = wave + jj * C::NW;
    if (li & 1) buf_load16_lds(rv, st + C::OFF_V + i * 1024, roff_v[jj], (uint32_t)kt * v_step);
    else buf_load16_lds(rk, st + C::OFF_K + i * 1024, roff_k[jj], (uint32_t)kt * k_step);
  };

  // ---- LDS read offsets: row-wise (K, V row perm32(col), chunk 2s + half) and
  // transposed (K^T block db, keys 16 t + 8 (g >> 1) + (0..3 | 4..7))
  constexpr int NSX = D == 256 ? 1 : KS;
  int sx[NSX];
#pragma unroll
  for (int s = 0; s < NSX; ++s) {
    const int r = perm32(col);
    sx[s] = r * ROWB + (((2 * s + half) ^ trswz<CR>(r & 15)) << 4);
  }
  auto sxo = [&](int s) -> int {
    if constexpr (NSX == 1) return sx[0] ^ (32 * s);
    else return sx[s];
  };
  int tx[DB][2];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, c = lane & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = 8 * (g >> 1) + 4 * hh + r;  // plus 16 t
        const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
        tx[db][hh] = row * ROWB + ((chunk ^ trswz<CR>(row & 15)) << 4) + 8 * (c & 1);
      }
    }
  }
  auto pin_offsets = [&]() {
#pragma unroll
    for (int s = 0; s < NSX; ++s) asm volatile("" : "+v"(sx[s]));
#pragma unroll
    for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(tx[db][0]), "+v"(tx[db][1]));
  };

  f32x16_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[d][v] = 0.f;
  }

  constexpr int PF = 4;
  constexpr int NMA = 2 * KS;  // S^T, dP^T MFMAs
  constexpr int NMB = 2 * DB;  // dQ^T MFMAs (two 16-key chunks)
  constexpr int NS = NMA + NMB;
  constexpr int NVAL = 16;     // P, dS values per lane per tile
  constexpr int VPS = (NVAL + NMA - 1) / NMA;  // values per score slot (1 for D = 128, 2 for D = 64)
  static_assert(VPS * NMA >= NVAL && VPS <= 2, "values ride in the score slots");
  const f32x16_t zero16 = {};
  auto load_op = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int m) -> i32x4_t {
    if (m < NMA) return *(lds_i32x4_t*)(s_next + ((m & 1) ? C::OFF_V : C::OFF_K) + sxo(m >> 1));
    const int mm = m - NMA, t = mm / DB, db = mm % DB;
    const lds_char_t* base = s_cur + C::OFF_K + t * 16 * ROWB;
    const u32x2_t lo = lds_read_tr16(base + tx[db][0]);
    const u32x2_t hi = lds_read_tr16(base + tx[db][1]);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };
  // value v = 8 t + e of the C tile: key 16 t + 8 half + e of the tile
  auto value = [&](int v, const f32x16_t& sc, const f32x16_t& dpc, float (&dsv)[2]) {
    const float pe = fast_exp2(fmaf(sc[v], p.scale_log2, -lse2));
    dsv[v & 1] = pe * (dpc[v] - dlt);
  };
  auto mfma_slot = [&](int m, i32x4_t op, f32x16_t& sn, f32x16_t& dpn, const i32x4_t (&dsb)[2]) {
    if (m < NMA) {
      const int s = m >> 1;
      if (m & 1) dpn = mfma32(op, doreg[s], s == 0 ? zero16 : dpn, T());
      else sn = mfma32(op, qreg[s], s == 0 ? zero16 : sn, T());
    } else {
      const int mm = m - NMA, t = mm / DB, db = mm % DB;
      acc[db] = mfma32(op, dsb[t], acc[db], T());
    }
  };

  // step j (j + 1 < ntiles, j % 4 == kk)
  auto step = [&](auto kk, int j, const f32x16_t& sc, const f32x16_t& dpc, f32x16_t& sn, f32x16_t& dpn) {
    constexpr int k = decltype(kk)::value;
    ring_sync<C::LOADS>();  // tile j + 1 has landed (tile j + 2 may be in flight)
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    i32x4_t opr[PF];
#pragma unroll
    for (int m = 0; m < PF; ++m) opr[m] = load_op(s_next, s_cur, m);
    i32x4_t dsb[2];
    float dsv[2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < NS; ++m) {
      mfma_slot(m, opr[m % PF], sn, dpn, dsb);
      if (m + PF < NS) opr[m % PF] = load_op(s_next, s_cur, m + PF);
#pragma unroll
      for (int w = 0; w < VPS; ++w) {
        const int v = VPS * m + w;
        if (m < NMA && v < NVAL) {
          value(v, sc, dpc, dsv);
          if (v & 1) dsb[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(dsv[0], dsv[1]);
        }
      }
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) {
        if (li * NS / C::LOADS == m) issue_load(s_req, j + 3, li);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto last_step = [&](auto kk, const f32x16_t& sc, const f32x16_t& dpc) {
    const lds_char_t* s_cur = stage(kk);
    i32x4_t dsb[2];
    float dsv[2];
#pragma unroll
    for (int v = 0; v < NVAL; ++v) {
      value(v, sc, dpc, dsv);
      if (v & 1) dsb[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(dsv[0], dsv[1]);
    }
    f32x16_t un_s, un_p;
#pragma unroll
    for (int m = NMA; m < NS; ++m) mfma_slot(m, load_op(s_cur, s_cur, m), un_s, un_p, dsb);
  };

  if (ntiles > 0) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    ring_sync<2 * C::LOADS>();  // Q, dO rows and tile 0
    f32x16_t sa, pa, sb, pbb;
    {
      const lds_char_t* s0 = stage(IC<0>{});
      i32x4_t dummy[2];
#pragma unroll
      for (int m = 0; m < NMA; ++m) mfma_slot(m, load_op(s0, s0, m), sa, pa, dummy);
    }
    int j = 0;
    for (; j + 4 < ntiles; j += 4) {
      step(IC<0>{}, j, sa, pa, sb, pbb);
      step(IC<1>{}, j + 1, sb, pbb, sa, pa);
      step(IC<2>{}, j + 2, sa, pa, sb, pbb);
      step(IC<3>{}, j + 3, sb, pbb, sa, pa);
    }
    const int rest = ntiles - j;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, j, sa, pa, sb, pbb);
    if (rest >= 3) step(IC<1>{}, j + 1, sb, pbb, sa, pa);
    if (rest >= 4) step(IC<2>{}, j + 2, sa, pa, sb, pbb);
    if (rest == 1) last_step(IC<0>{}, sa, pa);
    else if (rest == 2) last_step(IC<1>{}, sb, pbb);
    else if (rest == 3) last_step(IC<2>{}, sa, pa);
    else last_step(IC<3>{}, sb, pbb);
    wait_vmem();  // no requests beyond the last tile stay in flight
  }

  // ---- dQ = s (dQ^T)^T: lane holds query col, rows d = 32 db + 8 jj + 4 half + (0..3)
  if (query < p.Lq) {
    char* dqp = (char*)p.dq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)query * p.dq_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int dc = d * 32 + 8 * jj + 4 * half;
        u32x2_t w = {Elem<T>::pack2(acc[d][4 * jj] * p.scale, acc[d][4 * jj + 1] * p.scale),
                     Elem<T>::pack2(acc[d][4 * jj + 2] * p.scale, acc[d][4 * jj + 3] * p.scale)};
        *(u32x2_t*)(dqp + dc * 2) = w;
      }
    }
  }
}

}  // namespace dmad
