// Backward attention kernels for gfx950.
//
// The reference backward (_attention.backward,
// train/wan/rcm/utils/flash_attention_jvp_triton.py:534-579) hands dO, O and
// LSE to flash-attn's FA2 backward and discards the cotangent of the tangent
// output. Its arithmetic, restated from the mathematics:
//   P  = exp(s Q K^T - LSE),  D = rowsum(dO * O)
//   dP = dO V^T,  dS = P * (dP - D)
//   dQ = s dS K,  dK = s dS^T Q,  dV = P^T dO                         (mode A)
// The full derivative of (O, Od) (mode B), with Sd = s(Qd K^T + Q Kd^T),
// mu = rowsum(P*Sd), rho = rowsum(dOd*O), D' = rowsum(dO*O) + rowsum(dOd*Od) - mu*rho:
//   dPd = dOd V^T
//   dP  = dO V^T + dOd Vd^T + dPd*(Sd - mu) - Sd*rho
//   dS  = P*(dP - D'),  dSd = P*(dPd - rho),  Pd = P*(Sd - mu)
//   dQ = s(dS K + dSd Kd),  dK = s(dS^T Q + dSd^T Qd),  dV = P^T dO + Pd^T dOd
// and the tangent gradients dQd = s dSd K, dKd = s dSd^T Q, dVd = P^T dOd
// are mode A with (dO, D) replaced by (dOd, rho).
//
// This file holds the key-stationary pass (dK, dV and, for the full
// derivative, their Kd/Vd-independent sums); dQ comes from the query-stationary
// pass in attn_bwd_dq.h, so no gradient needs atomics.
//
// Work decomposition (one workgroup = 4 waves = 128 keys of one head):
//   * lane l of wave w owns key 32w + l%32; its K, V (and Kd, Vd) rows stay in
//     registers as the B operand of S = Q K^T and dP = dO V^T, so the C tiles
//     have lane <-> key and 16 query values per lane;
//   * query tiles stream through a double-buffered LDS ring by buffer->LDS
//     DMA: Q, dO rows (A operands of the score GEMMs, read in perm32 row order),
//     Q^T, dO^T (A operands of dK^T += Q^T dS, dV^T += dO^T P) and the per-row
//     statistics (log2-domain LSE, D or D', mu, rho) prepared by bwd_prep;
//   * P and dS leave the score C tiles already in B-operand layout (perm32),
//     so dK^T and dV^T accumulate in registers with no data movement;
#pragma once
#include "attn_fwd.h"
#include "common.h"

namespace dmad {

enum BwdMode : int { kBwdDoutOnly = 0, kBwdFull = 1 };

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* tq;
  const void* tk;
  const void* tv;
  const void* dout;  // dO rows  (mode A with tangent grads: dOd)
  const void* dto;   // dOd rows (mode B)
  const void* qT;    // Q^T   [BH][DP][LQP]
  const void* tqT;   // Qd^T  [BH][DP][LQP] (mode B)
  const void* doT;   // dO^T  [BH][DP][LQP]
  const void* dtoT;  // dOd^T [BH][DP][LQP] (mode B)
  const float* stats;  // [BH][LQP/BMQ][NSTAT][BMQ]
  void* dk;
  void* dv;
  int64_t q_sb, q_sh, q_sl;  // shared by Q, Qd
  int64_t k_sb, k_sh, k_sl;  // shared by K, Kd
  int64_t v_sb, v_sh, v_sl;  // shared by V, Vd
  int64_t do_sb, do_sh, do_sl;  // shared by dO, dOd
  int64_t dk_sb, dk_sh, dk_sl;
  int64_t dv_sb, dv_sh, dv_sl;
  int B, H, Lq, Lk, LQP;
  float scale, scale_log2;
  int xcd_order;  // work items contiguous per XCD (common.h)
  // Stored score gradients (key passes instantiated with STORE, 128-wide heads):
  // the launch covers (b, h) slices bh0 .. bh0 + grid / key tiles - 1, and slice
  // bh - bh0 of `sc` (sc_slice bytes apart) receives its dS [, dSd] in the layout
  // of ScLayout below.
  void* sc;
  int64_t sc_slice;
  int bh0;
};

// Layout of the score gradients a key pass stores for the query pass to read
// back (the dQ pass then multiplies them by K instead of recomputing S and dP).
// One (b, h) slice holds NT tensors (dS; or dS, dSd) in pieces of 32 queries x
// 32 keys (2 KiB, bf16/fp16):
//   [query block of 128][key block of 32][tensor][query tile of 32 (4)]
//     [16-query chunk u (2)][row (32)][query half (2)][8 queries]
// with row = (key % 32) ^ 4u. The key pass's wave owns one key block and holds,
// per lane (key, half), the 8 consecutive queries 16u + 8 half + 0..7 of its
// tile packed in 16 bytes, so each chunk leaves as one contiguous 1 KiB store.
// The query pass copies a (query block, key block) piece of NT x 8 KiB into LDS
// as it lies and reads dS^T straight from it as MFMA B operands with
// ds_read_b64_tr_b16 (lane = query, 8 consecutive keys); the row XOR puts the
// two chunks a 32-lane half reads at once in different 128-byte bank windows.
struct ScLayout {
  static constexpr int BQ = 128;          // queries per query block
  static constexpr int BK = 32;           // keys per key block
  static constexpr int PIECE = 8192;      // one tensor's (query block, key block) piece
  static constexpr int TILE = 2048;       // one 32-query tile of a piece
  static constexpr int CHUNK = 1024;      // one 16-query chunk of a tile
  // Query blocks' strips start STRIP_PAD bytes apart beyond their size: the
  // query pass streams all strips of a slice at once, and strips an exact
  // power of two apart read 2-4% slower (5.80 against 6.05 TB/s at the 14B shape).
  static constexpr int STRIP_PAD = 20480;
  __host__ __device__ static int64_t strip_stride(int64_t nkb, int nt) { return nkb * nt * PIECE + STRIP_PAD; }
  // byte offset of lane (key col, half)'s 16 bytes within chunk u
  __device__ __forceinline__ static uint32_t lane_off(int col, int half, int u) {
    return (uint32_t)((((col ^ (4 * u)) * 2) + half) * 16);
  }
};
// Bytes of one (b, h) slice: NT tensors over Lq rounded up to 128 queries and
// `nkb` key blocks (the key pass covers nkt * 128 keys: nkb = 4 nkt).
__host__ __device__ inline int64_t sc_slice_bytes(int64_t lq, int64_t nkb, int nt) {
  return (lq + ScLayout::BQ - 1) / ScLayout::BQ * ScLayout::strip_stride(nkb, nt);
}

template <int D, int MODE>
struct BwdCfg {
  static constexpr int NW = 4;
  static constexpr int BK = 32 * NW;  // keys per workgroup
  static constexpr int DP = D < 32 ? 32 : D;
  static constexpr bool FULL = MODE == kBwdFull;
  static constexpr int BMQ = (FULL || D > 128) ? 32 : 64;  // queries per tile
  static constexpr int NQB = BMQ / 32;
  static constexpr int KS = D / 16;   // d slices of the score GEMMs
  static constexpr int DB = DP / 32;  // 32-row d blocks of dK^T, dV^T, dQ^T
  static constexpr int CR = D / 8;    // 16-byte chunks per row-tile row
  static constexpr int CT = BMQ / 8;  // chunks per transposed-tile row
  static constexpr int NSTAT = FULL ? 4 : 2;
  static constexpr int NT = FULL ? 4 : 2;  // row tiles (Q, dO [, Qd, dOd]) = transposed tiles
  static constexpr int ROW_BYTES = BMQ * D * 2;
  static constexpr int TR_BYTES = DP * BMQ * 2;
  static constexpr int STAT_BYTES = NSTAT * BMQ * 4;
  static constexpr int OFF_ROW = 0;
  static constexpr int OFF_TR = NT * ROW_BYTES;
  static constexpr int OFF_STAT = OFF_TR + NT * TR_BYTES;
  static constexpr int STAGE = (OFF_STAT + STAT_BYTES + 1023) / 1024 * 1024;
  static constexpr int LDS_BYTES = 2 * STAGE;
  static constexpr int NRI = BMQ * CR / 64;  // wave-wide 1 KiB loads per row tile
  static constexpr int NTI = DP * CT / 64;   // ... per transposed tile
  static_assert(STAT_BYTES <= 1024, "statistics must fit one wave-wide load");
};

template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void attn_bwd_kernel(BwdParams p) {
  using C = BwdCfg<D, MODE>;
  constexpr int BMQ = C::BMQ, NQB = C::NQB, KS = C::KS, DB = C::DB, CR = C::CR, CT = C::CT;
  constexpr bool FULL = C::FULL;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nkt = (p.Lk + C::BK - 1) / C::BK;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nkt, kt = work - bh * nkt;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nqt = p.LQP / BMQ;

  const int key = kt * C::BK + wave * 32 + col;  // this lane's key (C-layout column)
  const bool key_ok = key < p.Lk;

  // ---- stationary K, V (and Kd, Vd) rows: B operands of the score GEMMs
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  __amdgpu_buffer_rsrc_t rtk = rk, rtv = rv;
  if constexpr (FULL) {
    rtk = make_rsrc((const char*)p.tk + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
    rtv = make_rsrc((const char*)p.tv + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  }
  i32x4_t kreg[KS], vreg[KS], tkreg[KS], tvreg[KS];
  {
    const uint32_t ko = (uint32_t)((int64_t)key * p.k_sl * 2) + half * 16;
    const uint32_t vo = (uint32_t)((int64_t)key * p.v_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kreg[s] = buf_load16(rk, ko + s * 32);
      vreg[s] = buf_load16(rv, vo + s * 32);
      if constexpr (FULL) {
        tkreg[s] = buf_load16(rtk, ko + s * 32);
        tvreg[s] = buf_load16(rtv, vo + s * 32);
      }
    }
  }
  // ---- DMA of one query tile into a stage
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const uint32_t tr_bytes = (uint32_t)((int64_t)C::DP * p.LQP * 2);
  const uint32_t st_bytes = (uint32_t)((int64_t)p.LQP * C::NSTAT * 4);
  const __amdgpu_buffer_rsrc_t rrow[4] = {
      make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes),
      make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes),
      make_rsrc((const char*)(FULL ? p.tq : p.q) + (b * p.q_sb + h * p.q_sh) * 2, q_bytes),
      make_rsrc((const char*)(FULL ? p.dto : p.dout) + (b * p.do_sb + h * p.do_sh) * 2, do_bytes)};
  const __amdgpu_buffer_rsrc_t rtr[4] = {
      make_rsrc((const char*)p.qT + (int64_t)bh * tr_bytes, tr_bytes),
      make_rsrc((const char*)p.doT + (int64_t)bh * tr_bytes, tr_bytes),
      make_rsrc((const char*)(FULL ? p.tqT : p.qT) + (int64_t)bh * tr_bytes, tr_bytes),
      make_rsrc((const char*)(FULL ? p.dtoT : p.doT) + (int64_t)bh * tr_bytes, tr_bytes)};
  const __amdgpu_buffer_rsrc_t rst = make_rsrc((const char*)p.stats + (int64_t)bh * st_bytes, st_bytes);
  const int64_t row_sl[4] = {p.q_sl, p.do_sl, p.q_sl, p.do_sl};

  constexpr int RPW = (C::NRI + C::NW - 1) / C::NW;
  constexpr int TPW = (C::NTI + C::NW - 1) / C::NW;
  uint32_t roff_q[RPW], roff_do[RPW], toff[TPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ swz<CR>(perm32(row & 31) & 15);
    roff_q[j] = (uint32_t)((int64_t)row * p.q_sl * 2) + logical * 16;
    roff_do[j] = (uint32_t)((int64_t)row * p.do_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CT, phys = pch % CT;
    const int logical = phys ^ swz<CT>(d & 15);
    toff[j] = (uint32_t)(d * p.LQP * 2) + logical * 16;
  }

  auto issue_tile = [&](int qt, int stage) {
    char* st = smem + stage * C::STAGE;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
      const uint32_t rs = (uint32_t)((int64_t)qt * BMQ * row_sl[t] * 2);
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const int i = wave + j * C::NW;
        if (i < C::NRI) buf_load16_lds(rrow[t], st + C::OFF_ROW + t * C::ROW_BYTES + i * 1024, (t & 1) ? roff_do[j] : roff_q[j], rs);
      }
      const uint32_t ts = (uint32_t)qt * BMQ * 2;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int i = wave + j * C::NW;
        if (i < C::NTI) buf_load16_lds(rtr[t], st + C::OFF_TR + t * C::TR_BYTES + i * 1024, toff[j], ts);
      }
    }
    if (wave == C::NW - 1 && lane * 16 < C::STAT_BYTES)
      buf_load16_lds(rst, st + C::OFF_STAT, lane * 16, (uint32_t)qt * C::STAT_BYTES);
  };

  // ---- LDS read offsets
  const int rswz = swz<CR>(col & 15), tswz = swz<CT>(col & 15);
  const int rrow_off = perm32(col) * CR * 16;
  const int trow_off = col * CT * 16;

  f32x16_t dkacc[DB], dvacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      dkacc[d][v] = 0.f;
      dvacc[d][v] = 0.f;
    }
  }

  issue_tile(0, 0);
  for (int qt = 0; qt < nqt; ++qt) {
    wait_vmem();
    __syncthreads();
    if (qt + 1 < nqt) issue_tile(qt + 1, (qt + 1) & 1);
    const char* st = smem + (qt & 1) * C::STAGE;
    const char* rq_t = st + C::OFF_ROW;
    const char* rdo_t = st + C::OFF_ROW + C::ROW_BYTES;
    const char* rtq_t = st + C::OFF_ROW + 2 * C::ROW_BYTES;
    const char* rdto_t = st + C::OFF_ROW + 3 * C::ROW_BYTES;
    const float* sst = (const float*)(st + C::OFF_STAT);

    // ---- phase 1: score tiles (rows = queries in perm32 order, cols = keys)
    f32x16_t sacc[NQB], dpacc[NQB], tsacc[NQB], dpdacc[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        sacc[qb][v] = 0.f;
        dpacc[qb][v] = 0.f;
        tsacc[qb][v] = 0.f;
        dpdacc[qb][v] = 0.f;
      }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        const int off = qb * 32 * CR * 16 + rrow_off + (((2 * s + half) ^ rswz) << 4);
        const i32x4_t aq = *(const i32x4_t*)(rq_t + off);
        const i32x4_t ado = *(const i32x4_t*)(rdo_t + off);
        sacc[qb] = mfma32(aq, kreg[s], sacc[qb], T());
        dpacc[qb] = mfma32(ado, vreg[s], dpacc[qb], T());
        if constexpr (FULL) {
          const i32x4_t atq = *(const i32x4_t*)(rtq_t + off);
          const i32x4_t adto = *(const i32x4_t*)(rdto_t + off);
          tsacc[qb] = mfma32(atq, kreg[s], tsacc[qb], T());
          tsacc[qb] = mfma32(aq, tkreg[s], tsacc[qb], T());
          dpacc[qb] = mfma32(adto, tvreg[s], dpacc[qb], T());
          dpdacc[qb] = mfma32(adto, vreg[s], dpdacc[qb], T());
        }
      }
    }

    // ---- phase 2: elementwise; value v of block qb is query qb*32 + 16t + 8*half + e (v = 8t + e)
    i32x4_t pb[NQB][2], dsb[NQB][2], tpb[NQB][2], tdsb[NQB][2];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int q0 = qb * 32 + 16 * t + 8 * half;
        float lse2[8], dlt[8], mu[8], rho[8];
#pragma unroll
        for (int e4 = 0; e4 < 2; ++e4) {
          const float4 a = *(const float4*)(sst + 0 * BMQ + q0 + 4 * e4);
          const float4 c = *(const float4*)(sst + 1 * BMQ + q0 + 4 * e4);
          lse2[4 * e4 + 0] = a.x; lse2[4 * e4 + 1] = a.y; lse2[4 * e4 + 2] = a.z; lse2[4 * e4 + 3] = a.w;
          dlt[4 * e4 + 0] = c.x; dlt[4 * e4 + 1] = c.y; dlt[4 * e4 + 2] = c.z; dlt[4 * e4 + 3] = c.w;
          if constexpr (FULL) {
            const float4 m4 = *(const float4*)(sst + 2 * BMQ + q0 + 4 * e4);
            const float4 r4 = *(const float4*)(sst + 3 * BMQ + q0 + 4 * e4);
            mu[4 * e4 + 0] = m4.x; mu[4 * e4 + 1] = m4.y; mu[4 * e4 + 2] = m4.z; mu[4 * e4 + 3] = m4.w;
            rho[4 * e4 + 0] = r4.x; rho[4 * e4 + 1] = r4.y; rho[4 * e4 + 2] = r4.z; rho[4 * e4 + 3] = r4.w;
          }
        }
        float pv[8], dsv[8], tpv[8], tdsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int v = 8 * t + e;
          // no key mask: a lane's key >= Lk reads K = V = 0, and its dK, dV
          // column (the only outputs its P, dS reach) is never stored
          const float pe = fast_exp2(fmaf(sacc[qb][v], p.scale_log2, -lse2[e]));
          pv[e] = pe;
          if constexpr (!FULL) {
            dsv[e] = pe * (dpacc[qb][v] - dlt[e]);
          } else {
            const float sd = tsacc[qb][v] * p.scale;
            const float c = sd - mu[e];
            const float dpd = dpdacc[qb][v];
            const float dp = dpacc[qb][v] + dpd * c - sd * rho[e];
            tpv[e] = pe * c;
            dsv[e] = pe * (dp - dlt[e]);
            tdsv[e] = pe * (dpd - rho[e]);
          }
        }
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          pb[qb][t][e2] = (int)Elem<T>::pack2(pv[2 * e2], pv[2 * e2 + 1]);
          dsb[qb][t][e2] = (int)Elem<T>::pack2(dsv[2 * e2], dsv[2 * e2 + 1]);
          if constexpr (FULL) {
            tpb[qb][t][e2] = (int)Elem<T>::pack2(tpv[2 * e2], tpv[2 * e2 + 1]);
            tdsb[qb][t][e2] = (int)Elem<T>::pack2(tdsv[2 * e2], tdsv[2 * e2 + 1]);
          }
        }
      }
    }

    // ---- phase 3: dV^T += dO^T P (+ dOd^T Pd), dK^T += Q^T dS (+ Qd^T dSd)
    const char* tq_t = st + C::OFF_TR;
    const char* tdo_t = st + C::OFF_TR + C::TR_BYTES;
    const char* ttq_t = st + C::OFF_TR + 2 * C::TR_BYTES;
    const char* tdto_t = st + C::OFF_TR + 3 * C::TR_BYTES;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ch = ((qb * 4 + 2 * t + half) ^ tswz) << 4;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const int off = d * 32 * CT * 16 + trow_off + ch;
          const i32x4_t ado = *(const i32x4_t*)(tdo_t + off);
          const i32x4_t aq = *(const i32x4_t*)(tq_t + off);
          dvacc[d] = mfma32(ado, pb[qb][t], dvacc[d], T());
          dkacc[d] = mfma32(aq, dsb[qb][t], dkacc[d], T());
          if constexpr (FULL) {
            const i32x4_t adto = *(const i32x4_t*)(tdto_t + off);
            const i32x4_t atq = *(const i32x4_t*)(ttq_t + off);
            dvacc[d] = mfma32(adto, tpb[qb][t], dvacc[d], T());
            dkacc[d] = mfma32(atq, tdsb[qb][t], dkacc[d], T());
          }
        }
      }
    }

  }

  // ---- store dK = s (dK^T)^T, dV = (dV^T)^T for this lane's key
  if (key_ok) {
    char* dkp = (char*)p.dk + ((b * p.dk_sb + h * p.dk_sh) + (int64_t)key * p.dk_sl) * 2;
    char* dvp = (char*)p.dv + ((b * p.dv_sb + h * p.dv_sh) + (int64_t)key * p.dv_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int dc = d * 32 + 8 * j + 4 * half;
        if (D >= 32 || dc < D) {
          u32x2_t wk = {Elem<T>::pack2(dkacc[d][4 * j] * p.scale, dkacc[d][4 * j + 1] * p.scale),
                        Elem<T>::pack2(dkacc[d][4 * j + 2] * p.scale, dkacc[d][4 * j + 3] * p.scale)};
          u32x2_t wv = {Elem<T>::pack2(dvacc[d][4 * j], dvacc[d][4 * j + 1]),
                        Elem<T>::pack2(dvacc[d][4 * j + 2], dvacc[d][4 * j + 3])};
          *(u32x2_t*)(dkp + dc * 2) = wk;
          *(u32x2_t*)(dvp + dc * 2) = wv;
        }
      }
    }
  }
}

// Pipelined dO-only dK/dV pass: 4 waves x 32 keys, 32x32x16 MFMAs, BMQ-query
// steps through a four-stage LDS ring whose tiles are requested three steps
// ahead. Step j (after one barrier) is a fixed stream of MFMAs:
//   S, dP of tile j+1 (with the VALU P, dS of tile j interleaved), then
//   dV^T += dO^T P, dK^T += Q^T dS of tile j (with tile j+3's requests interleaved);
// every MFMA's LDS operand is read four MFMAs ahead. S and dP alternate between
// two register sets, and the loop is unrolled by four so that each ring stage
// is a separate LDS object known at compile time (the compiler then waits for a
// buffer->LDS request only before reading the stage it fills). Keys at or
// beyond Lk read K = V = 0 and are never stored, so P needs no key mask;
// padded queries carry lse = +inf, so their P is 0.
template <int D, int BMQ_>
struct KvPipeCfg {
  static constexpr int NW = 4;
  static constexpr int BK = 32 * NW;   // keys per workgroup
  static constexpr int BMQ = BMQ_;     // queries per pipeline step
  static constexpr int NQB = BMQ / 32;
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;    // 32-row blocks of dK^T, dV^T
  static constexpr int CR = D / 8;     // chunks per Q / dO row
  static constexpr int CT = BMQ / 8;   // chunks per Q^T / dO^T row
  static constexpr int ROW_BYTES = BMQ * D * 2;
  static constexpr int TR_BYTES = D * BMQ * 2;
  static constexpr int OFF_Q = 0;
  static constexpr int OFF_DO = ROW_BYTES;
  static constexpr int OFF_QT = 2 * ROW_BYTES;
  static constexpr int OFF_DOT = 2 * ROW_BYTES + TR_BYTES;
  static constexpr int OFF_ST = 2 * ROW_BYTES + 2 * TR_BYTES;
  static constexpr int STAT_BYTES = 2 * BMQ * 4;
  static constexpr int STAGE = (OFF_ST + STAT_BYTES + 1023) / 1024 * 1024;
  static constexpr int NSTAGE = 4;
  static constexpr int NRI = BMQ * CR / 64;  // wave-wide 1 KiB loads per row tile
  static constexpr int NTI = D * CT / 64;    // ... per transposed tile
  static constexpr int ST_LANES = STAT_BYTES / 16 / NW;  // lanes per wave loading statistics
  // Requests per tile: the Q and dO row tiles (2 NRI), the Q^T and dO^T tiles
  // (2 NTI) and one for the statistics. A wave's k-th row request is request
  // (wave + NW k) of the row tiles taken together, so that every wave issues
  // the same number of loads per tile (counted waits) also when a tile has
  // fewer requests than there are waves.
  static constexpr int RLOADS = 2 * NRI / NW;  // row requests per wave per tile
  static constexpr int TLOADS = 2 * NTI / NW;  // transposed-tile requests per wave per tile
  static constexpr bool FITS = D >= 32 && D <= 128 && 2 * NRI % NW == 0 && 2 * NTI % NW == 0 &&
                               NSTAGE * STAGE <= 160 * 1024;
  static constexpr int LOADS = RLOADS + TLOADS + 1;  // per wave per tile
};

// Query tile used by the dO-only dK/dV kernel for head dim D (the layout of the
// backward statistics follows it). 32 queries per step: at D = 32 (the head dim
// this kernel serves) the two score-tile sets then take 64 registers and the
// kernel 188, so two waves share each SIMD (64-query steps took 328 registers,
// one wave per SIMD: 14.4 against 11.4 ms at B=4, H=32, L=16384, fp16).
template <int D>
constexpr int kv_pipe_bmq() { return 32; }

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_kv_pipe_kernel(BwdParams p) {
  using C = KvPipeCfg<D, kv_pipe_bmq<D>()>;
  constexpr int BMQ = C::BMQ, NQB = C::NQB, KS = C::KS, DB = C::DB, CR = C::CR, CT = C::CT, NST = C::NSTAGE;
  static_assert(C::FITS, "configuration does not fit");
  // one LDS object per ring stage: the compiler then orders LDS reads only
  // after the buffer->LDS requests into the same stage
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[C::STAGE];
  static_assert(NST == 4, "four ring stages");

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nkt = (p.Lk + C::BK - 1) / C::BK;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nkt, kt = work - bh * nkt;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nqt = p.LQP / BMQ;

  const int key = kt * C::BK + wave * 32 + col;

  // ---- stationary K, V rows: B operands of S = Q K^T and dP = dO V^T
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  i32x4_t kreg[KS], vreg[KS];
  {
    const uint32_t ko = (uint32_t)((int64_t)key * p.k_sl * 2) + half * 16;
    const uint32_t vo = (uint32_t)((int64_t)key * p.v_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kreg[s] = buf_load16(rk, ko + s * 32);
      vreg[s] = buf_load16(rv, vo + s * 32);
    }
  }

  // ---- query-side resources and per-lane DMA offsets
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const uint32_t tr_bytes = (uint32_t)((int64_t)D * p.LQP * 2);
  const uint32_t st_bytes = (uint32_t)((int64_t)p.LQP * 2 * 4);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
  const __amdgpu_buffer_rsrc_t rqt = make_rsrc((const char*)p.qT + (int64_t)bh * tr_bytes, tr_bytes);
  const __amdgpu_buffer_rsrc_t rdot = make_rsrc((const char*)p.doT + (int64_t)bh * tr_bytes, tr_bytes);
  const __amdgpu_buffer_rsrc_t rst = make_rsrc((const char*)p.stats + (int64_t)bh * st_bytes, st_bytes);
  // request g of the row tiles: tensor g / NRI (Q, dO), 1 KiB block g % NRI
  constexpr int RL = C::RLOADS, TL = C::TLOADS;
  uint32_t roff[RL], toff[TL];
#pragma unroll
  for (int j = 0; j < RL; ++j) {
    const int g = wave + j * C::NW;
    const int pch = (g % C::NRI) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ swz<CR>(perm32(row & 31) & 15);
    roff[j] = (uint32_t)((int64_t)row * (g < C::NRI ? p.q_sl : p.do_sl) * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < TL; ++j) {
    const int g = wave + j * C::NW;
    const int pch = (g % C::NTI) * 64 + lane;
    const int d = pch / CT, phys = pch % CT;
    const int logical = phys ^ swz<CT>(d & 15);
    toff[j] = (uint32_t)(d * p.LQP * 2) + logical * 16;
  }
  const uint32_t q_step = (uint32_t)((int64_t)BMQ * p.q_sl * 2);
  const uint32_t do_step = (uint32_t)((int64_t)BMQ * p.do_sl * 2);
  static_assert(C::ST_LANES * C::NW * 16 == C::STAT_BYTES, "statistics split evenly over the waves");
  const bool st_lane = lane >= wave * C::ST_LANES && lane < (wave + 1) * C::ST_LANES;

  // stage of tile qt is qt % 4, always known at compile time
  auto stage = [&](auto kk) -> lds_char_t* {
    constexpr int k = decltype(kk)::value & 3;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else if constexpr (k == 2) return (lds_char_t*)stg2;
    else return (lds_char_t*)stg3;
  };
  // Load li (0 <= li < C::LOADS) of tile qt into stage st. Tiles at or beyond
  // the end read zeros or in-range rows (buffer range checks) into a stage
  // nobody reads again.
  auto issue_load = [&](lds_char_t* st, int qt, int li) {
    if (li < RL) {
      const int g = wave + li * C::NW, i = g % C::NRI;
      if (g >= C::NRI) buf_load16_lds(rdo, st + C::OFF_DO + i * 1024, roff[li], (uint32_t)qt * do_step);
      else buf_load16_lds(rq, st + C::OFF_Q + i * 1024, roff[li], (uint32_t)qt * q_step);
    } else if (li < RL + TL) {
      const int jj = li - RL, g = wave + jj * C::NW, i = g % C::NTI;
      if (g >= C::NTI) buf_load16_lds(rdot, st + C::OFF_DOT + i * 1024, toff[jj], (uint32_t)qt * BMQ * 2);
      else buf_load16_lds(rqt, st + C::OFF_QT + i * 1024, toff[jj], (uint32_t)qt * BMQ * 2);
    } else {
      if (st_lane) buf_load16_lds(rst, st + C::OFF_ST, lane * 16, (uint32_t)qt * C::STAT_BYTES);
    }
  };

  const int rswz = swz<CR>(col & 15), tswz = swz<CT>(col & 15);
  const int rrow_off = perm32(col) * CR * 16;
  const int trow_off = col * CT * 16;

  f32x16_t dkacc[DB], dvacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      dkacc[d][v] = 0.f;
      dvacc[d][v] = 0.f;
    }
  }

  // One step is a fixed stream of MFMAs: NMA score MFMAs (S, dP of the next
  // tile; block qb holds queries 32 qb + perm32(row)) then NMB update MFMAs
  // (dV^T, dK^T of this tile). Each MFMA's LDS operand is read PF slots ahead;
  // the P, dS arithmetic of this tile rides in the score slots and the tile
  // requests three steps ahead ride in the update slots.
  constexpr int PF = 4;
  constexpr int NMA = 2 * KS * NQB;
  constexpr int NMB = 4 * NQB * DB;
  constexpr int NVAL = 16 * NQB;  // P, dS values per lane per tile
  static_assert(NVAL % NMA == 0 || NMA % NVAL == 0, "value slots");
  static_assert(C::LOADS <= NMB, "load slots");
  const f32x16_t zero16 = {};
  auto op_ptr = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int m) -> lds_i32x4_t* {
    if (m < NMA) {
      const int s = m / (2 * NQB), r = m % (2 * NQB), qb = r >> 1;
      return (lds_i32x4_t*)(s_next + ((r & 1) ? C::OFF_DO : C::OFF_Q) + qb * 32 * CR * 16 + rrow_off +
                              (((2 * s + half) ^ rswz) << 4));
    }
    const int mm = m - NMA, u = mm / (2 * DB), r = mm % (2 * DB), d = r >> 1;
    return (lds_i32x4_t*)(s_cur + ((r & 1) ? C::OFF_QT : C::OFF_DOT) + d * 32 * CT * 16 + trow_off +
                            (((2 * u + half) ^ tswz) << 4));
  };
  // statistics of one tile: lse (log2 units) and Delta for queries 32 qb + 16 t + 8 half + 0..7
  auto load_stats = [&](const lds_char_t* st, f32x4_t (&lsev)[2 * NQB][2], f32x4_t (&dltv)[2 * NQB][2]) {
    const lds_char_t* sst = st + C::OFF_ST;
#pragma unroll
    for (int u = 0; u < 2 * NQB; ++u) {
      const int q0 = 16 * u + 8 * half;
      lsev[u][0] = *(lds_f32x4_t*)(sst + 4 * q0);
      lsev[u][1] = *(lds_f32x4_t*)(sst + 4 * (q0 + 4));
      dltv[u][0] = *(lds_f32x4_t*)(sst + 4 * (BMQ + q0));
      dltv[u][1] = *(lds_f32x4_t*)(sst + 4 * (BMQ + q0 + 4));
    }
  };
  // value v of this tile: block v / 16, value (v % 16) of its C tile = query 32 qb + 16 t + 8 half + e
  auto value = [&](int v, const f32x16_t (&sc)[NQB], const f32x16_t (&dpc)[NQB], const f32x4_t (&lsev)[2 * NQB][2],
                   const f32x4_t (&dltv)[2 * NQB][2], float (&pv)[2], float (&dsv)[2]) {
    const int qb = v / 16, t = (v % 16) / 8, e = v % 8, u = 2 * qb + t;
    const float l2 = lsev[u][e >> 2][e & 3], dl = dltv[u][e >> 2][e & 3];
    const float pe = fast_exp2(fmaf(sc[qb][8 * t + e], p.scale_log2, -l2));
    pv[v & 1] = pe;
    dsv[v & 1] = pe * (dpc[qb][8 * t + e] - dl);
  };
  auto pack = [&](int v, const float (&pv)[2], const float (&dsv)[2], i32x4_t (&pb)[2 * NQB],
                  i32x4_t (&dsb)[2 * NQB]) {
    const int u = v / 8, e2 = (v % 8) >> 1;
    pb[u][e2] = (int)Elem<T>::pack2(pv[0], pv[1]);
    dsb[u][e2] = (int)Elem<T>::pack2(dsv[0], dsv[1]);
  };
  auto mfma_slot = [&](int m, i32x4_t op, f32x16_t (&sn)[NQB], f32x16_t (&dpn)[NQB],
                       const i32x4_t (&pb)[2 * NQB], const i32x4_t (&dsb)[2 * NQB]) {
    if (m < NMA) {
      const int s = m / (2 * NQB), r = m % (2 * NQB), qb = r >> 1;
      if (r & 1) dpn[qb] = mfma32(op, vreg[s], s == 0 ? zero16 : dpn[qb], T());
      else sn[qb] = mfma32(op, kreg[s], s == 0 ? zero16 : sn[qb], T());
    } else {
      const int mm = m - NMA, u = mm / (2 * DB), r = mm % (2 * DB), d = r >> 1;
      if (r & 1) dkacc[d] = mfma32(op, dsb[u], dkacc[d], T());
      else dvacc[d] = mfma32(op, pb[u], dvacc[d], T());
    }
  };

  // step j (j + 1 < nqt, j % 4 == kk): S, dP of tile j + 1 || P, dS of tile j; update with tile j;
  // request tile j + 3
  auto step = [&](auto kk, int j, const f32x16_t (&sc)[NQB], const f32x16_t (&dpc)[NQB], f32x16_t (&sn)[NQB],
                  f32x16_t (&dpn)[NQB]) {
    constexpr int k = decltype(kk)::value;
    ring_sync<C::LOADS>();  // tile j + 1 has landed (tile j + 2 may be in flight)
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    f32x4_t lsev[2 * NQB][2], dltv[2 * NQB][2];
    load_stats(s_cur, lsev, dltv);
    i32x4_t opr[PF];
#pragma unroll
    for (int m = 0; m < PF; ++m) opr[m] = *op_ptr(s_next, s_cur, m);
    i32x4_t pb[2 * NQB], dsb[2 * NQB];
    float pv[2], dsv[2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < NMA + NMB; ++m) {
      mfma_slot(m, opr[m % PF], sn, dpn, pb, dsb);
      if (m + PF < NMA + NMB) opr[m % PF] = *op_ptr(s_next, s_cur, m + PF);
      if (m < NMA) {
        constexpr int VPS = NVAL >= NMA ? NVAL / NMA : 1;
#pragma unroll
        for (int k = 0; k < VPS; ++k) {
          const int v = m * VPS + k;
          if (v < NVAL && (NVAL >= NMA || m % (NMA / NVAL) == 0)) {
            const int vv = NVAL >= NMA ? v : m / (NMA / NVAL);
            value(vv, sc, dpc, lsev, dltv, pv, dsv);
            if (vv & 1) pack(vv, pv, dsv, pb, dsb);
          }
        }
      }
      // tile j + 3's requests, spread evenly over the step
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) {
        if (li * (NMA + NMB) / C::LOADS == m) issue_load(s_req, j + 3, li);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // final tile: P, dS then the update MFMAs
  auto last_step = [&](auto kk, const f32x16_t (&sc)[NQB], const f32x16_t (&dpc)[NQB]) {
    const lds_char_t* s_cur = stage(kk);
    f32x4_t lsev[2 * NQB][2], dltv[2 * NQB][2];
    load_stats(s_cur, lsev, dltv);
    i32x4_t pb[2 * NQB], dsb[2 * NQB];
    float pv[2], dsv[2];
#pragma unroll
    for (int v = 0; v < NVAL; ++v) {
      value(v, sc, dpc, lsev, dltv, pv, dsv);
      if (v & 1) pack(v, pv, dsv, pb, dsb);
    }
    f32x16_t unused_s[NQB], unused_p[NQB];
#pragma unroll
    for (int m = NMA; m < NMA + NMB; ++m) mfma_slot(m, *op_ptr(s_cur, s_cur, m), unused_s, unused_p, pb, dsb);
  };

  if (nqt > 0) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    wait_vmem_n<2 * C::LOADS>();  // K, V rows and tile 0
    __syncthreads();
    f32x16_t sa[NQB], pa[NQB], sb[NQB], pbb[NQB];
    {
      const lds_char_t* s0 = stage(IC<0>{});
      i32x4_t dummy_p[2 * NQB], dummy_d[2 * NQB];
#pragma unroll
      for (int m = 0; m < NMA; ++m) mfma_slot(m, *op_ptr(s0, s0, m), sa, pa, dummy_p, dummy_d);
    }
    int j = 0;
    for (; j + 4 < nqt; j += 4) {
      step(IC<0>{}, j, sa, pa, sb, pbb);
      step(IC<1>{}, j + 1, sb, pbb, sa, pa);
      step(IC<2>{}, j + 2, sa, pa, sb, pbb);
      step(IC<3>{}, j + 3, sb, pbb, sa, pa);
    }
    const int rest = nqt - j;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, j, sa, pa, sb, pbb);
    if (rest >= 3) step(IC<1>{}, j + 1, sb, pbb, sa, pa);
    if (rest >= 4) step(IC<2>{}, j + 2, sa, pa, sb, pbb);
    if (rest == 1) last_step(IC<0>{}, sa, pa);
    else if (rest == 2) last_step(IC<1>{}, sb, pbb);
    else if (rest == 3) last_step(IC<2>{}, sa, pa);
    else last_step(IC<3>{}, sb, pbb);
    wait_vmem();  // no requests beyond the last tile stay in flight
  }

  // ---- store dK = s (dK^T)^T, dV = (dV^T)^T for this lane's key
  if (key < p.Lk) {
    char* dkp = (char*)p.dk + ((b * p.dk_sb + h * p.dk_sh) + (int64_t)key * p.dk_sl) * 2;
    char* dvp = (char*)p.dv + ((b * p.dv_sb + h * p.dv_sh) + (int64_t)key * p.dv_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int dc = d * 32 + 8 * jj + 4 * half;
        u32x2_t wk = {Elem<T>::pack2(dkacc[d][4 * jj] * p.scale, dkacc[d][4 * jj + 1] * p.scale),
                      Elem<T>::pack2(dkacc[d][4 * jj + 2] * p.scale, dkacc[d][4 * jj + 3] * p.scale)};
        u32x2_t wv = {Elem<T>::pack2(dvacc[d][4 * jj], dvacc[d][4 * jj + 1]),
                      Elem<T>::pack2(dvacc[d][4 * jj + 2], dvacc[d][4 * jj + 3])};
        *(u32x2_t*)(dkp + dc * 2) = wk;
        *(u32x2_t*)(dvp + dc * 2) = wv;
      }
    }
  }
}

// dO-only dK/dV pass reading the transposed operands Q^T, dO^T straight from
// the row-major Q, dO tiles with lds_read_tr16 (no transposed copies in HBM or
// LDS). 4 waves x 32 keys, 32-query steps through a four-stage ring. Step j is
// a fixed MFMA stream:
//   S, dP of tile j+1 (the second half of tile j's P, dS on the VALU), then
//   dV^T += dO^T P, dK^T += Q^T dS of tile j (the first half of tile j+1's P,
//   dS on the VALU; tile j+3 requested meanwhile).
template <int D, int BMQ_>
struct KvTrCfg {
  static constexpr int NW = 4;
  static constexpr int BK = 32 * NW;
  static constexpr int BMQ = BMQ_;
  static constexpr int NQB = BMQ / 32;
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;  // 16-byte chunks per Q / dO row
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BMQ * ROWB;
  static constexpr int OFF_Q = 0;
  static constexpr int OFF_DO = ROW_BYTES;
  static constexpr int OFF_ST = 2 * ROW_BYTES;
  static constexpr int STAT_BYTES = 2 * BMQ * 4;
  static constexpr int STAGE = (OFF_ST + STAT_BYTES + 1023) / 1024 * 1024;
  static constexpr int NSTAGE = 4;
  static constexpr int NRI = BMQ * CR / 64;  // wave-wide 1 KiB loads per row tile
  static constexpr int RPW = NRI / NW;
  static constexpr int ST_LANES = STAT_BYTES / 16 / NW;
  static constexpr bool FITS = (D == 128 || D == 64) && NRI % NW == 0 && NSTAGE * STAGE <= 160 * 1024;
  static constexpr int LOADS = 2 * RPW + 1;
};

// Query tile of attn_bwd_kv_tr_kernel.
constexpr int kKvTrBmq = 32;

// What attn_bwd_kv_tr_kernel does with stored score gradients (ScLayout).
enum KvScMode : int {
  kScNone = 0,   // nothing stored or read
  kScStore = 1,  // writes each tile's dS (dO-only backward: the query pass reads it back)
  kScLoad = 2    // reads dS (tensor 1 of a full-derivative layout: dSd) instead of computing dP, dS
};

// Compiled with MFMAs in VGPR form (bwd_kv_inst.hip): the S, dP MFMAs write
// VGPRs that the VALU reads directly, and the dK, dV accumulators stay in
// AGPRs through inline MFMAs (mfma32_acc).
// SCM == kScStore (128-wide heads): also writes each tile's dS (the bf16/fp16
// operand of the dK update, keys at or beyond Lk as zeros) to p.sc in the
// ScLayout for attn_bwd_dq_sc_kernel, chunk 0 of tile j in slot 14 of step j
// and chunk 1 (packed by slot 13) in slot 28, between the step's ring requests.
// The next barrier's vmcnt(LOADS) stays exact whatever order stores and loads
// complete in: a request of tile j + 2 still in flight means all LOADS requests
// of tile j + 3 are too.
// SCM == kScLoad (128-wide heads; the full derivative's tangent key pass, run on
// (dO, D) := (dOd, rho)): dS = P (dP - D) is the dSd the full key pass stored
// (tensor 1 of its layout), so the pass reads it instead of computing dP: each
// wave's two 1 KiB chunks of a tile ride in the ring stage with the Q and dO
// rows (a lane's 16 bytes land where it reads them), V is not read, and a step
// runs 8 S MFMAs and 16 update MFMAs instead of 32.
template <typename T, int D, int SCM = kScNone>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void attn_bwd_kv_tr_kernel(BwdParams p) {
  using C = KvTrCfg<D, kKvTrBmq>;
  constexpr int BMQ = C::BMQ, NQB = C::NQB, KS = C::KS, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  constexpr bool STORE = SCM == kScStore, LOAD = SCM == kScLoad;
  static_assert(C::FITS, "configuration does not fit");
  static_assert(SCM == kScNone || D == 128, "stored score gradients are laid out for 128-wide heads");
  // the loaded dS chunks follow the stage's rows and statistics: 2 KiB per wave
  constexpr int OFF_DS = C::STAGE, STAGE = C::STAGE + (LOAD ? C::NW * 2 * ScLayout::CHUNK : 0);
  constexpr int LOADS = C::LOADS + (LOAD ? 2 : 0);  // requests per wave per tile
  static_assert(4 * STAGE <= 160 * 1024, "the ring fits the LDS");
  __shared__ __attribute__((aligned(1024))) char stg0[STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nkt = (p.Lk + C::BK - 1) / C::BK;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int slice = work / nkt, kt = work - slice * nkt;
  const int bh = (SCM != kScNone ? p.bh0 : 0) + slice;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nqt = p.LQP / BMQ;

  const int key = kt * C::BK + wave * 32 + col;

  // ---- stored score gradients (STORE: dS written; LOAD: tensor 1 of a full
  // layout read): this wave's key block of the slice's strips
  constexpr int SC_NT = LOAD ? 2 : 1;
  const int64_t sc_strip = ScLayout::strip_stride(4 * nkt, SC_NT);  // one query block
  char* const sc_base = SCM != kScNone ? (char*)p.sc + (int64_t)slice * p.sc_slice : nullptr;
  const uint32_t sc_kb = (uint32_t)(kt * 4 + wave) * SC_NT * ScLayout::PIECE + (LOAD ? ScLayout::PIECE : 0);
  const uint32_t sc_lo0 = ScLayout::lane_off(col, half, 0), sc_lo1 = ScLayout::lane_off(col, half, 1);
  const bool sc_tail = (kt + 1) * C::BK > p.Lk;  // keys at or beyond Lk in this workgroup
  auto store_chunk = [&](int qt, int u, i32x4_t v) {
    if (sc_tail && key >= p.Lk) v = i32x4_t{0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(sc_base + (int64_t)(qt >> 2) * sc_strip, (uint32_t)(sc_strip - ScLayout::STRIP_PAD));
    buf_store16_stream(rs, v, u ? sc_lo1 : sc_lo0,
                       sc_kb + (uint32_t)(qt & 3) * ScLayout::TILE + (uint32_t)u * ScLayout::CHUNK);
  };

  // ---- stationary K, V rows: B operands of S = Q K^T and dP = dO V^T (LOAD: K only)
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + (b * p.v_sb + h * p.v_sh) * 2, v_bytes);
  i32x4_t kreg[KS], vreg[KS];
  {
    const uint32_t ko = (uint32_t)((int64_t)key * p.k_sl * 2) + half * 16;
    const uint32_t vo = (uint32_t)((int64_t)key * p.v_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kreg[s] = buf_load16(rk, ko + s * 32);
      if constexpr (!LOAD) vreg[s] = buf_load16(rv, vo + s * 32);
    }
  }

  // ---- query-side resources and per-lane DMA offsets
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const uint32_t st_bytes = (uint32_t)((int64_t)p.LQP * 2 * 4);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + (b * p.do_sb + h * p.do_sh) * 2, do_bytes);
  const __amdgpu_buffer_rsrc_t rst = make_rsrc((const char*)p.stats + (int64_t)bh * st_bytes, st_bytes);
  constexpr int RPW = C::RPW;
  uint32_t roff_q[RPW], roff_do[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ trswz<CR>(row & 15);
    roff_q[j] = (uint32_t)((int64_t)row * p.q_sl * 2) + logical * 16;
    roff_do[j] = (uint32_t)((int64_t)row * p.do_sl * 2) + logical * 16;
  }
  const uint32_t q_step = (uint32_t)((int64_t)BMQ * p.q_sl * 2);
  const uint32_t do_step = (uint32_t)((int64_t)BMQ * p.do_sl * 2);
  static_assert(C::ST_LANES * C::NW * 16 == C::STAT_BYTES, "statistics split evenly over the waves");
  const bool st_lane = lane >= wave * C::ST_LANES && lane < (wave + 1) * C::ST_LANES;

  auto stage = [&](auto kk) -> lds_char_t* {
    constexpr int k = decltype(kk)::value & 3;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else if constexpr (k == 2) return (lds_char_t*)stg2;
    else return (lds_char_t*)stg3;
  };
  // request li (0 <= li < LOADS) of tile qt into stage st; tiles at or beyond
  // the end read zeros or in-range rows into a stage nobody reads again (the
  // loaded dS chunks of such tiles are the last tile's again: a strip beyond the
  // slice does not exist)
  auto issue_load = [&](lds_char_t* st, int qt, int li) {
    if (li < 2 * RPW) {
      const int jj = li >> 1, i = wave + jj * C::NW;
      if (li & 1) buf_load16_lds(rdo, st + C::OFF_DO + i * 1024, roff_do[jj], (uint32_t)qt * do_step);
      else buf_load16_lds(rq, st + C::OFF_Q + i * 1024, roff_q[jj], (uint32_t)qt * q_step);
    } else if (li == 2 * RPW) {
      if (st_lane) buf_load16_lds(rst, st + C::OFF_ST, lane * 16, (uint32_t)qt * C::STAT_BYTES);
    } else if constexpr (LOAD) {
      const int u = li - 2 * RPW - 1, qc = qt < nqt ? qt : nqt - 1;
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(sc_base + (int64_t)(qc >> 2) * sc_strip, (uint32_t)(sc_strip - ScLayout::STRIP_PAD));
      buf_load16_lds(rs, st + OFF_DS + wave * 2 * ScLayout::CHUNK + u * ScLayout::CHUNK, u ? sc_lo1 : sc_lo0,
                     sc_kb + (uint32_t)(qc & 3) * ScLayout::TILE + (uint32_t)u * ScLayout::CHUNK);
    }
  };

  // ---- LDS read offsets. Row-wise reads (S, dP): row 32 qb + perm32(col), chunk 2s + half.
  int sx[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int r = perm32(col);
    sx[s] = r * ROWB + (((2 * s + half) ^ trswz<CR>(r & 15)) << 4);
  }
  // Transposed reads (dO^T, Q^T blocks): lane group g = lane / 16 covers d0 = 32 db + 16 (g & 1)
  // and queries 16 u + 8 (g >> 1) + (0..3 | 4..7); lane 4r + c of the group points at row r,
  // elements d0 + 4c .. d0 + 4c + 3.
  int tx[DB][2];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, c = lane & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = 8 * (g >> 1) + 4 * hh + r;  // plus 16 u
        const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
        tx[db][hh] = row * ROWB + ((chunk ^ trswz<CR>(row & 15)) << 4) + 8 * (c & 1);
      }
    }
  }
  auto pin_offsets = [&]() {
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+v"(sx[s]));
#pragma unroll
    for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(tx[db][0]), "+v"(tx[db][1]));
  };

  f32x16_t dkacc[DB], dvacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      dkacc[d][v] = 0.f;
      dvacc[d][v] = 0.f;
    }
  }

  // D = 128 keeps the dK, dV accumulators in AGPRs through inline MFMAs (462
  // registers, one wave per SIMD); D = 64 keeps everything in VGPRs (no AGPRs,
  // so the compiler can fit two waves per SIMD in 256 registers)
  constexpr bool kAccAgpr = D == 128;
  constexpr int PF = 4;
  constexpr int NMA = (LOAD ? 1 : 2) * KS * NQB;   // S, dP MFMAs (LOAD: S)
  constexpr int NMB = 4 * NQB * DB;   // dV^T, dK^T MFMAs
  constexpr int NS = NMA + NMB;
  constexpr int NVAL = 16 * NQB;      // P, dS values per lane per tile
  const f32x16_t zero16 = {};
  // operand m: m < NMA reads Q / dO rows of the next tile (s = m / (2 NQB)),
  // otherwise dO^T / Q^T of this tile (u = 16-query chunk, db = 32-row d block)
  auto load_op = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int m) -> i32x4_t {
    if constexpr (LOAD) {
      if (m < NMA) return *(lds_i32x4_t*)(s_next + C::OFF_Q + (m % NQB) * 32 * ROWB + sx[m / NQB]);
    }
    if (m < NMA) {
      const int s = m / (2 * NQB), r = m % (2 * NQB), qb = r >> 1;
      return *(lds_i32x4_t*)(s_next + ((r & 1) ? C::OFF_DO : C::OFF_Q) + qb * 32 * ROWB + sx[s]);
    }
    const int mm = m - NMA, u = mm / (2 * DB), r = mm % (2 * DB), db = r >> 1;
    const lds_char_t* base = s_cur + ((r & 1) ? C::OFF_Q : C::OFF_DO) + u * 16 * ROWB;
    const u32x2_t lo = lds_read_tr16(base + tx[db][0]);
    const u32x2_t hi = lds_read_tr16(base + tx[db][1]);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };
  // statistics of 16-query chunk u: lse (log2 units), Delta for queries 16 u + 8 half + 0..7
  struct Stats {
    f32x4_t l[2], d[2];
  };
  auto load_stats = [&](const lds_char_t* st, int u, Stats& sv) {
    const lds_char_t* sst = st + C::OFF_ST;
    const int q0 = 16 * u + 8 * half;
    sv.l[0] = *(lds_f32x4_t*)(sst + 4 * q0);
    sv.l[1] = *(lds_f32x4_t*)(sst + 4 * (q0 + 4));
    sv.d[0] = *(lds_f32x4_t*)(sst + 4 * (BMQ + q0));
    sv.d[1] = *(lds_f32x4_t*)(sst + 4 * (BMQ + q0 + 4));
  };
  // Values of a tile: 16 per lane, value v = C-tile value v of S, dP (query 16 t + 8 half + e for
  // v = 8 t + e). Chunk u = values 8u .. 8u + 7 feeds the update MFMAs of 16-query chunk u; pair i of
  // a chunk = values 8u + 2i, 8u + 2i + 1, packed into component i of pb[u] (P~) and dsb[u] (dS~).
  // A pair is computed in two halves placed in different MFMA slots, so that the exp latency is
  // covered by an MFMA: half 1 = exp2(s c - lse2) and dP - Delta, half 2 = the product and packs.
  struct Half {
    float p[2], dd[2];
  };
  auto pair_first = [&](int u, int i, const f32x16_t& sc, const f32x16_t& dpc, const Stats& sv, Half& hv) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int v = 8 * u + 2 * i + w, e = v % 8;
      const float l2 = sv.l[e >> 2][e & 3], dl = sv.d[e >> 2][e & 3];
      // re-define the inputs here (an empty asm) so the compiler cannot hoist the
      // arithmetic out of its MFMA slot and bunch the VALU work together
      if constexpr (LOAD) {
        float s_in = sc[v];
        asm volatile("" : "+v"(s_in));
        hv.p[w] = fast_exp2(fmaf(s_in, p.scale_log2, -l2));
      } else {
        float s_in = sc[v], d_in = dpc[v];
        asm volatile("" : "+v"(s_in), "+v"(d_in));
        hv.p[w] = fast_exp2(fmaf(s_in, p.scale_log2, -l2));
        hv.dd[w] = d_in - dl;
      }
    }
  };
  auto pair_second = [&](int i, Half& hv, i32x4_t& pbu, i32x4_t& dsbu) {
    if constexpr (LOAD) {  // P~ only: dS~ is loaded
      asm volatile("" : "+v"(hv.p[0]), "+v"(hv.p[1]));
      pbu[i] = (int)Elem<T>::pack2(hv.p[0], hv.p[1]);
      asm volatile("" : "+v"(pbu[i]));
    } else {
      asm volatile("" : "+v"(hv.p[0]), "+v"(hv.p[1]), "+v"(hv.dd[0]), "+v"(hv.dd[1]));
      pbu[i] = (int)Elem<T>::pack2(hv.p[0], hv.p[1]);
      dsbu[i] = (int)Elem<T>::pack2(hv.p[0] * hv.dd[0], hv.p[1] * hv.dd[1]);
      asm volatile("" : "+v"(pbu[i]), "+v"(dsbu[i]));
    }
  };
  // the loaded dS~ chunk u of the tile in stage st (LOAD)
  auto load_ds = [&](const lds_char_t* st, int u) -> i32x4_t {
    return *(lds_i32x4_t*)(st + OFF_DS + wave * 2 * ScLayout::CHUNK + u * ScLayout::CHUNK + lane * 16);
  };
  // all 16 values of a tile at once (prologue and last step)
  auto chunk_now = [&](const lds_char_t* st, int u, const f32x16_t& sc, const f32x16_t& dpc, i32x4_t& pbu,
                       i32x4_t& dsbu) {
    Stats sv;
    load_stats(st, u, sv);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Half hv;
      pair_first(u, i, sc, dpc, sv, hv);
      pair_second(i, hv, pbu, dsbu);
    }
  };
  auto mfma_slot = [&](int m, i32x4_t op, f32x16_t (&sn)[NQB], f32x16_t (&dpn)[NQB], const i32x4_t (&pb)[2 * NQB],
                       const i32x4_t (&dsb)[2 * NQB]) {
    if (LOAD && m < NMA) {
      const int s = m / NQB, qb = m % NQB;
      sn[qb] = mfma32(op, kreg[s], s == 0 ? zero16 : sn[qb], T());
    } else if (m < NMA) {
      const int s = m / (2 * NQB), r = m % (2 * NQB), qb = r >> 1;
      if (r & 1) dpn[qb] = mfma32(op, vreg[s], s == 0 ? zero16 : dpn[qb], T());
      else sn[qb] = mfma32(op, kreg[s], s == 0 ? zero16 : sn[qb], T());
    } else {
      const int mm = m - NMA, u = mm / (2 * DB), r = mm % (2 * DB), db = r >> 1;
      if constexpr (kAccAgpr) {
        if (r & 1) mfma32_acc(dkacc[db], op, dsb[u], T());
        else mfma32_acc(dvacc[db], op, pb[u], T());
      } else {
        if (r & 1) dkacc[db] = mfma32(op, dsb[u], dkacc[db], T());
        else dvacc[db] = mfma32(op, pb[u], dvacc[db], T());
      }
    }
  };
  static_assert(NQB == 1 && (NS == 32 || NS == 16 || (LOAD && NS == 24)),
                "slot plan below assumes one 32-query block per step");
  // Slot plan of step j (P~, dS~ of chunk 0 of tile j arrive computed by the previous step), D = 128:
  //   slots  0..15  S, dP MFMAs of tile j + 1; chunk 1 of tile j: pair i halves at 2 + 3i, 4 + 3i
  //   slots 16..23  dV, dK MFMAs of chunk 0; 24..31 of chunk 1
  //   slots 17..31  chunk 0 of tile j + 1 (S, dP of tile j + 1 complete after slot 15): halves at 17 + 4i, 19 + 4i
  // D = 64 (half the MFMAs, the same values): S, dP in slots 0..7, updates of chunk 0 in 8..11 and of chunk 1
  // in 12..15; chunk 1 of tile j: halves at i, 2 + i; chunk 0 of tile j + 1: halves at 9 + i, 11 + i.
  // LOAD (D = 128, P~ only): S in slots 0..7, updates of chunk 0 in 8..15 and of chunk 1 in 16..23; chunk 1 of
  // tile j: halves at 1 + 2i, 3 + 2i; chunk 0 of tile j + 1: halves at 9 + 3i, 11 + 3i; the loaded dS~ of tile j
  // read in slot 0.
  constexpr int A1 = NS == 32 ? 2 : LOAD ? 1 : 0, AS = NS == 32 ? 3 : LOAD ? 2 : 1;
  constexpr int B1 = NMA + 1, BS = NS == 32 ? 4 : LOAD ? 3 : 1;
  constexpr int STAT_SLOT = NS == 16 ? 6 : LOAD ? 6 : 12;  // statistics of tile j + 1 requested here
  constexpr int SC_SLOT0 = 14, SC_SLOT1 = 28;   // score stores of tile j (STORE, 32 slots per step)
  auto step = [&](auto kk, int j, const f32x16_t (&sc)[NQB], const f32x16_t (&dpc)[NQB], f32x16_t (&sn)[NQB],
                  f32x16_t (&dpn)[NQB], const i32x4_t& pb0, const i32x4_t& ds0, i32x4_t& pb0n, i32x4_t& ds0n) {
    constexpr int k = decltype(kk)::value;
    ring_sync<LOADS>();  // tile j + 1 has landed (tile j + 2 may be in flight)
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    Stats sv1, svn;  // chunk 1 of tile j, chunk 0 of tile j + 1
    load_stats(s_cur, 1, sv1);
    i32x4_t opr[PF];
#pragma unroll
    for (int m = 0; m < PF; ++m) opr[m] = load_op(s_next, s_cur, m);
    i32x4_t pb[2], dsb[2];
    pb[0] = pb0;
    if constexpr (LOAD) {
      dsb[0] = load_ds(s_cur, 0);
      dsb[1] = load_ds(s_cur, 1);
    } else {
      dsb[0] = ds0;
    }
    Half h1[4], hn[4];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < NS; ++m) {
      mfma_slot(m, opr[m % PF], sn, dpn, pb, dsb);
      if (m + PF < NS) opr[m % PF] = load_op(s_next, s_cur, m + PF);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (m == A1 + AS * i) pair_first(1, i, sc[0], dpc[0], sv1, h1[i]);
        if (m == A1 + 2 + AS * i) pair_second(i, h1[i], pb[1], dsb[1]);
        if (m == B1 + BS * i) pair_first(0, i, sn[0], dpn[0], svn, hn[i]);
        if (m == B1 + 2 + BS * i) pair_second(i, hn[i], pb0n, ds0n);
      }
      if (m == STAT_SLOT) load_stats(s_next, 0, svn);
      if constexpr (STORE) {
        if (m == SC_SLOT0) store_chunk(j, 0, ds0);
        if (m == SC_SLOT1) store_chunk(j, 1, dsb[1]);
      }
#pragma unroll
      for (int li = 0; li < LOADS; ++li) {
        if (li * NS / LOADS == m) issue_load(s_req, j + 3, li);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(A1 + 2 + AS * 3 < NMA + 2 * DB, "chunk 1 is packed before its first update MFMA");
  static_assert(B1 + 2 + BS * 3 < NS, "chunk 0 of the next tile is packed within the step");
  static_assert(STAT_SLOT < B1, "statistics of the next tile are requested before their first use");
  static_assert(!STORE || (NS == 32 && A1 + 2 + AS * 3 < SC_SLOT1), "chunk 1 is packed before its store");
  // final tile: chunk 1 values then the update MFMAs
  auto last_step = [&](auto kk, const f32x16_t (&sc)[NQB], const f32x16_t (&dpc)[NQB], const i32x4_t& pb0,
                       const i32x4_t& ds0) {
    const lds_char_t* s_cur = stage(kk);
    i32x4_t pb[2], dsb[2];
    pb[0] = pb0;
    dsb[0] = ds0;
    chunk_now(s_cur, 1, sc[0], dpc[0], pb[1], dsb[1]);
    if constexpr (LOAD) {
      dsb[0] = load_ds(s_cur, 0);
      dsb[1] = load_ds(s_cur, 1);
    }
    if constexpr (STORE) {
      store_chunk(nqt - 1, 0, dsb[0]);
      store_chunk(nqt - 1, 1, dsb[1]);
    }
    f32x16_t un_s[NQB], un_p[NQB];
#pragma unroll
    for (int m = NMA; m < NS; ++m) mfma_slot(m, load_op(s_cur, s_cur, m), un_s, un_p, pb, dsb);
  };

  if (nqt > 0) {
#pragma unroll
    for (int li = 0; li < LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    ring_sync<2 * LOADS>();  // K, V rows and tile 0
    f32x16_t sa[NQB], pa[NQB], sb[NQB], pbb[NQB];
    i32x4_t ca_p, ca_d, cb_p, cb_d;  // chunk-0 packs carried between steps (alternating)
    {
      const lds_char_t* s0 = stage(IC<0>{});
      i32x4_t dummy_p[2 * NQB], dummy_d[2 * NQB];
#pragma unroll
      for (int m = 0; m < NMA; ++m) mfma_slot(m, load_op(s0, s0, m), sa, pa, dummy_p, dummy_d);
      chunk_now(s0, 0, sa[0], pa[0], ca_p, ca_d);
    }
    int j = 0;
    for (; j + 4 < nqt; j += 4) {
      step(IC<0>{}, j, sa, pa, sb, pbb, ca_p, ca_d, cb_p, cb_d);
      step(IC<1>{}, j + 1, sb, pbb, sa, pa, cb_p, cb_d, ca_p, ca_d);
      step(IC<2>{}, j + 2, sa, pa, sb, pbb, ca_p, ca_d, cb_p, cb_d);
      step(IC<3>{}, j + 3, sb, pbb, sa, pa, cb_p, cb_d, ca_p, ca_d);
    }
    const int rest = nqt - j;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, j, sa, pa, sb, pbb, ca_p, ca_d, cb_p, cb_d);
    if (rest >= 3) step(IC<1>{}, j + 1, sb, pbb, sa, pa, cb_p, cb_d, ca_p, ca_d);
    if (rest >= 4) step(IC<2>{}, j + 2, sa, pa, sb, pbb, ca_p, ca_d, cb_p, cb_d);
    if (rest == 1) last_step(IC<0>{}, sa, pa, ca_p, ca_d);
    else if (rest == 2) last_step(IC<1>{}, sb, pbb, cb_p, cb_d);
    else if (rest == 3) last_step(IC<2>{}, sa, pa, ca_p, ca_d);
    else last_step(IC<3>{}, sb, pbb, cb_p, cb_d);
    wait_vmem();  // no requests beyond the last tile stay in flight
  }
  if constexpr (kAccAgpr) mfma_acc_drain();  // the last dK, dV MFMAs have finished before their AGPRs are read

  // ---- store dK = s (dK^T)^T, dV = (dV^T)^T for this lane's key
  if (key < p.Lk) {
    char* dkp = (char*)p.dk + ((b * p.dk_sb + h * p.dk_sh) + (int64_t)key * p.dk_sl) * 2;
    char* dvp = (char*)p.dv + ((b * p.dv_sb + h * p.dv_sh) + (int64_t)key * p.dv_sl) * 2;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int dc = d * 32 + 8 * jj + 4 * half;
        u32x2_t wk = {Elem<T>::pack2(dkacc[d][4 * jj] * p.scale, dkacc[d][4 * jj + 1] * p.scale),
                      Elem<T>::pack2(dkacc[d][4 * jj + 2] * p.scale, dkacc[d][4 * jj + 3] * p.scale)};
        u32x2_t wv = {Elem<T>::pack2(dvacc[d][4 * jj], dvacc[d][4 * jj + 1]),
                      Elem<T>::pack2(dvacc[d][4 * jj + 2], dvacc[d][4 * jj + 3])};
        *(u32x2_t*)(dkp + dc * 2) = wk;
        *(u32x2_t*)(dvp + dc * 2) = wv;
      }
    }
  }
}

// Query tile of the dO-only dK/dV kernel chosen for head dim D (it fixes the
// layout of the backward statistics).
template <int D>
constexpr int dout_only_kv_bmq() {
  if constexpr (KvTrCfg<D, kKvTrBmq>::FITS) return kKvTrBmq;
  else if constexpr (KvPipeCfg<D, kv_pipe_bmq<D>()>::FITS) return kv_pipe_bmq<D>();
  else return BwdCfg<D, kBwdDoutOnly>::BMQ;
}

// Per-row statistics for the backward, one thread per (b*h, query row):
//   A layout  [BH][LQP/BA][2][BA]: lse2 = LSE*log2(e), D = rowsum(dO*O)
//   B layout  [BH][LQP/32][4][32]: lse2, D' = rowsum(dO*O) + rowsum(dOd*Od) - mu*rho, mu, rho
//   BT layout [BH][LQP/BA][2][BA]: lse2, rho = rowsum(dOd*O)   (tangent gradients)
// BA is the query tile of the dO-only key-stationary kernel for this head dim.
// Rows past Lq get lse2 = +inf (so P = 0) and zeros.
struct PrepParams {
  const void* o;
  const void* to;
  const void* dout;
  const void* dto;
  const float* lse;
  const float* mu;
  float* stats_a;   // may be null
  float* stats_b;   // may be null
  float* stats_bt;  // may be null
  int64_t o_sb, o_sh, o_sl;
  int64_t do_sb, do_sh, do_sl;
  int H, Lq, LQP, D, BH, BA;
};


}  // namespace dmad
