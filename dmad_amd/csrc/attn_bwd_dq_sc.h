// Query pass over stored score gradients, 128-wide heads: dQ (and dQd) as a
// streaming GEMM over the dS (and dSd) tiles a STORE key pass wrote in the
// ScLayout (attn_bwd.h), instead of recomputing S and dP per (query, key) pair:
//   NT = 1 (dO-only gradients):    dQ = s dS K
//   NT = 2 (full derivative):      dQ = s (dS K + dSd Kd),  dQd = s dSd K
// Per (query, key) pair this reads the 2 NT bytes of stored gradients once from
// HBM and runs 2 (NT = 1) or 6 (NT = 2) units of MFMA work, where the
// recomputing passes run 6 or 18.
//
// One workgroup = 4 waves x 32 queries: wave w takes query tile w of the
// workgroup's 128-query block. 32-key steps run through a ring of NSTAGE LDS
// stages; a stage holds the step's K [and Kd] rows (row-major, chunk-swizzled
// for transposed reads, as the other row-reading passes stage them) and the
// (query block, key block) piece of the stored gradients, copied as it lies.
// Per step and wave, for each 16-key slice: the B operands dS^T [dSd^T]
// (lane = query, 8 consecutive keys) and the A operands K^T [Kd^T] (lane = d,
// 8 consecutive keys), both with ds_read_b64_tr_b16, then
//   dQ^T += K^T dS^T [+ Kd^T dSd^T],   [dQd^T += K^T dSd^T].
// Keys at or beyond Lk read K = Kd = 0 and their stored gradients are zeros.
#pragma once
#include "attn_bwd.h"
#include "attn_bwd_dq.h"

namespace dmad {

template <int NT>
struct DqScCfg {
  static constexpr int D = 128;
  static constexpr int NW = 4;
  static constexpr int BM = ScLayout::BQ;  // queries per workgroup
  static constexpr int BN = ScLayout::BK;  // keys per step
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BN * ROWB;  // K rows of one step
  static constexpr int OFF_K = 0, OFF_TK = ROW_BYTES;
  static constexpr int OFF_SC = NT * ROW_BYTES;
  static constexpr int STAGE = NT * ROW_BYTES + NT * ScLayout::PIECE;
  static constexpr int NSTAGE = 4;
  static constexpr int WG_PER_CU = NT == 1 ? 2 : 1;  // 64 KiB or 128 KiB of ring per workgroup
  static constexpr int NRI = ROW_BYTES / 1024;  // wave-wide 1 KiB requests per row tile
  static constexpr int RPW = NRI / NW;
  static constexpr int NSC = NT * ScLayout::PIECE / 1024;  // requests per stored piece
  static constexpr int SPW = NSC / NW;
  static constexpr int LOADS = NT * RPW + SPW;  // requests per wave per step
  static_assert(NRI % NW == 0 && NSC % NW == 0, "requests split evenly over the waves");
  static_assert(NSTAGE * STAGE <= 160 * 1024, "the ring fits the LDS");
  static_assert(3 * LOADS < 64, "vmcnt is a 6-bit field");
};

template <typename T, int NT>
__global__ __launch_bounds__(256, DqScCfg<NT>::WG_PER_CU) void attn_bwd_dq_sc_kernel(DqParams p) {
  using C = DqScCfg<NT>;
  constexpr int D = C::D, BN = C::BN, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  static_assert(C::NSTAGE == 4, "four stage arrays below");
  // one array per stage, addressed with compile-time stage numbers, so the
  // compiler can tell the stage being filled from the one being read (with one
  // array it waits for every in-flight request before each LDS read)
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nqb = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int slice = work / nqb, qb = work - slice * nqb;
  const int bh = p.bh0 + slice;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nsteps = (p.Lk + BN - 1) / BN;
  const int query = qb * C::BM + wave * 32 + col;

  // ---- K [, Kd] rows: per-lane request offsets (row, swizzled chunk)
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const int64_t khead = b * p.k_sb + h * p.k_sh;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + khead * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rtk = make_rsrc((const char*)(NT == 2 ? p.tk : p.k) + khead * 2, k_bytes);
  uint32_t roff_k[C::RPW];
#pragma unroll
  for (int j = 0; j < C::RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ trswz<CR>(row & 15);
    roff_k[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
  }
  const uint32_t k_step = (uint32_t)((int64_t)BN * p.k_sl * 2);
  // ---- stored gradients: this workgroup's strip [key block][tensor][piece]
  const uint32_t strip = (uint32_t)p.sc_nkb * NT * ScLayout::PIECE;
  const __amdgpu_buffer_rsrc_t rsc =
      make_rsrc((const char*)p.sc + (int64_t)slice * p.sc_slice + (int64_t)qb * strip, strip);

  // request li of step jj into stage st (steps past the end repeat the last one)
  auto issue_load = [&](lds_char_t* st, int jj, int li) {
    jj = jj < nsteps ? jj : nsteps - 1;
    if (li < NT * C::RPW) {
      const int t = li / C::RPW, r = li % C::RPW, i = wave + r * C::NW;
      buf_load16_lds(t ? rtk : rk, st + (t ? C::OFF_TK : C::OFF_K) + i * 1024, roff_k[r], (uint32_t)jj * k_step);
    } else {
      const int i = wave + (li - NT * C::RPW) * C::NW;
      buf_load16_lds(rsc, st + C::OFF_SC + i * 1024, (uint32_t)(i * 1024 + lane * 16),
                     (uint32_t)jj * NT * ScLayout::PIECE);
    }
  };

  // ---- transposed-read offsets
  // A = K^T (d x 16 keys): lane group g covers d0 = 32 db + 16 (g & 1), keys 8 (g >> 1) + 0..7
  int tx[DB][2];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, c = lane & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = 8 * (g >> 1) + 4 * hh + r;
        const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
        tx[db][hh] = row * ROWB + ((chunk ^ trswz<CR>(row & 15)) << 4) + 8 * (c & 1);
      }
    }
  }
  // B = dS^T (16 keys x 32 queries): lane group g reads chunk u = g & 1 of this
  // wave's tile (queries 16 u + 0..15 = lane % 32) at keys 8 (g >> 1) + 4 hh + 0..3
  int bx[2];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, c = lane & 3, u = g & 1;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = (8 * (g >> 1) + 4 * hh + r) ^ (4 * u);
      bx[hh] = wave * ScLayout::TILE + u * ScLayout::CHUNK + row * 32 + 8 * c;
    }
  }
  auto tr_pair = [&](const lds_char_t* base, int o0, int o1) -> i32x4_t {
    const u32x2_t lo = lds_read_tr16(base + o0);
    const u32x2_t hi = lds_read_tr16(base + o1);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };

  f32x16_t acc[DB], tacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc[d][v] = 0.f;
      tacc[d][v] = 0.f;
    }
  }

  auto stage = [&](auto kk) -> lds_char_t* {
    constexpr int k = decltype(kk)::value & 3;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else if constexpr (k == 2) return (lds_char_t*)stg2;
    else return (lds_char_t*)stg3;
  };
  // every operand of the step is read before its first MFMA, so one LDS
  // latency is paid per step rather than one per MFMA
  auto compute = [&](const lds_char_t* st) {
    i32x4_t bs[2], bd[2], a[2][DB], at[2][DB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const lds_char_t* sb = st + C::OFF_SC + ks * 16 * 32;
      bs[ks] = tr_pair(sb, bx[0], bx[1]);
      if constexpr (NT == 2) bd[ks] = tr_pair(sb + ScLayout::PIECE, bx[0], bx[1]);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const lds_char_t* kb = st + C::OFF_K + ks * 16 * ROWB;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        a[ks][db] = tr_pair(kb, tx[db][0], tx[db][1]);
        if constexpr (NT == 2) at[ks][db] = tr_pair(kb + C::OFF_TK, tx[db][0], tx[db][1]);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[db] = mfma32(a[ks][db], bs[ks], acc[db], T());
        if constexpr (NT == 2) {
          tacc[db] = mfma32(a[ks][db], bd[ks], tacc[db], T());
          acc[db] = mfma32(at[ks][db], bd[ks], acc[db], T());
        }
      }
    }
  };

  // step j (j % 4 == kk): once step j has landed, refill the stage step j - 1
  // used (every wave is past its reads) with step j + 3, then compute step j
  auto step = [&](auto kk, int j) {
    constexpr int k = decltype(kk)::value;
    ring_sync<2 * C::LOADS>();  // step j has landed; steps j + 1, j + 2 may be in flight
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<k + 3>{}), j + 3, li);
    compute(stage(IC<k>{}));
  };
  if (nsteps > 0) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    int j = 0;
    for (; j + 4 <= nsteps; j += 4) {
      step(IC<0>{}, j);
      step(IC<1>{}, j + 1);
      step(IC<2>{}, j + 2);
      step(IC<3>{}, j + 3);
    }
    if (j < nsteps) step(IC<0>{}, j);
    if (j + 1 < nsteps) step(IC<1>{}, j + 1);
    if (j + 2 < nsteps) step(IC<2>{}, j + 2);
    wait_vmem();  // no requests stay in flight
  }

  // ---- dQ = s (dQ^T)^T [, dQd = s (dQd^T)^T]: lane holds query col, d = 32 db + 8 jj + 4 half + 0..3
  if (query < p.Lq) {
    char* dqp = (char*)p.dq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)query * p.dq_sl) * 2;
    char* dtqp = NT == 2 ? (char*)p.dtq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)query * p.dq_sl) * 2 : nullptr;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int dc = d * 32 + 8 * jj + 4 * half;
        u32x2_t w = {Elem<T>::pack2(acc[d][4 * jj] * p.scale, acc[d][4 * jj + 1] * p.scale),
                     Elem<T>::pack2(acc[d][4 * jj + 2] * p.scale, acc[d][4 * jj + 3] * p.scale)};
        *(u32x2_t*)(dqp + dc * 2) = w;
        if constexpr (NT == 2) {
          if (p.dtq != nullptr) {
            u32x2_t wt = {Elem<T>::pack2(tacc[d][4 * jj] * p.scale, tacc[d][4 * jj + 1] * p.scale),
                          Elem<T>::pack2(tacc[d][4 * jj + 2] * p.scale, tacc[d][4 * jj + 3] * p.scale)};
            *(u32x2_t*)(dtqp + dc * 2) = wt;
          }
        }
      }
    }
  }
}

}  // namespace dmad
