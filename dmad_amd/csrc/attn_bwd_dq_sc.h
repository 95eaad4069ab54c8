// Query pass over stored score gradients, 128-wide heads: dQ (and dQd) as a
// streaming GEMM over the dS (and dSd) tiles a STORE key pass wrote in the
// ScLayout (attn_bwd.h), instead of recomputing S and dP per (query, key) pair:
//   NT = 1 (dO-only gradients):    dQ = s dS K
//   NT = 2 (full derivative):      dQ = s (dS K + dSd Kd),  dQd = s dSd K
// Per (query, key) pair this reads the 2 NT bytes of stored gradients once from
// HBM and runs 2 (NT = 1) or 6 (NT = 2) units of MFMA work, where the
// recomputing passes run 6 or 18.
//
// One workgroup = 8 waves over two 128-query blocks (two waves per SIMD): wave
// w takes query tile w % 4 of block 2 qbp + w / 4. 32-key steps run through a
// ring of NSTAGE LDS stages; a stage holds the step's K [and Kd] rows
// (row-major, chunk-swizzled for transposed reads, as the other row-reading
// passes stage them), shared by both blocks, and each block's (query block,
// key block) piece of the stored gradients, copied as it lies. Per step and
// wave, for each 16-key slice: the B operands dS^T [dSd^T] (lane = query, 8
// consecutive keys) and the A operands K^T [Kd^T] (lane = d, 8 consecutive
// keys), all with ds_read_b64_tr_b16 and all read before the step's first
// MFMA, then
//   dQ^T += K^T dS^T [+ Kd^T dSd^T],   [dQd^T += K^T dSd^T].
// Keys at or beyond Lk read K = Kd = 0 and their stored gradients are zeros.
#pragma once
#include "attn_bwd.h"
#include "attn_bwd_dq.h"

namespace dmad {

template <int NT>
struct DqScCfg {
  static constexpr int D = 128;
  static constexpr int NW = 8;             // waves per workgroup
  static constexpr int NBLK = 2;           // 128-query blocks per workgroup
  static constexpr int BQ = ScLayout::BQ;  // queries per block
  static constexpr int BN = ScLayout::BK;  // keys per step
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BN * ROWB;  // K rows of one step
  static constexpr int OFF_K = 0, OFF_TK = ROW_BYTES;
  static constexpr int OFF_SC = NT * ROW_BYTES;            // block b's pieces at OFF_SC + b * SC_BYTES
  static constexpr int SC_BYTES = NT * ScLayout::PIECE;
  static constexpr int STAGE = NT * ROW_BYTES + NBLK * SC_BYTES;
  static constexpr int NSTAGE = NT == 1 ? 4 : 3;           // 96 KiB or 144 KiB of ring
  static constexpr int NRI = ROW_BYTES / 1024;             // wave-wide 1 KiB requests per row tile
  static constexpr int NSC = NBLK * SC_BYTES / 1024;       // ... for the stored pieces
  static constexpr int NREQ = NT * NRI + NSC;
  static constexpr int LOADS = NREQ / NW;                  // requests per wave per step
  static_assert(NREQ % NW == 0, "requests split evenly over the waves");
  static_assert(NSTAGE * STAGE <= 160 * 1024, "the ring fits the LDS");
  static_assert((NSTAGE - 1) * LOADS < 64, "vmcnt is a 6-bit field");
};

template <typename T, int NT>
__global__ __launch_bounds__(512, 1) void attn_bwd_dq_sc_kernel(DqParams p) {
  using C = DqScCfg<NT>;
  constexpr int D = C::D, BN = C::BN, DB = C::DB, CR = C::CR, ROWB = C::ROWB, NSTAGE = C::NSTAGE;
  // one array per stage, addressed with compile-time stage numbers, so the
  // compiler can tell the stage being filled from the one being read (with one
  // array it waits for every in-flight request before each LDS read)
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[NSTAGE > 3 ? C::STAGE : 16];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int blk = wave >> 2, tile = wave & 3;

  const int nqb = (p.Lq + C::BQ - 1) / C::BQ;
  const int npair = (nqb + 1) / 2;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int slice = work / npair, qbp = work - slice * npair;
  const int bh = p.bh0 + slice;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nsteps = (p.Lk + BN - 1) / BN;
  const int qb = 2 * qbp + blk;  // this wave's query block (qb == nqb: none; its reads repeat block nqb - 1)
  const int query = qb * C::BQ + tile * 32 + col;

  // ---- K [, Kd] rows and the two blocks' strips of stored gradients
  // ([key block][tensor][piece]; a missing second block reads the first again)
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const int64_t khead = b * p.k_sb + h * p.k_sh;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + khead * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rtk = make_rsrc((const char*)(NT == 2 ? p.tk : p.k) + khead * 2, k_bytes);
  const uint32_t k_step = (uint32_t)((int64_t)BN * p.k_sl * 2);
  const uint32_t strip = (uint32_t)p.sc_nkb * NT * ScLayout::PIECE;
  const int64_t stride = ScLayout::strip_stride(p.sc_nkb, NT);
  const char* sc_slice = (const char*)p.sc + (int64_t)slice * p.sc_slice;
  const int qb0 = 2 * qbp, qb1 = 2 * qbp + 1 < nqb ? 2 * qbp + 1 : nqb - 1;
  const __amdgpu_buffer_rsrc_t rsc0 = make_rsrc(sc_slice + (int64_t)qb0 * stride, strip);
  const __amdgpu_buffer_rsrc_t rsc1 = make_rsrc(sc_slice + (int64_t)qb1 * stride, strip);

  // request i (0 <= i < NREQ; wave w issues i = w, w + NW, ...) of step jj into
  // stage st: rows of K [and Kd] (1 KiB each), then the pieces of block 0 and
  // block 1 (steps past the end repeat the last one)
  auto issue_req = [&](lds_char_t* st, int jj, int i) {
    jj = jj < nsteps ? jj : nsteps - 1;
    if (i < NT * C::NRI) {
      const int t = i / C::NRI, r = i % C::NRI;
      const int pch = r * 64 + lane;
      const int row = pch / CR, phys = pch % CR;
      const uint32_t off = (uint32_t)((int64_t)row * p.k_sl * 2) + (uint32_t)((phys ^ trswz<CR>(row & 15)) * 16);
      buf_load16_lds(t ? rtk : rk, st + (t ? C::OFF_TK : C::OFF_K) + r * 1024, off, (uint32_t)jj * k_step);
    } else {
      const int s = i - NT * C::NRI, bb = s / (C::SC_BYTES / 1024), r = s % (C::SC_BYTES / 1024);
      buf_load16_lds(bb ? rsc1 : rsc0, st + C::OFF_SC + bb * C::SC_BYTES + r * 1024, (uint32_t)(r * 1024 + lane * 16),
                     (uint32_t)jj * NT * ScLayout::PIECE);
    }
  };
  auto issue_step = [&](lds_char_t* st, int jj) {
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) issue_req(st, jj, wave + l * C::NW);
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
      bx[hh] = C::OFF_SC + blk * C::SC_BYTES + tile * ScLayout::TILE + u * ScLayout::CHUNK + row * 32 + 8 * c;
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
    constexpr int k = decltype(kk)::value % NSTAGE;
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
      const lds_char_t* sb = st + ks * 16 * 32;
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
  // step j (j % NSTAGE == kk): once step j has landed, refill the stage step
  // j - 1 used (every wave is past its reads) with step j + NSTAGE - 1, then
  // compute step j
  auto step = [&](auto kk, int j) {
    constexpr int k = decltype(kk)::value;
    ring_sync<(NSTAGE - 2) * C::LOADS>();  // step j has landed; later ones may be in flight
    issue_step(stage(IC<k + NSTAGE - 1>{}), j + NSTAGE - 1);
    compute(stage(IC<k>{}));
  };
  if (nsteps > 0) {
    issue_step(stage(IC<0>{}), 0);
    issue_step(stage(IC<1>{}), 1);
    if constexpr (NSTAGE == 4) issue_step(stage(IC<2>{}), 2);
    int j = 0;
    for (; j + NSTAGE <= nsteps; j += NSTAGE) {
      step(IC<0>{}, j);
      step(IC<1>{}, j + 1);
      step(IC<2>{}, j + 2);
      if constexpr (NSTAGE == 4) step(IC<3>{}, j + 3);
    }
    if (j < nsteps) step(IC<0>{}, j);
    if (j + 1 < nsteps) step(IC<1>{}, j + 1);
    if constexpr (NSTAGE == 4) {
      if (j + 2 < nsteps) step(IC<2>{}, j + 2);
    }
    wait_vmem();  // no requests stay in flight
  }

  // ---- dQ = s (dQ^T)^T [, dQd = s (dQd^T)^T]: lane holds query col, d = 32 db + 8 jj + 4 half + 0..3
  if (qb < nqb && query < p.Lq) {
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
