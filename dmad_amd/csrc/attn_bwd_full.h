// Full-derivative backward (the cotangent of Od included) for 128-wide heads,
// reading Q, Qd, dO, dOd, K, Kd, V, Vd row-major in place: their transposes
// are formed on the LDS read with ds_read_b64_tr_b16, so no transposed copies
// are made in HBM.
//
// With s the softmax scale, Sd = s(Qd K^T + Q Kd^T), mu = rowsum(P*Sd),
// rho = rowsum(dOd*O) and D' = rowsum(dO*O) + rowsum(dOd*Od) - mu*rho (the
// statistics bwd_prep writes in its B layout):
//   dPd = dOd V^T,   dP = dO V^T + dOd Vd^T + dPd*(Sd - mu) - Sd*rho
//   Pd = P*(Sd - mu),  dS = P*(dP - D'),  dSd = P*(dPd - rho)
//   dK = s(dS^T Q + dSd^T Qd),  dV = P^T dO + Pd^T dOd         (key pass)
//   dQ = s(dS K + dSd Kd),  dQd = s dSd K                       (query pass)
// and dKd = s dSd^T Q, dVd = P^T dOd come from the dO-only key pass run with
// (dO, D) := (dOd, rho). Per (query, key) pair the two passes here run six
// score GEMMs each (S, the two halves of Sd, dPd, the two halves of dP) and
// four (key pass) or three (query pass) update GEMMs.
//
// Both passes keep their stationary rows (K, Kd, V, Vd or Q, Qd, dO, dOd: the
// B operands of the score MFMAs) and their accumulators in AGPRs (256 of them),
// so the VGPRs hold two sets of score tiles: a step's MFMAs compute the score
// tiles of the next tile while the VALU turns the current tile's scores into
// the bf16/fp16 operands P, Pd, dS, dSd of its update MFMAs.
#pragma once
#include "attn_bwd.h"
#include "attn_bwd_dq.h"

namespace dmad {

// ---------------------------------------------------------------- key pass: dK, dV
// One workgroup = 4 waves x 32 keys; 32-query steps through a four-stage ring
// of Q, dO, Qd, dOd row tiles and the tile's statistics, requested three steps
// ahead. Step j:
//   phase A  score MFMAs of tile j+1 (S, Sd; dPd, dP) with tile j's P, Pd, dS,
//            dSd on the VALU between them (four values per 4 operand slots)
//   phase B  dV^T += dO^T P + dOd^T Pd, dK^T += Q^T dS + Qd^T dSd of tile j,
//            with the requests for tile j+3 spread between the MFMAs
// Keys at or beyond Lk read K = Kd = V = Vd = 0 and are never stored; padded
// queries carry lse2 = +inf (P = 0).
template <int D>
struct KvFullCfg {
  static constexpr int NW = 4;
  static constexpr int BK = 32 * NW;   // keys per workgroup
  static constexpr int BMQ = 32;       // queries per step
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BMQ * ROWB;
  static constexpr int OFF_Q = 0, OFF_DO = ROW_BYTES, OFF_TQ = 2 * ROW_BYTES, OFF_DTO = 3 * ROW_BYTES;
  static constexpr int OFF_ST = 4 * ROW_BYTES;
  static constexpr int STAT_BYTES = 4 * BMQ * 4;  // lse2, D', mu, rho
  static constexpr int STAGE = (OFF_ST + STAT_BYTES + 1023) / 1024 * 1024;
  static constexpr int NSTAGE = 4;
  static constexpr int NRI = BMQ * CR / 64;  // 1 KiB requests per row tile
  static constexpr int RPW = NRI / NW;
  static constexpr int ST_LANES = STAT_BYTES / 16 / NW;
  static constexpr int LOADS = 4 * RPW + 1;  // requests per wave per step
  static constexpr bool FITS = D == 128 && NRI % NW == 0 && NSTAGE * STAGE <= 160 * 1024;
};

// Elementwise step of the full derivative for one value: S, Sd (unscaled
// score sums), dPd, dPb = dO V^T + dOd Vd^T, and the row's statistics; returns
// P, Pd, dS, dSd.
struct FullVals {
  float p, pd, ds, dsd;
};
__device__ __forceinline__ FullVals full_values(float s, float sd_raw, float dpd, float dpb, float lse2, float dprime,
                                                float mu, float rho, float scale, float scale_log2) {
  FullVals r;
  r.p = fast_exp2(fmaf(s, scale_log2, -lse2));
  const float sd = sd_raw * scale;
  const float c = sd - mu;
  const float dp = fmaf(dpd, c, dpb) - sd * rho;
  r.pd = r.p * c;
  r.ds = r.p * (dp - dprime);
  r.dsd = r.p * (dpd - rho);
  return r;
}

// STORE: also writes each tile's dS and dSd (the operands of the dK updates,
// keys at or beyond Lk as zeros) to p.sc in the ScLayout (tensor 0 = dS,
// 1 = dSd) for attn_bwd_dq_sc_kernel: tile j's four chunks leave in phase B of
// step j, one every eight update MFMAs, between the ring requests. The next
// barrier's vmcnt(LOADS) stays exact whatever order stores and loads complete
// in: a request of tile j + 2 still in flight means all LOADS requests of tile
// j + 3 are too.
template <typename T, int D, bool STORE = false>
__global__ __launch_bounds__(256, 1) void attn_bwd_kv_full_kernel(BwdParams p) {
  using C = KvFullCfg<D>;
  constexpr int BMQ = C::BMQ, KS = C::KS, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  static_assert(C::FITS, "configuration does not fit");
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  const int nkt = (p.Lk + C::BK - 1) / C::BK;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int slice = work / nkt, kt = work - slice * nkt;
  const int bh = (STORE ? p.bh0 : 0) + slice;
  const int b = bh / p.H, h = bh - b * p.H;
  const int nqt = p.LQP / BMQ;
  const int key = kt * C::BK + wave * 32 + col;

  // ---- score-gradient stores (STORE): this wave's key block of the slice's strips
  const int64_t sc_strip = ScLayout::strip_stride(4 * nkt, 2);  // one query block, both tensors
  char* const sc_base = STORE ? (char*)p.sc + (int64_t)slice * p.sc_slice : nullptr;
  const uint32_t sc_kb = (uint32_t)(kt * 4 + wave) * 2 * ScLayout::PIECE;
  const uint32_t sc_lo0 = ScLayout::lane_off(col, half, 0), sc_lo1 = ScLayout::lane_off(col, half, 1);
  const bool sc_tail = (kt + 1) * C::BK > p.Lk;  // keys at or beyond Lk in this workgroup
  // chunk u of tensor t (0: dS, 1: dSd) of tile qt
  auto store_chunk = [&](int qt, int t, int u, i32x4_t v) {
    if (sc_tail && key >= p.Lk) v = i32x4_t{0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(sc_base + (int64_t)(qt >> 2) * sc_strip, (uint32_t)(sc_strip - ScLayout::STRIP_PAD));
    buf_store16_stream(rs, v, u ? sc_lo1 : sc_lo0,
                       sc_kb + (uint32_t)(qt & 3) * ScLayout::TILE + (uint32_t)t * ScLayout::PIECE +
                           (uint32_t)u * ScLayout::CHUNK);
  };

  // ---- stationary K, Kd, V, Vd rows (B operands of the score MFMAs), kept in AGPRs
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const int64_t khead = b * p.k_sb + h * p.k_sh, vhead = b * p.v_sb + h * p.v_sh;
  i32x4_t kreg[KS], tkreg[KS], vreg[KS], tvreg[KS];
  {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + khead * 2, k_bytes);
    const __amdgpu_buffer_rsrc_t rtk = make_rsrc((const char*)p.tk + khead * 2, k_bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + vhead * 2, v_bytes);
    const __amdgpu_buffer_rsrc_t rtv = make_rsrc((const char*)p.tv + vhead * 2, v_bytes);
    const uint32_t ko = (uint32_t)((int64_t)key * p.k_sl * 2) + half * 16;
    const uint32_t vo = (uint32_t)((int64_t)key * p.v_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kreg[s] = buf_load16(rk, ko + s * 32);
      tkreg[s] = buf_load16(rtk, ko + s * 32);
      vreg[s] = buf_load16(rv, vo + s * 32);
      tvreg[s] = buf_load16(rtv, vo + s * 32);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+a"(kreg[s]), "+a"(tkreg[s]), "+a"(vreg[s]), "+a"(tvreg[s]));
  }

  // ---- query-side resources and per-lane request offsets
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const uint32_t st_bytes = (uint32_t)((int64_t)p.LQP * 4 * 4);
  const int64_t qhead = b * p.q_sb + h * p.q_sh, dohead = b * p.do_sb + h * p.do_sh;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + qhead * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rtq = make_rsrc((const char*)p.tq + qhead * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + dohead * 2, do_bytes);
  const __amdgpu_buffer_rsrc_t rdto = make_rsrc((const char*)p.dto + dohead * 2, do_bytes);
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
  // request li (0 <= li < LOADS) of query tile qt into stage st: row pieces of
  // Q, dO, Qd, dOd, then the statistics; tiles at or beyond the end read zeros
  auto issue_load = [&](lds_char_t* st, int qt, int li) {
    if (li < 4 * RPW) {
      const int t = li % 4, jj = li / 4, i = wave + jj * C::NW;
      const uint32_t qs = (uint32_t)qt * q_step, ds = (uint32_t)qt * do_step;
      if (t == 0) buf_load16_lds(rq, st + C::OFF_Q + i * 1024, roff_q[jj], qs);
      else if (t == 1) buf_load16_lds(rdo, st + C::OFF_DO + i * 1024, roff_do[jj], ds);
      else if (t == 2) buf_load16_lds(rtq, st + C::OFF_TQ + i * 1024, roff_q[jj], qs);
      else buf_load16_lds(rdto, st + C::OFF_DTO + i * 1024, roff_do[jj], ds);
    } else {
      if (st_lane) buf_load16_lds(rst, st + C::OFF_ST, lane * 16, (uint32_t)qt * C::STAT_BYTES);
    }
  };

  // ---- LDS read offsets: rows (query perm32(col), chunk 2s + half) and
  // transposed blocks (lane group g: d0 = 32 db + 16 (g & 1), queries 16 u + 8 (g >> 1) + 0..7)
  int sx[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int r = perm32(col);
    sx[s] = r * ROWB + (((2 * s + half) ^ trswz<CR>(r & 15)) << 4);
  }
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
#pragma unroll
  for (int d = 0; d < DB; ++d) asm volatile("" : "+a"(dkacc[d]), "+a"(dvacc[d]));

  // score tiles of one query tile: S, Sd (unscaled), dPd, dPb
  struct Scores {
    f32x16_t s, sd, dpd, dpb;
  };
  constexpr int PF = 4;
  constexpr int NOPA = 4 * KS;       // Q, dO, dOd, Qd rows per k slice
  constexpr int NOPB = 2 * 4 * DB;   // (chunk, operand, d block): dO^T, dOd^T, Q^T, Qd^T
  constexpr int NOP = NOPA + NOPB;
  const f32x16_t zero16 = {};
  auto load_op = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int o) -> i32x4_t {
    if (o < NOPA) {
      const int s = o >> 2, w = o & 3;
      const int off = w == 0 ? C::OFF_Q : w == 1 ? C::OFF_DO : w == 2 ? C::OFF_DTO : C::OFF_TQ;
      return *(lds_i32x4_t*)(s_next + off + sx[s]);
    }
    const int j = o - NOPA, u = j / (4 * DB), w = (j / DB) % 4, db = j % DB;
    const int off = w == 0 ? C::OFF_DO : w == 1 ? C::OFF_DTO : w == 2 ? C::OFF_Q : C::OFF_TQ;
    const lds_char_t* base = s_cur + off + u * 16 * ROWB;
    const u32x2_t lo = lds_read_tr16(base + tx[db][0]);
    const u32x2_t hi = lds_read_tr16(base + tx[db][1]);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };
  // packs of the current tile: P, Pd, dS, dSd for 16-query chunks u = 0, 1
  struct Packs {
    i32x4_t p[2], pd[2], ds[2], dsd[2];
  };
  auto mfma_op = [&](int o, i32x4_t a, Scores& n, const Packs& pk) {
    if (o < NOPA) {
      const int s = o >> 2, w = o & 3;
      if (w == 0) {
        n.s = mfma32(a, kreg[s], s == 0 ? zero16 : n.s, T());
        n.sd = mfma32(a, tkreg[s], s == 0 ? zero16 : n.sd, T());
      } else if (w == 1) {
        n.dpb = mfma32(a, vreg[s], s == 0 ? zero16 : n.dpb, T());
      } else if (w == 2) {
        n.dpd = mfma32(a, vreg[s], s == 0 ? zero16 : n.dpd, T());
        n.dpb = mfma32(a, tvreg[s], n.dpb, T());
      } else {
        n.sd = mfma32(a, kreg[s], n.sd, T());
      }
    } else {
      const int j = o - NOPA, u = j / (4 * DB), w = (j / DB) % 4, db = j % DB;
      if (w == 0) mfma32_acc(dvacc[db], a, pk.p[u], T());
      else if (w == 1) mfma32_acc(dvacc[db], a, pk.pd[u], T());
      else if (w == 2) mfma32_acc(dkacc[db], a, pk.ds[u], T());
      else mfma32_acc(dkacc[db], a, pk.dsd[u], T());
    }
  };
  // statistics of the 4 queries of value group g (values 4g .. 4g+3: queries
  // 16 (g >> 1) + 8 half + 4 (g & 1) + 0..3)
  struct Stat4 {
    f32x4_t lse2, dpr, mu, rho;
  };
  auto load_stats = [&](const lds_char_t* st, int g, Stat4& sv) {
    const lds_char_t* sst = st + C::OFF_ST;
    const int q0 = 16 * (g >> 1) + 8 * half + 4 * (g & 1);
    sv.lse2 = *(lds_f32x4_t*)(sst + 4 * q0);
    sv.dpr = *(lds_f32x4_t*)(sst + 4 * (BMQ + q0));
    sv.mu = *(lds_f32x4_t*)(sst + 4 * (2 * BMQ + q0));
    sv.rho = *(lds_f32x4_t*)(sst + 4 * (3 * BMQ + q0));
  };
  // values 2i, 2i + 1 of tile scores sc -> component i & 3 of chunk i >> 2 of the packs
  auto pair = [&](int i, const Scores& sc, const Stat4& sv, Packs& pk) {
    FullVals r[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int v = 2 * i + w, e = v & 3;
      r[w] = full_values(sc.s[v], sc.sd[v], sc.dpd[v], sc.dpb[v], sv.lse2[e], sv.dpr[e], sv.mu[e], sv.rho[e], p.scale,
                         p.scale_log2);
    }
    const int u = i >> 2, c = i & 3;
    pk.p[u][c] = (int)Elem<T>::pack2(r[0].p, r[1].p);
    pk.pd[u][c] = (int)Elem<T>::pack2(r[0].pd, r[1].pd);
    pk.ds[u][c] = (int)Elem<T>::pack2(r[0].ds, r[1].ds);
    pk.dsd[u][c] = (int)Elem<T>::pack2(r[0].dsd, r[1].dsd);
  };

  // step j (j + 1 < nqt, j % 4 == kk): phase A on tile j+1 with tile j's
  // values, phase B on tile j; requests tile j+3
  auto step = [&](auto kk, int j, const Scores& sc, Scores& sn) {
    constexpr int k = decltype(kk)::value;
    ring_sync<C::LOADS>();  // tile j+1 has landed (tile j+2 may be in flight)
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    i32x4_t opr[PF];
#pragma unroll
    for (int o = 0; o < PF; ++o) opr[o] = load_op(s_next, s_cur, o);
    Packs pk;
    Stat4 sv;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 0; o < NOPA; ++o) {
      mfma_op(o, opr[o % PF], sn, pk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
      // value pair i in operand slot 4i + 1 (its group's statistics one slot earlier)
      if ((o & 3) == 0 && ((o >> 2) & 1) == 0) load_stats(s_cur, o >> 3, sv);
      if ((o & 3) == 1) pair(o >> 2, sc, sv, pk);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" : "+v"(pk.p[0]), "+v"(pk.p[1]), "+v"(pk.pd[0]), "+v"(pk.pd[1]));
    asm volatile("" : "+v"(pk.ds[0]), "+v"(pk.ds[1]), "+v"(pk.dsd[0]), "+v"(pk.dsd[1]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) {
      mfma_op(o, opr[o % PF], sn, pk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) {
        if (NOPA + li * NOPB / C::LOADS == o) issue_load(s_req, j + 3, li);
      }
      if constexpr (STORE) {
        // phase-B slots 4, 12, 20, 28: dS chunks 0, 1, then dSd chunks 0, 1
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (o == NOPA + 4 + 8 * c) store_chunk(j, c >> 1, c & 1, (c >> 1) ? pk.dsd[c & 1] : pk.ds[c & 1]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(NOPA == 32 && 4 * 7 + 1 < NOPA, "eight value pairs ride in the 32 phase-A slots");
  // last tile: its values, then its update MFMAs
  auto last_step = [&](auto kk, const Scores& sc) {
    const lds_char_t* s_cur = stage(kk);
    Packs pk;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      Stat4 sv;
      load_stats(s_cur, g, sv);
      pair(2 * g, sc, sv, pk);
      pair(2 * g + 1, sc, sv, pk);
    }
    asm volatile("" : "+v"(pk.p[0]), "+v"(pk.p[1]), "+v"(pk.pd[0]), "+v"(pk.pd[1]));
    asm volatile("" : "+v"(pk.ds[0]), "+v"(pk.ds[1]), "+v"(pk.dsd[0]), "+v"(pk.dsd[1]));
    if constexpr (STORE) {
#pragma unroll
      for (int c = 0; c < 4; ++c) store_chunk(nqt - 1, c >> 1, c & 1, (c >> 1) ? pk.dsd[c & 1] : pk.ds[c & 1]);
    }
    Scores un;
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) mfma_op(o, load_op(s_cur, s_cur, o), un, pk);
  };

  if (nqt > 0) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    ring_sync<2 * C::LOADS>();  // K, Kd, V, Vd rows and tile 0
    Scores sa, sb;
    {
      const lds_char_t* s0 = stage(IC<0>{});
      Packs none;
#pragma unroll
      for (int o = 0; o < NOPA; ++o) mfma_op(o, load_op(s0, s0, o), sa, none);
    }
    int j = 0;
    for (; j + 4 < nqt; j += 4) {
      step(IC<0>{}, j, sa, sb);
      step(IC<1>{}, j + 1, sb, sa);
      step(IC<2>{}, j + 2, sa, sb);
      step(IC<3>{}, j + 3, sb, sa);
    }
    const int rest = nqt - j;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, j, sa, sb);
    if (rest >= 3) step(IC<1>{}, j + 1, sb, sa);
    if (rest >= 4) step(IC<2>{}, j + 2, sa, sb);
    if (rest == 1) last_step(IC<0>{}, sa);
    else if (rest == 2) last_step(IC<1>{}, sb);
    else if (rest == 3) last_step(IC<2>{}, sa);
    else last_step(IC<3>{}, sb);
    wait_vmem();  // no requests beyond the last tile stay in flight
  }
  mfma_acc_drain();  // the last dK, dV MFMAs have finished before their AGPRs are read

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

// ---------------------------------------------------------------- query pass: dQ (and dQd)
// One workgroup = 4 waves x 32 queries (lane <-> query, so the statistics are
// per-lane scalars); 32-key steps through a four-stage ring of K, Kd, V, Vd row
// tiles. Step j:
//   phase A  S^T = K Q^T, Sd^T = K Qd^T + Kd Q^T, dPd^T = V dOd^T,
//            dPb^T = V dO^T + Vd dOd^T of tile j+1, with tile j's dS, dSd on
//            the VALU between them
//   phase B  dQ^T += K^T dS^T + Kd^T dSd^T (and dQd^T += K^T dSd^T) of tile j
// Keys at or beyond Lk read K = Kd = V = Vd = 0: their (finite) dS, dSd meet
// zero K^T, Kd^T columns, so no key mask is needed.
template <int D>
struct DqFullCfg {
  static constexpr int NW = 4;
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 32;
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CR = D / 8;
  static constexpr int ROWB = D * 2;
  static constexpr int ROW_BYTES = BN * ROWB;
  static constexpr int OFF_K = 0, OFF_V = ROW_BYTES, OFF_TK = 2 * ROW_BYTES, OFF_TV = 3 * ROW_BYTES;
  static constexpr int STAGE = 4 * ROW_BYTES;
  static constexpr int NSTAGE = 4;
  static constexpr int NRI = BN * CR / 64;
  static constexpr int RPW = NRI / NW;
  static constexpr bool FITS = D == 128 && NRI % NW == 0 && NSTAGE * STAGE <= 160 * 1024;
  static constexpr int LOADS = 4 * RPW;
};

// TG: also the tangent gradient dQd = s dSd K.
template <typename T, int D, bool TG>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_full_kernel(DqParams p) {
  using C = DqFullCfg<D>;
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

  // ---- this lane's query: Q, Qd, dO, dOd rows (B operands, AGPRs) and statistics
  const int query = qt * C::BM + wave * 32 + col;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const uint32_t do_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.do_sl + D) * 2);
  const int64_t qhead = b * p.q_sb + h * p.q_sh, dohead = b * p.do_sb + h * p.do_sh;
  i32x4_t qreg[KS], tqreg[KS], doreg[KS], dtoreg[KS];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + qhead * 2, q_bytes);
    const __amdgpu_buffer_rsrc_t rtq = make_rsrc((const char*)p.tq + qhead * 2, q_bytes);
    const __amdgpu_buffer_rsrc_t rdo = make_rsrc((const char*)p.dout + dohead * 2, do_bytes);
    const __amdgpu_buffer_rsrc_t rdto = make_rsrc((const char*)p.dto + dohead * 2, do_bytes);
    const uint32_t qo = (uint32_t)((int64_t)query * p.q_sl * 2) + half * 16;
    const uint32_t oo = (uint32_t)((int64_t)query * p.do_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qreg[s] = buf_load16(rq, qo + s * 32);
      tqreg[s] = buf_load16(rtq, qo + s * 32);
      doreg[s] = buf_load16(rdo, oo + s * 32);
      dtoreg[s] = buf_load16(rdto, oo + s * 32);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+a"(qreg[s]), "+a"(tqreg[s]), "+a"(doreg[s]), "+a"(dtoreg[s]));
  }
  // statistics in the B layout [BH][LQP/32][4][32]: lse2, D', mu, rho
  float lse2 = __builtin_inff(), dpr = 0.f, mu = 0.f, rho = 0.f;
  if (query < p.LQP) {
    const float* st = p.stats + ((int64_t)bh * (p.LQP / 32) + query / 32) * 4 * 32 + query % 32;
    lse2 = st[0];
    dpr = st[32];
    mu = st[64];
    rho = st[96];
  }

  // ---- key-side resources and per-lane request offsets
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + D) * 2);
  const int64_t khead = b * p.k_sb + h * p.k_sh, vhead = b * p.v_sb + h * p.v_sh;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + khead * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rtk = make_rsrc((const char*)p.tk + khead * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + vhead * 2, v_bytes);
  const __amdgpu_buffer_rsrc_t rtv = make_rsrc((const char*)p.tv + vhead * 2, v_bytes);
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
  auto issue_load = [&](lds_char_t* st, int kt, int li) {
    const int t = li % 4, jj = li / 4, i = wave + jj * C::NW;
    const uint32_t ks = (uint32_t)kt * k_step, vs = (uint32_t)kt * v_step;
    if (t == 0) buf_load16_lds(rk, st + C::OFF_K + i * 1024, roff_k[jj], ks);
    else if (t == 1) buf_load16_lds(rv, st + C::OFF_V + i * 1024, roff_v[jj], vs);
    else if (t == 2) buf_load16_lds(rtk, st + C::OFF_TK + i * 1024, roff_k[jj], ks);
    else buf_load16_lds(rtv, st + C::OFF_TV + i * 1024, roff_v[jj], vs);
  };

  int sx[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int r = perm32(col);
    sx[s] = r * ROWB + (((2 * s + half) ^ trswz<CR>(r & 15)) << 4);
  }
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
  auto pin_offsets = [&]() {
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+v"(sx[s]));
#pragma unroll
    for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(tx[db][0]), "+v"(tx[db][1]));
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
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    asm volatile("" : "+a"(acc[d]));
    if constexpr (TG) asm volatile("" : "+a"(tacc[d]));
  }

  struct Scores {
    f32x16_t s, sd, dpd, dpb;
  };
  struct Packs {
    i32x4_t ds[2], dsd[2];
  };
  constexpr int PF = 4;
  constexpr int NOPA = 4 * KS;      // K, V, Vd, Kd rows per k slice
  constexpr int NOPB = 2 * 2 * DB;  // (chunk, operand, d block): K^T, Kd^T
  constexpr int NOP = NOPA + NOPB;
  const f32x16_t zero16 = {};
  auto load_op = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int o) -> i32x4_t {
    if (o < NOPA) {
      const int s = o >> 2, w = o & 3;
      const int off = w == 0 ? C::OFF_K : w == 1 ? C::OFF_V : w == 2 ? C::OFF_TV : C::OFF_TK;
      return *(lds_i32x4_t*)(s_next + off + sx[s]);
    }
    const int j = o - NOPA, t = j / (2 * DB), w = (j / DB) % 2, db = j % DB;
    const lds_char_t* base = s_cur + (w == 0 ? C::OFF_K : C::OFF_TK) + t * 16 * ROWB;
    const u32x2_t lo = lds_read_tr16(base + tx[db][0]);
    const u32x2_t hi = lds_read_tr16(base + tx[db][1]);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };
  auto mfma_op = [&](int o, i32x4_t a, Scores& n, const Packs& pk) {
    if (o < NOPA) {
      const int s = o >> 2, w = o & 3;
      if (w == 0) {
        n.s = mfma32(a, qreg[s], s == 0 ? zero16 : n.s, T());
        n.sd = mfma32(a, tqreg[s], s == 0 ? zero16 : n.sd, T());
      } else if (w == 1) {
        n.dpb = mfma32(a, doreg[s], s == 0 ? zero16 : n.dpb, T());
        n.dpd = mfma32(a, dtoreg[s], s == 0 ? zero16 : n.dpd, T());
      } else if (w == 2) {
        n.dpb = mfma32(a, dtoreg[s], n.dpb, T());
      } else {
        n.sd = mfma32(a, qreg[s], n.sd, T());
      }
    } else {
      const int j = o - NOPA, t = j / (2 * DB), w = (j / DB) % 2, db = j % DB;
      if (w == 0) {
        mfma32_acc(acc[db], a, pk.ds[t], T());
        if constexpr (TG) mfma32_acc(tacc[db], a, pk.dsd[t], T());
      } else {
        mfma32_acc(acc[db], a, pk.dsd[t], T());
      }
    }
  };
  // values 2i, 2i + 1 (keys 16 (i >> 2) + 8 half + 2 (i & 3) + 0, 1) -> component i & 3 of chunk i >> 2
  auto pair = [&](int i, const Scores& sc, Packs& pk) {
    FullVals r[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int v = 2 * i + w;
      r[w] = full_values(sc.s[v], sc.sd[v], sc.dpd[v], sc.dpb[v], lse2, dpr, mu, rho, p.scale, p.scale_log2);
    }
    const int t = i >> 2, c = i & 3;
    pk.ds[t][c] = (int)Elem<T>::pack2(r[0].ds, r[1].ds);
    pk.dsd[t][c] = (int)Elem<T>::pack2(r[0].dsd, r[1].dsd);
  };

  auto step = [&](auto kk, int j, const Scores& sc, Scores& sn) {
    constexpr int k = decltype(kk)::value;
    ring_sync<C::LOADS>();  // tile j+1 has landed (tile j+2 may be in flight)
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    i32x4_t opr[PF];
#pragma unroll
    for (int o = 0; o < PF; ++o) opr[o] = load_op(s_next, s_cur, o);
    Packs pk;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 0; o < NOPA; ++o) {
      mfma_op(o, opr[o % PF], sn, pk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
      if ((o & 3) == 1) pair(o >> 2, sc, pk);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" : "+v"(pk.ds[0]), "+v"(pk.ds[1]), "+v"(pk.dsd[0]), "+v"(pk.dsd[1]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) {
      mfma_op(o, opr[o % PF], sn, pk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) {
        if (NOPA + li * NOPB / C::LOADS == o) issue_load(s_req, j + 3, li);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto last_step = [&](auto kk, const Scores& sc) {
    const lds_char_t* s_cur = stage(kk);
    Packs pk;
#pragma unroll
    for (int i = 0; i < 8; ++i) pair(i, sc, pk);
    asm volatile("" : "+v"(pk.ds[0]), "+v"(pk.ds[1]), "+v"(pk.dsd[0]), "+v"(pk.dsd[1]));
    Scores un;
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) mfma_op(o, load_op(s_cur, s_cur, o), un, pk);
  };

  if (ntiles > 0) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    ring_sync<2 * C::LOADS>();  // Q, Qd, dO, dOd rows and tile 0
    Scores sa, sb;
    {
      const lds_char_t* s0 = stage(IC<0>{});
      Packs none;
#pragma unroll
      for (int o = 0; o < NOPA; ++o) mfma_op(o, load_op(s0, s0, o), sa, none);
    }
    int j = 0;
    for (; j + 4 < ntiles; j += 4) {
      step(IC<0>{}, j, sa, sb);
      step(IC<1>{}, j + 1, sb, sa);
      step(IC<2>{}, j + 2, sa, sb);
      step(IC<3>{}, j + 3, sb, sa);
    }
    const int rest = ntiles - j;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, j, sa, sb);
    if (rest >= 3) step(IC<1>{}, j + 1, sb, sa);
    if (rest >= 4) step(IC<2>{}, j + 2, sa, sb);
    if (rest == 1) last_step(IC<0>{}, sa);
    else if (rest == 2) last_step(IC<1>{}, sb);
    else if (rest == 3) last_step(IC<2>{}, sa);
    else last_step(IC<3>{}, sb);
    wait_vmem();  // no requests beyond the last tile stay in flight
  }
  mfma_acc_drain();

  // ---- dQ = s (dQ^T)^T [, dQd = s (dQd^T)^T]: lane holds query col, d = 32 db + 8 jj + 4 half + 0..3
  if (query < p.Lq) {
    char* dqp = (char*)p.dq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)query * p.dq_sl) * 2;
    char* dtqp = TG ? (char*)p.dtq + ((b * p.dq_sb + h * p.dq_sh) + (int64_t)query * p.dq_sl) * 2 : nullptr;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int dc = d * 32 + 8 * jj + 4 * half;
        u32x2_t w = {Elem<T>::pack2(acc[d][4 * jj] * p.scale, acc[d][4 * jj + 1] * p.scale),
                     Elem<T>::pack2(acc[d][4 * jj + 2] * p.scale, acc[d][4 * jj + 3] * p.scale)};
        *(u32x2_t*)(dqp + dc * 2) = w;
        if constexpr (TG) {
          u32x2_t wt = {Elem<T>::pack2(tacc[d][4 * jj] * p.scale, tacc[d][4 * jj + 1] * p.scale),
                        Elem<T>::pack2(tacc[d][4 * jj + 2] * p.scale, tacc[d][4 * jj + 3] * p.scale)};
          *(u32x2_t*)(dtqp + dc * 2) = wt;
        }
      }
    }
  }
}

}  // namespace dmad
