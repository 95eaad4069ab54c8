// Forward for the K, V tangent-free mode (Kd = Vd = 0: Wan's text
// cross-attention, Lq = 32760 queries over 512 text keys) of 128-wide heads,
// at two workgroups per CU.
//
// attn_fwd32_kernel keeps Q and Qd in registers, one wave per SIMD: the
// online softmax between a tile's score MFMAs and its P V MFMAs can then
// overlap the matrix unit only through the wave's own instruction order, and
// with 16 key steps per 128-query tile the tile's fixed work (Q reads, ring
// fill, O stores) is as long as its key loop. Here Qd stays
// in a wave-private LDS region and is read slice by slice as the B operand of
// Sd^T = K Qd^T, the score tiles are single (not double-buffered) and the key
// ring has three stages: 80 KiB of LDS and at most 256 registers per lane, so
// two workgroups share a CU and every SIMD runs two waves of different
// workgroups. While one wave runs its softmax, the other's MFMAs keep the
// matrix unit busy; one workgroup's Q reads and O stores overlap the other's
// key loop.
//
// Arithmetic: that of attn_fwd32_kernel<T, kFwdJvpQOnly> (the reference
// kernel `_attn_fwd`, train/wan/rcm/utils/flash_attention_jvp_triton.py:107-232,
// with K-dot = V-dot = 0): the same score slices in the same order, the same
// log2-domain online softmax with lazy rescale, P~ and H~ rounded to the
// input type before the P V products, fp32 accumulators and the :216-223
// epilogue. Its outputs are bitwise those of that kernel.
//
// Step i (one barrier):
//   request tile i+2 into the stage step i-1 read;
//   phase A  S^T, Sd^T of tile i (K slices from the ring, Q from registers,
//            Qd slices from the wave's region);
//   softmax of tile i's first 16-key chunk on the VALU (V^T operands of phase B
//            read meanwhile);
//   phase B  O~^T += V^T P~^T, C~^T += V^T H~^T, the second chunk's softmax
//            beside the first chunk's MFMAs.
#pragma once
#include "attn_fwd32.h"

namespace dmad {

struct Fwd32X2Cfg {
  static constexpr int D = 128;
  static constexpr int NW = 4;        // waves per workgroup (one per SIMD)
  static constexpr int BM = 32 * NW;  // query rows per workgroup
  static constexpr int BN = 32;       // keys per step
  static constexpr int KS = D / 16;   // 16-wide k slices of Q K^T
  static constexpr int DB = D / 32;   // 32-row blocks of O^T
  static constexpr int CR = D / 8;    // 16-byte chunks per row
  static constexpr int ROWB = D * 2;
  static constexpr int TILE = BN * ROWB;  // 32 key rows
  static constexpr int OFF_K = 0, OFF_V = TILE;
  static constexpr int STAGE = 2 * TILE;  // K, V
  static constexpr int NSTAGE = 3;
  static constexpr int QREGION = 32 * ROWB;        // a wave's 32 Qd rows
  static constexpr int QPT = QREGION / 1024;       // 1 KiB requests for them
  static constexpr int RPW = BN * CR / 64 / NW;    // 1 KiB requests per tile per wave
  static constexpr int LOADS = 2 * RPW;            // requests per wave per step
  static constexpr int LDS_BYTES = NSTAGE * STAGE + NW * QREGION;
  static_assert(BN * CR % (64 * NW) == 0, "tile requests split evenly over the waves");
  static_assert(LDS_BYTES <= 80 * 1024, "two workgroups per CU share its 160 KiB of LDS");
  static_assert(2 * RowStage<D>::BYTES <= QREGION + STAGE / 2, "a wave's O, Od rows fit its staging bytes");
};

// Shapes attn_fwd32_x2_kernel serves.
constexpr bool fwd32x2_supported(int mode, int dqk, int dv) { return mode == kFwdJvpQOnly && dqk == 128 && dv == 128; }

template <typename T>
__global__ __launch_bounds__(256, 2) void attn_fwd32_x2_kernel(FwdParams p) {
  using C = Fwd32X2Cfg;
  constexpr int D = C::D, BN = C::BN, KS = C::KS, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  constexpr float kSlack = RescaleSlack<T>::value;
  // bf16 forms H~ = P~ Sd without the softmax scale and applies it to C~ and r
  // in the epilogue, as attn_fwd32_kernel does in this mode (the same bits)
  constexpr bool kHScaled = !std::is_same<T, __bf16>::value;
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char qdr[C::NW][C::QREGION];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;
  lds_char_t* const my = (lds_char_t*)qdr[wave];

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;
  const int ntiles = (p.Lk + BN - 1) / BN;  // >= 1 (the launcher takes Lk >= 1)
  const int row0 = qt * C::BM + wave * 32;
  const int query = row0 + col;

  // ---- Q rows: B operands of S^T = K Q^T, in registers; this wave's 32 Qd
  // rows into its region (chunk c of row r at slot c ^ trswz(r)), rows >= Lq
  // read as zeros
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const int64_t qhead = b * p.q_sb + h * p.q_sh;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + qhead * 2, q_bytes);
  const __amdgpu_buffer_rsrc_t rtq = make_rsrc((const char*)p.tq + qhead * 2, q_bytes);
  i32x4_t qreg[KS];
  {
    const uint32_t qo = (uint32_t)((int64_t)query * p.q_sl * 2) + half * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s) qreg[s] = buf_load16(rq, qo + s * 32);
    const uint32_t base = (uint32_t)((int64_t)row0 * p.q_sl * 2);
#pragma unroll
    for (int j = 0; j < C::QPT; ++j) {
      const int pch = j * 64 + lane, row = pch / CR, phys = pch % CR;
      const uint32_t off = (uint32_t)((int64_t)row * p.q_sl * 2) + ((phys ^ trswz<CR>(row & 15)) << 4);
      buf_load16_lds(rtq, my + j * 1024, off, base);
    }
  }

  // ---- key-side resources and per-lane request offsets
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
    constexpr int k = decltype(kk)::value % 3;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else return (lds_char_t*)stg2;
  };
  // request li of key tile kt into stage st; tiles at or beyond the end read
  // zeros or in-range rows into a stage nobody reads again
  auto issue_load = [&](lds_char_t* st, int kt, int li) {
    const int jj = li >> 1, i = wave + jj * C::NW;
    if (li & 1) buf_load16_lds(rv, st + C::OFF_V + i * 1024, roff_v[jj], (uint32_t)kt * v_step);
    else buf_load16_lds(rk, st + C::OFF_K + i * 1024, roff_k[jj], (uint32_t)kt * k_step);
  };

  // ---- LDS read offsets. Slice s of a row-wise read is chunk 2s + half,
  // stored at slot (2s + half) ^ trswz(r) = 2s ^ (half ^ trswz(r)) (2s has no
  // low bit), i.e. at byte offset off0 ^ 32s; V^T block db sits at off0 ^ 64db.
  // Only the s = 0 / db = 0 offsets are kept and re-defined at each step (an
  // empty asm) so the compiler rebuilds the others with one XOR at their use
  // instead of holding 24 offsets in registers.
  int kx0, qx0, tx0[2];
  {
    const int r = perm32(col);
    kx0 = r * ROWB + ((half ^ trswz<CR>(r & 15)) << 4);
    qx0 = col * ROWB + ((half ^ trswz<CR>(col & 15)) << 4);
    const int g = lane >> 4, rr = (lane & 15) >> 2, c = lane & 3;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 8 * (g >> 1) + 4 * hh + rr;  // plus 16 t
      const int chunk = 2 * (g & 1) + (c >> 1);
      tx0[hh] = row * ROWB + ((chunk ^ trswz<CR>(row & 15)) << 4) + 8 * (c & 1);
    }
  }

  // everything in VGPRs (no AGPRs: 256 per lane at two waves per SIMD); the
  // accumulators take 128 of them. Step 0 starts them (its first 16-key
  // chunk's MFMAs take a zero C operand), so they need no clearing.
  f32x16_t oacc[DB], cacc[DB];
  const f32x16_t zero16 = {};
  float m_i = -__builtin_inff(), l_i = 0.f, r_i = 0.f;

  // Online softmax of one tile (log2 domain; lanes l and l^32 share a query):
  // value v of the score tile is key 16 (v >> 3) + 8 half + (v & 7); P~, H~ are
  // packed as the B operands of the two 16-key chunks. soft_head takes the row
  // max and the lazy-rescale decision (and rescales O~, C~ before any of the
  // tile's MFMAs), soft_pair finishes one pair of values (exps, running sums,
  // packs). The running sums are re-defined after each pair (an empty asm):
  // the compiler would otherwise sink them to the end of the step and keep all
  // 32 values live.
  float neg_m = 0.f;
  auto soft_head = [&](const f32x16_t& sc, auto first) -> float {
    float a = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    float b2 = fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]));
    float c2 = fmaxf(fmaxf(sc[8], sc[9]), fmaxf(sc[10], sc[11]));
    float d2 = fmaxf(fmaxf(sc[12], sc[13]), fmaxf(sc[14], sc[15]));
    float mx = fmaxf(fmaxf(a, b2), fmaxf(c2, d2));
    mx = fmaxf(mx, other_half(mx)) * p.scale_log2;
    const bool moved = __builtin_amdgcn_ballot_w64(mx > m_i + kSlack) != 0;
    const float m_new = moved ? fmaxf(m_i, mx) : m_i;
    const float alpha = fast_exp2(m_i - m_new);
    m_i = m_new;
    neg_m = -exp_base<T>(m_new);
    if (!decltype(first)::value && moved) {  // rare with the slack; nothing to rescale at step 0
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          oacc[d][v] *= alpha;
          cacc[d][v] *= alpha;
        }
      }
    }
    return alpha;
  };
  auto soft_pair = [&](int v, const f32x16_t& sc, const f32x16_t& tc, i32x4_t (&pk)[2], i32x4_t (&hk)[2], float& ls,
                       float& rs) {
    const float p0 = fast_exp2(fmaf(sc[v], p.scale_log2, neg_m));
    const float p1 = fast_exp2(fmaf(sc[v + 1], p.scale_log2, neg_m));
    ls += p0;
    const float h0 = kHScaled ? p0 * (tc[v] * p.scale) : p0 * tc[v];
    rs += h0;
    ls += p1;
    const float h1 = kHScaled ? p1 * (tc[v + 1] * p.scale) : p1 * tc[v + 1];
    rs += h1;
    pk[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(p0, p1);
    hk[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(h0, h1);
    asm volatile("" : "+v"(ls), "+v"(rs));
  };

  constexpr int PFA = 2;  // phase-A operand pairs (K slice, Qd slice) read ahead
  constexpr int NB = 2 * DB;
  constexpr int PFB = 4;  // phase-B operands read ahead (the first ones during the softmax)
  // step i: tile i sits in stage kk % 3 (first: step 0, which starts the accumulators)
  auto step = [&](auto kk, int i, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    ring_sync<C::LOADS>();  // tile i has landed (tile i+1 may be in flight); all waves are past step i-1
    asm volatile("" : "+v"(kx0), "+v"(qx0), "+v"(tx0[0]), "+v"(tx0[1]));
    const lds_char_t* s_cur = stage(kk);
    lds_char_t* s_req = stage(IC<decltype(kk)::value + 2>{});
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(s_req, i + 2, li);

    auto load_k = [&](int s) -> i32x4_t { return *(lds_i32x4_t*)(s_cur + C::OFF_K + (kx0 ^ (32 * s))); };
    auto load_qd = [&](int s) -> i32x4_t { return *(lds_i32x4_t*)(my + (qx0 ^ (32 * s))); };
    auto load_vt = [&](int j) -> i32x4_t {  // V^T block db = j % DB of 16-key chunk t = j / DB
      const int t = j / DB, db = j % DB;
      const lds_char_t* base = s_cur + C::OFF_V + t * 16 * ROWB;
      const u32x2_t lo = lds_read_tr16(base + (tx0[0] ^ (64 * db)));
      const u32x2_t hi = lds_read_tr16(base + (tx0[1] ^ (64 * db)));
      return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
    };

    // phase A: S^T, Sd^T of tile i
    f32x16_t sc, tc;
    i32x4_t ka[PFA], qa[PFA];
#pragma unroll
    for (int s = 0; s < PFA; ++s) {
      ka[s] = load_k(s);
      qa[s] = load_qd(s);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the MFMA phases run at wave priority 1 and the softmax at 0, so that on a
    // SIMD shared with another workgroup's wave the matrix unit goes to the wave
    // in its MFMA phase and the other's softmax fills the gaps (0.8% faster)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const i32x4_t a = ka[s % PFA], qd = qa[s % PFA];
      if (s + PFA < KS) {
        ka[s % PFA] = load_k(s + PFA);
        qa[s % PFA] = load_qd(s + PFA);
      }
      sc = mfma32(a, qreg[s], s == 0 ? zero16 : sc, T());
      tc = mfma32(a, qd, s == 0 ? zero16 : tc, T());
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    // the last tile may hold keys >= Lk
    if (i == ntiles - 1) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        if (i * BN + 16 * (v >> 3) + 8 * half + (v & 7) >= p.Lk) sc[v] = -__builtin_inff();
      }
    }
    i32x4_t vb[PFB];
#pragma unroll
    for (int j = 0; j < PFB; ++j) vb[j] = load_vt(j);
    // softmax of the first 16-key chunk (two pairs per scheduling group)
    i32x4_t pk[2], hk[2];
    float ls = 0.f, rs = 0.f;
    const float alpha = soft_head(sc, first);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int v = 0; v < 8; v += 2) {
      soft_pair(v, sc, tc, pk, hk, ls, rs);
      if (v & 2) __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(1);
    // phase B: O~^T += V^T P~^T, C~^T += V^T H~^T (per 16-key chunk t, block db);
    // the second chunk's values are computed beside the first chunk's MFMAs
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int t = j / DB, db = j % DB;
      const i32x4_t a = vb[j % PFB];
      if (j + PFB < NB) vb[j % PFB] = load_vt(j + PFB);
      oacc[db] = mfma32(a, pk[t], (FIRST && t == 0) ? zero16 : oacc[db], T());
      cacc[db] = mfma32(a, hk[t], (FIRST && t == 0) ? zero16 : cacc[db], T());
      if (j < DB) soft_pair(8 + 2 * j, sc, tc, pk, hk, ls, rs);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    l_i = l_i * alpha + ls;
    r_i = r_i * alpha + rs;
  };

  // ---- prologue: key tiles 0, 1 (behind the Q and Qd requests)
#pragma unroll
  for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
  for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
  step(IC<0>{}, 0, IC<1>{});  // ntiles >= 1
  int i = 1;
  for (; i + 3 <= ntiles; i += 3) {
    step(IC<1>{}, i, IC<0>{});
    step(IC<2>{}, i + 1, IC<0>{});
    step(IC<3>{}, i + 2, IC<0>{});
  }
  if (i < ntiles) step(IC<1>{}, i, IC<0>{});
  if (i + 1 < ntiles) step(IC<2>{}, i + 1, IC<0>{});
  wait_vmem();  // no request beyond the last tile stays in flight

  // ---- epilogue: lane (query col, half) holds d = 32 db + 8 jj + 4 half + (0..3)
  const float l = l_i + other_half(l_i);
  const float inv_l = 1.0f / l;
  const float inv_lh = kHScaled ? inv_l : inv_l * p.scale;  // 1 / l, with the scale H~ left out
  const float mu = (r_i + other_half(r_i)) * inv_lh;
  const int64_t obase = b * p.o_sb + h * p.o_sh;
  const uint32_t o_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.o_sl + D) * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc((char*)p.o + obase * 2, o_bytes);
  const __amdgpu_buffer_rsrc_t rto = make_rsrc((char*)p.to + obase * 2, o_bytes);
  // O and Od leave as whole rows through LDS once every wave has finished its
  // last step: O through the wave's Qd region, Od through half a ring stage
  ring_sync<0>();
  lds_char_t* const ostage = my;
  lds_char_t* const tstage = (wave < 2 ? stage(IC<0>{}) : stage(IC<1>{})) + (wave & 1) * RowStage<D>::BYTES;
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float ov[4], tv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = oacc[d][4 * jj + e] * inv_l;
        tv[e] = cacc[d][4 * jj + e] * inv_lh - mu * ov[e];
      }
      stage_put<D>(ostage, col, half, d, jj, u32x2_t{Elem<T>::pack2(ov[0], ov[1]), Elem<T>::pack2(ov[2], ov[3])});
      stage_put<D>(tstage, col, half, d, jj, u32x2_t{Elem<T>::pack2(tv[0], tv[1]), Elem<T>::pack2(tv[2], tv[3])});
    }
  }
  auto row_off = [&](int r) -> uint32_t {
    return row0 + r < p.Lq ? (uint32_t)((int64_t)(row0 + r) * p.o_sl * 2) : o_bytes;
  };
#pragma unroll
  for (int kk = 0; kk < RowStage<D>::NST; ++kk) {
    stage_store<D>(ostage, kk, lane, ro, row_off);
    stage_store<D>(tstage, kk, lane, rto, row_off);
  }
  if (half == 0 && query < p.Lq) {
    const int64_t si = (int64_t)bh * p.Lq + query;
    p.lse[si] = (exp_base<T>(m_i) + __builtin_log2f(l)) * 0.6931471805599453f;
    p.mu[si] = mu;
  }
}

}  // namespace dmad
