// Forward(+JVP) kernel for 64-, 128- and (dense) 256-wide heads on 32x32x16 MFMAs.
//
// Same semantics as attn_fwd_kernel (the reference kernel `_attn_fwd`,
// train/wan/rcm/utils/flash_attention_jvp_triton.py:107-232): log2-domain
// online softmax, P~ and H~ rounded to the input type before the P V products,
// fp32 accumulators, the :216-223 epilogue, LSE and mu per query row.
//
// Work decomposition: one workgroup = 4 waves (one per SIMD) = 128 query rows
// of one head. Lane l of a wave owns query l%32; its Q (and Qd) row stays in
// registers as the B operand of S^T = K Q^T (and Sd^T = K Qd^T + Kd Q^T), so a
// 32x32 score tile gives each lane 16 keys of its own query and the row
// statistics are per-lane scalars (the other 16 keys sit in lane l^32).
// K, Kd, V, Vd stream as row-major 32-key tiles through a four-stage LDS ring
// filled by buffer->LDS requests three steps ahead (three stages, two steps
// ahead, where four stages do not fit: 256-wide heads with Kd, Vd). K rows are read in perm32
// order (A operand), so P~ and H~ leave the score tile already in the
// B-operand layout of O^T += V^T P^T; V^T is read from the row-major V tile
// with ds_read_b64_tr_b16, so V needs no transposed copy.
//
// Compared with 16-query waves, every K/V byte read from LDS feeds twice the
// MFMA work, which halves the LDS traffic per flop (the 16-query kernel is
// bound by LDS bandwidth at this head size).
//
// Step i (after one barrier) is a fixed stream of MFMAs:
//   phase A  S^T, Sd^T of tile i+1 (K, Kd of stage i+1), with the online
//            softmax of tile i on the VALU between them
//   (rescale of O~, C~ when some row's running max moved)
//   phase B  O~^T += V^T P~^T, C~^T += V^T H~^T + Vd^T P~^T of tile i, with
//            the requests for tile i+3 (i+2) spread between the MFMAs
// Every MFMA's LDS operand is read four operands ahead.
#pragma once
#include "attn_fwd.h"

namespace dmad {

// 256-wide heads in the JVP modes split V (and Vd, O, Od) into two 128-column
// chunks, one per workgroup (the O~ and C~ accumulators of 256 columns do not
// fit beside Q, Qd): each chunk's workgroup computes the full 256-wide scores
// (S, Sd twice over per query tile) and the 128 output columns of its chunk.
// K, Kd rows are then 512 bytes and V, Vd rows 256 bytes in the ring; with Kd,
// Vd a stage is 48 KiB, so the ring has three stages. The plain forward keeps
// all 256 columns in one workgroup (512-byte V rows, four stages).
template <int MODE, int DH = 128>
struct Fwd32Cfg {
  static constexpr int D = DH;  // Q, K width
  static constexpr int DVC = DH == 256 && MODE != kFwdPlain ? 128 : DH;  // V, O columns per workgroup
  static constexpr int CHUNKS = D / DVC;
  static constexpr int NW = 4;        // waves per workgroup
  static constexpr int BM = 32 * NW;  // query rows per workgroup
  static constexpr int BN = 32;       // keys per pipeline step
  static constexpr int KS = D / 16;   // 16-wide k slices of Q K^T
  static constexpr int DB = DVC / 32;  // 32-row blocks of O^T
  static constexpr int CR = D / 8;    // 16-byte chunks per K row
  static constexpr int CRV = DVC / 8;  // 16-byte chunks per V row (its chunk)
  static constexpr int ROWB = D * 2;
  static constexpr int ROWBV = DVC * 2;
  static constexpr int TILE = BN * ROWB;    // K (Kd) tile
  static constexpr int TILEV = BN * ROWBV;  // V (Vd) tile
  static constexpr bool JVP = MODE != kFwdPlain;
  static constexpr bool KVT = MODE == kFwdJvp;
  static constexpr int NTILE = KVT ? 4 : 2;  // row tiles per stage: K, V [, Kd, Vd]
  static constexpr int OFF_K = 0, OFF_V = TILE, OFF_KT = TILE + TILEV, OFF_VT = 2 * TILE + TILEV;
  static constexpr int STAGE = (KVT ? 2 : 1) * (TILE + TILEV);
  static constexpr int NSTAGE = 4 * STAGE <= 160 * 1024 ? 4 : 3;
  static constexpr int RPW = BN * CR / 64 / NW;    // 1 KiB requests per K tile per wave
  static constexpr int RPWV = BN * CRV / 64 / NW;  // 1 KiB requests per V tile per wave
  static constexpr int LOADS = (KVT ? 2 : 1) * (RPW + RPWV);  // requests per wave per step
  static constexpr int NOPA = KS * (KVT ? 2 : 1);     // LDS operands of phase A
  static constexpr int NOPB = 2 * DB * (KVT ? 2 : 1);  // LDS operands of phase B
  static_assert(BN * CRV % (64 * NW) == 0, "tile requests split evenly over the waves");
  static_assert(NSTAGE * STAGE <= 160 * 1024, "ring exceeds the LDS");
};

// Head shapes served by attn_fwd32_kernel (the others use attn_fwd_kernel and
// its variants, which read a transposed copy of V).
constexpr bool fwd32_supported(int dqk, int dv) { return (dqk == 128 && dv == 128) || (dqk == 64 && dv == 64); }
// 256-wide heads (Dqk = Dv = 256), dense and block-sparse launches.
constexpr bool fwd32_wide_supported(int dqk, int dv) { return dqk == 256 && dv == 256; }
// Workgroups per query tile (column chunks of V).
constexpr int fwd32_chunks(int mode, int d) { return d == 256 && mode != kFwdPlain ? 2 : 1; }
static_assert(fwd32_chunks(kFwdJvp, 256) == Fwd32Cfg<kFwdJvp, 256>::CHUNKS &&
                  fwd32_chunks(kFwdJvpQOnly, 256) == Fwd32Cfg<kFwdJvpQOnly, 256>::CHUNKS &&
                  fwd32_chunks(kFwdPlain, 256) == Fwd32Cfg<kFwdPlain, 256>::CHUNKS,
              "chunk counts of the launch plan");

// ---------------------------------------------------------------- row-staged stores
// One wave's 32 x D output tile, held in the MFMA C layout (lane: row `col`,
// columns 32 db + 8 jj + 4 half + 0..3), is written to a wave-private LDS
// region as row-major rows (16-byte chunk c of row r at slot c ^ trswz(r)) and
// read back as whole rows: each 16-byte-per-lane store instruction then writes
// 64 / (D/8) complete rows, so every 128-byte line of the output is written by
// one instruction (8-byte stores straight from the C layout reach each line
// from eight instructions, and HBM saw partly filled lines).
template <int D>
struct RowStage {
  static constexpr int CR = D / 8;         // 16-byte chunks per row
  static constexpr int ROWB = D * 2;       // bytes per row
  static constexpr int BYTES = 32 * ROWB;  // one 32-row tile
  static constexpr int RPI = 64 / CR;      // rows per store instruction
  static constexpr int NST = 32 / RPI;     // store instructions per tile
};

template <int D>
__device__ __forceinline__ void stage_put(lds_char_t* region, int col, int half, int db, int jj, u32x2_t v) {
  using R = RowStage<D>;
  typedef __attribute__((address_space(3))) u32x2_t lds_u32x2_t;
  const int chunk = 4 * db + jj;
  *(lds_u32x2_t*)(region + col * R::ROWB + ((chunk ^ trswz<R::CR>(col & 15)) << 4) + 8 * half) = v;
}

// Store instruction k of the tile in `region` (rows k RPI .. k RPI + RPI - 1).
// row_off(r) is the byte offset of tile row r in `rs`, or at least the range
// of `rs` for a row that must not be written (the store is then dropped).
template <int D, typename RowOff>
__device__ __forceinline__ void stage_store(const lds_char_t* region, int k, int lane, __amdgpu_buffer_rsrc_t rs,
                                            RowOff row_off) {
  using R = RowStage<D>;
  const int row = k * R::RPI + lane / R::CR, phys = lane % R::CR;
  const int logical = phys ^ trswz<R::CR>(row & 15);
  const i32x4_t v = *(lds_i32x4_t*)(region + row * R::ROWB + phys * 16);
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, (int)(row_off(row) + (uint32_t)logical * 16), 0, 0);
}

// MAGI: the block-sparse variant (the reference's `_attn_fwd_magi`,
// flash_attention_jvp_triton.py:242-409). The workgroup runs one (query group,
// 128-query tile) task (256-wide heads in the JVP modes: one 128-column chunk of
// V of it, two adjacent workgroups per task); its key tiles walk the group's key ranges in order, a
// range starting at a 32-key boundary below its first key, and keys outside the
// current range score -inf (the reference's n_mask, :338-343). Only the tile's
// rows inside the group's query range are stored (:386-409).
//
// Waves per SIMD: one at D = 128 and 256 (the JVP modes hold 416-468
// registers); two at D = 64, four for its dense plain forward (128 registers,
// 32 KiB of LDS per workgroup; 1-2% faster than two, bitwise equal).
template <typename T, int MODE, bool MAGI = false, int DH = 128>
__global__ __launch_bounds__(256, DH == 64 ? (MODE == kFwdPlain && !MAGI ? 4 : 2) : 1) void attn_fwd32_kernel(
    FwdParams p) {
  using C = Fwd32Cfg<MODE, DH>;
  constexpr int D = C::D, BN = C::BN, KS = C::KS, DB = C::DB, CR = C::CR, ROWB = C::ROWB;
  constexpr int DVC = C::DVC, CRV = C::CRV, ROWBV = C::ROWBV, NSTAGE = C::NSTAGE;
  constexpr int NOPA = C::NOPA, NOPB = C::NOPB, NOP = NOPA + NOPB, PF = 4;
  constexpr float kSlack = RescaleSlack<T>::value;
  // Without Kd, Vd (C~ = V^T H~ alone) and in bf16 (fp32's range), H~ = P~ Sd
  // is formed without the softmax scale, which the epilogue applies to C~ and
  // to r once per row: one multiply per score value fewer. fp16, whose range
  // the unscaled H~ could leave, and the full JVP (C~ also sums Vd^T P~) keep
  // the reference's H~ = P~ (s Sd).
  constexpr bool kHScaled = C::KVT || !std::is_same<T, __bf16>::value;
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[NSTAGE == 4 ? C::STAGE : 16];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  int bh, qt, ntiles, chunk = 0;
  int q_lo = 0, q_hi = p.Lq;  // rows this workgroup stores
  int r_beg = 0, r_end = 0;   // key ranges of the group (MAGI)
  if constexpr (MAGI) {
    int work = xcd_remap(blockIdx.x, p.T * p.B * p.H * C::CHUNKS);
    if constexpr (C::CHUNKS > 1) {
      chunk = work % C::CHUNKS;  // the chunks of one task are adjacent work items
      work /= C::CHUNKS;
    }
    bh = work / p.T;
    const MagiTask t = magi_task(p, work - bh * p.T, C::BM);
    qt = t.row0 / C::BM;
    q_lo = t.q_lo;
    q_hi = t.q_hi;
    r_beg = t.r_beg;
    r_end = t.r_end;
    ntiles = magi_ntiles(p, t, BN);
    if (ntiles == 0) {  // uniform over the workgroup: nothing requested yet
      if (chunk == 0) magi_store_empty<T, D, C::JVP>(p, bh, t, C::BM);  // every column of the rows
      return;
    }
  } else {
    const int nqt = (p.Lq + C::BM - 1) / C::BM;
    int work = work_item(p.xcd_order);  // block order (common.h)
    if constexpr (C::CHUNKS > 1) {
      chunk = work % C::CHUNKS;  // the chunks of one query tile are adjacent work items
      work /= C::CHUNKS;
    }
    bh = work / nqt;
    qt = work - bh * nqt;
    ntiles = (p.Lk + BN - 1) / BN;
  }
  const int b = bh / p.H, h = bh - b * p.H;

  // ---- this lane's query: Q (and Qd) row slices, B operands of the score MFMAs
  const int query = qt * C::BM + wave * 32 + col;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + D) * 2);
  const int64_t qhead = b * p.q_sb + h * p.q_sh;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc((const char*)p.q + qhead * 2, q_bytes);
  i32x4_t qreg[KS], tqreg[KS];
  {
    const uint32_t qo = (uint32_t)((int64_t)query * p.q_sl * 2) + half * 16;
    __amdgpu_buffer_rsrc_t rtq = rq;
    if constexpr (C::JVP) rtq = make_rsrc((const char*)p.tq + qhead * 2, q_bytes);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qreg[s] = buf_load16(rq, qo + s * 32);
      if constexpr (C::JVP) tqreg[s] = buf_load16(rtq, qo + s * 32);
    }
  }
  // 128-wide heads: Q and Qd live in AGPRs for the whole kernel (MFMA operands
  // read them there); the VGPRs hold the accumulators, the score tiles and the
  // softmax. This unit is compiled with MFMAs in VGPR form
  // (-amdgpu-mfma-vgpr-form). 64-wide heads keep everything in VGPRs, two waves
  // per SIMD.
  if constexpr (DH >= 128) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      asm volatile("" : "+a"(qreg[s]));
      if constexpr (C::JVP) asm volatile("" : "+a"(tqreg[s]));
    }
  }

  // ---- key-side resources and per-lane request offsets (tile independent)
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + D) * 2);
  // V (Vd) resources start at this workgroup's column chunk
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.v_sl + DVC) * 2);
  const int64_t khead = b * p.k_sb + h * p.k_sh, vhead = b * p.v_sb + h * p.v_sh + chunk * DVC;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const char*)p.k + khead * 2, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.v + vhead * 2, v_bytes);
  __amdgpu_buffer_rsrc_t rtk = rk, rtv = rv;
  if constexpr (C::KVT) {
    rtk = make_rsrc((const char*)p.tk + khead * 2, k_bytes);
    rtv = make_rsrc((const char*)p.tv + vhead * 2, v_bytes);
  }
  constexpr int RPW = C::RPW, RPWV = C::RPWV;
  uint32_t roff_k[RPW], roff_v[RPWV];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CR, phys = pch % CR;
    const int logical = phys ^ trswz<CR>(row & 15);
    roff_k[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
    if constexpr (RPWV == RPW) roff_v[j] = (uint32_t)((int64_t)row * p.v_sl * 2) + logical * 16;
  }
  if constexpr (RPWV != RPW) {
#pragma unroll
    for (int j = 0; j < RPWV; ++j) {
      const int pch = (wave + j * C::NW) * 64 + lane;
      const int row = pch / CRV, phys = pch % CRV;
      const int logical = phys ^ trswz<CRV>(row & 15);
      roff_v[j] = (uint32_t)((int64_t)row * p.v_sl * 2) + logical * 16;
    }
  }
  const uint32_t k_step = (uint32_t)((int64_t)BN * p.k_sl * 2);
  const uint32_t v_step = (uint32_t)((int64_t)BN * p.v_sl * 2);

  auto stage = [&](auto kk) -> lds_char_t* {
    constexpr int k = decltype(kk)::value % NSTAGE;
    if constexpr (k == 0) return (lds_char_t*)stg0;
    else if constexpr (k == 1) return (lds_char_t*)stg1;
    else if constexpr (k == 2) return (lds_char_t*)stg2;
    else return (lds_char_t*)stg3;
  };
  // request li (0 <= li < LOADS) of tile kt into stage st (MAGI: of the tile
  // whose first key row is kt); tiles at or beyond the end read zeros or
  // in-range rows into a stage nobody reads again
  auto issue_load = [&](lds_char_t* st, int kt, int li) {
    // request li: tile t, 1 KiB slot jj of this wave. Equal K and V rows: the
    // tiles interleave; otherwise K's requests, then Kd's, then V's and Vd's
    int t = li % C::NTILE, jj = li / C::NTILE;
    if constexpr (RPWV != RPW) {
      constexpr int NK = (C::KVT ? 2 : 1) * RPW;
      if (li < NK) {
        t = C::KVT ? 2 * (li / RPW) : 0;
        jj = li % RPW;
      } else {
        t = 1 + (C::KVT ? 2 * ((li - NK) / RPWV) : 0);
        jj = (li - NK) % RPWV;
      }
    }
    const int i = wave + jj * C::NW;
    uint32_t ks, vs;
    if constexpr (MAGI) {
      ks = (uint32_t)kt * (uint32_t)(p.k_sl * 2);
      vs = (uint32_t)kt * (uint32_t)(p.v_sl * 2);
    } else {
      ks = (uint32_t)kt * k_step;
      vs = (uint32_t)kt * v_step;
    }
    if (t == 0) buf_load16_lds(rk, st + C::OFF_K + i * 1024, roff_k[jj], ks);
    else if (t == 1) buf_load16_lds(rv, st + C::OFF_V + i * 1024, roff_v[jj], vs);
    else if (t == 2) buf_load16_lds(rtk, st + C::OFF_KT + i * 1024, roff_k[jj], ks);
    else buf_load16_lds(rtv, st + C::OFF_VT + i * 1024, roff_v[jj], vs);
  };

  // ---- LDS read offsets: K rows (row perm32(col), chunk 2s + half) and V^T
  // through lds_read_tr16 (block db, keys 16 t + 8 (g >> 1) + (0..3 | 4..7))
  // 256-wide heads keep only slice 0's offset: slice s of a 512-byte row sits
  // at sx[0] ^ 32 s (the row bits lie above the XOR), rebuilt at each read
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
        const int ch = 4 * db + 2 * (g & 1) + (c >> 1);
        tx[db][hh] = row * ROWBV + ((ch ^ trswz<CRV>(row & 15)) << 4) + 8 * (c & 1);
      }
    }
  }
  // Re-defines the offsets at each step (an empty asm), so that stage base +
  // offset folds into the LDS instructions' immediate per step.
  auto pin_offsets = [&]() {
#pragma unroll
    for (int s = 0; s < NSX; ++s) asm volatile("" : "+v"(sx[s]));
#pragma unroll
    for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(tx[db][0]), "+v"(tx[db][1]));
  };

  // Phase A operand o: K slice (KVT: even o) or Kd slice (odd o) s.
  // Phase B operand o - NOPA = j: key chunk t = j / (NOPB / 2); within a chunk
  // the order is V^T blocks (0, 1), Vd^T blocks (0, 1), V^T (2, 3), Vd^T (2, 3)
  // so the two C~ updates of one block are two operands apart.
  struct OpB {
    int t, db;
    bool vd;
  };
  auto op_b = [&](int j) -> OpB {
    constexpr int PER_T = NOPB / 2;
    const int t = j / PER_T, jj = j % PER_T;
    if constexpr (C::KVT) {
      const int pair = jj / 4, w = jj % 4;
      return OpB{t, 2 * pair + (w & 1), w >= 2};
    } else {
      return OpB{t, jj, false};
    }
  };
  auto load_op = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int o) -> i32x4_t {
    if (o < NOPA) {
      const int s = C::KVT ? o >> 1 : o;
      const int off = (C::KVT && (o & 1)) ? C::OFF_KT : C::OFF_K;
      return *(lds_i32x4_t*)(s_next + off + sxo(s));
    }
    const OpB ob = op_b(o - NOPA);
    const lds_char_t* base = s_cur + (ob.vd ? C::OFF_VT : C::OFF_V) + ob.t * 16 * ROWBV;
    const u32x2_t lo = lds_read_tr16(base + tx[ob.db][0]);
    const u32x2_t hi = lds_read_tr16(base + tx[ob.db][1]);
    return i32x4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  };

  f32x16_t oacc[DB], cacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      oacc[d][v] = 0.f;
      cacc[d][v] = 0.f;
    }
  }
  const f32x16_t zero16 = {};
  // O~, C~ accumulation. In the bf16 JVP mode for 128-wide heads (dense and
  // block-sparse) the accumulators stay in AGPRs through inline MFMAs, which
  // frees the VGPRs for the score tiles and the softmax (0.6-1% faster dense,
  // 0.4-0.6% block-sparse, once the rescale went block by block; before, the
  // block-sparse kernel spilled and ran 3% slower). Measured slower for fp16
  // (6%: 59.8 against 56.3 ms at the Wan2.1-14B shape; still 8% with the
  // rescale done block by block and no spills: 51.5 against 47.5 ms at B=4,
  // H=32, L=16384 -- fp16 MFMAs writing AGPRs cost more than the copies they
  // save); 256-wide heads need them for every type. The plain forward keeps
  // them in VGPRs, where it fits two waves per SIMD. Code that touches AGPR accumulators with the VALU (the
  // rescale, the epilogue) waits for the MFMAs first.
  constexpr bool kAccAgpr = MODE == kFwdJvp && ((DH == 128 && !__is_same(T, _Float16)) || DH == 256);
  auto acc_mfma = [&](f32x16_t& c, i32x4_t a, i32x4_t b) {
    if constexpr (kAccAgpr) mfma32_acc(c, a, b, T());
    else c = mfma32(a, b, c, T());
  };
  // the MFMAs of operand o (pk, hk: P~, H~ of the current tile, two 16-key chunks)
  auto mfma_op = [&](int o, i32x4_t a, f32x16_t& sn, f32x16_t& tn, const i32x4_t (&pk)[2],
                     const i32x4_t (&hk)[2]) {
    if (o < NOPA) {
      const int s = C::KVT ? o >> 1 : o;
      if (C::KVT && (o & 1)) {
        tn = mfma32(a, qreg[s], tn, T());
      } else {
        sn = mfma32(a, qreg[s], s == 0 ? zero16 : sn, T());
        if constexpr (C::JVP) tn = mfma32(a, tqreg[s], s == 0 ? zero16 : tn, T());
      }
    } else {
      const OpB ob = op_b(o - NOPA);
      if (ob.vd) {
        acc_mfma(cacc[ob.db], a, pk[ob.t]);
      } else {
        acc_mfma(oacc[ob.db], a, pk[ob.t]);
        if constexpr (C::JVP) acc_mfma(cacc[ob.db], a, hk[ob.t]);
      }
    }
  };

  // Online softmax of one tile in NMICRO micro-steps (log2 domain; lanes l and
  // l^32 share a query and its running max). Value v of the score tile is key
  // 16 (v >> 3) + 8 half + (v & 7); P~, H~ are packed as the B operands of the
  // two 16-key chunks.
  constexpr int NMICRO = 18;
  float m_i = -__builtin_inff(), l_i = 0.f, r_i = 0.f;
  struct Soft {
    float mx, alpha, neg_m, ls, rs, pv;
    float hv;
    bool moved;
  };
  auto soft_micro = [&](int u, Soft& sm, const f32x16_t& sc, const f32x16_t& tc, i32x4_t (&pk)[2],
                        i32x4_t (&hk)[2]) {
    if (u == 0) {
      float a = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      float b2 = fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]));
      float c2 = fmaxf(fmaxf(sc[8], sc[9]), fmaxf(sc[10], sc[11]));
      float d2 = fmaxf(fmaxf(sc[12], sc[13]), fmaxf(sc[14], sc[15]));
      sm.mx = fmaxf(fmaxf(a, b2), fmaxf(c2, d2));
      sm.ls = 0.f;
      sm.rs = 0.f;
    } else if (u == 1) {
      sm.mx = fmaxf(sm.mx, other_half(sm.mx)) * p.scale_log2;
      sm.moved = __builtin_amdgcn_ballot_w64(sm.mx > m_i + kSlack) != 0;
      const float m_new = sm.moved ? fmaxf(m_i, sm.mx) : m_i;
      sm.alpha = fast_exp2(m_i - m_new);
      m_i = m_new;
      sm.neg_m = -exp_base<T>(m_new);
    } else {
      const int v = u - 2;
      const float pe = fast_exp2(fmaf(sc[v], p.scale_log2, sm.neg_m));
      sm.ls += pe;
      float he = 0.f;
      if constexpr (C::JVP) {
        he = kHScaled ? pe * (tc[v] * p.scale) : pe * tc[v];
        sm.rs += he;
      }
      if (v & 1) {
        pk[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(sm.pv, pe);
        if constexpr (C::JVP) hk[v >> 3][(v & 7) >> 1] = (int)Elem<T>::pack2(sm.hv, he);
      } else {
        sm.pv = pe;
        sm.hv = he;
      }
    }
  };
  auto rescale = [&](float alpha) {
    if constexpr (kAccAgpr) {
      // one 16-value block at a time, so the copies through VGPRs need 16 of
      // them rather than all 128 (which spilled: 256-wide heads leave no AGPR
      // free; 128-wide ones spilled 5 registers and ran 0.3% slower)
#pragma unroll
      for (int d = 0; d < 2 * DB; ++d) {
        f32x16_t& a = d < DB ? oacc[d] : cacc[d - DB];
        asm volatile("" : "+a"(a));  // read after the previous block's write-back
#pragma unroll
        for (int v = 0; v < 16; ++v) a[v] *= alpha;
        asm volatile("" : "+a"(a));
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          oacc[d][v] *= alpha;
          if constexpr (C::JVP) cacc[d][v] *= alpha;
        }
      }
    }
  };

  // keys of the cursor's tile outside its range score -inf
  auto mask_range = [&](f32x16_t& sc, const MagiCursor& c) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      if (c.masked(c.start + 16 * (v >> 3) + 8 * half + (v & 7))) sc[v] = -__builtin_inff();
    }
  };
  MagiCursor ci{r_beg, r_end, 0, 0, 0};  // MAGI: tile requested next
  if constexpr (MAGI) ci.seek(p, BN);
  MagiCursor cm = ci;  // MAGI: tile whose softmax runs next

  // step i (i + 1 < ntiles, i % 4 == kk): phase A on tile i+1's K, softmax of
  // tile i (sc, tc); phase B on tile i's V; requests tile i+3
  auto step = [&](auto kk, int i, const f32x16_t& sc, const f32x16_t& tc, f32x16_t& sn, f32x16_t& tn) {
    constexpr int k = decltype(kk)::value;
    // tile i+1 has landed (four stages: tile i+2 may be in flight)
    ring_sync<(NSTAGE - 3) * C::LOADS>();
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + NSTAGE - 1>{});
    i32x4_t opr[PF];
#pragma unroll
    for (int o = 0; o < PF; ++o) opr[o] = load_op(s_next, s_cur, o);
    Soft sm;
    i32x4_t pk[2], hk[2];
    if constexpr (MAGI) {
      if (cm.partial(BN)) mask_range(const_cast<f32x16_t&>(sc), cm);
      cm.next(p, BN);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 0; o < NOPA; ++o) {
      mfma_op(o, opr[o % PF], sn, tn, pk, hk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
#pragma unroll
      for (int u = o * NMICRO / NOPA; u < (o + 1) * NMICRO / NOPA; ++u) soft_micro(u, sm, sc, tc, pk, hk);
      __builtin_amdgcn_sched_barrier(0);
    }
    l_i = l_i * sm.alpha + sm.ls;
    if constexpr (C::JVP) r_i = r_i * sm.alpha + sm.rs;
    // keep the softmax in phase A: the values are used here, before the branch
    asm volatile("" : "+v"(pk[0]), "+v"(pk[1]), "+v"(l_i));
    if constexpr (C::JVP) asm volatile("" : "+v"(hk[0]), "+v"(hk[1]), "+v"(r_i));
    if (sm.moved) {
      rescale(sm.alpha);
      if constexpr (kAccAgpr) asm volatile("s_nop 2" ::: "memory");  // AGPR writes before the next MFMA reads them
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) {
      mfma_op(o, opr[o % PF], sn, tn, pk, hk);
      if (o + PF < NOP) opr[o % PF] = load_op(s_next, s_cur, o + PF);
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) {
        if (NOPA + li * NOPB / C::LOADS == o) issue_load(s_req, MAGI ? ci.start : i + NSTAGE - 1, li);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MAGI) ci.next(p, BN);
  };
  // last tile (may hold keys >= Lk): masked softmax, rescale, PV
  auto last_step = [&](auto kk, int i, f32x16_t& sc, const f32x16_t& tc) {
    const lds_char_t* s_cur = stage(kk);
    if constexpr (MAGI) {
      mask_range(sc, cm);
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        if (i * BN + 16 * (v >> 3) + 8 * half + (v & 7) >= p.Lk) sc[v] = -__builtin_inff();
      }
    }
    Soft sm;
    i32x4_t pk[2], hk[2];
#pragma unroll
    for (int u = 0; u < NMICRO; ++u) soft_micro(u, sm, sc, tc, pk, hk);
    l_i = l_i * sm.alpha + sm.ls;
    if constexpr (C::JVP) r_i = r_i * sm.alpha + sm.rs;
    rescale(sm.alpha);
    if constexpr (kAccAgpr) asm volatile("s_nop 2" ::: "memory");
    f32x16_t un_s, un_t;
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) mfma_op(o, load_op(s_cur, s_cur, o), un_s, un_t, pk, hk);
  };

  // ---- prologue: tiles 0..NSTAGE-2 requested, scores of tile 0
  if constexpr (MAGI) {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), ci.start, li);
    ci.next(p, BN);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), ci.start, li);
    ci.next(p, BN);
    if constexpr (NSTAGE == 4) {
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), ci.start, li);
      ci.next(p, BN);
    }
  } else {
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
    for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
    if constexpr (NSTAGE == 4) {
#pragma unroll
      for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
    }
  }
  ring_sync<(NSTAGE - 2) * C::LOADS>();  // Q slices and tile 0
  f32x16_t sa, ta, sb, tb;
  {
    const lds_char_t* s0 = stage(IC<0>{});
    const i32x4_t none[2] = {};
#pragma unroll
    for (int o = 0; o < NOPA; ++o) mfma_op(o, load_op(s0, s0, o), sa, ta, none, none);
  }
  int i = 0;
  if constexpr (NSTAGE == 4) {
    for (; i + 4 < ntiles; i += 4) {
      step(IC<0>{}, i, sa, ta, sb, tb);
      step(IC<1>{}, i + 1, sb, tb, sa, ta);
      step(IC<2>{}, i + 2, sa, ta, sb, tb);
      step(IC<3>{}, i + 3, sb, tb, sa, ta);
    }
    const int rest = ntiles - i;  // 1..4 tiles left
    if (rest >= 2) step(IC<0>{}, i, sa, ta, sb, tb);
    if (rest >= 3) step(IC<1>{}, i + 1, sb, tb, sa, ta);
    if (rest >= 4) step(IC<2>{}, i + 2, sa, ta, sb, tb);
    if (rest == 1) last_step(IC<0>{}, i, sa, ta);
    else if (rest == 2) last_step(IC<1>{}, i + 1, sb, tb);
    else if (rest == 3) last_step(IC<2>{}, i + 2, sa, ta);
    else last_step(IC<3>{}, i + 3, sb, tb);
  } else {
    // three stages: six steps per pass keep both the stage (k % 3) and the
    // score-tile pair (k % 2) compile-time
    for (; i + 6 < ntiles; i += 6) {
      step(IC<0>{}, i, sa, ta, sb, tb);
      step(IC<1>{}, i + 1, sb, tb, sa, ta);
      step(IC<2>{}, i + 2, sa, ta, sb, tb);
      step(IC<3>{}, i + 3, sb, tb, sa, ta);
      step(IC<4>{}, i + 4, sa, ta, sb, tb);
      step(IC<5>{}, i + 5, sb, tb, sa, ta);
    }
    const int rest = ntiles - i;  // 1..6 tiles left
    if (rest >= 2) step(IC<0>{}, i, sa, ta, sb, tb);
    if (rest >= 3) step(IC<1>{}, i + 1, sb, tb, sa, ta);
    if (rest >= 4) step(IC<2>{}, i + 2, sa, ta, sb, tb);
    if (rest >= 5) step(IC<3>{}, i + 3, sb, tb, sa, ta);
    if (rest >= 6) step(IC<4>{}, i + 4, sa, ta, sb, tb);
    if (rest == 1) last_step(IC<0>{}, i, sa, ta);
    else if (rest == 2) last_step(IC<1>{}, i + 1, sb, tb);
    else if (rest == 3) last_step(IC<2>{}, i + 2, sa, ta);
    else if (rest == 4) last_step(IC<3>{}, i + 3, sb, tb);
    else if (rest == 5) last_step(IC<4>{}, i + 4, sa, ta);
    else last_step(IC<5>{}, i + 5, sb, tb);
  }
  wait_vmem();  // no requests beyond the last tile stay in flight
  if constexpr (kAccAgpr) mfma_acc_drain();

  // ---- epilogue: lane (query col, half) holds d = 32 db + 8 jj + 4 half + (0..3)
  const float l = l_i + other_half(l_i);
  const float inv_l = 1.0f / l;
  const float inv_lh = kHScaled ? inv_l : inv_l * p.scale;  // 1 / l, with the scale H~ left out
  float mu = 0.f;
  if constexpr (C::JVP) mu = (r_i + other_half(r_i)) * inv_lh;
  // O (Od) resources start at this workgroup's column chunk
  const int64_t obase = b * p.o_sb + h * p.o_sh + chunk * DVC;
  const uint32_t o_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.o_sl + DVC) * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc((char*)p.o + obase * 2, o_bytes);
  __amdgpu_buffer_rsrc_t rto = ro;
  if constexpr (C::JVP) rto = make_rsrc((char*)p.to + obase * 2, o_bytes);
  // O (and Od) leave as whole rows through LDS: once every wave has finished
  // its last step the ring is free, and wave w stages its 32 rows in ring bytes
  // [w WST, (w + 1) WST)
  ring_sync<0>();
  // (regions that do not pack into a stage take one stage per wave)
  constexpr int WST = (C::JVP ? 2 : 1) * RowStage<DVC>::BYTES;
  constexpr bool kPacked = C::STAGE % WST == 0;
  static_assert(kPacked ? C::NW * WST <= NSTAGE * C::STAGE : WST <= C::STAGE && C::NW <= NSTAGE,
                "staging fits the ring");
  const int wst_stage = kPacked ? wave * WST / C::STAGE : wave;
  lds_char_t* const region = (wst_stage == 0 ? stage(IC<0>{}) : wst_stage == 1 ? stage(IC<1>{})
                              : wst_stage == 2 ? stage(IC<2>{}) : stage(IC<3>{})) +
                             (kPacked ? (wave * WST) % C::STAGE : 0);
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float ov[4], tv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = oacc[d][4 * jj + e] * inv_l;
        if constexpr (C::JVP) tv[e] = cacc[d][4 * jj + e] * inv_lh - mu * ov[e];
      }
      stage_put<DVC>(region, col, half, d, jj, u32x2_t{Elem<T>::pack2(ov[0], ov[1]), Elem<T>::pack2(ov[2], ov[3])});
      if constexpr (C::JVP)
        stage_put<DVC>(region + RowStage<DVC>::BYTES, col, half, d, jj,
                     u32x2_t{Elem<T>::pack2(tv[0], tv[1]), Elem<T>::pack2(tv[2], tv[3])});
    }
    if constexpr (kAccAgpr) __builtin_amdgcn_sched_barrier(0);  // one block's copies at a time
  }
  // rows >= Lq fall outside the resource; MAGI stores only the group's rows
  const bool keep = !MAGI || (query >= q_lo && query < q_hi);
  const int row0 = qt * C::BM + wave * 32;
  auto row_off = [&](int r) -> uint32_t {
    const int qrow = row0 + r;
    const bool ok = qrow < p.Lq && (!MAGI || (qrow >= q_lo && qrow < q_hi));
    return ok ? (uint32_t)((int64_t)qrow * p.o_sl * 2) : o_bytes;
  };
#pragma unroll
  for (int kk = 0; kk < RowStage<DVC>::NST; ++kk) {
    stage_store<DVC>(region, kk, lane, ro, row_off);
    if constexpr (C::JVP) stage_store<DVC>(region + RowStage<DVC>::BYTES, kk, lane, rto, row_off);
  }
  // every chunk's workgroup holds the same statistics; chunk 0 stores them
  if (half == 0 && query < p.Lq && keep && chunk == 0) {
    const int64_t si = (int64_t)bh * p.Lq + query;
    p.lse[si] = (exp_base<T>(m_i) + __builtin_log2f(l)) * 0.6931471805599453f;
    if constexpr (C::JVP) p.mu[si] = mu;
  }
}

}  // namespace dmad
