// Forward attention kernels for gfx950: plain (O, LSE) and forward+JVP
// (O, tangent output, LSE, mu) in a single online-softmax pass.
//
// Semantics follow the reference Triton kernel `_attn_fwd`
// (train/wan/rcm/utils/flash_attention_jvp_triton.py:107-232):
//   S  = s * Q K^T                     (log2 domain: qk = S * log2(e))
//   P~ = exp2(qk - m)                  running max m per query row
//   Sd = s * (Qd K^T + Q Kd^T)         tangent scores (natural domain)
//   H~ = P~ * Sd,  r = rowsum(H~)
//   O~ += bf16(P~) V,  C~ += bf16(P~) Vd + bf16(H~) V     (fp32 accumulators)
//   O = O~/l,  Od = C~/l - (r/l) O,  LSE = (m + log2 l) ln 2,  mu = r/l
// The reference keeps A~ = P~ Vd and B~ = H~ V apart and adds them in its
// epilogue (:216-223); they receive identical rescales, so one accumulator
// C~ = A~ + B~ holds the same sum.
//
// Kernels in this file (128-wide Q/K and V heads use attn_fwd32_kernel in
// attn_fwd32.h instead):
//   attn_fwd_kernel / attn_fwd_stream_kernel: one workgroup = 8 waves (2 per
//     SIMD) = 128 query rows of one head; wave w owns 16 query rows, whose Q
//     and Qd slices stay in registers as the B operand of S^T = K Q^T on
//     16x16x32 MFMAs (lane l <-> query l%16);
//   attn_fwd_simple_kernel: 4 waves x 32 queries on 32x32x16 MFMAs, one
//     tile per step, for head dims whose four-stage ring does not fit in LDS.
// In all of them:
//   * K, Kd tiles [BN keys][D] and V^T, Vd^T tiles [D][BN keys] are streamed
//     through an LDS ring by buffer->LDS DMA (16 B per lane);
//   * the C layout of S^T (lane <-> query, key values per lane) feeds the
//     B operand of O^T = V^T P^T directly, because the K rows of every key
//     block are read in a permuted order that makes a lane's values cover
//     consecutive keys;
//   * O~^T and C~^T accumulate in registers with lane <-> query, so the
//     per-row rescale is a per-lane scalar multiply.
// V and Vd are read from a pre-transposed copy ([BH][DVP][LKP], zero padded),
// produced by transpose_pad_kernel; that costs one extra HBM pass over V and
// Vd, far below the O(L^2) work of the pass itself.
#pragma once
#include <type_traits>

#include "common.h"

namespace dmad {

enum FwdMode : int { kFwdPlain = 0, kFwdJvp = 1, kFwdJvpQOnly = 2 };

struct FwdParams {
  const void* q;
  const void* k;
  const void* tq;
  const void* tk;
  const void* vt;   // V^T  [B*H][DVP][LKP]  (kernels that read a transposed copy)
  const void* tvt;  // Vd^T [B*H][DVP][LKP]
  const void* v;    // V, Vd rows (kernels that transpose on the LDS read)
  const void* tv;
  void* o;
  void* to;
  float* lse;  // [B*H][Lq]
  float* mu;   // [B*H][Lq]
  int64_t q_sb, q_sh, q_sl;  // element strides, shared by Q and Qd
  int64_t k_sb, k_sh, k_sl;  // shared by K and Kd
  int64_t v_sb, v_sh, v_sl;  // shared by V and Vd
  int64_t o_sb, o_sh, o_sl;  // shared by O and Od
  int B, H, Lq, Lk, LKP;
  float scale;       // softmax scale s
  float scale_log2;  // s * log2(e)
  // block-sparse (MagiMask) mode of attn_fwd32_kernel: query groups partition
  // [0, Lq); group g attends to the sorted, disjoint key ranges
  // k_ranges[qk_map[g] .. qk_map[g+1]); a task is a (group, 128-query tile) pair
  const int* q_ranges;    // [G][2]
  const int* k_ranges;    // [R][2]
  const int* qk_map;      // [G+1]
  const int* task_group;  // [T]
  const int* task_qtile;  // [T]
  int G, R, T;
  int xcd_order;  // dense kernels: work items contiguous per XCD (common.h)
};

// One (query group, 128-query tile) task of the block-sparse forward: group
// and key-range indices clamped into the arrays, the query range and the key
// ranges clipped to the sequences, so malformed tables read nothing outside
// them. The query tile is 128 rows from row0.
struct MagiTask {
  int row0, q_lo, q_hi, r_beg, r_end;
};
__device__ __forceinline__ MagiTask magi_task(const FwdParams& p, int task, int bm) {
  MagiTask t;
  const int g = min(max(__builtin_amdgcn_readfirstlane(p.task_group[task]), 0), p.G - 1);
  t.row0 = __builtin_amdgcn_readfirstlane(p.task_qtile[task]) * bm;
  t.q_lo = max(__builtin_amdgcn_readfirstlane(p.q_ranges[2 * g]), 0);
  t.q_hi = min(__builtin_amdgcn_readfirstlane(p.q_ranges[2 * g + 1]), p.Lq);
  t.r_beg = min(max(__builtin_amdgcn_readfirstlane(p.qk_map[g]), 0), p.R);
  t.r_end = min(max(__builtin_amdgcn_readfirstlane(p.qk_map[g + 1]), t.r_beg), p.R);
  return t;
}
// Key range r clipped to [0, Lk) (empty when k1 <= k0).
__device__ __forceinline__ void magi_range(const FwdParams& p, int r, int& k0, int& k1) {
  k0 = max(__builtin_amdgcn_readfirstlane(p.k_ranges[2 * r]), 0);
  k1 = min(__builtin_amdgcn_readfirstlane(p.k_ranges[2 * r + 1]), p.Lk);
}
// 32-key (BN-key) tiles the task walks: per range, from the tile holding its
// first key to the one holding its last.
__device__ __forceinline__ int magi_ntiles(const FwdParams& p, const MagiTask& t, int bn) {
  int n = 0;
  for (int r = t.r_beg; r < t.r_end; ++r) {
    int k0, k1;
    magi_range(p, r, k0, k1);
    if (k1 > k0) n += (k1 + bn - 1) / bn - k0 / bn;
  }
  return n;
}
// Walks the key tiles of a task: current range r (clipped to [k0, k1)) and
// the first key row of the current BN-key tile; past the last range it
// points at row Lk and beyond (tiles of zeros, never used).
struct MagiCursor {
  int r, r_end, start, k0, k1;
  __device__ __forceinline__ void seek(const FwdParams& p, int bn) {  // first non-empty range from r on
    for (; r < r_end; ++r) {
      magi_range(p, r, k0, k1);
      if (k1 > k0) {
        start = k0 / bn * bn;
        return;
      }
    }
    start = k0 = k1 = p.Lk;
  }
  __device__ __forceinline__ void next(const FwdParams& p, int bn) {
    start += bn;
    if (start >= k1 && r < r_end) {
      ++r;
      seek(p, bn);
    }
  }
  // key lies outside the current range (the reference's n_mask, :338-343)
  __device__ __forceinline__ bool masked(int key) const { return (unsigned)(key - k0) >= (unsigned)(k1 - k0); }
  // the current tile has keys outside the range
  __device__ __forceinline__ bool partial(int bn) const { return start < k0 || start + bn > k1; }
};

// Rows of a task whose group has no key in [0, Lk): O = Od = 0 and LSE = -inf,
// what the reference's epilogue gives for l_i == 0 (:386-400); mu = 0. The
// whole workgroup (any size) writes 16-byte chunks.
template <typename T, int DV, bool JVP>
__device__ void magi_store_empty(const FwdParams& p, int bh, const MagiTask& t, int bm) {
  const int b = bh / p.H, h = bh - b * p.H;
  const int lo = max(t.row0, t.q_lo), hi = min(t.row0 + bm, t.q_hi);
  constexpr int CH = DV / 8;
  const int64_t obase = b * p.o_sb + h * p.o_sh;
  for (int idx = threadIdx.x; idx < (hi - lo) * CH; idx += blockDim.x) {
    const int r = lo + idx / CH, c = idx - (idx / CH) * CH;
    const int64_t off = (obase + (int64_t)r * p.o_sl + 8 * c) * 2;
    *(i32x4_t*)((char*)p.o + off) = i32x4_t{0, 0, 0, 0};
    if constexpr (JVP) *(i32x4_t*)((char*)p.to + off) = i32x4_t{0, 0, 0, 0};
  }
  for (int r = lo + (int)threadIdx.x; r < hi; r += blockDim.x) {
    p.lse[(int64_t)bh * p.Lq + r] = -__builtin_inff();
    if constexpr (JVP) p.mu[(int64_t)bh * p.Lq + r] = 0.f;
  }
}

// Lazy rescale (log2 units): the running max m only moves when a row's tile
// max exceeds it by more than `value`, so the accumulators are rescaled only
// on those steps, and P~ = exp2(x - m - offset). bf16 shares fp32's exponent
// range: offset 0, P~ <= 2^8. fp16 subtracts offset = value, so P~ <= 1 and
// H~ = P~ s Sd stay within the reference's bounds (its P~ <= 1 with the exact
// max) and nothing new can overflow; l, r and the accumulators all carry the
// same factor, which cancels in O, Od and mu, and LSE adds the offset back.
template <typename T> struct RescaleSlack {
  static constexpr float value = 8.0f;
  static constexpr float offset = 0.0f;
};
template <> struct RescaleSlack<_Float16> {
  static constexpr float value = 4.0f;
  static constexpr float offset = 4.0f;
};
// m + offset (m itself when the offset is 0, bit for bit)
template <typename T>
__device__ __forceinline__ float exp_base(float m) {
  if constexpr (RescaleSlack<T>::offset != 0.0f) return m + RescaleSlack<T>::offset;
  else return m;
}

template <int DQK, int DV, int MODE>
struct FwdCfg {
  static constexpr int NW = 8;         // waves per workgroup, 2 per SIMD
  static constexpr int QW = 16;        // query rows per wave
  static constexpr int BM = QW * NW;   // query rows per workgroup
  static constexpr int DVP = DV;       // V^T rows read (16-row MFMA blocks)
  static constexpr int VT_ROWS = DV < 32 ? 32 : DV;  // rows per head of the V^T workspace
  static constexpr int BN = 32;        // keys per pipeline step (two 16-key score blocks)
  static constexpr int KS = DQK / 32;  // 32-wide k slices of Q K^T
  static constexpr int DB = DV / 16;   // 16-row blocks of O^T
  static constexpr int CK = DQK / 8;   // 16-byte chunks per K row
  static constexpr int CV = BN / 8;    // 16-byte chunks per V^T row
  static constexpr bool JVP = MODE != kFwdPlain;
  static constexpr bool KVT = MODE == kFwdJvp;
  static constexpr int K_BYTES = BN * DQK * 2;
  static constexpr int V_BYTES = DVP * BN * 2;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_V = K_BYTES;
  static constexpr int OFF_KT = K_BYTES + V_BYTES;
  static constexpr int OFF_VT = 2 * K_BYTES + V_BYTES;
  static constexpr int STAGE = (KVT ? 2 : 1) * (K_BYTES + V_BYTES);
  static constexpr int NSTAGE = 4;  // tiles i-1 (V), i (V), i+1 (K) in use, i+2 landing
  // this kernel needs 32-wide score slices and a four-stage ring that fits the LDS
  static constexpr bool FITS = DQK >= 32 && NSTAGE * STAGE <= 160 * 1024;
  static constexpr int NKI = BN * CK / 64;   // wave-wide 1 KiB loads per K tile
  static constexpr int NVI = DVP * CV / 64;  // ... per V^T tile
  static constexpr int KPW = (NKI + NW - 1) / NW;
  static constexpr int VPW = (NVI + NW - 1) / NW;
};

// Key row of score block b (0, 1), MFMA row r (0..15), inside a 32-key tile.
// Lane group g (rows 4g..4g+3) of block b then holds keys 8g + 4b + v, so the
// two blocks together give each lane group 8 consecutive keys: the B-operand
// layout of the following 32-key P V^T product, with no data movement.
__device__ __forceinline__ int key_of_row16(int b, int r) { return ((r >> 2) << 3) + (b << 2) + (r & 3); }

// XOR swizzle of the 16-byte chunk index of K-tile row R (0..31) for C chunks
// per row: the 16 rows one lane group reads (fixed b, r = 0..15) land in 16
// distinct 16-byte slots of the 256-byte LDS bank window.
template <int C>
__device__ __forceinline__ int kswz16(int R) {
  const int u = ((R >> 1) & 12) | (R & 3);  // distinct for the 16 rows of either block
  if constexpr (C >= 16) return u;
  else if constexpr (C == 8) return u >> 1;
  else return (u >> 2) & (C - 1);
}

// Value held by lane l^16, via v_permlane16_swap (rows of 16 lanes swap pairwise).
__device__ __forceinline__ float other_row16(float x) {
  uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}

// Software pipeline over 32-key tiles, step i:
//   top      wait for tile i+1's DMA, barrier, start the DMA of tile i+2
//   phase A  MFMA: O~^T, C~^T += V^T P^T ... of tile i-1  ||  VALU: softmax of tile i
//   phase B  MFMA: S^T, Sd^T of tile i+1 (overwrites tile i's score registers)
// Each wave owns 16 query rows (lane l <-> query l%16); two waves share a SIMD,
// so one wave's MFMA chain runs while the other waits on LDS or does softmax.
template <typename T, int DQK, int DV, int MODE>
__global__ __launch_bounds__(512) void attn_fwd_kernel(FwdParams p) {
  struct C : FwdCfg<DQK, DV, MODE> {
    static constexpr float rescale_log2() { return RescaleSlack<T>::value; }
  };
  constexpr int BN = C::BN, KS = C::KS, DB = C::DB, CK = C::CK, CV = C::CV, NST = C::NSTAGE;
  __shared__ __attribute__((aligned(1024))) char smem[NST * C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;

  const char* qbase = (const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2;
  const char* kbase = (const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + DQK) * 2);
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + DQK) * 2);
  const uint32_t vt_bytes = (uint32_t)((int64_t)C::VT_ROWS * p.LKP * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qbase, q_bytes);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.vt + (int64_t)bh * vt_bytes, vt_bytes);
  __amdgpu_buffer_rsrc_t rtq = rq, rtk = rk, rtv = rv;
  if constexpr (C::JVP) rtq = make_rsrc((const char*)p.tq + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  if constexpr (C::KVT) {
    rtk = make_rsrc((const char*)p.tk + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
    rtv = make_rsrc((const char*)p.tvt + (int64_t)bh * vt_bytes, vt_bytes);
  }

  // ---- Q (and Qd) slices in registers: B operand of S^T = K Q^T
  const int qrow = qt * C::BM + wave * C::QW + col;
  const uint32_t qoff = (uint32_t)((int64_t)qrow * p.q_sl * 2) + grp * 16;
  i32x4_t qr[KS], tqr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qr[s] = buf_load16(rq, qoff + s * 64);
    if constexpr (C::JVP) tqr[s] = buf_load16(rtq, qoff + s * 64);
  }

  // ---- per-lane DMA offsets (tile independent)
  uint32_t koff[C::KPW], voff[C::VPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CK, phys = pch % CK;
    const int logical = phys ^ kswz16<CK>(row);
    koff[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < C::VPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CV, phys = pch % CV;
    const int logical = phys ^ swz4r(d & 15);
    voff[j] = (uint32_t)(d * p.LKP * 2) + logical * 16;
  }
  const uint32_t k_tile_step = (uint32_t)((int64_t)BN * p.k_sl * 2);

  auto stage_ptr = [&](int kt) -> const char* { return smem + (kt & (NST - 1)) * C::STAGE; };
  auto issue_tile = [&](int kt) {
    char* st = smem + (kt & (NST - 1)) * C::STAGE;
    const uint32_t ks = (uint32_t)kt * k_tile_step;
    const uint32_t vs = (uint32_t)kt * BN * 2;
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NKI) {
        buf_load16_lds(rk, st + C::OFF_K + i * 1024, koff[j], ks);
        if constexpr (C::KVT) buf_load16_lds(rtk, st + C::OFF_KT + i * 1024, koff[j], ks);
      }
    }
#pragma unroll
    for (int j = 0; j < C::VPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NVI) {
        buf_load16_lds(rv, st + C::OFF_V + i * 1024, voff[j], vs);
        if constexpr (C::KVT) buf_load16_lds(rtv, st + C::OFF_VT + i * 1024, voff[j], vs);
      }
    }
  };

  // ---- LDS read offsets (tile independent)
  int krow_off[2], kswzv[2];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int R = key_of_row16(sb, col);
    krow_off[sb] = R * CK * 16;
    kswzv[sb] = kswz16<CK>(R);
  }
  const int vrow_off = col * CV * 16 + ((grp ^ swz4r(col)) << 4);

  f32x4_t oacc[DB], cacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      oacc[d][v] = 0.f;
      cacc[d][v] = 0.f;
    }
  }
  float m_i = -__builtin_inff(), l_i = 0.f, r_i = 0.f;
  const int ntiles = (p.Lk + BN - 1) / BN;

  // S^T (and Sd^T) of one 32-key tile: two 16-key blocks, A = K rows from LDS, B = Q slices
  f32x4_t sc[2], tc[2];
  auto scores = [&](const char* st) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int off = krow_off[sb] + (((4 * s + grp) ^ kswzv[sb]) << 4);
        const i32x4_t ak = *(const i32x4_t*)(st + C::OFF_K + off);
        if (s == 0) {
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
          sc[sb] = mfma16(ak, qr[0], z, T());
          if constexpr (C::JVP) tc[sb] = mfma16(ak, tqr[0], z, T());
        } else {
          sc[sb] = mfma16(ak, qr[s], sc[sb], T());
          if constexpr (C::JVP) tc[sb] = mfma16(ak, tqr[s], tc[sb], T());
        }
        if constexpr (C::KVT) {
          const i32x4_t akt = *(const i32x4_t*)(st + C::OFF_KT + off);
          tc[sb] = mfma16(akt, qr[s], tc[sb], T());
        }
      }
    }
  };

  // Online softmax of one tile (log2 domain; the 4 lane groups of a query share m).
  // Leaves P~ and H~ packed as B operands (keys 8*grp + e in pk, hk) and returns
  // the accumulator rescale factor (1 when the running max did not move).
  auto softmax = [&](int kt, auto TAIL, i32x4_t& pk, i32x4_t& hk) -> float {
    if constexpr (decltype(TAIL)::value) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if (kt * BN + 8 * grp + 4 * sb + v >= p.Lk) sc[sb][v] = -__builtin_inff();
        }
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    mx = fmaxf(mx, other_row16(mx));
    mx = fmaxf(mx, other_half(mx)) * p.scale_log2;
    const bool moved = __builtin_amdgcn_ballot_w64(mx > m_i + C::rescale_log2()) != 0;
    const float m_new = moved ? fmaxf(m_i, mx) : m_i;
    const float alpha = fast_exp2(m_i - m_new);
    m_i = m_new;
    const float neg_m = -exp_base<T>(m_new);
    float pv[8], hv[8], ls = 0.f, rs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sb = e >> 2, v = e & 3;
      pv[e] = fast_exp2(fmaf(sc[sb][v], p.scale_log2, neg_m));
      ls += pv[e];
      if constexpr (C::JVP) {
        hv[e] = pv[e] * (tc[sb][v] * p.scale);
        rs += hv[e];
      }
    }
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      pk[e2] = (int)Elem<T>::pack2(pv[2 * e2], pv[2 * e2 + 1]);
      if constexpr (C::JVP) hk[e2] = (int)Elem<T>::pack2(hv[2 * e2], hv[2 * e2 + 1]);
    }
    l_i = l_i * alpha + ls;
    if constexpr (C::JVP) r_i = r_i * alpha + rs;
    return alpha;
  };

  auto rescale = [&](float alpha) {
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        oacc[d][v] *= alpha;
        if constexpr (C::JVP) cacc[d][v] *= alpha;
      }
    }
  };

  // O~^T += V^T P^T ; C~^T += Vd^T P^T + V^T H^T  (one 32-key MFMA per 16-row d block)
  auto pv_update = [&](const char* st, const i32x4_t& pk, const i32x4_t& hk) {
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int off = d * 16 * CV * 16 + vrow_off;
      const i32x4_t av = *(const i32x4_t*)(st + C::OFF_V + off);
      oacc[d] = mfma16(av, pk, oacc[d], T());
      if constexpr (C::KVT) {
        const i32x4_t avt = *(const i32x4_t*)(st + C::OFF_VT + off);
        cacc[d] = mfma16(avt, pk, cacc[d], T());
      }
      if constexpr (C::JVP) cacc[d] = mfma16(av, hk, cacc[d], T());
    }
  };

  // ---- prologue: tiles 0..2 in flight, scores + softmax of tile 0, scores of tile 1
  issue_tile(0);
  if (ntiles > 1) issue_tile(1);
  if (ntiles > 2) issue_tile(2);
  wait_vmem();
  __syncthreads();
  i32x4_t pk, hk;
  scores(stage_ptr(0));
  if (ntiles == 1) {
    softmax(0, std::true_type(), pk, hk);  // accumulators are still zero
  } else {
    softmax(0, std::false_type(), pk, hk);
    scores(stage_ptr(1));
  }
  // ---- steady state: step i runs PV of tile i-1, softmax of tile i, scores of tile i+1
  // The rescale for step i's alpha runs at the top of step i+1: after the PV
  // of tile i-1 and before that of tile i, and in its own (rarely taken)
  // branch, so the softmax of step i stays in one block with its MFMAs.
  bool moved = false;
  float alpha = 1.f;
  int i = 1;
  for (; i + 1 < ntiles; ++i) {
    wait_vmem();
    __syncthreads();
    if (i + 2 < ntiles) issue_tile(i + 2);  // reuses the stage of tile i-2
    if (moved) rescale(alpha);
    i32x4_t pn, hn;
    pv_update(stage_ptr(i - 1), pk, hk);
    alpha = softmax(i, std::false_type(), pn, hn);
    moved = alpha != 1.f;
    moved = __builtin_amdgcn_ballot_w64(moved) != 0;
    scores(stage_ptr(i + 1));
    pk = pn;
    hk = hn;
  }
  if (moved) rescale(alpha);
  // ---- last step: tile ntiles-1 may hold keys >= Lk
  if (ntiles > 1) {
    i32x4_t pn, hn;
    pv_update(stage_ptr(i - 1), pk, hk);
    alpha = softmax(i, std::true_type(), pn, hn);
    rescale(alpha);
    pk = pn;
    hk = hn;
  }
  pv_update(stage_ptr(ntiles - 1), pk, hk);

  // ---- epilogue: lane (query col, group g) holds d = 16*dblk + 4g + v
  float l = l_i + other_row16(l_i);
  l = l + other_half(l);
  const float inv_l = 1.0f / l;
  float mu = 0.f;
  if constexpr (C::JVP) {
    float r = r_i + other_row16(r_i);
    r = r + other_half(r);
    mu = r * inv_l;
  }
  const int64_t obase = b * p.o_sb + h * p.o_sh;
  const uint32_t o_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.o_sl + DV) * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc((char*)p.o + obase * 2, o_bytes);
  __amdgpu_buffer_rsrc_t rto = ro;
  if constexpr (C::JVP) rto = make_rsrc((char*)p.to + obase * 2, o_bytes);
  const uint32_t orow = (uint32_t)((int64_t)qrow * p.o_sl * 2);
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    const int dc = d * 16 + 4 * grp;
    float ov[4], tv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ov[v] = oacc[d][v] * inv_l;
      if constexpr (C::JVP) tv[v] = cacc[d][v] * inv_l - mu * ov[v];
    }
    const uint32_t off = orow + dc * 2;
    u32x2_t w = {Elem<T>::pack2(ov[0], ov[1]), Elem<T>::pack2(ov[2], ov[3])};
    buf_store8(ro, w, off);
    if constexpr (C::JVP) {
      u32x2_t wt = {Elem<T>::pack2(tv[0], tv[1]), Elem<T>::pack2(tv[2], tv[3])};
      buf_store8(rto, wt, off);
    }
  }
  if (grp == 0 && qrow < p.Lq) {
    const int64_t si = (int64_t)bh * p.Lq + qrow;
    p.lse[si] = (exp_base<T>(m_i) + __builtin_log2f(l)) * 0.6931471805599453f;
    if constexpr (C::JVP) p.mu[si] = mu;
  }
}

// Streamed variant of attn_fwd_kernel for shapes whose K and V^T tiles split
// evenly over the eight waves (DQK = DV = 128 in particular). Step i, after one
// barrier, is a fixed stream of MFMAs:
//   phase A  S^T, Sd^T of tile i+1, with the online softmax of tile i on the VALU
//   (rescale of the accumulators, only when some row's running max moved)
//   phase B  O~^T, C~^T += V^T P^T ... of tile i, with tile i+3's requests
// Every MFMA's LDS operand is read four operands ahead. The ring has four
// stages, each its own LDS object, and the loop is unrolled by four so each
// stage reference is known at compile time: the compiler then waits for a
// buffer->LDS request only before reading the stage it fills, and tiles are
// requested three steps before use.
template <int DQK, int DV, int MODE>
struct FwdStreamCfg : FwdCfg<DQK, DV, MODE> {
  using Base = FwdCfg<DQK, DV, MODE>;
  static constexpr int KSPLIT = Base::KVT ? 2 : 1;  // K tile loads come as K (, Kd) pairs
  static constexpr bool OK = Base::FITS && Base::NKI % Base::NW == 0 && Base::NVI % Base::NW == 0;
  static constexpr int KPW = Base::NKI / Base::NW, VPW = Base::NVI / Base::NW;
  static constexpr int LOADS = (KPW + VPW) * KSPLIT;  // vector-memory requests per wave per tile
  static constexpr int NOPA = 2 * Base::KS * KSPLIT;  // LDS operands of phase A
  static constexpr int NOPB = Base::DB * KSPLIT;      // LDS operands of phase B
};

template <typename T, int DQK, int DV, int MODE>
__global__ __launch_bounds__(512) void attn_fwd_stream_kernel(FwdParams p) {
  struct C : FwdStreamCfg<DQK, DV, MODE> {
    static constexpr float rescale_log2() { return RescaleSlack<T>::value; }
  };
  static_assert(C::OK, "shape not supported by the streamed kernel");
  constexpr int BN = C::BN, KS = C::KS, DB = C::DB, CK = C::CK, CV = C::CV;
  constexpr int KSPLIT = C::KSPLIT, NOPA = C::NOPA, NOPB = C::NOPB, NOP = NOPA + NOPB, PF = 4;
  __shared__ __attribute__((aligned(1024))) char stg0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char stg3[C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;

  const int nqt = (p.Lq + C::BM - 1) / C::BM;
  const int work = work_item(p.xcd_order);  // block order (common.h)
  const int bh = work / nqt, qt = work - bh * nqt;
  const int b = bh / p.H, h = bh - b * p.H;

  const char* qbase = (const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2;
  const char* kbase = (const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + DQK) * 2);
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + DQK) * 2);
  const uint32_t vt_bytes = (uint32_t)((int64_t)C::VT_ROWS * p.LKP * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qbase, q_bytes);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.vt + (int64_t)bh * vt_bytes, vt_bytes);
  __amdgpu_buffer_rsrc_t rtq = rq, rtk = rk, rtv = rv;
  if constexpr (C::JVP) rtq = make_rsrc((const char*)p.tq + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  if constexpr (C::KVT) {
    rtk = make_rsrc((const char*)p.tk + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
    rtv = make_rsrc((const char*)p.tvt + (int64_t)bh * vt_bytes, vt_bytes);
  }

  // ---- Q (and Qd) slices in registers: B operand of S^T = K Q^T
  const int qrow = qt * C::BM + wave * C::QW + col;
  const uint32_t qoff = (uint32_t)((int64_t)qrow * p.q_sl * 2) + grp * 16;
  i32x4_t qr[KS], tqr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qr[s] = buf_load16(rq, qoff + s * 64);
    if constexpr (C::JVP) tqr[s] = buf_load16(rtq, qoff + s * 64);
  }

  // ---- per-lane DMA offsets (tile independent)
  uint32_t koff[C::KPW], voff[C::VPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CK, phys = pch % CK;
    const int logical = phys ^ kswz16<CK>(row);
    koff[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < C::VPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CV, phys = pch % CV;
    const int logical = phys ^ swz4r(d & 15);
    voff[j] = (uint32_t)(d * p.LKP * 2) + logical * 16;
  }
  const uint32_t k_tile_step = (uint32_t)((int64_t)BN * p.k_sl * 2);

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
    if (li < C::KPW * KSPLIT) {
      const int jj = li / KSPLIT, i = wave + jj * C::NW;
      const uint32_t ks = (uint32_t)kt * k_tile_step;
      if (KSPLIT == 2 && (li & 1)) buf_load16_lds(rtk, st + C::OFF_KT + i * 1024, koff[jj], ks);
      else buf_load16_lds(rk, st + C::OFF_K + i * 1024, koff[jj], ks);
    } else {
      const int lv = li - C::KPW * KSPLIT, jj = lv / KSPLIT, i = wave + jj * C::NW;
      const uint32_t vs = (uint32_t)kt * BN * 2;
      if (KSPLIT == 2 && (lv & 1)) buf_load16_lds(rtv, st + C::OFF_VT + i * 1024, voff[jj], vs);
      else buf_load16_lds(rv, st + C::OFF_V + i * 1024, voff[jj], vs);
    }
  };

  // ---- LDS read offsets (tile independent): kx[2 s + sb] for K chunk s of
  // 16-key block sb, vx for V^T rows; stage, tile part and d block are immediates
  int kx[2 * KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int R = key_of_row16(sb, col);
      kx[2 * s + sb] = R * CK * 16 + (((4 * s + grp) ^ kswz16<CK>(R)) << 4);
    }
  }
  int vx = col * CV * 16 + ((grp ^ swz4r(col)) << 4);
  // Re-defines the offsets at each step (an empty asm), so that stage base +
  // offset is formed per step and folds into the LDS instructions' immediate
  // instead of being hoisted into one register per stage.
  auto pin_offsets = [&]() {
#pragma unroll
    for (int x = 0; x < 2 * KS; ++x) asm volatile("" : "+v"(kx[x]));
    asm volatile("" : "+v"(vx));
  };

  f32x4_t oacc[DB], cacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      oacc[d][v] = 0.f;
      cacc[d][v] = 0.f;
    }
  }
  float m_i = -__builtin_inff(), l_i = 0.f, r_i = 0.f;
  const int ntiles = (p.Lk + BN - 1) / BN;

  // LDS operand o of a step: o < NOPA reads a K (then Kd) chunk of the next
  // tile (s = k slice, sb = 16-key block), o >= NOPA a V^T (then Vd^T) block of this tile
  auto op_ptr = [&](const lds_char_t* s_next, const lds_char_t* s_cur, int o) -> lds_i32x4_t* {
    if (o < NOPA) {
      const int kd = o / (2 * KS), r = o % (2 * KS);
      return (lds_i32x4_t*)(s_next + (kd ? C::OFF_KT : C::OFF_K) + kx[r]);
    }
    const int ob = o - NOPA, vd = ob / DB, d = ob % DB;
    return (lds_i32x4_t*)(s_cur + (vd ? C::OFF_VT : C::OFF_V) + d * 16 * CV * 16 + vx);
  };
  const f32x4_t zero4 = {};
  // the MFMAs of operand o
  auto mfma_op = [&](int o, i32x4_t a, f32x4_t (&sc)[2], f32x4_t (&tc)[2], i32x4_t pk, i32x4_t hk) {
    if (o < NOPA) {
      const int kd = o / (2 * KS), r = o % (2 * KS), s = r >> 1, sb = r & 1;
      if (kd == 0) {
        sc[sb] = mfma16(a, qr[s], s == 0 ? zero4 : sc[sb], T());
        if constexpr (C::JVP) tc[sb] = mfma16(a, tqr[s], s == 0 ? zero4 : tc[sb], T());
      } else {
        tc[sb] = mfma16(a, qr[s], tc[sb], T());
      }
    } else {
      const int ob = o - NOPA, vd = ob / DB, d = ob % DB;
      if (vd == 0) {
        oacc[d] = mfma16(a, pk, oacc[d], T());
        if constexpr (C::JVP) cacc[d] = mfma16(a, hk, cacc[d], T());
      } else {
        cacc[d] = mfma16(a, pk, cacc[d], T());
      }
    }
  };

  // Online softmax of one tile split into 16 micro-steps (log2 domain; the 4
  // lane groups of a query share m). Leaves P~ and H~ packed as B operands
  // (keys 8*grp + e in pk, hk) and alpha, the accumulator rescale factor.
  struct Soft {
    float mx, alpha, neg_m, ls, rs;
    float pv[2], hv[2];
    bool moved;
  };
  auto soft_micro = [&](int u, Soft& sm, const f32x4_t (&sc)[2], const f32x4_t (&tc)[2], i32x4_t& pk,
                        i32x4_t& hk) {
    if (u == 0) {
      sm.mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                    fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
      sm.ls = 0.f;
      sm.rs = 0.f;
    } else if (u == 1) {
      sm.mx = fmaxf(sm.mx, other_row16(sm.mx));
    } else if (u == 2) {
      sm.mx = fmaxf(sm.mx, other_half(sm.mx)) * p.scale_log2;
      sm.moved = __builtin_amdgcn_ballot_w64(sm.mx > m_i + C::rescale_log2()) != 0;
      const float m_new = sm.moved ? fmaxf(m_i, sm.mx) : m_i;
      sm.alpha = fast_exp2(m_i - m_new);
      m_i = m_new;
      sm.neg_m = -exp_base<T>(m_new);
    } else if (u < 11) {
      const int e = u - 3, sb = e >> 2, v = e & 3;
      sm.pv[e & 1] = fast_exp2(fmaf(sc[sb][v], p.scale_log2, sm.neg_m));
      sm.ls += sm.pv[e & 1];
      if constexpr (C::JVP) {
        sm.hv[e & 1] = sm.pv[e & 1] * (tc[sb][v] * p.scale);
        sm.rs += sm.hv[e & 1];
      }
      if (e & 1) {
        pk[e >> 1] = (int)Elem<T>::pack2(sm.pv[0], sm.pv[1]);
        if constexpr (C::JVP) hk[e >> 1] = (int)Elem<T>::pack2(sm.hv[0], sm.hv[1]);
      }
    } else if (u < 15) {
    } else {
      l_i = l_i * sm.alpha + sm.ls;
      if constexpr (C::JVP) r_i = r_i * sm.alpha + sm.rs;
    }
  };
  auto rescale = [&](float alpha) {
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        oacc[d][v] *= alpha;
        if constexpr (C::JVP) cacc[d][v] *= alpha;
      }
    }
  };

  // step i (i + 1 < ntiles, i % 4 == kk): phase A on tile i+1's K, softmax of tile i (sc, tc);
  // phase B on tile i's V; requests tile i+3
  auto step = [&](auto kk, int i, const f32x4_t (&sc)[2], const f32x4_t (&tc)[2], f32x4_t (&sn)[2],
                  f32x4_t (&tn)[2]) {
    constexpr int k = decltype(kk)::value;
    ring_sync<C::LOADS>();  // tile i+1 has landed (tile i+2 may be in flight)
    pin_offsets();
    const lds_char_t* s_next = stage(IC<k + 1>{});
    const lds_char_t* s_cur = stage(IC<k>{});
    lds_char_t* s_req = stage(IC<k + 3>{});
    i32x4_t opr[PF];
#pragma unroll
    for (int o = 0; o < PF; ++o) opr[o] = *op_ptr(s_next, s_cur, o);
    Soft sm;
    i32x4_t pk, hk;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 0; o < NOPA; ++o) {
      mfma_op(o, opr[o % PF], sn, tn, pk, hk);
      if (o + PF < NOP) opr[o % PF] = *op_ptr(s_next, s_cur, o + PF);
#pragma unroll
      for (int u = o * 16 / NOPA; u < (o + 1) * 16 / NOPA; ++u) soft_micro(u, sm, sc, tc, pk, hk);
      __builtin_amdgcn_sched_barrier(0);
    }
    // keep the softmax in phase A: the values are used here, before the branch
    asm volatile("" : "+v"(pk), "+v"(hk), "+v"(l_i), "+v"(r_i));
    if (sm.moved) rescale(sm.alpha);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) {
      mfma_op(o, opr[o % PF], sn, tn, pk, hk);
      if (o + PF < NOP) opr[o % PF] = *op_ptr(s_next, s_cur, o + PF);
      if (o - NOPA < C::LOADS) issue_load(s_req, i + 3, o - NOPA);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // last tile (may hold keys >= Lk): masked softmax, rescale, PV
  auto last_step = [&](auto kk, int i, f32x4_t (&sc)[2], const f32x4_t (&tc)[2]) {
    const lds_char_t* s_cur = stage(kk);
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (i * BN + 8 * grp + 4 * sb + v >= p.Lk) sc[sb][v] = -__builtin_inff();
      }
    }
    Soft sm;
    i32x4_t pk, hk;
#pragma unroll
    for (int u = 0; u < 16; ++u) soft_micro(u, sm, sc, tc, pk, hk);
    rescale(sm.alpha);
    f32x4_t un_s[2], un_t[2];
#pragma unroll
    for (int o = NOPA; o < NOP; ++o) mfma_op(o, *op_ptr(s_cur, s_cur, o), un_s, un_t, pk, hk);
  };

  // ---- prologue: tiles 0..2 requested, scores of tile 0
#pragma unroll
  for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<0>{}), 0, li);
#pragma unroll
  for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<1>{}), 1, li);
#pragma unroll
  for (int li = 0; li < C::LOADS; ++li) issue_load(stage(IC<2>{}), 2, li);
  ring_sync<2 * C::LOADS>();  // Q slices and tile 0
  f32x4_t sa[2], ta[2], sb2[2], tb[2];
  {
    const lds_char_t* s0 = stage(IC<0>{});
    i32x4_t pk0 = {}, hk0 = {};
#pragma unroll
    for (int o = 0; o < NOPA; ++o) mfma_op(o, *op_ptr(s0, s0, o), sa, ta, pk0, hk0);
  }
  int i = 0;
  for (; i + 4 < ntiles; i += 4) {
    step(IC<0>{}, i, sa, ta, sb2, tb);
    step(IC<1>{}, i + 1, sb2, tb, sa, ta);
    step(IC<2>{}, i + 2, sa, ta, sb2, tb);
    step(IC<3>{}, i + 3, sb2, tb, sa, ta);
  }
  const int rest = ntiles - i;  // 1..4 tiles left
  if (rest >= 2) step(IC<0>{}, i, sa, ta, sb2, tb);
  if (rest >= 3) step(IC<1>{}, i + 1, sb2, tb, sa, ta);
  if (rest >= 4) step(IC<2>{}, i + 2, sa, ta, sb2, tb);
  if (rest == 1) last_step(IC<0>{}, i, sa, ta);
  else if (rest == 2) last_step(IC<1>{}, i + 1, sb2, tb);
  else if (rest == 3) last_step(IC<2>{}, i + 2, sa, ta);
  else last_step(IC<3>{}, i + 3, sb2, tb);
  wait_vmem();  // no requests beyond the last tile stay in flight

  // ---- epilogue: lane (query col, group g) holds d = 16*dblk + 4g + v
  float l = l_i + other_row16(l_i);
  l = l + other_half(l);
  const float inv_l = 1.0f / l;
  float mu = 0.f;
  if constexpr (C::JVP) {
    float r = r_i + other_row16(r_i);
    r = r + other_half(r);
    mu = r * inv_l;
  }
  const int64_t obase = b * p.o_sb + h * p.o_sh;
  const uint32_t o_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.o_sl + DV) * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc((char*)p.o + obase * 2, o_bytes);
  __amdgpu_buffer_rsrc_t rto = ro;
  if constexpr (C::JVP) rto = make_rsrc((char*)p.to + obase * 2, o_bytes);
  const uint32_t orow = (uint32_t)((int64_t)qrow * p.o_sl * 2);
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    const int dc = d * 16 + 4 * grp;
    float ov[4], tv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ov[v] = oacc[d][v] * inv_l;
      if constexpr (C::JVP) tv[v] = cacc[d][v] * inv_l - mu * ov[v];
    }
    const uint32_t off = orow + dc * 2;
    u32x2_t w = {Elem<T>::pack2(ov[0], ov[1]), Elem<T>::pack2(ov[2], ov[3])};
    buf_store8(ro, w, off);
    if constexpr (C::JVP) {
      u32x2_t wt = {Elem<T>::pack2(tv[0], tv[1]), Elem<T>::pack2(tv[2], tv[3])};
      buf_store8(rto, wt, off);
    }
  }
  if (grp == 0 && qrow < p.Lq) {
    const int64_t si = (int64_t)bh * p.Lq + qrow;
    p.lse[si] = (exp_base<T>(m_i) + __builtin_log2f(l)) * 0.6931471805599453f;
    if constexpr (C::JVP) p.mu[si] = mu;
  }
}

// Columns of V one workgroup of attn_fwd_simple_kernel handles: a 256-wide V
// in the JVP modes is split into two 128-column halves, each workgroup
// recomputing the scores (3 of the 6 GEMMs run twice), because O~ and C~ for
// all 256 columns next to Q, Qd and the score tiles spill registers (~650
// bytes per lane at Dqk = 256, 100-360 at the other Dqk).
constexpr int fwd_simple_dvc(int mode, int dv) { return (mode != kFwdPlain && dv == 256) ? 128 : dv; }

// Single-stage-per-tile variant for head dims whose four-stage ring does not
// fit in LDS (a 256-wide Q/K or V head in the full JVP mode): scores, softmax
// and PV of each 64- or 32-key tile run back to back.
template <int DQK, int DV, int MODE>
struct FwdSimpleCfg {
  static constexpr int NW = 4;
  static constexpr int BM = 32 * NW;
  static constexpr int DVP = DV < 32 ? 32 : DV;
  static constexpr int BN = (DQK > 128 || DVP > 128) ? 32 : 64;
  static constexpr int NB = BN / 32;  // 32-key blocks per tile
  static constexpr int KS = DQK / 16;  // 16-wide k slices of Q K^T
  static constexpr int DB = DVP / 32;  // 32-row blocks of O^T
  static constexpr int CK = DQK / 8;   // 16-byte chunks per K row
  static constexpr int CV = BN / 8;    // 16-byte chunks per V^T row
  static constexpr bool JVP = MODE != kFwdPlain;
  static constexpr bool KVT = MODE == kFwdJvp;
  static constexpr int K_BYTES = BN * DQK * 2;
  static constexpr int V_BYTES = DVP * BN * 2;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_V = K_BYTES;
  static constexpr int OFF_KT = K_BYTES + V_BYTES;
  static constexpr int OFF_VT = 2 * K_BYTES + V_BYTES;
  static constexpr int STAGE = (KVT ? 2 : 1) * (K_BYTES + V_BYTES);
  static constexpr int NKI = BN * CK / 64;   // wave-wide 1 KiB loads per K tile
  static constexpr int NVI = DVP * CV / 64;  // ... per V^T tile
  static constexpr int KPW = (NKI + NW - 1) / NW;
  static constexpr int VPW = (NVI + NW - 1) / NW;
};

// MAGI: the block-sparse variant for every head shape (the reference's
// `_attn_fwd_magi`, flash_attention_jvp_triton.py:242-409): one (query group,
// 128-query tile) task per workgroup, key tiles walking the group's ranges,
// keys outside the current range at -inf, only the group's rows stored.
template <typename T, int DQK, int DV, int MODE, bool MAGI = false>
__global__ __launch_bounds__(256) void attn_fwd_simple_kernel(FwdParams p) {
  constexpr int DVC = fwd_simple_dvc(MODE, DV);  // V columns of this workgroup
  constexpr int NCH = DV / DVC;                  // workgroups per query tile
  using C = FwdSimpleCfg<DQK, DVC, MODE>;
  constexpr int BN = C::BN, NB = C::NB, KS = C::KS, DB = C::DB, CK = C::CK, CV = C::CV;
  __shared__ __attribute__((aligned(1024))) char smem[2 * C::STAGE];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;

  int bh, qt, ntiles, chunk;
  int q_lo = 0, q_hi = p.Lq;         // rows this workgroup stores
  MagiCursor cm{0, 0, 0, 0, 0};      // MAGI: tile in use
  if constexpr (MAGI) {
    const int work = xcd_remap(blockIdx.x, p.T * p.B * p.H * NCH);
    chunk = work % NCH;
    const int w2 = work / NCH;
    bh = w2 / p.T;
    const MagiTask t = magi_task(p, w2 - bh * p.T, C::BM);
    qt = t.row0 / C::BM;
    q_lo = t.q_lo;
    q_hi = t.q_hi;
    ntiles = magi_ntiles(p, t, BN);
    if (ntiles == 0) {  // uniform over the workgroup: nothing requested yet
      if (chunk == 0) magi_store_empty<T, DV, C::JVP>(p, bh, t, C::BM);  // every column of the rows
      return;
    }
    cm = MagiCursor{t.r_beg, t.r_end, 0, 0, 0};
    cm.seek(p, BN);
  } else {
    const int nqt = (p.Lq + C::BM - 1) / C::BM;
    const int work = work_item(p.xcd_order);  // block order (common.h)
    chunk = work % NCH;
    const int w2 = work / NCH;
    bh = w2 / nqt;
    qt = w2 - bh * nqt;
    ntiles = (p.Lk + BN - 1) / BN;
  }
  MagiCursor ci = cm;  // MAGI: tile requested next
  const int b = bh / p.H, h = bh - b * p.H;

  const char* qbase = (const char*)p.q + (b * p.q_sb + h * p.q_sh) * 2;
  const char* kbase = (const char*)p.k + (b * p.k_sb + h * p.k_sh) * 2;
  const uint32_t q_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.q_sl + DQK) * 2);
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Lk - 1) * p.k_sl + DQK) * 2);
  // V^T copy [B*H][DV padded to 32][LKP]; this workgroup reads rows
  // [chunk * DVC, (chunk + 1) * DVC) of its head
  const int64_t vt_head = (int64_t)(DV < 32 ? 32 : DV) * p.LKP * 2;
  const uint32_t vt_bytes = (uint32_t)((int64_t)C::DVP * p.LKP * 2);
  const int64_t vt_off = (int64_t)bh * vt_head + (int64_t)chunk * DVC * p.LKP * 2;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qbase, q_bytes);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const char*)p.vt + vt_off, vt_bytes);
  __amdgpu_buffer_rsrc_t rtq = rq, rtk = rk, rtv = rv;
  if constexpr (C::JVP) rtq = make_rsrc((const char*)p.tq + (b * p.q_sb + h * p.q_sh) * 2, q_bytes);
  if constexpr (C::KVT) {
    rtk = make_rsrc((const char*)p.tk + (b * p.k_sb + h * p.k_sh) * 2, k_bytes);
    rtv = make_rsrc((const char*)p.tvt + vt_off, vt_bytes);
  }

  // ---- Q (and Qd) slices in registers: B operand of S^T = K Q^T
  const int qrow = qt * C::BM + wave * 32 + col;
  const uint32_t qoff = (uint32_t)((int64_t)qrow * p.q_sl * 2) + half * 16;
  i32x4_t qr[KS], tqr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qr[s] = buf_load16(rq, qoff + s * 32);
    if constexpr (C::JVP) tqr[s] = buf_load16(rtq, qoff + s * 32);
  }

  // ---- per-lane DMA offsets (tile independent)
  uint32_t koff[C::KPW], voff[C::VPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int row = pch / CK, phys = pch % CK;
    const int logical = phys ^ swz<CK>(perm32(row & 31) & 15);
    koff[j] = (uint32_t)((int64_t)row * p.k_sl * 2) + logical * 16;
  }
#pragma unroll
  for (int j = 0; j < C::VPW; ++j) {
    const int pch = (wave + j * C::NW) * 64 + lane;
    const int d = pch / CV, phys = pch % CV;
    const int logical = phys ^ swz<CV>(d & 15);
    voff[j] = (uint32_t)(d * p.LKP * 2) + logical * 16;
  }
  const uint32_t k_tile_step = (uint32_t)((int64_t)BN * p.k_sl * 2);

  // tile kt (MAGI: the tile whose first key row is kt) into stage `stage`
  auto issue_tile = [&](int kt, int stage) {
    char* st = smem + stage * C::STAGE;
    uint32_t ks, vs;
    if constexpr (MAGI) {
      ks = (uint32_t)kt * (uint32_t)(p.k_sl * 2);
      vs = (uint32_t)kt * 2;
    } else {
      ks = (uint32_t)kt * k_tile_step;
      vs = (uint32_t)kt * BN * 2;
    }
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NKI) {
        buf_load16_lds(rk, st + C::OFF_K + i * 1024, koff[j], ks);
        if constexpr (C::KVT) buf_load16_lds(rtk, st + C::OFF_KT + i * 1024, koff[j], ks);
      }
    }
#pragma unroll
    for (int j = 0; j < C::VPW; ++j) {
      const int i = wave + j * C::NW;
      if (i < C::NVI) {
        buf_load16_lds(rv, st + C::OFF_V + i * 1024, voff[j], vs);
        if constexpr (C::KVT) buf_load16_lds(rtv, st + C::OFF_VT + i * 1024, voff[j], vs);
      }
    }
  };

  // ---- LDS read offsets (tile independent)
  const int kswz = swz<CK>(col & 15), vswz = swz<CV>(col & 15);
  const int krow_off = perm32(col) * CK * 16;
  const int vrow_off = col * CV * 16;

  f32x16_t oacc[DB], cacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      oacc[d][v] = 0.f;
      cacc[d][v] = 0.f;
    }
  }
  float m_i = -__builtin_inff(), l_i = 0.f, r_i = 0.f;

  issue_tile(MAGI ? ci.start : 0, 0);
  for (int kt = 0; kt < ntiles; ++kt) {
    wait_vmem();
    __syncthreads();
    if constexpr (MAGI) ci.next(p, BN);
    if (kt + 1 < ntiles) issue_tile(MAGI ? ci.start : kt + 1, (kt + 1) & 1);
    const char* st = smem + (kt & 1) * C::STAGE;

    // ---- S^T and Sd^T for BN keys x 32 queries
    f32x16_t sacc[NB], tacc[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        sacc[kb][v] = 0.f;
        tacc[kb][v] = 0.f;
      }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
        const int off = kb * 32 * CK * 16 + krow_off + (((2 * s + half) ^ kswz) << 4);
        const i32x4_t ak = *(const i32x4_t*)(st + C::OFF_K + off);
        sacc[kb] = mfma32(ak, qr[s], sacc[kb], T());
        if constexpr (C::JVP) tacc[kb] = mfma32(ak, tqr[s], tacc[kb], T());
        if constexpr (C::KVT) {
          const i32x4_t akt = *(const i32x4_t*)(st + C::OFF_KT + off);
          tacc[kb] = mfma32(akt, qr[s], tacc[kb], T());
        }
      }
    }

    // ---- tail keys (MAGI: keys outside the current range) -> -inf
    if constexpr (MAGI) {
      if (cm.partial(BN)) {
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int j = v >> 2;
            const int key = cm.start + kb * 32 + ((j >> 1) << 4) + (half << 3) + ((j & 1) << 2) + (v & 3);
            if (cm.masked(key)) sacc[kb][v] = -__builtin_inff();
          }
        }
      }
      cm.next(p, BN);
    } else if ((kt + 1) * BN > p.Lk) {
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int j = v >> 2;
          const int key = kt * BN + kb * 32 + ((j >> 1) << 4) + (half << 3) + ((j & 1) << 2) + (v & 3);
          if (key >= p.Lk) sacc[kb][v] = -__builtin_inff();
        }
      }
    }

    // ---- online softmax (log2 domain); both halves of the wave share m
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[kb][v]);
    }
    mx = fmaxf(mx, other_half(mx));
    const float m_new = fmaxf(m_i, mx * p.scale_log2);
    const float alpha = fast_exp2(m_i - m_new);
    const float neg_m = -m_new;
    float ls = 0.f, rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float pv = fast_exp2(fmaf(sacc[kb][v], p.scale_log2, neg_m));
        sacc[kb][v] = pv;
        ls += pv;
        if constexpr (C::JVP) {
          const float hv = pv * (tacc[kb][v] * p.scale);
          tacc[kb][v] = hv;
          rs += hv;
        }
      }
    }
    l_i = l_i * alpha + ls;
    m_i = m_new;
    if constexpr (C::JVP) r_i = r_i * alpha + rs;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        oacc[d][v] *= alpha;
        if constexpr (C::JVP) cacc[d][v] *= alpha;
      }
    }

    // ---- O~^T += V^T P^T ; C~^T += Vd^T P^T + V^T H^T
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        i32x4_t pb, hb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pb[e] = (int)Elem<T>::pack2(sacc[kb][8 * t + 2 * e], sacc[kb][8 * t + 2 * e + 1]);
          if constexpr (C::JVP) hb[e] = (int)Elem<T>::pack2(tacc[kb][8 * t + 2 * e], tacc[kb][8 * t + 2 * e + 1]);
        }
        const int vch = ((kb * 4 + 2 * t + half) ^ vswz) << 4;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const int off = d * 32 * CV * 16 + vrow_off + vch;
          const i32x4_t av = *(const i32x4_t*)(st + C::OFF_V + off);
          oacc[d] = mfma32(av, pb, oacc[d], T());
          if constexpr (C::KVT) {
            const i32x4_t avt = *(const i32x4_t*)(st + C::OFF_VT + off);
            cacc[d] = mfma32(avt, pb, cacc[d], T());
          }
          if constexpr (C::JVP) cacc[d] = mfma32(av, hb, cacc[d], T());
        }
      }
    }
  }

  // ---- epilogue
  const float l = l_i + other_half(l_i);
  const float inv_l = 1.0f / l;
  float mu = 0.f;
  if constexpr (C::JVP) mu = (r_i + other_half(r_i)) * inv_l;

  const int64_t obase = b * p.o_sb + h * p.o_sh;
  const uint32_t o_bytes = (uint32_t)(((int64_t)(p.Lq - 1) * p.o_sl + DV) * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc((char*)p.o + obase * 2, o_bytes);
  __amdgpu_buffer_rsrc_t rto = ro;
  if constexpr (C::JVP) rto = make_rsrc((char*)p.to + obase * 2, o_bytes);
  // rows >= Lq fall outside the resource; MAGI stores only the group's rows
  const bool keep = !MAGI || (qrow >= q_lo && qrow < q_hi);
  const uint32_t orow = keep ? (uint32_t)((int64_t)qrow * p.o_sl * 2) : o_bytes;
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int dc = d * 32 + 8 * j + 4 * half;
      if (DVC >= 32 || dc < DVC) {
        float ov[4], tv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ov[r] = oacc[d][4 * j + r] * inv_l;
          if constexpr (C::JVP) tv[r] = cacc[d][4 * j + r] * inv_l - mu * ov[r];
        }
        const uint32_t off = orow + (chunk * DVC + dc) * 2;
        u32x2_t w = {Elem<T>::pack2(ov[0], ov[1]), Elem<T>::pack2(ov[2], ov[3])};
        buf_store8(ro, w, off);
        if constexpr (C::JVP) {
          u32x2_t wt = {Elem<T>::pack2(tv[0], tv[1]), Elem<T>::pack2(tv[2], tv[3])};
          buf_store8(rto, wt, off);
        }
      }
    }
  }
  if (half == 0 && qrow < p.Lq && keep && chunk == 0) {
    const int64_t si = (int64_t)bh * p.Lq + qrow;
    p.lse[si] = (m_i + __builtin_log2f(l)) * 0.6931471805599453f;
    if constexpr (C::JVP) p.mu[si] = mu;
  }
}

// Transpose X [B,H,L,D] (element strides sb, sh, sl; unit stride in D) ->
// Y [B*H][DP][LP] contiguous, zero where l >= L or d >= D.
struct TransposeParams {
  const void* x;
  void* y;
  int64_t sb, sh, sl;
  int H, L, D, LP, DP;
};

}  // namespace dmad
