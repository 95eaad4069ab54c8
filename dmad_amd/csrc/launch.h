// Launcher table shared by the per-(dtype, head-dim) instantiation units and
// the C ABI. Each unit is one compilation of fwd_inst.hip / bwd_inst.hip with
// DMAD_T and DMAD_D set, so the kernels build in parallel.
#pragma once
#include <hip/hip_runtime.h>
#include "attn_fwd.h"
#include "attn_fwd32.h"
#include "attn_fwd32_x2.h"
#include "attn_bwd.h"
#include "attn_bwd_dq.h"
#include "attn_bwd_full.h"
#include "attn_bwd_dq_sc.h"
#include "attn_f32.h"

namespace dmad {

typedef hipError_t (*FwdLaunchFn)(const FwdParams&, int grid, hipStream_t);

// Launcher for attn_fwd_kernel<T, DQK, DV, MODE>, or nullptr if (DV, MODE) is unsupported.
template <typename T, int DQK>
FwdLaunchFn fwd_select(int dv, int mode);

// Launcher for attn_fwd32_kernel<T, MODE> (128-wide heads; fwd32_inst.hip).
template <typename T>
FwdLaunchFn fwd32_select(int mode, int d);
template <> FwdLaunchFn fwd32_select<__bf16>(int, int);
template <> FwdLaunchFn fwd32_select<_Float16>(int, int);

// Two-workgroups-per-CU forward (attn_fwd32_x2_kernel; mode kFwdJvpQOnly,
// 128-wide heads): one workgroup per 128-query tile.
template <typename T>
FwdLaunchFn fwd32x2_select(int mode, int d);
template <> FwdLaunchFn fwd32x2_select<__bf16>(int, int);
template <> FwdLaunchFn fwd32x2_select<_Float16>(int, int);

// Block-sparse (MagiMask) forward launchers, JVP modes only; the grid is
// tasks * B * H workgroups of 256 threads, each task a 128-query tile.
template <typename T, int DQK>
FwdLaunchFn fwd_magi_select(int dv, int mode);
template <typename T>
FwdLaunchFn fwd32_magi_select(int mode, int d);
template <> FwdLaunchFn fwd32_magi_select<__bf16>(int, int);
template <> FwdLaunchFn fwd32_magi_select<_Float16>(int, int);
// Query rows per task of the block-sparse kernels.
constexpr int kMagiBlockM = 128;

// Generic bf16/fp16 forward kernels (the head-dim pairs attn_fwd32_kernel does
// not take): JVP modes with a 256-wide V run attn_fwd_simple_kernel on
// 128-column halves of V, two workgroups per 128-query tile, where the other
// kernels' registers would spill (Dqk = 16, 128, 256, and every block-sparse
// launch, which always runs attn_fwd_simple_kernel).
constexpr bool fwd_generic_uses_halves(int mode, int dqk, int dv, bool magi) {
  return mode != kFwdPlain && dv == 256 && (magi || dqk == 16 || dqk >= 128);
}
constexpr int fwd_generic_chunks(int mode, int dqk, int dv, bool magi) {
  return fwd_generic_uses_halves(mode, dqk, dv, magi) ? 2 : 1;
}

typedef hipError_t (*BwdLaunchFn)(const BwdParams&, int grid, hipStream_t);

// Launcher for attn_bwd_kernel<T, D, MODE>, or nullptr if unsupported.
template <typename T, int D>
BwdLaunchFn bwd_select(int mode);

typedef hipError_t (*DqLaunchFn)(const DqParams&, int grid, hipStream_t);

// Launcher for attn_bwd_dq_kernel<T, D, MODE>, or nullptr if unsupported.
template <typename T, int D>
DqLaunchFn dq_select(int mode);

// Launcher for the dO-only attn_bwd_kv_tr_kernel<T, D>, D = 64 or 128 (bwd_kv_inst.hip).
template <typename T, int D>
BwdLaunchFn kv_tr_select();
template <> BwdLaunchFn kv_tr_select<__bf16, 64>();
template <> BwdLaunchFn kv_tr_select<__bf16, 128>();
template <> BwdLaunchFn kv_tr_select<_Float16, 64>();
template <> BwdLaunchFn kv_tr_select<_Float16, 128>();

// Launcher for the dO-only attn_bwd_dq_tr_kernel<T, D>, D = 64, 128 or 256 (bwd_dq_inst.hip).
template <typename T, int D>
DqLaunchFn dq_tr_select();
template <> DqLaunchFn dq_tr_select<__bf16, 64>();
template <> DqLaunchFn dq_tr_select<__bf16, 128>();
template <> DqLaunchFn dq_tr_select<_Float16, 64>();
template <> DqLaunchFn dq_tr_select<_Float16, 128>();
template <> DqLaunchFn dq_tr_select<__bf16, 256>();
template <> DqLaunchFn dq_tr_select<_Float16, 256>();

// Full-derivative passes for 128-wide heads (bwd_full_inst.hip): the key pass
// (dK, dV) and the query pass (dQ, and dQd when tangent_grads).
template <typename T>
BwdLaunchFn kv_full_select();
template <> BwdLaunchFn kv_full_select<__bf16>();
template <> BwdLaunchFn kv_full_select<_Float16>();
template <typename T>
DqLaunchFn dq_full_select(bool tangent_grads);
template <> DqLaunchFn dq_full_select<__bf16>(bool);
template <> DqLaunchFn dq_full_select<_Float16>(bool);
// Head dims whose full derivative runs on those passes.
inline bool full_reads_rows(int d) { return d == 128; }

// Stored-score backward of 128-wide heads: the key pass that also writes dS
// (dO only: attn_bwd_kv_tr_kernel<T, 128, true>, bwd_kv_inst.hip) or dS, dSd
// (full derivative: attn_bwd_kv_full_kernel<T, 128, true>, bwd_full_inst.hip),
// and the query pass over them (attn_bwd_dq_sc_kernel<T, 1 | 2>).
template <typename T>
BwdLaunchFn kv_sc_dout_only();
template <> BwdLaunchFn kv_sc_dout_only<__bf16>();
template <> BwdLaunchFn kv_sc_dout_only<_Float16>();
template <typename T>
DqLaunchFn dq_sc_dout_only();
template <> DqLaunchFn dq_sc_dout_only<__bf16>();
template <> DqLaunchFn dq_sc_dout_only<_Float16>();
template <typename T>
BwdLaunchFn kv_sc_tangent();  // attn_bwd_kv_tr_kernel<T, 128, kScLoad>
template <> BwdLaunchFn kv_sc_tangent<__bf16>();
template <> BwdLaunchFn kv_sc_tangent<_Float16>();
template <typename T>
BwdLaunchFn kv_sc_select(bool full);
template <> BwdLaunchFn kv_sc_select<__bf16>(bool);
template <> BwdLaunchFn kv_sc_select<_Float16>(bool);
template <typename T>
DqLaunchFn dq_sc_select(bool full);
template <> DqLaunchFn dq_sc_select<__bf16>(bool);
template <> DqLaunchFn dq_sc_select<_Float16>(bool);

// Query tile of the dK/dV kernel, which fixes the layout of the backward
// statistics (the full-derivative kernel always uses 32-query tiles).
inline int bwd_bmq(int d, int mode) {
  if (mode == kBwdFull) return BwdCfg<128, kBwdFull>::BMQ;
  switch (d) {
    case 16: return dout_only_kv_bmq<16>();
    case 32: return dout_only_kv_bmq<32>();
    case 64: return dout_only_kv_bmq<64>();
    case 128: return dout_only_kv_bmq<128>();
    default: return dout_only_kv_bmq<256>();
  }
}

// True when the dO-only dK/dV pass for head dim d reads Q, dO row-major
// (transposing on the LDS read), so it needs no transposed copies of them.
inline bool kv_dout_only_reads_rows(int d) {
  switch (d) {
    case 16: return KvTrCfg<16, kKvTrBmq>::FITS;
    case 32: return KvTrCfg<32, kKvTrBmq>::FITS;
    case 64: return KvTrCfg<64, kKvTrBmq>::FITS;
    case 128: return KvTrCfg<128, kKvTrBmq>::FITS;
    default: return KvTrCfg<256, kKvTrBmq>::FITS;
  }
}
// The same for the dQ pass and K.
inline bool dq_dout_only_reads_rows(int d) {
  switch (d) {
    case 16: return DqTrCfg<16>::FITS;
    case 32: return DqTrCfg<32>::FITS;
    case 64: return DqTrCfg<64>::FITS;
    case 128: return DqTrCfg<128>::FITS;
    default: return DqTrCfg<256>::FITS;
  }
}

// fp32 operands (attn_f32.h; f32_inst.hip, one compilation per head dim).
// Forward launcher for (Dqk, Dv, mode), dense or block-sparse, or nullptr; the
// grid is (f32_fwd_bm-query tiles, or tasks * kMagiBlockM / f32_fwd_bm) * B * H * f32_fwd_chunks(mode, Dqk, Dv)
// workgroups.
template <int DQK>
FwdLaunchFn f32_fwd_select(int dv, int mode, bool magi);
template <> FwdLaunchFn f32_fwd_select<16>(int, int, bool);
template <> FwdLaunchFn f32_fwd_select<32>(int, int, bool);
template <> FwdLaunchFn f32_fwd_select<64>(int, int, bool);
template <> FwdLaunchFn f32_fwd_select<128>(int, int, bool);
template <> FwdLaunchFn f32_fwd_select<256>(int, int, bool);
// V columns per workgroup: 128 in the JVP modes, all of V with 256-wide Q, K
// (one wave per SIMD, f32_fwd_wide); the plain forward takes up to 256 columns
// at every Q, K width
constexpr int f32_fwd_chunks(int mode, int dqk, int dv) {
  const int dvc = f32_fwd_wide(mode, dqk) || mode == kFwdPlain ? 256 : 128;
  return dv > dvc ? dv / dvc : 1;
}
// Query rows per workgroup of the fp32 forward (a block-sparse task's 128 rows
// take kMagiBlockM / f32_fwd_bm workgroups)
constexpr int f32_fwd_bm(int mode, int dqk) { return f32_fwd_wide(mode, dqk) ? 64 : 128; }
// dO-only backward: statistics, key pass, query pass (each sizes its own grid).
struct F32BwdFns {
  hipError_t (*prep)(const F32PrepParams&, hipStream_t);
  hipError_t (*kv)(const BwdParams&, const float* lse2, const float* dd, hipStream_t);
  hipError_t (*dq)(const DqParams&, const float* lse2, const float* dd, hipStream_t);
};
template <int D>
F32BwdFns f32_bwd_select();
template <> F32BwdFns f32_bwd_select<16>();
template <> F32BwdFns f32_bwd_select<32>();
template <> F32BwdFns f32_bwd_select<64>();
template <> F32BwdFns f32_bwd_select<128>();
template <> F32BwdFns f32_bwd_select<256>();

// Fused RMSNorm(+tangent) + interleaved RoPE prologue (prologue.hip).
constexpr int kPrologueMaxChunks = 20;  // 16-byte chunks per lane: C <= 64 * 8 * 20
struct PrologueParams {
  const void* y;      // [rows, C] (row stride y_stride elements)
  const void* ty;     // tangent, same strides; null for the primal only
  const void* w;      // [C] weight; null skips the norm (rotation only)
  const float* freqs;  // [L, D/2] angles; null skips the rotation
  void* out;          // [rows, C] (row stride o_stride)
  void* tout;         // tangent output; null iff ty is null
  int64_t rows, y_stride, o_stride;
  int L, C, D;
  float eps, inv_c;
};
hipError_t launch_rmsnorm_rope(const PrologueParams& p, int dtype, hipStream_t s);

hipError_t launch_transpose_pad(const TransposeParams& p, int BH, hipStream_t s);
// MFMA ceiling probe (probe.hip): `blocks` workgroups of 4 waves, each wave 256 * rounds
// back-to-back 32x32x16 MFMAs (bf16, or fp16 when f16).
hipError_t launch_mfma_probe(bool f16, int blocks, int rounds, float* sink, hipStream_t s);
hipError_t launch_bwd_prep(const PrepParams& p, int dtype, hipStream_t s);

// ---------------------------------------------------------------- kernel choice per shape
// The generic forward kernels (transposed V) by (Dqk, Dv, mode): fwd_inst.hip
// launches, and the launch-plan query names, the kernel this returns.
enum class GenericFwd { kSimple, kStream, kTiled };
template <int DQK, int DV, int MODE>
constexpr GenericFwd generic_fwd_kind() {
  // registers spill on the other kernels for these (the JVP modes with a
  // 256-wide V, and the K, V tangent-free mode with 256-wide Q, K and 128-wide V)
  if constexpr (fwd_generic_uses_halves(MODE, DQK, DV, false) || (MODE == kFwdJvpQOnly && DQK == 256 && DV == 128))
    return GenericFwd::kSimple;
  else if constexpr (FwdStreamCfg<DQK, DV, MODE>::OK) return GenericFwd::kStream;
  else if constexpr (FwdCfg<DQK, DV, MODE>::FITS) return GenericFwd::kTiled;
  else return GenericFwd::kSimple;
}
template <int DQK, int DV>
inline GenericFwd generic_fwd_kind_of_mode(int mode) {
  return mode == kFwdPlain ? generic_fwd_kind<DQK, DV, kFwdPlain>()
         : mode == kFwdJvp ? generic_fwd_kind<DQK, DV, kFwdJvp>()
                           : generic_fwd_kind<DQK, DV, kFwdJvpQOnly>();
}
template <int DQK>
inline GenericFwd generic_fwd_kind_of(int dv, int mode) {
  switch (dv) {
    case 16: return generic_fwd_kind_of_mode<DQK, 16>(mode);
    case 32: return generic_fwd_kind_of_mode<DQK, 32>(mode);
    case 64: return generic_fwd_kind_of_mode<DQK, 64>(mode);
    case 128: return generic_fwd_kind_of_mode<DQK, 128>(mode);
    default: return generic_fwd_kind_of_mode<DQK, 256>(mode);
  }
}
inline const char* generic_fwd_name(int dqk, int dv, int mode) {
  GenericFwd k = GenericFwd::kSimple;
  switch (dqk) {
    case 16: k = generic_fwd_kind_of<16>(dv, mode); break;
    case 32: k = generic_fwd_kind_of<32>(dv, mode); break;
    case 64: k = generic_fwd_kind_of<64>(dv, mode); break;
    case 128: k = generic_fwd_kind_of<128>(dv, mode); break;
    default: k = generic_fwd_kind_of<256>(dv, mode); break;
  }
  return k == GenericFwd::kStream ? "attn_fwd_stream_kernel" : k == GenericFwd::kTiled ? "attn_fwd_kernel"
                                                                                       : "attn_fwd_simple_kernel";
}

// Keys (queries) per workgroup of the fp32 dK/dV (dQ) pass for head dim d.
inline int f32_kv_block(int d) {
  switch (d) {
    case 16: return F32KvCfg<16>::BK;
    case 32: return F32KvCfg<32>::BK;
    case 64: return F32KvCfg<64>::BK;
    case 128: return F32KvCfg<128>::BK;
    default: return F32KvCfg<256>::BK;
  }
}
inline int f32_dq_block(int d) {
  switch (d) {
    case 16: return F32DqCfg<16>::BM;
    case 32: return F32DqCfg<32>::BM;
    case 64: return F32DqCfg<64>::BM;
    case 128: return F32DqCfg<128>::BM;
    default: return F32DqCfg<256>::BM;
  }
}

// The dO-only backward passes by head dim: bwd_inst.hip launches, and the
// launch-plan query names, these kernels.
template <int D>
constexpr bool kv_dout_only_rows() { return KvTrCfg<D, kKvTrBmq>::FITS; }
template <int D>
constexpr bool kv_dout_only_pipe() { return !kv_dout_only_rows<D>() && KvPipeCfg<D, kv_pipe_bmq<D>()>::FITS; }
template <int D>
constexpr bool dq_dout_only_rows() { return DqTrCfg<D>::FITS; }
template <int D>
constexpr bool dq_dout_only_pipe() { return !dq_dout_only_rows<D>() && DqPipeCfg<D>::FITS; }
template <int D>
inline const char* kv_dout_only_name_of() {
  return kv_dout_only_rows<D>() ? "attn_bwd_kv_tr_kernel" : kv_dout_only_pipe<D>() ? "attn_bwd_kv_pipe_kernel" : "attn_bwd_kernel";
}
template <int D>
inline const char* dq_dout_only_name_of() {
  return dq_dout_only_rows<D>() ? "attn_bwd_dq_tr_kernel" : dq_dout_only_pipe<D>() ? "attn_bwd_dq_pipe_kernel"
                                                                                   : "attn_bwd_dq_kernel";
}
inline const char* kv_dout_only_name(int d) {
  switch (d) {
    case 16: return kv_dout_only_name_of<16>();
    case 32: return kv_dout_only_name_of<32>();
    case 64: return kv_dout_only_name_of<64>();
    case 128: return kv_dout_only_name_of<128>();
    default: return kv_dout_only_name_of<256>();
  }
}
inline const char* dq_dout_only_name(int d) {
  switch (d) {
    case 16: return dq_dout_only_name_of<16>();
    case 32: return dq_dout_only_name_of<32>();
    case 64: return dq_dout_only_name_of<64>();
    case 128: return dq_dout_only_name_of<128>();
    default: return dq_dout_only_name_of<256>();
  }
}

}  // namespace dmad
