// C ABI entry points (include/dmad_attn.h): argument validation, workspace
// carving and kernel dispatch. Nothing here allocates device memory; the
// allocation-free backward uses this file's static device array `scratch`.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "dmad_attn.h"
#include "launch.h"

namespace dmad {
// explicit specialisations live in the fwd_inst.hip compilations
template <> FwdLaunchFn fwd_select<__bf16, 16>(int, int);
template <> FwdLaunchFn fwd_select<__bf16, 32>(int, int);
template <> FwdLaunchFn fwd_select<__bf16, 64>(int, int);
template <> FwdLaunchFn fwd_select<__bf16, 128>(int, int);
template <> FwdLaunchFn fwd_select<__bf16, 256>(int, int);
template <> FwdLaunchFn fwd_select<_Float16, 16>(int, int);
template <> FwdLaunchFn fwd_select<_Float16, 32>(int, int);
template <> FwdLaunchFn fwd_select<_Float16, 64>(int, int);
template <> FwdLaunchFn fwd_select<_Float16, 128>(int, int);
template <> FwdLaunchFn fwd_select<_Float16, 256>(int, int);
template <> BwdLaunchFn bwd_select<__bf16, 16>(int);
template <> BwdLaunchFn bwd_select<__bf16, 32>(int);
template <> BwdLaunchFn bwd_select<__bf16, 64>(int);
template <> BwdLaunchFn bwd_select<__bf16, 128>(int);
template <> BwdLaunchFn bwd_select<__bf16, 256>(int);
template <> BwdLaunchFn bwd_select<_Float16, 16>(int);
template <> BwdLaunchFn bwd_select<_Float16, 32>(int);
template <> BwdLaunchFn bwd_select<_Float16, 64>(int);
template <> BwdLaunchFn bwd_select<_Float16, 128>(int);
template <> BwdLaunchFn bwd_select<_Float16, 256>(int);
template <> DqLaunchFn dq_select<__bf16, 16>(int);
template <> DqLaunchFn dq_select<__bf16, 32>(int);
template <> DqLaunchFn dq_select<__bf16, 64>(int);
template <> DqLaunchFn dq_select<__bf16, 128>(int);
template <> DqLaunchFn dq_select<__bf16, 256>(int);
template <> DqLaunchFn dq_select<_Float16, 16>(int);
template <> DqLaunchFn dq_select<_Float16, 32>(int);
template <> DqLaunchFn dq_select<_Float16, 64>(int);
template <> DqLaunchFn dq_select<_Float16, 128>(int);
template <> DqLaunchFn dq_select<_Float16, 256>(int);
template <> FwdLaunchFn fwd_magi_select<__bf16, 16>(int, int);
template <> FwdLaunchFn fwd_magi_select<__bf16, 32>(int, int);
template <> FwdLaunchFn fwd_magi_select<__bf16, 64>(int, int);
template <> FwdLaunchFn fwd_magi_select<__bf16, 128>(int, int);
template <> FwdLaunchFn fwd_magi_select<__bf16, 256>(int, int);
template <> FwdLaunchFn fwd_magi_select<_Float16, 16>(int, int);
template <> FwdLaunchFn fwd_magi_select<_Float16, 32>(int, int);
template <> FwdLaunchFn fwd_magi_select<_Float16, 64>(int, int);
template <> FwdLaunchFn fwd_magi_select<_Float16, 128>(int, int);
template <> FwdLaunchFn fwd_magi_select<_Float16, 256>(int, int);
}  // namespace dmad

namespace {

thread_local std::string g_last_error;
constexpr int kMaxEvents = 256;
thread_local hipEvent_t g_events[kMaxEvents];
thread_local int g_nevents = 0;

// Records the before (after == false) or after event of main kernel `i`.
void mark(int i, bool after, hipStream_t s) {
  const int e = 2 * i + (after ? 1 : 0);
  if (e < g_nevents && g_events[e] != nullptr) (void)hipEventRecord(g_events[e], s);
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return DMAD_OK;
}

bool head_dim_ok(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

constexpr int64_t kMaxHeadBytes = (int64_t)1 << 31;  // buffer offsets are 32-bit
constexpr int64_t kLkAlign = 64;                       // key padding of transposed copies

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Checks one [B,H,L,D] operand of `esz`-byte elements: pointer, unit inner
// stride, 16-byte alignment of every row start, and that one (b, h) slice fits
// 32-bit byte offsets (with 256 rows of slack for tile overrun).
int check_operand(const char* name, const void* ptr, const int64_t* st, int64_t L, int64_t D, int esz = 2) {
  if (ptr == nullptr) return fail(DMAD_ERR_INVALID, "%s: null pointer", name);
  if (st == nullptr) return fail(DMAD_ERR_INVALID, "%s: null strides", name);
  if (st[3] != 1) return fail(DMAD_ERR_INVALID, "%s: stride of the head dim must be 1, got %lld", name, (long long)st[3]);
  const int align = 16 / esz;
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0) return fail(DMAD_ERR_INVALID, "%s: negative stride %lld", name, (long long)st[i]);
    if (st[i] % align != 0)
      return fail(DMAD_ERR_INVALID, "%s: strides must be multiples of %d elements (16 bytes), got %lld", name, align,
                  (long long)st[i]);
  }
  if (L > 1 && st[2] < D) return fail(DMAD_ERR_INVALID, "%s: rows overlap (stride %lld < D %lld)", name, (long long)st[2], (long long)D);
  if (((uintptr_t)ptr & 15) != 0) return fail(DMAD_ERR_INVALID, "%s: base pointer must be 16-byte aligned", name);
  if (((L + 256) * st[2] + D) * esz >= kMaxHeadBytes)
    return fail(DMAD_ERR_UNSUPPORTED, "%s: one (batch, head) slice spans more than 2 GiB", name);
  return DMAD_OK;
}

int elem_size(int dtype) { return dtype == DMAD_F32 ? 4 : 2; }

dmad::FwdLaunchFn pick_fwd_f32(int64_t dqk, int64_t dv, int mode, bool magi) {
  using namespace dmad;
  switch (dqk) {
    case 16: return f32_fwd_select<16>((int)dv, mode, magi);
    case 32: return f32_fwd_select<32>((int)dv, mode, magi);
    case 64: return f32_fwd_select<64>((int)dv, mode, magi);
    case 128: return f32_fwd_select<128>((int)dv, mode, magi);
    case 256: return f32_fwd_select<256>((int)dv, mode, magi);
  }
  return nullptr;
}

dmad::F32BwdFns pick_bwd_f32(int64_t d) {
  using namespace dmad;
  switch (d) {
    case 16: return f32_bwd_select<16>();
    case 32: return f32_bwd_select<32>();
    case 64: return f32_bwd_select<64>();
    case 128: return f32_bwd_select<128>();
    case 256: return f32_bwd_select<256>();
  }
  return F32BwdFns{};
}

// Bytes of the transposed, key-padded V (and Vd) copies the generic forward
// kernels read. The row-reading kernel serves every bf16/fp16 forward of 64-
// and 128-wide heads and of Dqk = Dv = 256 heads, dense and block-sparse, and
// reads V in place: those need no workspace (plan_fwd gives one launch's size).
int64_t fwd_ws_bytes(int mode, int64_t B, int64_t H, int64_t Lk, int64_t Dqk, int64_t Dv) {
  if (dmad::fwd32_supported((int)Dqk, (int)Dv) || dmad::fwd32_wide_supported((int)Dqk, (int)Dv)) return 0;
  const int64_t dvp = Dv < 32 ? 32 : Dv;
  const int64_t one = B * H * dvp * round_up(Lk, kLkAlign) * 2;
  return round_up(one, 256) * (mode == DMAD_FWD_JVP ? 2 : 1);
}

dmad::FwdLaunchFn pick_fwd(int dtype, int64_t dqk, int64_t dv, int mode) {
  using namespace dmad;
  if (dtype == DMAD_BF16) {
    switch (dqk) {
      case 16: return fwd_select<__bf16, 16>((int)dv, mode);
      case 32: return fwd_select<__bf16, 32>((int)dv, mode);
      case 64: return fwd_select<__bf16, 64>((int)dv, mode);
      case 128: return fwd_select<__bf16, 128>((int)dv, mode);
      case 256: return fwd_select<__bf16, 256>((int)dv, mode);
    }
  } else if (dtype == DMAD_F16) {
    switch (dqk) {
      case 16: return fwd_select<_Float16, 16>((int)dv, mode);
      case 32: return fwd_select<_Float16, 32>((int)dv, mode);
      case 64: return fwd_select<_Float16, 64>((int)dv, mode);
      case 128: return fwd_select<_Float16, 128>((int)dv, mode);
      case 256: return fwd_select<_Float16, 256>((int)dv, mode);
    }
  }
  return nullptr;
}

dmad::FwdLaunchFn pick_fwd_magi(int dtype, int64_t dqk, int64_t dv, int mode) {
  using namespace dmad;
  if (dtype == DMAD_BF16) {
    switch (dqk) {
      case 16: return fwd_magi_select<__bf16, 16>((int)dv, mode);
      case 32: return fwd_magi_select<__bf16, 32>((int)dv, mode);
      case 64: return fwd_magi_select<__bf16, 64>((int)dv, mode);
      case 128: return fwd_magi_select<__bf16, 128>((int)dv, mode);
      case 256: return fwd_magi_select<__bf16, 256>((int)dv, mode);
    }
  } else if (dtype == DMAD_F16) {
    switch (dqk) {
      case 16: return fwd_magi_select<_Float16, 16>((int)dv, mode);
      case 32: return fwd_magi_select<_Float16, 32>((int)dv, mode);
      case 64: return fwd_magi_select<_Float16, 64>((int)dv, mode);
      case 128: return fwd_magi_select<_Float16, 128>((int)dv, mode);
      case 256: return fwd_magi_select<_Float16, 256>((int)dv, mode);
    }
  }
  return nullptr;
}

dmad::FwdLaunchFn pick_fwd32x2(int dtype, int64_t d, int mode) {
  if (dtype == DMAD_BF16) return dmad::fwd32x2_select<__bf16>(mode, (int)d);
  if (dtype == DMAD_F16) return dmad::fwd32x2_select<_Float16>(mode, (int)d);
  return nullptr;
}

// Key-tile counts (32 keys each) up to which the K, V tangent-free forward of
// 128-wide heads runs on attn_fwd32_x2_kernel: measured at H=40, Lq=32760,
// 17-18% faster than the one-workgroup-per-CU kernels at 128-256 keys, 7-8% at
// 512-1024, 3% at 2048; 1-2% slower at 4096-8192 keys.
constexpr int64_t kX2MaxKeyTiles = 64;

// ---------------------------------------------------------------- launch plans
// The fixed per-shape table that stands in for the reference's Triton
// autotuning (configs over BLOCK_M, BLOCK_N, stages and warps keyed on
// SEQ_LEN_Q, SEQ_LEN_KV, HEAD_DIM_QK, HEAD_DIM_V:
// train/wan/rcm/utils/flash_attention_jvp_triton.py:98-107). Its keys are the
// dtype, the mode, the mask, Lq (query tiles per head), Lk (key tiles) and the
// head dims; the entry points launch what it says, and dmad_attn_fwd_plan /
// dmad_attn_bwd_plan report it. Inputs are validated by the callers.
enum class FwdFamily { kRows, kRowsX2, kGeneric, kF32 };
struct FwdPlan {
  FwdFamily family;
  const char* kernel;
  int64_t grid, chunks;
  int xcd_order, copies;
  int64_t ws;
};

// magi_tasks < 0: dense; otherwise the block-sparse forward with that many tasks
FwdPlan plan_fwd(int dtype, int mode, int64_t magi_tasks, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk,
                 int64_t Dv) {
  const bool magi = magi_tasks >= 0;
  FwdPlan pl{};
  int64_t bm = 128;  // query rows per workgroup (a block-sparse task is 128 rows)
  if (dtype == DMAD_F32) {
    // fp32 operands: fp32-MFMA kernels, V in column chunks for wide heads
    pl.family = FwdFamily::kF32;
    pl.kernel = "attn_f32_fwd_kernel";
    pl.chunks = dmad::f32_fwd_chunks(mode, (int)Dqk, (int)Dv);
    bm = dmad::f32_fwd_bm(mode, (int)Dqk);
  } else if (!magi && dmad::fwd32x2_supported(mode, (int)Dqk, (int)Dv) && (Lk + 31) / 32 <= kX2MaxKeyTiles) {
    // short key sequences with Kd = Vd = 0 (the text cross-attention): two workgroups per CU
    pl.family = FwdFamily::kRowsX2;
    pl.kernel = "attn_fwd32_x2_kernel";
    pl.chunks = 1;
  } else if (dmad::fwd32_supported((int)Dqk, (int)Dv)) {
    // 64- and 128-wide heads: 32-query waves reading K, V row-major
    pl.family = FwdFamily::kRows;
    pl.kernel = "attn_fwd32_kernel";
    pl.chunks = 1;
  } else if (dmad::fwd32_wide_supported((int)Dqk, (int)Dv)) {
    // 256-wide heads: the same kernel; the JVP modes run one workgroup per 128-column chunk of V
    // (per query tile, or per block-sparse task)
    pl.family = FwdFamily::kRows;
    pl.kernel = "attn_fwd32_kernel";
    pl.chunks = dmad::fwd32_chunks(mode, 256);
  } else {
    // the other head dims: generic kernels on transposed copies of V (and Vd)
    pl.family = FwdFamily::kGeneric;
    pl.kernel = magi ? "attn_fwd_simple_kernel" : dmad::generic_fwd_name((int)Dqk, (int)Dv, mode);
    pl.chunks = dmad::fwd_generic_chunks(mode, (int)Dqk, (int)Dv, magi);
    pl.copies = mode == DMAD_FWD_JVP ? 2 : 1;
  }
  const int64_t units = magi ? magi_tasks * (dmad::kMagiBlockM / bm) : (Lq + bm - 1) / bm;  // query tiles
  pl.grid = units * B * H * pl.chunks;
  // block order (common.h): the block-sparse kernels always deal contiguous work items per XCD
  pl.xcd_order = magi ? 1 : units < dmad::kHeadMajorMinTiles;
  // the row-reading kernels read V in place; the generic ones need the copies
  pl.ws = pl.family == FwdFamily::kGeneric ? fwd_ws_bytes(mode, B, H, Lk, Dqk, Dv) : 0;
  return pl;
}

// Block-sparse tables of dmad_attn_jvp_fwd_magi (device pointers).
struct MagiArgs {
  const int32_t *q_ranges, *k_ranges, *qk_map, *task_group, *task_qtile;
  int64_t G, R, T;
};

dmad::BwdLaunchFn pick_bwd(int dtype, int64_t d, int mode) {
  using namespace dmad;
  if (dtype == DMAD_BF16) {
    switch (d) {
      case 16: return bwd_select<__bf16, 16>(mode);
      case 32: return bwd_select<__bf16, 32>(mode);
      case 64: return bwd_select<__bf16, 64>(mode);
      case 128: return bwd_select<__bf16, 128>(mode);
      case 256: return bwd_select<__bf16, 256>(mode);
    }
  } else if (dtype == DMAD_F16) {
    switch (d) {
      case 16: return bwd_select<_Float16, 16>(mode);
      case 32: return bwd_select<_Float16, 32>(mode);
      case 64: return bwd_select<_Float16, 64>(mode);
      case 128: return bwd_select<_Float16, 128>(mode);
      case 256: return bwd_select<_Float16, 256>(mode);
    }
  }
  return nullptr;
}

dmad::BwdLaunchFn pick_kv_full(int dtype) {
  if (dtype == DMAD_BF16) return dmad::kv_full_select<__bf16>();
  if (dtype == DMAD_F16) return dmad::kv_full_select<_Float16>();
  return nullptr;
}

dmad::DqLaunchFn pick_dq_full(int dtype, bool tangent_grads) {
  if (dtype == DMAD_BF16) return dmad::dq_full_select<__bf16>(tangent_grads);
  if (dtype == DMAD_F16) return dmad::dq_full_select<_Float16>(tangent_grads);
  return nullptr;
}

dmad::BwdLaunchFn pick_kv_sc(int dtype, bool full) {
  if (dtype == DMAD_BF16) return dmad::kv_sc_select<__bf16>(full);
  if (dtype == DMAD_F16) return dmad::kv_sc_select<_Float16>(full);
  return nullptr;
}

dmad::BwdLaunchFn pick_kv_sc_tangent(int dtype) {
  if (dtype == DMAD_BF16) return dmad::kv_sc_tangent<__bf16>();
  if (dtype == DMAD_F16) return dmad::kv_sc_tangent<_Float16>();
  return nullptr;
}

dmad::DqLaunchFn pick_dq_sc(int dtype, bool full) {
  if (dtype == DMAD_BF16) return dmad::dq_sc_select<__bf16>(full);
  if (dtype == DMAD_F16) return dmad::dq_sc_select<_Float16>(full);
  return nullptr;
}

dmad::DqLaunchFn pick_dq(int dtype, int64_t d, int mode) {
  using namespace dmad;
  if (dtype == DMAD_BF16) {
    switch (d) {
      case 16: return dq_select<__bf16, 16>(mode);
      case 32: return dq_select<__bf16, 32>(mode);
      case 64: return dq_select<__bf16, 64>(mode);
      case 128: return dq_select<__bf16, 128>(mode);
      case 256: return dq_select<__bf16, 256>(mode);
    }
  } else if (dtype == DMAD_F16) {
    switch (d) {
      case 16: return dq_select<_Float16, 16>(mode);
      case 32: return dq_select<_Float16, 32>(mode);
      case 64: return dq_select<_Float16, 64>(mode);
      case 128: return dq_select<_Float16, 128>(mode);
      case 256: return dq_select<_Float16, 256>(mode);
    }
  }
  return nullptr;
}

// Backward workspace, carved in this order (each piece 256-byte aligned):
//   transposed Q, dO [, Qd, dOd]   [BH][DP][LQP] each (input dtype)
//   transposed K [, Kd]            [BH][DP][LKP] each
//   statistics (A or B layout) [, BT layout]   float32
struct BwdWs {
  int64_t trq, trk, stats, stats_bt, total;
  int nq, nk;
  bool tgrad;
};

BwdWs bwd_ws(int full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D) {
  const int64_t BH = B * H, dp = D < 32 ? 32 : D, lqp = round_up(Lq, 64), lkp = round_up(Lk, kLkAlign);
  BwdWs w{};
  // transposed copies of Q, dO (and Qd, dOd) and K (and Kd): the full derivative
  // and the dO-only passes of the head dims whose kernels read transposed copies
  // (Q, dO for the dK/dV pass, K for the dQ pass)
  if (full != 0) {
    const bool copies = !dmad::full_reads_rows((int)D);
    w.nq = copies ? 4 : 0;
    w.nk = copies ? 2 : 0;
  } else {
    w.nq = dmad::kv_dout_only_reads_rows((int)D) ? 0 : 2;
    w.nk = dmad::dq_dout_only_reads_rows((int)D) ? 0 : 1;
  }
  w.tgrad = full == 2;
  w.trq = round_up(BH * dp * lqp * 2, 256);
  w.trk = round_up(BH * dp * lkp * 2, 256);
  w.stats = round_up(BH * lqp * (full ? 4 : 2) * 4, 256);
  w.stats_bt = w.tgrad ? round_up(BH * lqp * 2 * 4, 256) : 0;
  w.total = w.nq * w.trq + w.nk * w.trk + w.stats + w.stats_bt;
  return w;
}

// Workspace of a backward with operands of the given dtype. The fp32 passes
// (dO only) make no transposed copies and keep only the log2 LSE and D
// statistics, [BH][LQP] floats each.
BwdWs bwd_ws_of(int dtype, int full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D) {
  if (dtype != DMAD_F32) return bwd_ws(full, B, H, Lq, Lk, D);
  BwdWs w{};
  w.stats = round_up(B * H * round_up(Lq, 64) * 2 * 4, 256);
  w.total = w.stats;
  return w;
}

// Stored score gradients (attn_bwd_dq_sc.h): bf16/fp16 operands of 128-wide
// heads. Bytes per (b, h) slice: dS (and dSd for the full derivative) over Lq
// rounded up to 128 queries and the key pass's 128-key tiles, bf16/fp16.
bool score_store_ok(int dtype, int64_t D) { return (dtype == DMAD_BF16 || dtype == DMAD_F16) && D == 128; }
int64_t score_slice_bytes(bool full, int64_t Lq, int64_t Lk) {
  const int64_t nkt = (Lk + 127) / 128;
  return round_up(dmad::sc_slice_bytes(Lq, 4 * nkt, full ? 2 : 1), 256);
}
// (b, h) slices per launch pair that `workspace_bytes` holds beyond the minimum
// workspace `base` (0: the recomputing query pass runs)
int64_t score_slices(int dtype, bool full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, int64_t base,
                     int64_t workspace_bytes) {
  if (!score_store_ok(dtype, D) || B * H == 0 || Lq == 0 || Lk == 0 || workspace_bytes <= base) return 0;
  const int64_t one = score_slice_bytes(full, Lq, Lk);
  const int64_t n = (workspace_bytes - base) / one;
  return n < B * H ? n : B * H;
}

// Backward plan: the key-stationary pass (dK, dV), the query-stationary pass
// (dQ [, dQd]), and with tangent gradients the dO-only passes run on (dOd, rho)
// (the query one only where the full query pass does not give dQd). With
// score slices (sc > 0) the key pass also stores the score gradients and the
// query pass reads them back, sc (b, h) slices per launch pair.
struct BwdPlan {
  const char *kv, *dq, *kv_t, *dq_t;
  int64_t grid_kv, grid_dq;
  int xcd_kv, xcd_dq, copies;
  int64_t ws;
  int64_t sc;
};

BwdPlan plan_bwd(int dtype, bool full, bool tgrad, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D) {
  BwdPlan pl{};
  const int64_t BH = B * H;
  if (dtype == DMAD_F32) {
    // fp32 operands (dO only): fp32-MFMA passes, head-major order
    const int64_t bk = dmad::f32_kv_block((int)D), bm = dmad::f32_dq_block((int)D);
    pl.kv = "attn_f32_bwd_kv_kernel";
    pl.dq = "attn_f32_bwd_dq_kernel";
    pl.grid_kv = (Lk + bk - 1) / bk * BH;
    pl.grid_dq = (Lq + bm - 1) / bm * BH;
    pl.ws = bwd_ws_of(DMAD_F32, 0, B, H, Lq, Lk, D).total;
    return pl;
  }
  const bool rows = full && dmad::full_reads_rows((int)D);
  pl.kv = rows ? "attn_bwd_kv_full_kernel" : full ? "attn_bwd_kernel" : dmad::kv_dout_only_name((int)D);
  pl.dq = rows ? "attn_bwd_dq_full_kernel" : full ? "attn_bwd_dq_kernel" : dmad::dq_dout_only_name((int)D);
  pl.kv_t = tgrad ? dmad::kv_dout_only_name((int)D) : nullptr;
  pl.dq_t = tgrad && !rows ? dmad::dq_dout_only_name((int)D) : nullptr;
  const int64_t nkt = (Lk + 127) / 128, nqt = (Lq + 127) / 128;  // 128 keys / queries per workgroup
  pl.grid_kv = nkt * BH;
  pl.grid_dq = nqt * BH;
  pl.xcd_kv = nkt < dmad::kHeadMajorMinTiles;  // block order (common.h)
  pl.xcd_dq = nqt < dmad::kHeadMajorMinTiles;
  const BwdWs w = bwd_ws(full ? (tgrad ? 2 : 1) : 0, B, H, Lq, Lk, D);
  pl.copies = w.nq + w.nk;
  pl.ws = w.total;
  return pl;
}

// The plan of a call given its workspace: the stored-score passes where the
// workspace holds at least one (b, h) slice of score gradients beyond the minimum.
BwdPlan plan_bwd_ws(int dtype, bool full, bool tgrad, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                    int64_t workspace_bytes) {
  BwdPlan pl = plan_bwd(dtype, full, tgrad, B, H, Lq, Lk, D);
  pl.sc = score_slices(dtype, full, B, H, Lq, Lk, D, pl.ws, workspace_bytes);
  if (pl.sc > 0) {
    pl.kv = full ? "attn_bwd_kv_full_kernel<store>" : "attn_bwd_kv_tr_kernel<store>";
    pl.dq = "attn_bwd_dq_sc_kernel";
    if (tgrad) pl.kv_t = "attn_bwd_kv_tr_kernel<load>";  // per launch pair, on the stored dSd
    const int64_t npair = ((Lq + 127) / 128 + 1) / 2;  // two 128-query blocks per query-pass workgroup
    pl.grid_kv = (Lk + 127) / 128 * pl.sc;
    pl.grid_dq = npair * pl.sc;
    pl.xcd_dq = npair < dmad::kHeadMajorMinTiles;
    pl.ws += pl.sc * score_slice_bytes(full, Lq, Lk);
  }
  return pl;
}

// Shared body of the dense and block-sparse forwards (mg == nullptr: dense).
int fwd_impl(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv, const void* q,
             const void* k, const void* v, const void* tq, const void* tk, const void* tv, const int64_t q_strides[4],
             const int64_t k_strides[4], const int64_t v_strides[4], void* o, void* to, const int64_t o_strides[4],
             float* lse, float* mu, float sm_scale, void* workspace, size_t workspace_bytes, void* stream,
             const MagiArgs* mg) {
  if (dtype != DMAD_BF16 && dtype != DMAD_F16 && dtype != DMAD_F32)
    return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if (mode < DMAD_FWD_PLAIN || mode > DMAD_FWD_JVP_KV_TANGENT_ZERO) return fail(DMAD_ERR_INVALID, "unknown mode %d", mode);
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0) return fail(DMAD_ERR_INVALID, "negative size");
  if (!head_dim_ok(Dqk) || !head_dim_ok(Dv))
    return fail(DMAD_ERR_UNSUPPORTED, "head dims must be in {16,32,64,128,256}, got Dqk=%lld Dv=%lld", (long long)Dqk,
                (long long)Dv);
  if (!(sm_scale > 0.f)) return fail(DMAD_ERR_UNSUPPORTED, "sm_scale must be positive");
  if (mg != nullptr && mode == DMAD_FWD_PLAIN)
    return fail(DMAD_ERR_UNSUPPORTED, "the block-sparse forward has JVP modes only");
  if (B == 0 || H == 0 || Lq == 0 || (mg != nullptr && mg->T == 0)) return ok();
  if (Lk == 0) return fail(DMAD_ERR_INVALID, "Lk must be at least 1");
  if (B * H > ((int64_t)1 << 24) || Lq >= ((int64_t)1 << 26) || Lk >= ((int64_t)1 << 26))
    return fail(DMAD_ERR_UNSUPPORTED, "sizes too large");
  const bool jvp = mode != DMAD_FWD_PLAIN, kvt = mode == DMAD_FWD_JVP;
  const bool f32 = dtype == DMAD_F32;
  const int esz = elem_size(dtype);
  int rc;
  if ((rc = check_operand("q", q, q_strides, Lq, Dqk, esz))) return rc;
  if ((rc = check_operand("k", k, k_strides, Lk, Dqk, esz))) return rc;
  if ((rc = check_operand("v", v, v_strides, Lk, Dv, esz))) return rc;
  if ((rc = check_operand("o", o, o_strides, Lq, Dv, esz))) return rc;
  if (jvp) {
    if ((rc = check_operand("tq", tq, q_strides, Lq, Dqk, esz))) return rc;
    if ((rc = check_operand("to", to, o_strides, Lq, Dv, esz))) return rc;
    if (mu == nullptr) return fail(DMAD_ERR_INVALID, "mu: null pointer");
  }
  if (kvt) {
    if ((rc = check_operand("tk", tk, k_strides, Lk, Dqk, esz))) return rc;
    if ((rc = check_operand("tv", tv, v_strides, Lk, Dv, esz))) return rc;
  }
  if (lse == nullptr) return fail(DMAD_ERR_INVALID, "lse: null pointer");
  // the launch plan (kernel, grid, block order, copies, workspace) for this shape
  const FwdPlan plan = plan_fwd(dtype, mode, mg ? mg->T : -1, B, H, Lq, Lk, Dqk, Dv);
  const int64_t need = plan.ws;
  if (need > 0 && (workspace == nullptr || (int64_t)workspace_bytes < need))
    return fail(DMAD_ERR_WORKSPACE, "workspace needs %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  if (((uintptr_t)workspace & 255) != 0) return fail(DMAD_ERR_INVALID, "workspace must be 256-byte aligned");
  const int64_t dvp = Dv < 32 ? 32 : Dv, lkp = round_up(Lk, kLkAlign);
  if (dvp * lkp * 2 >= kMaxHeadBytes) return fail(DMAD_ERR_UNSUPPORTED, "Lk too large");

  dmad::FwdLaunchFn fn = plan.family == FwdFamily::kF32      ? pick_fwd_f32(Dqk, Dv, mode, mg != nullptr)
                         : plan.family == FwdFamily::kRowsX2 ? pick_fwd32x2(dtype, Dqk, mode)
                         : mg                                ? pick_fwd_magi(dtype, Dqk, Dv, mode)
                                                             : pick_fwd(dtype, Dqk, Dv, mode);
  if (fn == nullptr) return fail(DMAD_ERR_UNSUPPORTED, "no kernel for Dqk=%lld Dv=%lld", (long long)Dqk, (long long)Dv);

  hipStream_t s = (hipStream_t)stream;
  const int BH = (int)(B * H);
  char* ws = (char*)workspace;
  const int64_t vt_bytes = round_up(B * H * dvp * lkp * 2, 256);
  // the row-reading kernels transpose V on the LDS read; the others read a
  // transposed, key-padded copy made here
  const bool need_vt = plan.copies > 0;
  hipError_t e = hipSuccess;
  dmad::TransposeParams tp{v, ws, v_strides[0], v_strides[1], v_strides[2], (int)H, (int)Lk, (int)Dv, (int)lkp, (int)dvp};
  if (need_vt) e = dmad::launch_transpose_pad(tp, BH, s);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));
  if (kvt && need_vt) {
    dmad::TransposeParams tt = tp;
    tt.x = tv;
    tt.y = ws + vt_bytes;
    e = dmad::launch_transpose_pad(tt, BH, s);
    if (e != hipSuccess) return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));
  }

  dmad::FwdParams p{};
  p.q = q;
  p.k = k;
  p.tq = jvp ? tq : q;
  p.tk = kvt ? tk : k;
  p.vt = ws;
  p.tvt = kvt ? (const void*)(ws + vt_bytes) : (const void*)ws;
  p.v = v;
  p.tv = kvt ? tv : v;
  p.v_sb = v_strides[0];
  p.v_sh = v_strides[1];
  p.v_sl = v_strides[2];
  p.o = o;
  p.to = jvp ? to : o;
  p.lse = lse;
  p.mu = mu;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_sl = q_strides[2];
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_sl = k_strides[2];
  p.o_sb = o_strides[0];
  p.o_sh = o_strides[1];
  p.o_sl = o_strides[2];
  p.B = (int)B;
  p.H = (int)H;
  p.Lq = (int)Lq;
  p.Lk = (int)Lk;
  p.LKP = (int)lkp;
  p.scale = sm_scale;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  if (mg != nullptr) {
    p.q_ranges = mg->q_ranges;
    p.k_ranges = mg->k_ranges;
    p.qk_map = mg->qk_map;
    p.task_group = mg->task_group;
    p.task_qtile = mg->task_qtile;
    p.G = (int)mg->G;
    p.R = (int)mg->R;
    p.T = (int)mg->T;
  }
  if (plan.grid >= ((int64_t)1 << 31)) return fail(DMAD_ERR_UNSUPPORTED, "grid too large");
  const int64_t grid = plan.grid;
  p.xcd_order = plan.xcd_order;  // block order (common.h)
  mark(0, false, s);
  e = fn(p, (int)grid, s);
  mark(0, true, s);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "attention launch: %s", hipGetErrorString(e));
  return ok();
}

// Workspace of dmad_attn_jvp_bwd_noalloc: a static device array, one copy per
// GPU at that GPU's own address, held until the process ends. Host code never
// uses the name `scratch` as a device address (on the host it is a stand-in
// object); it uses the address hipGetSymbolAddress returns for the device.
// Every call on one GPU shares that GPU's copy: calls that overlap on one GPU
// (two streams, two threads) race. Each call's statistics pass rewrites every
// byte the backward kernels read before they read it, so nothing needs clearing.
static __device__ __attribute__((aligned(256))) char scratch[DMAD_BWD_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call on each device (that device current) and kept. `stream` must belong to
// the current device.
int scratch_of_device(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(DMAD_ERR_UNSUPPORTED, "device ordinal %d out of range", dev);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return fail(DMAD_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(DMAD_ERR_INVALID, "the stream belongs to device %d but device %d is current", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(DMAD_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    if (((uintptr_t)p & 255) != 0) return fail(DMAD_ERR_HIP, "scratch is not 256-byte aligned on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DMAD_OK;
}

// Shared body of dmad_attn_jvp_bwd (caller workspace) and
// dmad_attn_jvp_bwd_noalloc (use_scratch: the device's copy of `scratch`).
int bwd_impl(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q, const void* k,
             const void* v, const void* tq, const void* tk, const void* tv, const int64_t q_strides[4],
             const int64_t k_strides[4], const int64_t v_strides[4], const void* o, const void* to,
             const int64_t o_strides[4], const float* lse, const float* mu, const void* dout, const void* dto,
             const int64_t do_strides[4], void* dq, void* dk, void* dv, void* dtq, void* dtk, void* dtv,
             const int64_t dq_strides[4], const int64_t dk_strides[4], const int64_t dv_strides[4], float sm_scale,
             void* workspace, size_t workspace_bytes, void* stream, bool use_scratch) {
  if (dtype != DMAD_BF16 && dtype != DMAD_F16 && dtype != DMAD_F32)
    return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0) return fail(DMAD_ERR_INVALID, "negative size");
  if (!head_dim_ok(D)) return fail(DMAD_ERR_UNSUPPORTED, "head dim must be in {16,32,64,128,256}, got %lld", (long long)D);
  if (!(sm_scale > 0.f)) return fail(DMAD_ERR_UNSUPPORTED, "sm_scale must be positive");
  const bool full = dto != nullptr;
  const bool tgrad = dtq != nullptr || dtk != nullptr || dtv != nullptr;
  if (tgrad && !(dtq && dtk && dtv)) return fail(DMAD_ERR_INVALID, "dtq, dtk, dtv must be all set or all null");
  if (tgrad && !full) return fail(DMAD_ERR_INVALID, "tangent gradients need the cotangent dto");
  if (full && D > 128) return fail(DMAD_ERR_UNSUPPORTED, "the full backward supports head dims up to 128");
  const bool f32 = dtype == DMAD_F32;
  if (full && f32) return fail(DMAD_ERR_UNSUPPORTED, "the full backward takes bf16 or fp16 operands (fp32: dO only)");
  const int esz = elem_size(dtype);
  if (B == 0 || H == 0 || (Lq == 0 && Lk == 0)) return ok();
  if (Lk == 0) return fail(DMAD_ERR_INVALID, "Lk must be at least 1");
  if (Lq == 0) return fail(DMAD_ERR_INVALID, "Lq must be at least 1 (with no query rows dK and dV are zero)");
  if (B * H > ((int64_t)1 << 24) || Lq >= ((int64_t)1 << 26) || Lk >= ((int64_t)1 << 26))
    return fail(DMAD_ERR_UNSUPPORTED, "sizes too large");
  int rc;
  if ((rc = check_operand("q", q, q_strides, Lq, D, esz))) return rc;
  if ((rc = check_operand("k", k, k_strides, Lk, D, esz))) return rc;
  if ((rc = check_operand("v", v, v_strides, Lk, D, esz))) return rc;
  if ((rc = check_operand("o", o, o_strides, Lq, D, esz))) return rc;
  if ((rc = check_operand("dout", dout, do_strides, Lq, D, esz))) return rc;
  if ((rc = check_operand("dq", dq, dq_strides, Lq, D, esz))) return rc;
  if ((rc = check_operand("dk", dk, dk_strides, Lk, D, esz))) return rc;
  if ((rc = check_operand("dv", dv, dv_strides, Lk, D, esz))) return rc;
  if (lse == nullptr) return fail(DMAD_ERR_INVALID, "lse: null pointer");
  if (full) {
    if ((rc = check_operand("tq", tq, q_strides, Lq, D, esz))) return rc;
    if ((rc = check_operand("tk", tk, k_strides, Lk, D, esz))) return rc;
    if ((rc = check_operand("tv", tv, v_strides, Lk, D, esz))) return rc;
    if ((rc = check_operand("to", to, o_strides, Lq, D, esz))) return rc;
    if ((rc = check_operand("dto", dto, do_strides, Lq, D, esz))) return rc;
    if (mu == nullptr) return fail(DMAD_ERR_INVALID, "mu: null pointer");
  }
  if (tgrad) {
    if ((rc = check_operand("dtq", dtq, dq_strides, Lq, D, esz))) return rc;
    if ((rc = check_operand("dtk", dtk, dk_strides, Lk, D, esz))) return rc;
    if ((rc = check_operand("dtv", dtv, dv_strides, Lk, D, esz))) return rc;
  }
  const int fl = full ? (tgrad ? 2 : 1) : 0;
  const BwdWs w = bwd_ws_of(dtype, fl, B, H, Lq, Lk, D);
  if (use_scratch) {
    if (w.total > (int64_t)DMAD_BWD_SCRATCH_BYTES)
      return fail(DMAD_ERR_UNSUPPORTED,
                  "this backward needs %lld bytes of workspace; the static scratch of dmad_attn_jvp_bwd_noalloc "
                  "holds %lld (call dmad_attn_jvp_bwd with a workspace instead)",
                  (long long)w.total, (long long)DMAD_BWD_SCRATCH_BYTES);
    int rc_s;
    if ((rc_s = scratch_of_device(stream, &workspace))) return rc_s;
    workspace_bytes = DMAD_BWD_SCRATCH_BYTES;
  }
  if (workspace == nullptr || (int64_t)workspace_bytes < w.total)
    return fail(DMAD_ERR_WORKSPACE, "workspace needs %lld bytes, got %lld", (long long)w.total, (long long)workspace_bytes);
  // workspace beyond the minimum holds stored score gradients (128-wide bf16/fp16 heads)
  const int64_t sc = use_scratch ? 0 : score_slices(dtype, full, B, H, Lq, Lk, D, w.total, (int64_t)workspace_bytes);
  if (((uintptr_t)workspace & 255) != 0) return fail(DMAD_ERR_INVALID, "workspace must be 256-byte aligned");
  const int64_t dp = D < 32 ? 32 : D, lqp = round_up(Lq, 64), lkp = round_up(Lk, kLkAlign), BH = B * H;
  if (dp * lqp * 2 >= kMaxHeadBytes || dp * lkp * 2 >= kMaxHeadBytes) return fail(DMAD_ERR_UNSUPPORTED, "sequence too long");
  if (f32) {
    // fp32 (dO only): the workspace holds just the statistics [BH][LQP]
    // (log2 LSE, then D)
    const dmad::F32BwdFns f = pick_bwd_f32(D);
    if (f.prep == nullptr || f.kv == nullptr || f.dq == nullptr)
      return fail(DMAD_ERR_UNSUPPORTED, "no fp32 backward kernel for D=%lld", (long long)D);
    hipStream_t s = (hipStream_t)stream;
    float* lse2 = (float*)workspace;
    float* dd = lse2 + BH * lqp;
    dmad::F32PrepParams pp{(const float*)o, (const float*)dout, lse, lse2, dd, o_strides[0], o_strides[1],
                           o_strides[2], do_strides[0], do_strides[1], do_strides[2], (int)H, (int)Lq, (int)lqp,
                           (int)BH};
    dmad::BwdParams p{};
    p.q = q; p.k = k; p.v = v; p.dout = dout; p.dk = dk; p.dv = dv;
    p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_sl = q_strides[2];
    p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_sl = k_strides[2];
    p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_sl = v_strides[2];
    p.do_sb = do_strides[0]; p.do_sh = do_strides[1]; p.do_sl = do_strides[2];
    p.dk_sb = dk_strides[0]; p.dk_sh = dk_strides[1]; p.dk_sl = dk_strides[2];
    p.dv_sb = dv_strides[0]; p.dv_sh = dv_strides[1]; p.dv_sl = dv_strides[2];
    p.B = (int)B; p.H = (int)H; p.Lq = (int)Lq; p.Lk = (int)Lk; p.LQP = (int)lqp;
    p.scale = sm_scale;
    p.scale_log2 = sm_scale * 1.4426950408889634f;
    dmad::DqParams pq{};
    pq.q = q; pq.dout = dout; pq.k = k; pq.v = v; pq.dq = dq;
    pq.q_sb = q_strides[0]; pq.q_sh = q_strides[1]; pq.q_sl = q_strides[2];
    pq.do_sb = do_strides[0]; pq.do_sh = do_strides[1]; pq.do_sl = do_strides[2];
    pq.k_sb = k_strides[0]; pq.k_sh = k_strides[1]; pq.k_sl = k_strides[2];
    pq.v_sb = v_strides[0]; pq.v_sh = v_strides[1]; pq.v_sl = v_strides[2];
    pq.dq_sb = dq_strides[0]; pq.dq_sh = dq_strides[1]; pq.dq_sl = dq_strides[2];
    pq.B = (int)B; pq.H = (int)H; pq.Lq = (int)Lq; pq.Lk = (int)Lk; pq.LQP = (int)lqp; pq.LKP = (int)lkp;
    pq.scale = sm_scale;
    pq.scale_log2 = sm_scale * 1.4426950408889634f;
    hipError_t e;
    if ((e = f.prep(pp, s)) != hipSuccess) return fail(DMAD_ERR_HIP, "prep launch: %s", hipGetErrorString(e));
    mark(0, false, s);
    if ((e = f.kv(p, lse2, dd, s)) != hipSuccess) return fail(DMAD_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
    mark(0, true, s);
    mark(1, false, s);
    if ((e = f.dq(pq, lse2, dd, s)) != hipSuccess) return fail(DMAD_ERR_HIP, "backward dq launch: %s", hipGetErrorString(e));
    mark(1, true, s);
    return ok();
  }
  const int mode = full ? dmad::kBwdFull : dmad::kBwdDoutOnly;
  // 128-wide heads: the full derivative's query pass also gives dQd, so the
  // tangent gradients need only the dO-only key pass (dKd, dVd)
  const bool full_rows = full && dmad::full_reads_rows((int)D);
  dmad::BwdLaunchFn fn = full_rows ? pick_kv_full(dtype) : pick_bwd(dtype, D, mode);
  dmad::DqLaunchFn fq = full_rows ? pick_dq_full(dtype, tgrad) : pick_dq(dtype, D, mode);
  dmad::BwdLaunchFn fn_a = tgrad ? pick_bwd(dtype, D, dmad::kBwdDoutOnly) : nullptr;
  dmad::DqLaunchFn fq_a = tgrad && !full_rows ? pick_dq(dtype, D, dmad::kBwdDoutOnly) : nullptr;
  if (fn == nullptr || fq == nullptr || (tgrad && (fn_a == nullptr || (!full_rows && fq_a == nullptr))))
    return fail(DMAD_ERR_UNSUPPORTED, "no backward kernel for D=%lld", (long long)D);

  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  char* trq = w.nq ? ws : nullptr;
  char* trdo = w.nq ? ws + w.trq : nullptr;
  char* trtq = full && w.nq ? ws + 2 * w.trq : nullptr;
  char* trdto = full && w.nq ? ws + 3 * w.trq : nullptr;
  char* trk = w.nk ? ws + w.nq * w.trq : nullptr;
  char* trtk = full && w.nk ? trk + w.trk : nullptr;
  float* stats = (float*)(ws + w.nq * w.trq + w.nk * w.trk);
  float* stats_bt = w.tgrad ? (float*)((char*)stats + w.stats) : nullptr;

  hipError_t e;
  auto tr = [&](const void* x, const int64_t* st, char* y, int64_t L, int64_t LP) {
    dmad::TransposeParams tp{x, y, st[0], st[1], st[2], (int)H, (int)L, (int)D, (int)LP, (int)dp};
    return dmad::launch_transpose_pad(tp, (int)BH, s);
  };
  // the full-derivative kernels of head dims other than 128, and the dO-only
  // ones of some head dims, read transposed copies of Q, dO (and Qd, dOd) and K
  // (and Kd)
  const bool need_tr = w.nq > 0;
  if (need_tr && ((e = tr(q, q_strides, trq, Lq, lqp)) != hipSuccess || (e = tr(dout, do_strides, trdo, Lq, lqp)) != hipSuccess))
    return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));
  if (w.nk > 0 && (e = tr(k, k_strides, trk, Lk, lkp)) != hipSuccess)
    return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));
  if (need_tr && full && ((e = tr(tq, q_strides, trtq, Lq, lqp)) != hipSuccess || (e = tr(dto, do_strides, trdto, Lq, lqp)) != hipSuccess ||
               (e = tr(tk, k_strides, trtk, Lk, lkp)) != hipSuccess))
    return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));

  const int ba = dmad::bwd_bmq((int)D, dmad::kBwdDoutOnly);
  dmad::PrepParams pp{};
  pp.o = o;
  pp.to = full ? to : nullptr;
  pp.dout = dout;
  pp.dto = full ? dto : nullptr;
  pp.lse = lse;
  pp.mu = full ? mu : nullptr;
  pp.stats_a = full ? nullptr : stats;
  pp.stats_b = full ? stats : nullptr;
  pp.stats_bt = stats_bt;
  pp.o_sb = o_strides[0];
  pp.o_sh = o_strides[1];
  pp.o_sl = o_strides[2];
  pp.do_sb = do_strides[0];
  pp.do_sh = do_strides[1];
  pp.do_sl = do_strides[2];
  pp.H = (int)H;
  pp.Lq = (int)Lq;
  pp.LQP = (int)lqp;
  pp.D = (int)D;
  pp.BH = (int)BH;
  pp.BA = ba;
  if ((e = dmad::launch_bwd_prep(pp, dtype, s)) != hipSuccess) return fail(DMAD_ERR_HIP, "prep launch: %s", hipGetErrorString(e));

  // key-stationary pass: dK, dV
  dmad::BwdParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.tq = full ? tq : q;
  p.tk = full ? tk : k;
  p.tv = full ? tv : v;
  p.dout = dout;
  p.dto = full ? dto : dout;
  p.qT = trq;
  p.tqT = full ? trtq : trq;
  p.doT = trdo;
  p.dtoT = full ? trdto : trdo;
  p.stats = stats;
  p.dk = dk;
  p.dv = dv;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_sl = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_sl = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_sl = v_strides[2];
  p.do_sb = do_strides[0]; p.do_sh = do_strides[1]; p.do_sl = do_strides[2];
  p.dk_sb = dk_strides[0]; p.dk_sh = dk_strides[1]; p.dk_sl = dk_strides[2];
  p.dv_sb = dv_strides[0]; p.dv_sh = dv_strides[1]; p.dv_sl = dv_strides[2];
  p.B = (int)B;
  p.H = (int)H;
  p.Lq = (int)Lq;
  p.Lk = (int)Lk;
  p.LQP = (int)lqp;
  p.scale = sm_scale;
  p.scale_log2 = sm_scale * 1.4426950408889634f;

  // query-stationary pass: dQ
  dmad::DqParams pq{};
  pq.q = q;
  pq.tq = full ? tq : q;
  pq.dout = dout;
  pq.dto = full ? dto : dout;
  pq.k = k;
  pq.tk = full ? tk : k;
  pq.v = v;
  pq.tv = full ? tv : v;
  pq.kT = trk;
  pq.tkT = full ? trtk : trk;
  pq.stats = stats;
  pq.dq = dq;
  pq.dtq = dtq;
  pq.q_sb = q_strides[0]; pq.q_sh = q_strides[1]; pq.q_sl = q_strides[2];
  pq.do_sb = do_strides[0]; pq.do_sh = do_strides[1]; pq.do_sl = do_strides[2];
  pq.k_sb = k_strides[0]; pq.k_sh = k_strides[1]; pq.k_sl = k_strides[2];
  pq.v_sb = v_strides[0]; pq.v_sh = v_strides[1]; pq.v_sl = v_strides[2];
  pq.dq_sb = dq_strides[0]; pq.dq_sh = dq_strides[1]; pq.dq_sl = dq_strides[2];
  pq.B = (int)B;
  pq.H = (int)H;
  pq.Lq = (int)Lq;
  pq.Lk = (int)Lk;
  pq.LQP = (int)lqp;
  pq.LKP = (int)lkp;
  pq.stat_tile = full ? 32 : ba;
  pq.scale = sm_scale;
  pq.scale_log2 = sm_scale * 1.4426950408889634f;

  // grids and block order from the launch plan (128 keys / queries per workgroup)
  const BwdPlan plan = plan_bwd(dtype, full, tgrad, B, H, Lq, Lk, D);
  if (plan.grid_kv >= ((int64_t)1 << 31) || plan.grid_dq >= ((int64_t)1 << 31))
    return fail(DMAD_ERR_UNSUPPORTED, "grid too large");
  p.xcd_order = plan.xcd_kv;  // block order (common.h)
  pq.xcd_order = plan.xcd_dq;
  if (sc > 0) {
    // stored score gradients: per launch pair, the key pass over sc (b, h)
    // slices writes their dS [, dSd] after the minimum workspace, the query
    // pass reads them back, and with tangent gradients the dO-only key pass on
    // (dOd, rho) reads the stored dSd for dKd, dVd; main kernels in launch order
    const dmad::BwdLaunchFn fs = pick_kv_sc(dtype, full);
    const dmad::DqLaunchFn fqs = pick_dq_sc(dtype, full);
    const dmad::BwdLaunchFn fts = tgrad ? pick_kv_sc_tangent(dtype) : nullptr;
    if (fs == nullptr || fqs == nullptr || (tgrad && fts == nullptr))
      return fail(DMAD_ERR_UNSUPPORTED, "no stored-score backward kernel");
    const int64_t nkt = (Lk + 127) / 128, nqw = ((Lq + 127) / 128 + 1) / 2;  // query-pass workgroups per slice
    p.sc = ws + w.total;
    p.sc_slice = score_slice_bytes(full, Lq, Lk);
    pq.sc = p.sc;
    pq.sc_slice = p.sc_slice;
    // tangent key pass: dKd, dVd from (dOd, rho) and the stored dSd (a copy of p
    // made after the score fields are set: it reads the same slices)
    dmad::BwdParams pt = p;
    pt.dout = dto;
    pt.stats = stats_bt;
    pt.dk = dtk;
    pt.dv = dtv;
    pq.sc_nkb = (int)(4 * nkt);
    pq.xcd_order = nqw < dmad::kHeadMajorMinTiles;
    int ev = 0;
    for (int64_t bh0 = 0; bh0 < BH; bh0 += sc) {
      const int64_t n = BH - bh0 < sc ? BH - bh0 : sc;
      p.bh0 = pq.bh0 = pt.bh0 = (int)bh0;
      mark(ev, false, s);
      if ((e = fs(p, (int)(n * nkt), s)) != hipSuccess) return fail(DMAD_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
      mark(ev++, true, s);
      mark(ev, false, s);
      if ((e = fqs(pq, (int)(n * nqw), s)) != hipSuccess)
        return fail(DMAD_ERR_HIP, "backward dq launch: %s", hipGetErrorString(e));
      mark(ev++, true, s);
      if (tgrad) {
        mark(ev, false, s);
        if ((e = fts(pt, (int)(n * nkt), s)) != hipSuccess)
          return fail(DMAD_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
        mark(ev++, true, s);
      }
    }
    return ok();
  }
  mark(0, false, s);
  if ((e = fn(p, (int)plan.grid_kv, s)) != hipSuccess) return fail(DMAD_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  mark(0, true, s);
  mark(1, false, s);
  if (plan.grid_dq > 0 && (e = fq(pq, (int)plan.grid_dq, s)) != hipSuccess)
    return fail(DMAD_ERR_HIP, "backward dq launch: %s", hipGetErrorString(e));
  mark(1, true, s);
  if (tgrad) {
    // tangent gradients: the dO-only passes with (dO, D) := (dOd, rho) (the
    // query pass only where the full derivative's query pass did not give dQd)
    dmad::BwdParams pt = p;
    pt.dout = dto;
    pt.doT = trdto;
    pt.stats = stats_bt;
    pt.dk = dtk;
    pt.dv = dtv;
    mark(2, false, s);
    if ((e = fn_a(pt, (int)plan.grid_kv, s)) != hipSuccess)
      return fail(DMAD_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
    mark(2, true, s);
    dmad::DqParams pqt = pq;
    pqt.dout = dto;
    pqt.stats = stats_bt;
    pqt.stat_tile = ba;
    pqt.dq = dtq;
    if (fq_a != nullptr) {
      mark(3, false, s);
      if (plan.grid_dq > 0 && (e = fq_a(pqt, (int)plan.grid_dq, s)) != hipSuccess)
        return fail(DMAD_ERR_HIP, "backward dq launch: %s", hipGetErrorString(e));
      mark(3, true, s);
    }
  }
  return ok();
}


}  // namespace

extern "C" {

int dmad_abi_version(void) { return 2; }

const char* dmad_last_error(void) { return g_last_error.c_str(); }

int dmad_set_kernel_events(void* const* events, int count) {
  if (count < 0 || count > kMaxEvents || (count % 2) != 0)
    return fail(DMAD_ERR_INVALID, "count must be an even number in [0, %d]", kMaxEvents);
  if (count > 0 && events == nullptr) return fail(DMAD_ERR_INVALID, "events: null pointer");
  for (int i = 0; i < count; ++i) g_events[i] = (hipEvent_t)events[i];
  g_nevents = count;
  return ok();
}

int dmad_attn_fwd_workspace_bytes(int mode, int64_t B, int64_t H, int64_t Lk, int64_t Dqk, int64_t Dv,
                                  size_t* bytes) {
  if (bytes == nullptr) return fail(DMAD_ERR_INVALID, "bytes: null pointer");
  if (mode < DMAD_FWD_PLAIN || mode > DMAD_FWD_JVP_KV_TANGENT_ZERO) return fail(DMAD_ERR_INVALID, "unknown mode %d", mode);
  if (B < 0 || H < 0 || Lk < 0 || !head_dim_ok(Dqk) || !head_dim_ok(Dv)) return fail(DMAD_ERR_INVALID, "bad sizes");
  *bytes = (size_t)fwd_ws_bytes(mode, B, H, Lk, Dqk, Dv);
  return ok();
}

int dmad_attn_jvp_fwd(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv,
                      const void* q, const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4], void* o,
                      void* to, const int64_t o_strides[4], float* lse, float* mu, float sm_scale, void* workspace,
                      size_t workspace_bytes, void* stream) {
  return fwd_impl(dtype, mode, B, H, Lq, Lk, Dqk, Dv, q, k, v, tq, tk, tv, q_strides, k_strides, v_strides, o, to,
                  o_strides, lse, mu, sm_scale, workspace, workspace_bytes, stream, nullptr);
}

int dmad_attn_jvp_fwd_magi(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv,
                           const void* q, const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                           const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                           void* o, void* to, const int64_t o_strides[4], float* lse, float* mu, float sm_scale,
                           const int32_t* q_ranges, const int32_t* k_ranges, const int32_t* qk_map, int64_t G,
                           int64_t R, const int32_t* task_group, const int32_t* task_qtile, int64_t T,
                           int64_t block_m, void* workspace, size_t workspace_bytes, void* stream) {
  if (block_m != dmad::kMagiBlockM)
    return fail(DMAD_ERR_UNSUPPORTED, "tasks must be built for %d-query tiles, got BLOCK_M=%lld", dmad::kMagiBlockM,
                (long long)block_m);
  if (G < 1 || R < 0 || T < 0 || G >= ((int64_t)1 << 30) || R >= ((int64_t)1 << 30) || T >= ((int64_t)1 << 30))
    return fail(DMAD_ERR_INVALID, "bad table sizes G=%lld R=%lld T=%lld", (long long)G, (long long)R, (long long)T);
  if (q_ranges == nullptr || qk_map == nullptr || (R > 0 && k_ranges == nullptr) ||
      (T > 0 && (task_group == nullptr || task_qtile == nullptr)))
    return fail(DMAD_ERR_INVALID, "block-sparse tables: null pointer");
  const MagiArgs mg{q_ranges, k_ranges, qk_map, task_group, task_qtile, G, R, T};
  return fwd_impl(dtype, mode, B, H, Lq, Lk, Dqk, Dv, q, k, v, tq, tk, tv, q_strides, k_strides, v_strides, o, to,
                  o_strides, lse, mu, sm_scale, workspace, workspace_bytes, stream, &mg);
}

int dmad_attn_fwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv, const void* q,
                  const void* k, const void* v, const int64_t q_strides[4], const int64_t k_strides[4],
                  const int64_t v_strides[4], void* o, const int64_t o_strides[4], float* lse, float sm_scale,
                  void* workspace, size_t workspace_bytes, void* stream) {
  return dmad_attn_jvp_fwd(dtype, DMAD_FWD_PLAIN, B, H, Lq, Lk, Dqk, Dv, q, k, v, nullptr, nullptr, nullptr,
                           q_strides, k_strides, v_strides, o, nullptr, o_strides, lse, nullptr, sm_scale, workspace,
                           workspace_bytes, stream);
}

int dmad_attn_fwd_plan(int dtype, int mode, int64_t magi_tasks, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                       int64_t Dqk, int64_t Dv, dmad_plan* out) {
  if (out == nullptr) return fail(DMAD_ERR_INVALID, "plan: null pointer");
  if (dtype != DMAD_BF16 && dtype != DMAD_F16 && dtype != DMAD_F32)
    return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if (mode < DMAD_FWD_PLAIN || mode > DMAD_FWD_JVP_KV_TANGENT_ZERO) return fail(DMAD_ERR_INVALID, "unknown mode %d", mode);
  if (magi_tasks >= 0 && mode == DMAD_FWD_PLAIN) return fail(DMAD_ERR_INVALID, "the block-sparse forward has JVP modes only");
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0 || !head_dim_ok(Dqk) || !head_dim_ok(Dv)) return fail(DMAD_ERR_INVALID, "bad sizes");
  const FwdPlan pl = plan_fwd(dtype, mode, magi_tasks, B, H, Lq, Lk, Dqk, Dv);
  *out = dmad_plan{};
  out->kernel = pl.kernel;
  out->grid = pl.grid;
  out->xcd_order = pl.xcd_order;
  out->chunks = (int32_t)pl.chunks;
  out->transposed_copies = pl.copies;
  out->workspace_bytes = pl.ws;
  return ok();
}
int dmad_attn_bwd_plan(int dtype, int full, int tangent_grads, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                       dmad_plan* out) {
  if (out == nullptr) return fail(DMAD_ERR_INVALID, "plan: null pointer");
  if (dtype != DMAD_BF16 && dtype != DMAD_F16 && dtype != DMAD_F32)
    return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if ((full != 0 && full != 1) || (tangent_grads != 0 && tangent_grads != 1))
    return fail(DMAD_ERR_INVALID, "full and tangent_grads must be 0 or 1");
  if (tangent_grads && !full) return fail(DMAD_ERR_INVALID, "tangent gradients need the cotangent dto");
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0 || !head_dim_ok(D)) return fail(DMAD_ERR_INVALID, "bad sizes");
  if (full && D > 128) return fail(DMAD_ERR_UNSUPPORTED, "the full backward supports head dims up to 128");
  if (full && dtype == DMAD_F32) return fail(DMAD_ERR_UNSUPPORTED, "the full backward takes bf16 or fp16 operands");
  const BwdPlan pl = plan_bwd(dtype, full != 0, tangent_grads != 0, B, H, Lq, Lk, D);
  *out = dmad_plan{};
  out->kernel = pl.kv;
  out->kernel2 = pl.dq;
  out->kernel3 = pl.kv_t;
  out->kernel4 = pl.dq_t;
  out->grid = pl.grid_kv;
  out->grid2 = pl.grid_dq;
  out->xcd_order = pl.xcd_kv;
  out->xcd_order2 = pl.xcd_dq;
  out->chunks = 1;
  out->transposed_copies = pl.copies;
  out->workspace_bytes = pl.ws;
  return ok();
}
int dmad_attn_bwd_plan_ws(int dtype, int full, int tangent_grads, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                          int64_t D, size_t workspace_bytes, dmad_plan* out) {
  const int rc = dmad_attn_bwd_plan(dtype, full, tangent_grads, B, H, Lq, Lk, D, out);
  if (rc != DMAD_OK) return rc;
  const BwdPlan pl = plan_bwd_ws(dtype, full != 0, tangent_grads != 0, B, H, Lq, Lk, D, (int64_t)workspace_bytes);
  if (pl.sc > 0) {
    out->kernel = pl.kv;
    out->kernel2 = pl.dq;
    out->kernel3 = pl.kv_t;
    out->grid = pl.grid_kv;
    out->grid2 = pl.grid_dq;
    out->xcd_order2 = pl.xcd_dq;
    out->workspace_bytes = pl.ws;
    out->score_slices = pl.sc;
  }
  return ok();
}
int dmad_attn_bwd_score_bytes(int dtype, int full, int64_t Lq, int64_t Lk, int64_t D, size_t* bytes) {
  if (bytes == nullptr) return fail(DMAD_ERR_INVALID, "bytes: null pointer");
  if (full != 0 && full != 1) return fail(DMAD_ERR_INVALID, "full must be 0 or 1");
  if (Lq < 0 || Lk < 0 || !head_dim_ok(D)) return fail(DMAD_ERR_INVALID, "bad sizes");
  *bytes = score_store_ok(dtype, D) && Lq > 0 && Lk > 0 ? (size_t)score_slice_bytes(full != 0, Lq, Lk) : 0;
  return ok();
}
int dmad_attn_bwd_workspace_bytes(int full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, size_t* bytes) {
  if (bytes == nullptr) return fail(DMAD_ERR_INVALID, "bytes: null pointer");
  if (full < 0 || full > 2) return fail(DMAD_ERR_INVALID, "full must be 0, 1 or 2");
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0 || !head_dim_ok(D)) return fail(DMAD_ERR_INVALID, "bad sizes");
  *bytes = (size_t)bwd_ws(full, B, H, Lq, Lk, D).total;
  return ok();
}

int dmad_attn_jvp_bwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q,
                      const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                      const void* o, const void* to, const int64_t o_strides[4], const float* lse, const float* mu,
                      const void* dout, const void* dto, const int64_t do_strides[4], void* dq, void* dk, void* dv,
                      void* dtq, void* dtk, void* dtv, const int64_t dq_strides[4], const int64_t dk_strides[4],
                      const int64_t dv_strides[4], float sm_scale, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return bwd_impl(dtype, B, H, Lq, Lk, D, q, k, v, tq, tk, tv, q_strides, k_strides, v_strides, o, to, o_strides, lse,
                  mu, dout, dto, do_strides, dq, dk, dv, dtq, dtk, dtv, dq_strides, dk_strides, dv_strides, sm_scale,
                  workspace, workspace_bytes, stream, false);
}

int dmad_attn_jvp_bwd_noalloc(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q,
                              const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                              const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                              const void* o, const void* to, const int64_t o_strides[4], const float* lse,
                              const float* mu, const void* dout, const void* dto, const int64_t do_strides[4],
                              void* dq, void* dk, void* dv, void* dtq, void* dtk, void* dtv,
                              const int64_t dq_strides[4], const int64_t dk_strides[4], const int64_t dv_strides[4],
                              float sm_scale, void* stream) {
  return bwd_impl(dtype, B, H, Lq, Lk, D, q, k, v, tq, tk, tv, q_strides, k_strides, v_strides, o, to, o_strides, lse,
                  mu, dout, dto, do_strides, dq, dk, dv, dtq, dtk, dtv, dq_strides, dk_strides, dv_strides, sm_scale,
                  nullptr, 0, stream, true);
}

int dmad_rmsnorm_rope_jvp(int dtype, int64_t rows, int64_t L, int64_t H, int64_t D, const void* y, const void* ty,
                          int64_t y_stride, const void* weight, const float* freqs, float eps, void* out, void* tout,
                          int64_t out_stride, void* stream) {
  if (dtype != DMAD_BF16 && dtype != DMAD_F16) return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if (rows < 0 || H <= 0 || D <= 0) return fail(DMAD_ERR_INVALID, "bad sizes rows=%lld H=%lld D=%lld", (long long)rows,
                                                (long long)H, (long long)D);
  if (D % 8 != 0 || D > 512) return fail(DMAD_ERR_UNSUPPORTED, "head dim must be a multiple of 8 up to 512, got %lld",
                                         (long long)D);
  const int64_t C = H * D;
  if (C > 64 * 8 * dmad::kPrologueMaxChunks)
    return fail(DMAD_ERR_UNSUPPORTED, "model dim H*D = %lld exceeds %d", (long long)C, 64 * 8 * dmad::kPrologueMaxChunks);
  if ((ty == nullptr) != (tout == nullptr)) return fail(DMAD_ERR_INVALID, "ty and tout must be both set or both null");
  if (!(eps >= 0.f)) return fail(DMAD_ERR_INVALID, "eps must be non-negative");
  if (rows == 0) return ok();
  if (y == nullptr || out == nullptr) return fail(DMAD_ERR_INVALID, "null pointer");
  if (weight == nullptr && freqs == nullptr) return fail(DMAD_ERR_INVALID, "weight and freqs are both null: nothing to do");
  for (const void* ptr : {y, ty, weight, (const void*)out, (const void*)tout})
    if (ptr != nullptr && ((uintptr_t)ptr & 15) != 0) return fail(DMAD_ERR_INVALID, "pointers must be 16-byte aligned");
  if (y_stride < C || out_stride < C || y_stride % 8 != 0 || out_stride % 8 != 0)
    return fail(DMAD_ERR_INVALID, "row strides must be multiples of 8 and at least H*D");
  if (freqs != nullptr && (L <= 0 || rows % L != 0))
    return fail(DMAD_ERR_INVALID, "rows (%lld) must be a multiple of L (%lld)", (long long)rows, (long long)L);
  if (rows > ((int64_t)1 << 34)) return fail(DMAD_ERR_UNSUPPORTED, "too many rows");
  dmad::PrologueParams p{};
  p.y = y;
  p.ty = ty;
  p.w = weight;
  p.freqs = freqs;
  p.out = out;
  p.tout = tout;
  p.rows = rows;
  p.y_stride = y_stride;
  p.o_stride = out_stride;
  p.L = freqs != nullptr ? (int)L : 1;
  p.C = (int)C;
  p.D = (int)D;
  p.eps = eps;
  p.inv_c = 1.0f / (float)C;
  hipStream_t s = (hipStream_t)stream;
  mark(0, false, s);
  const hipError_t e = dmad::launch_rmsnorm_rope(p, dtype, s);
  mark(0, true, s);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "prologue launch: %s", hipGetErrorString(e));
  return ok();
}

int dmad_probe_mfma(int dtype, int64_t blocks, int64_t mfmas_per_wave, float* sink, void* stream) {
  if (dtype != DMAD_BF16 && dtype != DMAD_F16) return fail(DMAD_ERR_UNSUPPORTED, "the MFMA probe takes bf16 or fp16");
  if (blocks < 1 || blocks > (1 << 20)) return fail(DMAD_ERR_INVALID, "blocks must be in [1, 2^20]");
  if (mfmas_per_wave < 256 || mfmas_per_wave % 256 != 0 || mfmas_per_wave > ((int64_t)1 << 30))
    return fail(DMAD_ERR_INVALID, "mfmas_per_wave must be a positive multiple of 256 up to 2^30");
  if (sink == nullptr) return fail(DMAD_ERR_INVALID, "sink: null pointer");
  const hipError_t e = dmad::launch_mfma_probe(dtype == DMAD_F16, (int)blocks, (int)(mfmas_per_wave / 256), sink,
                                               (hipStream_t)stream);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "probe launch: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
