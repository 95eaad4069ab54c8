// C ABI entry points (include/dmad_attn.h): argument validation, workspace
// carving and kernel dispatch. Nothing here allocates device memory.
#include <cstdarg>
#include <cstdio>
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
}  // namespace dmad

namespace {

thread_local std::string g_last_error;

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

// Checks one [B,H,L,D] operand: pointer, unit inner stride, 16-byte alignment
// of every row start, and that one (b, h) slice fits 32-bit byte offsets
// (with 256 rows of slack for tile overrun).
int check_operand(const char* name, const void* ptr, const int64_t* st, int64_t L, int64_t D) {
  if (ptr == nullptr) return fail(DMAD_ERR_INVALID, "%s: null pointer", name);
  if (st == nullptr) return fail(DMAD_ERR_INVALID, "%s: null strides", name);
  if (st[3] != 1) return fail(DMAD_ERR_INVALID, "%s: stride of the head dim must be 1, got %lld", name, (long long)st[3]);
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0) return fail(DMAD_ERR_INVALID, "%s: negative stride %lld", name, (long long)st[i]);
    if (st[i] % 8 != 0)
      return fail(DMAD_ERR_INVALID, "%s: strides must be multiples of 8 elements (16 bytes), got %lld", name,
                  (long long)st[i]);
  }
  if (L > 1 && st[2] < D) return fail(DMAD_ERR_INVALID, "%s: rows overlap (stride %lld < D %lld)", name, (long long)st[2], (long long)D);
  if (((uintptr_t)ptr & 15) != 0) return fail(DMAD_ERR_INVALID, "%s: base pointer must be 16-byte aligned", name);
  if (((L + 256) * st[2] + D) * 2 >= kMaxHeadBytes)
    return fail(DMAD_ERR_UNSUPPORTED, "%s: one (batch, head) slice spans more than 2 GiB", name);
  return DMAD_OK;
}

int64_t fwd_ws_bytes(int mode, int64_t B, int64_t H, int64_t Lk, int64_t Dv) {
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

}  // namespace

extern "C" {

int dmad_abi_version(void) { return 1; }

const char* dmad_last_error(void) { return g_last_error.c_str(); }

int dmad_attn_fwd_workspace_bytes(int mode, int64_t B, int64_t H, int64_t Lk, int64_t Dv, size_t* bytes) {
  if (bytes == nullptr) return fail(DMAD_ERR_INVALID, "bytes: null pointer");
  if (mode < DMAD_FWD_PLAIN || mode > DMAD_FWD_JVP_KV_TANGENT_ZERO) return fail(DMAD_ERR_INVALID, "unknown mode %d", mode);
  if (B < 0 || H < 0 || Lk < 0 || !head_dim_ok(Dv)) return fail(DMAD_ERR_INVALID, "bad sizes");
  *bytes = (size_t)fwd_ws_bytes(mode, B, H, Lk, Dv);
  return ok();
}

int dmad_attn_jvp_fwd(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv,
                      const void* q, const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4], void* o,
                      void* to, const int64_t o_strides[4], float* lse, float* mu, float sm_scale, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (dtype != DMAD_BF16 && dtype != DMAD_F16) return fail(DMAD_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  if (mode < DMAD_FWD_PLAIN || mode > DMAD_FWD_JVP_KV_TANGENT_ZERO) return fail(DMAD_ERR_INVALID, "unknown mode %d", mode);
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0) return fail(DMAD_ERR_INVALID, "negative size");
  if (!head_dim_ok(Dqk) || !head_dim_ok(Dv))
    return fail(DMAD_ERR_UNSUPPORTED, "head dims must be in {16,32,64,128,256}, got Dqk=%lld Dv=%lld", (long long)Dqk,
                (long long)Dv);
  if (!(sm_scale > 0.f)) return fail(DMAD_ERR_UNSUPPORTED, "sm_scale must be positive");
  if (B == 0 || H == 0 || Lq == 0) return ok();
  if (Lk == 0) return fail(DMAD_ERR_INVALID, "Lk must be at least 1");
  if (B * H > ((int64_t)1 << 24) || Lq >= ((int64_t)1 << 26) || Lk >= ((int64_t)1 << 26))
    return fail(DMAD_ERR_UNSUPPORTED, "sizes too large");
  const bool jvp = mode != DMAD_FWD_PLAIN, kvt = mode == DMAD_FWD_JVP;
  int rc;
  if ((rc = check_operand("q", q, q_strides, Lq, Dqk))) return rc;
  if ((rc = check_operand("k", k, k_strides, Lk, Dqk))) return rc;
  if ((rc = check_operand("v", v, v_strides, Lk, Dv))) return rc;
  if ((rc = check_operand("o", o, o_strides, Lq, Dv))) return rc;
  if (jvp) {
    if ((rc = check_operand("tq", tq, q_strides, Lq, Dqk))) return rc;
    if ((rc = check_operand("to", to, o_strides, Lq, Dv))) return rc;
    if (mu == nullptr) return fail(DMAD_ERR_INVALID, "mu: null pointer");
  }
  if (kvt) {
    if ((rc = check_operand("tk", tk, k_strides, Lk, Dqk))) return rc;
    if ((rc = check_operand("tv", tv, v_strides, Lk, Dv))) return rc;
  }
  if (lse == nullptr) return fail(DMAD_ERR_INVALID, "lse: null pointer");
  const int64_t need = fwd_ws_bytes(mode, B, H, Lk, Dv);
  if (workspace == nullptr || (int64_t)workspace_bytes < need)
    return fail(DMAD_ERR_WORKSPACE, "workspace needs %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  if (((uintptr_t)workspace & 255) != 0) return fail(DMAD_ERR_INVALID, "workspace must be 256-byte aligned");
  const int64_t dvp = Dv < 32 ? 32 : Dv, lkp = round_up(Lk, kLkAlign);
  if (dvp * lkp * 2 >= kMaxHeadBytes) return fail(DMAD_ERR_UNSUPPORTED, "Lk too large");

  dmad::FwdLaunchFn fn = pick_fwd(dtype, Dqk, Dv, mode);
  if (fn == nullptr) return fail(DMAD_ERR_UNSUPPORTED, "no kernel for Dqk=%lld Dv=%lld", (long long)Dqk, (long long)Dv);

  hipStream_t s = (hipStream_t)stream;
  const int BH = (int)(B * H);
  char* ws = (char*)workspace;
  const int64_t vt_bytes = round_up(B * H * dvp * lkp * 2, 256);
  dmad::TransposeParams tp{v, ws, v_strides[0], v_strides[1], v_strides[2], (int)H, (int)Lk, (int)Dv, (int)lkp, (int)dvp};
  hipError_t e = dmad::launch_transpose_pad(tp, BH, s);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "transpose launch: %s", hipGetErrorString(e));
  if (kvt) {
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
  const int64_t nqt = (Lq + 127) / 128;
  if (nqt * BH >= ((int64_t)1 << 31)) return fail(DMAD_ERR_UNSUPPORTED, "grid too large");
  e = fn(p, (int)(nqt * BH), s);
  if (e != hipSuccess) return fail(DMAD_ERR_HIP, "attention launch: %s", hipGetErrorString(e));
  return ok();
}

int dmad_attn_fwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv, const void* q,
                  const void* k, const void* v, const int64_t q_strides[4], const int64_t k_strides[4],
                  const int64_t v_strides[4], void* o, const int64_t o_strides[4], float* lse, float sm_scale,
                  void* workspace, size_t workspace_bytes, void* stream) {
  return dmad_attn_jvp_fwd(dtype, DMAD_FWD_PLAIN, B, H, Lq, Lk, Dqk, Dv, q, k, v, nullptr, nullptr, nullptr,
                           q_strides, k_strides, v_strides, o, nullptr, o_strides, lse, nullptr, sm_scale, workspace,
                           workspace_bytes, stream);
}

int dmad_attn_bwd_workspace_bytes(int full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, size_t* bytes) {
  (void)full; (void)B; (void)H; (void)Lq; (void)Lk; (void)D;
  if (bytes) *bytes = 0;
  return fail(DMAD_ERR_UNSUPPORTED, "backward not built yet");
}

int dmad_attn_jvp_bwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q,
                      const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                      const void* o, const void* to, const int64_t o_strides[4], const float* lse, const float* mu,
                      const void* dout, const void* dto, const int64_t do_strides[4], void* dq, void* dk, void* dv,
                      void* dtq, void* dtk, void* dtv, const int64_t dq_strides[4], const int64_t dk_strides[4],
                      const int64_t dv_strides[4], float sm_scale, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return fail(DMAD_ERR_UNSUPPORTED, "backward not built yet");
}

}  // extern "C"
