/*
 * dmad_attn.h -- C ABI of the MI355X (gfx950) flash-attention JVP library.
 *
 * The library replaces the device side of the reference op
 *   _attention.apply(q, k, v, tq, tk, tv, sm_scale=None, magi_mask=None) -> (o, to)
 * (train/wan/rcm/utils/flash_attention_jvp_triton.py:450-582) and of the
 * plain attention it is paired with. All buffers are owned by the caller;
 * the library allocates nothing and keeps no state between calls. Every
 * call enqueues work on `stream` (a hipStream_t) and returns without a host
 * synchronisation.
 *
 * Tensor convention: logical shape [B, H, L, D] (BHSD) with arbitrary element
 * strides given as int64_t[4] = {stride_b, stride_h, stride_l, stride_d}.
 * stride_d must be 1. Tangent tensors share the strides of their primal
 * (the reference asserts the same, :473-474). lse and mu are dense
 * [B, H, Lq] float32.
 *
 * Every function returns DMAD_OK (0) or a non-zero status; dmad_last_error()
 * then describes the failure (thread-local, valid until the next call).
 */
#ifndef DMAD_ATTN_H
#define DMAD_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dmad_status {
  DMAD_OK = 0,
  DMAD_ERR_INVALID = 1,     /* bad pointer, shape, stride or argument */
  DMAD_ERR_UNSUPPORTED = 2, /* head dim / dtype / size outside what the kernels handle */
  DMAD_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  DMAD_ERR_HIP = 4          /* the HIP runtime reported an error at launch */
};

/* Operand types. bf16 and fp16: bf16/fp16 MFMAs with fp32 accumulation, every
 * entry point. fp32 (what the reference's Triton forward also accepts, and what
 * rcm/utils/attention.py:120-167 routes to PyTorch's SDPA): fp32 MFMAs, the
 * forward in every mode, dense and block-sparse, and the dO-only backward; the
 * full-derivative backward and the RMSNorm/RoPE prologue are DMAD_ERR_UNSUPPORTED.
 * Operand rows must start 16-byte aligned: strides are multiples of 8 elements
 * for bf16/fp16 and of 4 for fp32. fp32 needs no forward workspace. */
enum dmad_dtype { DMAD_BF16 = 0, DMAD_F16 = 1, DMAD_F32 = 2 };

enum dmad_fwd_mode {
  DMAD_FWD_PLAIN = 0,           /* O and LSE only */
  DMAD_FWD_JVP = 1,             /* O, tangent output, LSE, mu */
  DMAD_FWD_JVP_KV_TANGENT_ZERO = 2 /* as DMAD_FWD_JVP with tk = tv = 0 (tk, tv unused) */
};

/* Version of this ABI; bumped when a signature changes. */
int dmad_abi_version(void);

/* Description of the last failure on this thread ("" if none). */
const char* dmad_last_error(void);

/* Bytes of workspace dmad_attn_jvp_fwd / dmad_attn_fwd / dmad_attn_jvp_fwd_magi need
 * for these sizes with bf16/fp16 operands: 0 for Dqk = Dv = 64, 128 or 256 (V is read
 * in place; the workspace pointer may then be NULL), else room for transposed copies
 * of V (and Vd). fp32 operands need none. It covers every forward entry
 * (dmad_attn_fwd_plan gives the exact size of one launch). */
int dmad_attn_fwd_workspace_bytes(int mode, int64_t B, int64_t H, int64_t Lk, int64_t Dqk, int64_t Dv, size_t* bytes);

/*
 * Forward (+JVP): replaces the `_attn_fwd` launch of _attention.forward
 * (flash_attention_jvp_triton.py:463-499, kernel :107-232).
 *   o, to : [B,H,Lq,Dv] outputs in the input dtype (to unused in DMAD_FWD_PLAIN)
 *   lse   : natural-log logsumexp of the scaled scores, [B,H,Lq] float32
 *   mu    : r/l = rowsum(P * Sdot), [B,H,Lq] float32 (JVP modes; needed by the
 *           full backward)
 * Dqk, Dv in {16, 32, 64, 128, 256} (as asserted at :471-472); sm_scale > 0.
 */
int dmad_attn_jvp_fwd(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv,
                      const void* q, const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4], void* o,
                      void* to, const int64_t o_strides[4], float* lse, float* mu, float sm_scale, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Block-sparse forward (+JVP): replaces the `_attn_fwd_magi` launch of
 * _attention.forward with a MagiMask (flash_attention_jvp_triton.py:502-531,
 * kernel :242-409). The tables are the MagiMask fields
 * (train/wan/rcm/utils/magimask.py:240-283), int32 in device memory:
 *   q_ranges [G][2]  query range [q0, q1) of group g
 *   k_ranges [R][2]  key ranges; group g uses k_ranges[qk_map[g] .. qk_map[g+1])
 *   qk_map   [G+1]
 *   task_group, task_qtile [T]  one task per (group, 128-query tile) that
 *                    intersect; the tiles are block_m = 128 rows (the
 *                    reference's BLOCK_M; other values are DMAD_ERR_UNSUPPORTED)
 * Query row i of a task's tile attends to the keys of its group's ranges and
 * is stored only if it lies in the group's query range; rows no task covers
 * are left untouched (the reference allocates o, to, lse uninitialised). A
 * group without keys in [0, Lk) gets o = to = 0, lse = -inf, mu = 0. Ranges
 * are clipped to the sequences and table indices to the tables, so malformed
 * tables cannot read outside them. mode: DMAD_FWD_JVP or
 * DMAD_FWD_JVP_KV_TANGENT_ZERO (the reference has no plain masked forward).
 * Workspace as dmad_attn_fwd_workspace_bytes.
 */
int dmad_attn_jvp_fwd_magi(int dtype, int mode, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv,
                           const void* q, const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                           const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                           void* o, void* to, const int64_t o_strides[4], float* lse, float* mu, float sm_scale,
                           const int32_t* q_ranges, const int32_t* k_ranges, const int32_t* qk_map, int64_t G,
                           int64_t R, const int32_t* task_group, const int32_t* task_qtile, int64_t T,
                           int64_t block_m, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Plain forward (O and LSE), the attention used by the non-JVP Wan forward
 * (train/wan/rcm/utils/jvp_helper.py:305-308 and rcm/utils/attention.py:120-167).
 */
int dmad_attn_fwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t Dqk, int64_t Dv, const void* q,
                  const void* k, const void* v, const int64_t q_strides[4], const int64_t k_strides[4],
                  const int64_t v_strides[4], void* o, const int64_t o_strides[4], float* lse, float sm_scale,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace dmad_attn_jvp_bwd needs. full: 0 = dO-only gradients,
 * 1 = full derivative (dto given), 2 = full derivative plus tangent gradients
 * (dto, dtq, dtk, dtv given). The per-row statistics always; transposed copies
 * of Q, dO, K (and the tangents) for the full derivative of head dims other
 * than 128 and for the dO-only gradients of head dims other than 64 and 128.
 * The size is that of bf16/fp16 operands and bounds every dtype: fp32 operands
 * need only the statistics, round_up(B*H*round_up(Lq,64)*8, 256) bytes
 * (dmad_attn_bwd_plan reports the exact figure for each dtype). */
int dmad_attn_bwd_workspace_bytes(int full, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, size_t* bytes);

/*
 * Backward: replaces _attention.backward (flash_attention_jvp_triton.py:534-579),
 * whose arithmetic the reference delegates to flash-attn's _flash_attn_backward
 * (:540-555) and _flash_attn_varlen_backward (:556-578).
 *   dto == NULL : dO-only gradients dq, dk, dv, exactly what the reference
 *                 computes (its cotangent of `to` is discarded, :535).
 *   dto != NULL : full derivative of (o, to) w.r.t. (q, k, v), and, when dtq,
 *                 dtk, dtv are non-NULL, w.r.t. the tangents (tq, tk, tv).
 * Requires Dqk == Dv == D (as asserted at :537). o, to, lse, mu are the
 * outputs of dmad_attn_jvp_fwd for the same inputs. Gradients have the
 * strides given in dq_strides (shared by dq, dtq), dk_strides (dk, dtk) and
 * dv_strides (dv, dtv); do/dto share do_strides. B, H or Lq = Lk = 0 is a
 * no-op; Lq = 0 with Lk > 0 (where dk, dv are zero) is DMAD_ERR_INVALID: the
 * caller fills the zeros. A workspace larger than dmad_attn_bwd_workspace_bytes
 * by whole slices of dmad_attn_bwd_score_bytes selects the stored-score passes
 * (128-wide bf16/fp16 heads; the gradients agree with the recomputing passes
 * to rounding).
 */
int dmad_attn_jvp_bwd(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q,
                      const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                      const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                      const void* o, const void* to, const int64_t o_strides[4], const float* lse, const float* mu,
                      const void* dout, const void* dto, const int64_t do_strides[4], void* dq, void* dk, void* dv,
                      void* dtq, void* dtk, void* dtv, const int64_t dq_strides[4], const int64_t dk_strides[4],
                      const int64_t dv_strides[4], float sm_scale, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Size of the static device scratch of dmad_attn_jvp_bwd_noalloc (64 MiB). */
#define DMAD_BWD_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * Allocation-free backward. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc). Same arguments, results and
 * errors as dmad_attn_jvp_bwd without the workspace: the per-row statistics
 * (and any transposed copies) go to a static device array of
 * DMAD_BWD_SCRATCH_BYTES in the library, one copy per GPU, held until the
 * process ends. Problems whose workspace (dmad_attn_bwd_plan's workspace_bytes
 * for the dtype) exceeds that size fail with DMAD_ERR_UNSUPPORTED (e.g. the dO-only backward of 64- and 128-wide
 * heads fits up to B*H*Lq ~ 8.4M rows: Wan2.1-14B at 720p needs 24 MB; the full
 * derivative of 128-wide heads with tangent gradients up to ~2.8M rows). The
 * call allocates nothing; the first call on a device looks up that device's
 * copy of the array. Calls that overlap on one GPU (concurrent streams or
 * threads) share the array and race; serialise them. `stream` must belong to
 * the current device.
 */
int dmad_attn_jvp_bwd_noalloc(int dtype, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, const void* q,
                              const void* k, const void* v, const void* tq, const void* tk, const void* tv,
                              const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                              const void* o, const void* to, const int64_t o_strides[4], const float* lse,
                              const float* mu, const void* dout, const void* dto, const int64_t do_strides[4],
                              void* dq, void* dk, void* dv, void* dtq, void* dtk, void* dtv,
                              const int64_t dq_strides[4], const int64_t dk_strides[4], const int64_t dv_strides[4],
                              float sm_scale, void* stream);

/*
 * Fused attention-input prologue: RMSNorm over the model dim C = H*D, then the
 * interleaved rotary embedding, for a Linear output and its tangent in one HBM
 * pass. Replaces WanRMSNorm._forward under torch.func.jvp
 * (train/wan/rcm/networks/wan2pt1_jvp.py:207-216, applied to q and k at
 * :312-317) followed by apply_rope_with_tangent (train/wan/rcm/utils/rope.py:
 * 56-70, 106-114) as MinimalA2AAttnOpWithT.forward applies it
 * (train/wan/rcm/utils/jvp_helper.py:180-196); the rounding points are the
 * reference's (norm in float32, cast to the input type, times the weight in
 * the input type; rotation in float32, cast back).
 *   y, ty     : [rows, C] inputs (rows = B*L), row stride y_stride elements;
 *               ty == NULL computes the primal only (then tout must be NULL)
 *   weight    : [C] RMSNorm weight, same dtype; NULL: no norm, the rotation
 *               alone (apply_rope_with_tangent, rope.py:106-114, by itself)
 *   freqs     : [L, D/2] float32 angles, token l = row mod L; NULL: no rotation
 *               (weight and freqs may not both be NULL)
 *   out, tout : [rows, C] = [B, L, H, D] outputs, row stride out_stride
 * D a multiple of 8 and <= 512, C = H*D <= 10240, pointers 16-byte aligned,
 * strides multiples of 8 and >= C, rows a multiple of L when freqs is given.
 */
int dmad_rmsnorm_rope_jvp(int dtype, int64_t rows, int64_t L, int64_t H, int64_t D, const void* y, const void* ty,
                          int64_t y_stride, const void* weight, const float* freqs, float eps, void* out, void* tout,
                          int64_t out_stride, void* stream);

/*
 * Launch plan of a call (host only: needs no GPU). The library chooses its
 * kernels from a fixed per-shape table -- the dtype, the mode, the mask, Lq,
 * Lk and the head dims -- where the reference autotunes its Triton forward
 * over 48 configs keyed on (SEQ_LEN_Q, SEQ_LEN_KV, HEAD_DIM_QK, HEAD_DIM_V)
 * (train/wan/rcm/utils/flash_attention_jvp_triton.py:98-107). The entry points
 * launch what the plan reports. Kernel names are static strings.
 */
typedef struct dmad_plan {
  const char* kernel;        /* forward kernel; backward: key-stationary pass (dK, dV) */
  const char* kernel2;       /* backward: query-stationary pass (dQ [, dQd]); forward: NULL */
  const char* kernel3;       /* backward with tangent gradients: key pass on (dOd, rho) for dKd, dVd; else NULL */
  const char* kernel4;       /* ... and its query pass for dQd where kernel2 does not give it; else NULL */
  int64_t grid;              /* workgroups of `kernel` (and of kernel3) */
  int64_t grid2;             /* workgroups of `kernel2` (and of kernel4); 0 for the forward */
  int32_t xcd_order;         /* 1: work items dealt contiguously per XCD; 0: head-major (of `kernel`) */
  int32_t xcd_order2;        /* the same for `kernel2` */
  int32_t chunks;            /* forward: workgroups per query tile (column chunks of a wide V); the query tile
                                is 128 rows (a block-sparse task), 64 for fp32 with 256-wide Q, K in the JVP
                                modes (two per task) */
  int32_t transposed_copies; /* operands copied transposed into the workspace before the kernels */
  int64_t workspace_bytes;   /* workspace the call needs */
  int64_t score_slices;      /* backward (dmad_attn_bwd_plan_ws): (b, h) slices per launch pair of the stored-score
                                passes (`kernel` stores dS [, dSd], `kernel2` reads them back, `kernel3` with tangent
                                gradients reads the stored dSd; grids are per pair); 0: the query pass recomputes
                                the scores */
} dmad_plan;

/* Plan of dmad_attn_jvp_fwd / dmad_attn_fwd (magi_tasks < 0) or of
 * dmad_attn_jvp_fwd_magi with magi_tasks tasks; mode as there. */
int dmad_attn_fwd_plan(int dtype, int mode, int64_t magi_tasks, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                       int64_t Dqk, int64_t Dv, dmad_plan* plan);

/* Plan of dmad_attn_jvp_bwd with the minimum workspace; full and tangent_grads: 0 or 1 (dto and dtq/dtk/dtv
 * given). */
int dmad_attn_bwd_plan(int dtype, int full, int tangent_grads, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                       dmad_plan* plan);

/* Plan of dmad_attn_jvp_bwd called with `workspace_bytes` of workspace (see dmad_attn_bwd_score_bytes). */
int dmad_attn_bwd_plan_ws(int dtype, int full, int tangent_grads, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                          int64_t D, size_t workspace_bytes, dmad_plan* plan);

/*
 * Bytes of stored score gradients per (b, h) slice (no counterpart in the
 * reference; the reference's backward is flash-attn's, which recomputes).
 * For bf16/fp16 operands of 128-wide heads the backward's key pass can write
 * the dS (full = 1: and dSd) tiles it computes, in bf16/fp16, so that the
 * query pass becomes a streaming GEMM over them instead of recomputing S and
 * dP. dmad_attn_jvp_bwd takes that path when its workspace exceeds
 * dmad_attn_bwd_workspace_bytes by at least these bytes, processing as many
 * (b, h) slices per launch pair as the excess holds (e.g. Wan2.1-14B,
 * L = 32760: 2.15 GB per slice dO-only, 4.3 GB with dOd). 0 for other head dims
 * and for fp32 (the path does not exist there).
 */
int dmad_attn_bwd_score_bytes(int dtype, int full, int64_t Lq, int64_t Lk, int64_t D, size_t* bytes);

/*
 * Timing hook (no counterpart in the reference; for benchmarks and profilers
 * that time kernels live). `events` points to `count` hipEvent_t handles; while
 * set, every dmad_attn_jvp_fwd / dmad_attn_fwd / dmad_attn_jvp_bwd call on
 * this thread records events[2i] and events[2i+1] on its stream immediately
 * before and after its i-th main kernel, excluding the layout and statistics
 * passes. Main kernels in order: forward -> {attention}; backward -> {dK/dV
 * pass, dQ pass[, tangent dK/dV pass[, tangent dQ pass]]} (for 128-wide heads
 * the full derivative's dQ pass also gives dQd: no tangent dQ pass); a
 * backward on stored score gradients -> {dK/dV pass, dQ pass[, tangent dK/dV
 * pass]} once per launch pair. Kernels without a pair of events are not
 * timed. count <= 256; count = 0 (events may be NULL) stops.
 */
int dmad_set_kernel_events(void* const* events, int count);

/*
 * MFMA ceiling probe (no counterpart in the reference; a measurement aid for
 * benchmarks). Launches `blocks` workgroups of four waves on `stream`; every
 * wave issues `mfmas_per_wave` (a multiple of 256) back-to-back 32x32x16 MFMAs
 * of the dtype (DMAD_BF16 or DMAD_F16, 32768 flops each) on four independent
 * accumulators, with new operand bits every 32 MFMAs, and writes one float per
 * thread to `sink` (blocks * 256 floats). With one workgroup per CU it runs the
 * matrix units flat out under the board's power limit: the MFMA rate the
 * attention kernels can be measured against on the same board.
 */
int dmad_probe_mfma(int dtype, int64_t blocks, int64_t mfmas_per_wave, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DMAD_ATTN_H */
