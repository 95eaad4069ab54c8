"""Flash-attention JVP op for gfx950: drop-in for the reference ``_attention``.

Reference: ``train/wan/rcm/utils/flash_attention_jvp_triton.py:450-582``.
``_attention.apply(q, k, v, tq, tk, tv, sm_scale=None, magi_mask=None)`` returns
``(o, to)``: the attention output and its directional derivative along the
tangents ``(tq, tk, tv)``. Tensors are logical ``[B, H, L, D]`` with any
strides (the Wan callers pass ``[B, L, H, D]`` storage viewed as BHSD).

Device work is hand-written HIP (the forward+JVP kernel and its block-sparse
variant, the dK/dV and dQ backward passes) reached through the C ABI of
``libdmad_attn.so`` (``include/dmad_attn.h``); this module only checks
arguments, allocates outputs with the torch caching allocator and launches on
torch's current stream. There is no CPU or PyTorch fallback.

Differences from the reference, all additive:
  * ``tk``/``tv`` may be ``None`` (tangents of K and V known to be zero, as in
    Wan cross-attention): the forward then skips the two GEMMs they feed. O is
    the same bit for bit as with zero tangents; in bf16 ``to`` differs from the
    zero-tangent result by the rounding of P~ * Sd (formed without the softmax
    scale, which is applied once per row), as close to the exact value.
  * backward (``backward_mode`` for a scope, ``set_backward_mode`` for the
    process default): by default the reference's dO-only
    gradients, with the reference's saved tensors (q, k, v, o, LSE; the
    cotangent of ``to`` is ignored, :535), unless a tangent requires grad: then
    the full derivative, including the cotangent of ``to`` and gradients for
    the tangents (the reference returns None for them, :579). Mode "full" gives
    the full derivative whenever that cotangent arrives; mode "reference" never.
  * ``magi_mask`` (block-sparse masks, :502-531) runs the block-sparse kernel
    as the reference does (forward only: RuntimeError when q, k or v require
    grad, :504-505, and likewise when a tangent does). Masks built with any
    BLOCK_M are accepted (``dmad_amd.magimask.tasks_for_kernel``).
"""
from __future__ import annotations

import contextlib
import contextvars
import os
from typing import Iterator, Optional, Tuple

import torch

from . import _native as nat

_BACKWARD_MODES = ("auto", "reference", "full")
# process-wide default, and the mode of the innermost ``backward_mode`` scope of
# the calling thread or task (None outside any scope)
_DEFAULT_BACKWARD_MODE = "auto"
_SCOPED_BACKWARD_MODE: contextvars.ContextVar = contextvars.ContextVar("dmad_backward_mode", default=None)


def _check_backward_mode(mode: str) -> None:
    if mode not in _BACKWARD_MODES:
        raise ValueError(f"backward mode must be one of {_BACKWARD_MODES}, got {mode!r}")


@torch._dynamo.assume_constant_result
def _scoped_mode_at_trace() -> Optional[str]:
    return _SCOPED_BACKWARD_MODE.get()


def current_backward_mode() -> str:
    """The mode a forward called here would record: the innermost ``backward_mode``
    scope of this thread or task, else the process default.

    Under ``torch.compile`` the scope is read once, when the graph is traced
    (TorchDynamo cannot trace a context variable); the process default is a
    module global, which the compiled graph guards on, so ``set_backward_mode``
    retraces it.
    """
    m = _scoped_mode_at_trace() if torch.compiler.is_compiling() else _SCOPED_BACKWARD_MODE.get()
    return _DEFAULT_BACKWARD_MODE if m is None else m


@contextlib.contextmanager
def backward_mode(mode: str) -> Iterator[None]:
    """Scope in which forwards record ``mode`` for their backward (modes as in
    ``set_backward_mode``). The scope belongs to the calling thread or asyncio
    task (a ``contextvars`` variable): other threads keep their own mode, and
    scopes nest. The mode is read when the forward runs and kept on the autograd
    node, so a backward run after the scope has closed still follows it.
    """
    _check_backward_mode(mode)
    token = _SCOPED_BACKWARD_MODE.set(mode)
    try:
        yield
    finally:
        _SCOPED_BACKWARD_MODE.reset(token)


def set_backward_mode(mode: str) -> None:
    """Process-wide default of how ``attention``'s backward treats the cotangent
    of ``to`` (``backward_mode`` overrides it for a scope):

    "auto" (default): as the reference (dO-only gradients; only q, k, v, o and
        the LSE are kept for the backward) unless a tangent requires grad; then
        the full derivative, with gradients for the tangents.
    "reference": always as the reference (tangents get None).
    "full": the full derivative whenever the cotangent of ``to`` reaches the op
        (the tangents, ``to`` and mu are then kept for the backward too).
    """
    global _DEFAULT_BACKWARD_MODE
    _check_backward_mode(mode)
    _DEFAULT_BACKWARD_MODE = mode


# Device memory (bytes) the backward of 128-wide bf16/fp16 heads may take, per
# call and on top of its minimum workspace, for stored score gradients: its key
# pass then writes dS (and dSd) and the query pass reads them back instead of
# recomputing the scores, up to as many (b, h) slices per launch pair as fit. 0
# turns the path off. Environment default: DMAD_BWD_SCORE_BUDGET_MB (36 GiB, an eighth
# of an MI355X's HBM: sixteen dO-only or eight full-derivative slices of a Wan2.1-14B
# layer at 480p, 2.15 / 4.3 GB each, or three dO-only slices at 720p, 11.5 GB each;
# 18 GiB held only one 720p slice, too few key-pass workgroups for a launch pair).
_SCORE_BUDGET = int(os.environ.get("DMAD_BWD_SCORE_BUDGET_MB", "36864")) << 20


def set_backward_score_budget(nbytes: int) -> None:
    """Set how much device memory (bytes) each backward may use for stored score gradients
    (0: the query pass recomputes the scores; the memory is workspace, freed with the call)."""
    global _SCORE_BUDGET
    if int(nbytes) < 0:
        raise ValueError("the budget must be >= 0")
    _SCORE_BUDGET = int(nbytes)


def backward_score_budget() -> int:
    return _SCORE_BUDGET


# The dO-only backward stores its scores from this many queries and keys on: at 1024
# the recomputing query pass measured as fast (B=4, H=32, fp16: within 1% either way;
# 2048: the stored scores 4-7% faster). The stores cost the key pass about 15% of its
# time; the full derivative's query pass saves more than that at every length.
_SCORE_MIN_LEN_DOUT_ONLY = 2048


# A launch pair covering fewer slices than B*H should give its key pass at least
# this many workgroups (four per CU): with fewer, the last partly filled round of
# every pair idles a large share of the CUs (720p, one 11.4 GB slice per pair:
# 591 workgroups, 2.3 rounds), and the recomputing passes are kept instead.
_SCORE_MIN_KEY_WORKGROUPS = 4 * 256


def _score_bytes(code: int, full: bool, B: int, H: int, Lq: int, Lk: int, D: int) -> int:
    """Workspace bytes for stored score gradients within the budget (whole (b, h) slices)."""
    if not full and min(Lq, Lk) < _SCORE_MIN_LEN_DOUT_ONLY:
        return 0
    one = nat.bwd_score_bytes(code, full, Lq, Lk, D) if _SCORE_BUDGET > 0 else 0
    if one == 0 or _SCORE_BUDGET < one:
        return 0
    n = _score_slices(B * H, min(B * H, _SCORE_BUDGET // one), Lq, Lk)
    if n < B * H and n * ((Lk + 127) // 128) < _SCORE_MIN_KEY_WORKGROUPS:
        return 0
    return n * one


def _backward_workspace(code: int, ws_mode: int, B: int, H: int, Lq: int, Lk: int, D: int, device):
    """(pointer, size, owner) of a backward's workspace: the minimum plus the stored score
    gradients the budget allows. The stored scores only save time, so when the device cannot
    hold them the call takes the minimum and the query pass recomputes the scores (the same
    dQ bit for bit); an allocation failure of the minimum itself propagates."""
    base = nat.bwd_workspace_bytes_of(code, ws_mode, B, H, Lq, Lk, D)
    extra = _score_bytes(code, ws_mode > 0, B, H, Lq, Lk, D)
    if extra > 0:
        try:
            return nat.workspace(base + extra, device)
        except torch.cuda.OutOfMemoryError:
            pass
    return nat.workspace(base, device)


def _score_slices(bh: int, n_max: int, Lq: int, Lk: int) -> int:
    """(b, h) slices per launch pair, at most n_max: the count whose pairs fill the 256 CUs
    best. A pair of n slices runs n * key tiles key-pass workgroups and n * query-block
    pairs query-pass workgroups, one per CU at a time; every partly filled last round
    costs a whole round. Rounds are weighted by their measured lengths (a key-pass round
    ~1.4 query-pass rounds at equal Lq = Lk); ties go to more slices."""
    nkt = (Lk + 127) // 128
    nqw = ((Lq + 127) // 128 + 1) // 2

    def rounds(m):
        return 1.4 * (-(-m * nkt // 256)) + (-(-m * nqw // 256))

    best, best_cost = n_max, None
    for n in range(n_max, max(1, n_max // 2) - 1, -1):
        full, rest = divmod(bh, n)
        cost = full * rounds(n) + (rounds(rest) if rest else 0.0)
        if best_cost is None or cost < best_cost - 1e-9:
            best, best_cost = n, cost
    return best


def backward_plan(dtype: torch.dtype, B: int, H: int, Lq: int, Lk: int, D: int, full: bool = False,
                  tangent_grads: bool = False) -> dict:
    """The launch plan of the backward this op runs for these sizes under the current score
    budget (no GPU needed): kernels, grids, workspace and ``score_slices``; with score slices
    the key and query passes run ``pairs`` times, one pair per group of slices."""
    code = nat.dtype_code(dtype)
    mode = (2 if tangent_grads else 1) if full else 0
    ws = nat.bwd_workspace_bytes_of(code, mode, B, H, Lq, Lk, D) + _score_bytes(code, full, B, H, Lq, Lk, D)
    pl = nat.bwd_plan(code, B, H, Lq, Lk, D, full=full, tangent_grads=full and tangent_grads, workspace_bytes=ws)
    n = pl["score_slices"]
    pl["pairs"] = -(-(B * H) // n) if n else 1
    return pl


def set_reference_backward(flag: bool) -> None:
    """True: ``set_backward_mode("reference")``; False: ``set_backward_mode("full")``."""
    set_backward_mode("reference" if flag else "full")


_HEAD_DIMS = {16, 32, 64, 128, 256}

# Largest head dim the full-derivative backward kernels are built for.
FULL_BWD_MAX_HEAD_DIM = 128
_warned_full_fallback = False


def _full_backward_unavailable(mode: str, dqk: int, dv: int, dtype: torch.dtype) -> bool:
    """Backward mode for inputs the full derivative does not cover (head dims
    above 128, fp32 operands).

    Mode "auto" falls back to the reference's backward (dO-only gradients, None
    for the tangents, :534-579) with a one-time warning, so the op runs wherever
    the reference runs; mode "full" asked for the full derivative explicitly and
    raises here, in the forward, before any work is done.
    """
    global _warned_full_fallback
    what = (f"head dims up to {FULL_BWD_MAX_HEAD_DIM} (got Dqk={dqk}, Dv={dv})" if max(dqk, dv) > FULL_BWD_MAX_HEAD_DIM
            else f"bfloat16 and float16 operands (got {dtype})")
    if mode == "full":
        raise NotImplementedError(
            f"the full-derivative backward supports {what}; use backward mode 'auto' or 'reference' "
            "for the reference's dO-only gradients"
        )
    if not _warned_full_fallback:
        import warnings

        warnings.warn(
            f"the full-derivative backward supports {what}: the tangents get no gradients and the "
            "cotangent of `to` is ignored (the reference backward's behaviour)",
            stacklevel=3,
        )
        _warned_full_fallback = True
    return False


_layout_ok: dict = {}

# The kernels address one (batch, head) slice with 32-bit byte offsets: the rows
# a slice spans, plus 256 rows of slack for tile overrun, must stay under 2 GiB.
MAX_SLICE_BYTES = 1 << 31


def slice_fits(rows: int, row_stride: int, head_dim: int, elem_size: int) -> bool:
    """Whether a [rows, head_dim] slice with this row stride (elements) fits the kernels'
    32-bit offsets. Wan's BSHD views have row stride H*D, so one head of a 14B layer
    (H=40, D=128, bf16) stops fitting at about 209k tokens; a contiguous BHSD copy (row
    stride D) fits up to about 8.4M."""
    return ((rows + 256) * row_stride + head_dim) * elem_size < MAX_SLICE_BYTES


def _kernel_ready(t: torch.Tensor) -> bool:
    """Unit inner stride, 16-byte aligned rows and a (batch, head) slice within the 32-bit
    offsets (what the kernels load from). The layout part is a function of the strides, the
    element size and the last two sizes, decided once per key (this sits on every call's
    host path)."""
    st = t.stride()
    key = (st, t.element_size(), t.shape[-2], t.shape[-1])
    ok = _layout_ok.get(key)
    if ok is None:
        per16 = 16 // key[1]
        ok = st[-1] == 1 and all(x % per16 == 0 for x in st[:-1])
        ok = ok and slice_fits(key[2], st[-2], key[3], key[1])
        if len(_layout_ok) > 4096:
            _layout_ok.clear()
        _layout_ok[key] = ok
    return ok and t.data_ptr() % 16 == 0


def _prep(*ts):
    """Copy operands whose layout the kernels cannot read (among them views whose
    (batch, head) slice spans 2 GiB or more: the copy is contiguous BHSD, whose slice is
    only L*D elements); tangents stay stride-identical to their primals because both go
    through the same rule."""
    return tuple(None if t is None else (t if _kernel_ready(t) else t.contiguous()) for t in ts)


def _pair(x, tx):
    """(primal, tangent) in a layout the kernels read, with equal strides."""
    if tx is None:
        return (x if _kernel_ready(x) else x.contiguous()), None
    if x.stride() == tx.stride() and _kernel_ready(x) and _kernel_ready(tx):
        return x, tx
    return x.contiguous(), tx.contiguous()


def _fwd_ws_bytes(dtype, mode, B, H, Lk, Dqk, Dv) -> int:
    """Workspace of any forward entry (the block-sparse one included): transposed V copies of
    the bf16/fp16 kernels for some head dims; none for fp32."""
    return 0 if dtype == torch.float32 else nat.fwd_workspace_bytes(mode, B, H, Lk, Dqk, Dv)


_dense_needs_ws: dict = {}


def _fwd_dense_ws_bytes(dtype, mode, B, H, Lk, Dqk, Dv) -> int:
    """Workspace of the dense forward: the launch plan says whether its kernel reads V in
    place (asked once per dtype, mode and head dims; then none is allocated)."""
    key = (dtype, mode, Dqk, Dv)
    need = _dense_needs_ws.get(key)
    if need is None:
        need = dtype != torch.float32 and \
            nat.fwd_plan(nat.dtype_code(dtype), mode, 1, 1, 128, 128, Dqk, Dv)["workspace_bytes"] > 0
        _dense_needs_ws[key] = need
    return _fwd_ws_bytes(dtype, mode, B, H, Lk, Dqk, Dv) if need else 0


def _check_device(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "dmad_amd attention runs on the GPU only (HIP kernels); got a tensor on " + str(t.device)
            )


def jvp_attention_forward(q, k, v, tq, tk, tv, sm_scale, need_mu=True):
    """Launch the forward(+JVP) kernel; returns (o, to, lse, mu).

    ``tq is None`` selects the plain forward (to and mu are None).
    """
    B, H, Lq, Dqk = q.shape
    Lk, Dv = v.shape[-2], v.shape[-1]
    _check_device(q, k, v, tq, tk, tv)
    code = nat.dtype_code(q.dtype)
    if tq is None:
        mode = nat.DMAD_FWD_PLAIN
    elif tk is None and tv is None:
        mode = nat.DMAD_FWD_JVP_KV_TANGENT_ZERO
    else:
        if tk is None:
            tk = torch.zeros_like(k)
        if tv is None:
            tv = torch.zeros_like(v)
        mode = nat.DMAD_FWD_JVP
    q, tq = _pair(q, tq)
    k, tk = _pair(k, tk)
    v, tv = _pair(v, tv)
    dev = q.device
    o = torch.empty((B, H, Lq, Dv), device=dev, dtype=q.dtype)
    to = torch.empty_like(o) if tq is not None else None
    lse = torch.empty((B, H, Lq), device=dev, dtype=torch.float32)
    mu = torch.empty_like(lse) if tq is not None else None
    lib = nat.lib()
    ws_ptr, ws_size, ws = nat.workspace(_fwd_dense_ws_bytes(q.dtype, mode, B, H, Lk, Dqk, Dv), dev)
    nat.check(
        lib.dmad_attn_jvp_fwd(
            code, mode, B, H, Lq, Lk, Dqk, Dv,
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(tq), nat.ptr(tk), nat.ptr(tv),
            nat.strides4(q), nat.strides4(k), nat.strides4(v),
            nat.ptr(o), nat.ptr(to), nat.strides4(o), nat.ptr(lse), nat.ptr(mu),
            float(sm_scale), ws_ptr, ws_size, nat.stream_ptr(dev),
        )
    )
    return o, to, lse, mu


def jvp_attention_forward_magi(q, k, v, tq, tk, tv, sm_scale, magi_mask):
    """Launch the block-sparse forward+JVP kernel; returns (o, to, lse, mu).

    Rows that no task of the mask covers are left as allocated (uninitialised),
    as in the reference. ``tk is None and tv is None`` skips their GEMMs.
    """
    from . import magimask as mm

    B, H, Lq, Dqk = q.shape
    Lk, Dv = v.shape[-2], v.shape[-1]
    _check_device(q, k, v, tq, tk, tv)
    if tq is None:
        raise ValueError("the block-sparse forward needs the query tangent tq")
    code = nat.dtype_code(q.dtype)
    if tk is None and tv is None:
        mode = nat.DMAD_FWD_JVP_KV_TANGENT_ZERO
    else:
        if tk is None:
            tk = torch.zeros_like(k)
        if tv is None:
            tv = torch.zeros_like(v)
        mode = nat.DMAD_FWD_JVP
    q, tq = _pair(q, tq)
    k, tk = _pair(k, tk)
    v, tv = _pair(v, tv)
    dev = q.device
    q_unique = mm.as_int32(magi_mask.q_unique, dev)
    k_flat = mm.as_int32(magi_mask.k_flat, dev)
    qk_map = mm.as_int32(magi_mask.qk_map, dev)
    G, R = q_unique.numel() // 2, k_flat.numel() // 2
    if qk_map.numel() != G + 1:
        raise ValueError(f"qk_map has {qk_map.numel()} entries for {G} query groups (expected {G + 1})")
    task_group, task_qtile, T = mm.tasks_for_kernel(magi_mask, Lq, dev)
    o = torch.empty((B, H, Lq, Dv), device=dev, dtype=q.dtype)
    to = torch.empty_like(o)
    lse = torch.empty((B, H, Lq), device=dev, dtype=torch.float32)
    mu = torch.empty_like(lse)
    lib = nat.lib()
    ws_ptr, ws_size, ws = nat.workspace(_fwd_ws_bytes(q.dtype, mode, B, H, Lk, Dqk, Dv), dev)
    nat.check(
        lib.dmad_attn_jvp_fwd_magi(
            code, mode, B, H, Lq, Lk, Dqk, Dv,
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(tq), nat.ptr(tk), nat.ptr(tv),
            nat.strides4(q), nat.strides4(k), nat.strides4(v),
            nat.ptr(o), nat.ptr(to), nat.strides4(o), nat.ptr(lse), nat.ptr(mu), float(sm_scale),
            nat.ptr(q_unique), nat.ptr(k_flat), nat.ptr(qk_map), G, R,
            nat.ptr(task_group), nat.ptr(task_qtile), T, mm.KERNEL_BLOCK_M,
            ws_ptr, ws_size, nat.stream_ptr(dev),
        )
    )
    return o, to, lse, mu


def jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, dout, dto, sm_scale, want_tangent_grads):
    """Launch the backward kernels; returns (dq, dk, dv, dtq, dtk, dtv)."""
    B, H, Lq, D = q.shape
    Lk = k.shape[-2]
    _check_device(q, k, v, o, dout)
    code = nat.dtype_code(q.dtype)
    full = dto is not None
    if B * H * Lq == 0:
        # no query rows: every gradient is zero (dQ, dQ̇ are empty)
        tg = full and want_tangent_grads
        zq, zk, zv = (torch.zeros(x.shape, device=q.device, dtype=q.dtype) for x in (q, k, v))
        return zq, zk, zv, (torch.zeros_like(zq) if tg else None), (torch.zeros_like(zk) if tg else None), \
            (torch.zeros_like(zv) if tg else None)
    if full:
        if tk is None:
            tk = torch.zeros_like(k)
        if tv is None:
            tv = torch.zeros_like(v)
        q, tq = _pair(q, tq)
        k, tk = _pair(k, tk)
        v, tv = _pair(v, tv)
        o, to = _pair(o, to)
        dout = torch.zeros_like(o) if dout is None else dout
        dout, dto = _pair(dout, dto)
    else:
        q, k, v, o, dout = _prep(q, k, v, o, dout)
        tq = tk = tv = to = None
    dq = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    dk = torch.empty(k.shape, device=q.device, dtype=q.dtype)
    dv = torch.empty(v.shape, device=q.device, dtype=q.dtype)
    tgrads = full and want_tangent_grads
    dtq = torch.empty_like(dq) if tgrads else None
    dtk = torch.empty_like(dk) if tgrads else None
    dtv = torch.empty_like(dv) if tgrads else None
    lib = nat.lib()
    ws_mode = (2 if tgrads else 1) if full else 0
    ws_ptr, ws_size, ws = _backward_workspace(code, ws_mode, B, H, Lq, Lk, D, q.device)
    nat.check(
        lib.dmad_attn_jvp_bwd(
            code, B, H, Lq, Lk, D,
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(tq), nat.ptr(tk), nat.ptr(tv),
            nat.strides4(q), nat.strides4(k), nat.strides4(v),
            nat.ptr(o), nat.ptr(to), nat.strides4(o), nat.ptr(lse), nat.ptr(mu),
            nat.ptr(dout), nat.ptr(dto), nat.strides4(dout),
            nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.ptr(dtq), nat.ptr(dtk), nat.ptr(dtv),
            nat.strides4(dq), nat.strides4(dk), nat.strides4(dv),
            float(sm_scale), ws_ptr, ws_size, nat.stream_ptr(q.device),
        )
    )
    return dq, dk, dv, dtq, dtk, dtv


class _attention(torch.autograd.Function):
    """
    Arguments:
        q, tq: (batch_size, nheads, seqlen_q, d_qk)
        k, tk: (batch_size, nheads, seqlen_kv, d_qk)
        v, tv: (batch_size, nheads, seqlen_kv, d_v)
    Returns:
        o, to: (batch_size, nheads, seqlen_q, d_v)

    Backward is only supported when d_qk=d_v.
    """

    @staticmethod
    def forward(ctx, q, k, v, tq, tk, tv, sm_scale=None, magi_mask=None):
        # argument contract of flash_attention_jvp_triton.py:464-476
        is_grad = any(x is not None and x.requires_grad for x in (q, k, v))
        assert q.shape[:-2] == k.shape[:-2] and k.shape[:-2] == v.shape[:-2]
        assert k.shape[-2] == v.shape[-2] and q.shape[-1] == k.shape[-1]
        HEAD_DIM_QK, HEAD_DIM_V = q.shape[-1], v.shape[-1]
        assert HEAD_DIM_QK in _HEAD_DIMS
        assert HEAD_DIM_V in _HEAD_DIMS
        assert tq.shape == q.shape
        assert tk is None or tk.shape == k.shape
        assert tv is None or tv.shape == v.shape
        assert tq.stride() == q.stride()
        assert tk is None or tk.stride() == k.stride()
        assert tv is None or tv.stride() == v.stride()
        if q.dim() != 4:
            raise ValueError("expected 4-d [B, H, L, D] tensors")
        if sm_scale is None:
            sm_scale = HEAD_DIM_QK ** (-0.5)
        if magi_mask is not None:
            if is_grad or any(x is not None and x.requires_grad for x in (tq, tk, tv)):
                raise RuntimeError("Backward with MagiMask is not supported.")
            o, to, _, _ = jvp_attention_forward_magi(q, k, v, tq, tk, tv, sm_scale, magi_mask)
            return o, to
        tangent_grad = any(x is not None and x.requires_grad for x in (tq, tk, tv))
        # the full derivative needs the tangent side; otherwise keep only what the
        # reference keeps (q, k, v, o, LSE: :500-502), so tangent activations and
        # `to` are not held until the backward
        mode = current_backward_mode()
        full = mode == "full" or (mode == "auto" and tangent_grad)
        if full and (is_grad or tangent_grad) and (max(HEAD_DIM_QK, HEAD_DIM_V) > FULL_BWD_MAX_HEAD_DIM
                                                   or q.dtype == torch.float32):
            full = _full_backward_unavailable(mode, HEAD_DIM_QK, HEAD_DIM_V, q.dtype)
        # an output that does not reach the loss arrives in backward as None
        # (not zeros), so an unused `to` keeps the dO-only kernel
        ctx.set_materialize_grads(False)
        o, to, lse, mu = torch.ops.dmad.flash_attn_jvp_fwd(q, k, v, tq, tk, tv, float(sm_scale))
        if is_grad or tangent_grad:
            if full:
                ctx.save_for_backward(q, k, v, tq, tk, tv, o, to, lse, mu)
            else:
                ctx.save_for_backward(q, k, v, o, lse)
            ctx.full = full
            ctx.sm_scale = float(sm_scale)
            ctx.tangent_grad = tangent_grad
        return o, to

    @staticmethod
    def backward(ctx, dout, dto):
        if not ctx.full:
            # the reference's backward: dO-only gradients, the cotangent of `to` ignored (:534-579)
            q, k, v, o, lse = ctx.saved_tensors
            assert q.shape[-1] == k.shape[-1] and k.shape[-1] == v.shape[-1], (
                "Backward not supported with different headdim."
            )
            if dout is None:
                return (None,) * 8
            dq, dk, dv = torch.ops.dmad.flash_attn_bwd(dout, q, k, v, o, lse, ctx.sm_scale)
            return dq, dk, dv, None, None, None, None, None
        q, k, v, tq, tk, tv, o, to, lse, mu = ctx.saved_tensors
        assert q.shape[-1] == k.shape[-1] and k.shape[-1] == v.shape[-1], (
            "Backward not supported with different headdim."
        )
        if dout is None and dto is None:
            return (None,) * 8
        if dout is None:
            dout = torch.zeros_like(o)
        dq, dk, dv, dtq, dtk, dtv = torch.ops.dmad.flash_attn_jvp_bwd(
            q, k, v, tq, tk, tv, o, to, lse, mu, dout, dto, ctx.sm_scale, ctx.tangent_grad
        )
        # absent gradients come back from the op as 0-element tensors
        dtq, dtk, dtv = (None if g.numel() == 0 and x.numel() != 0 else g for g, x in ((dtq, q), (dtk, k), (dtv, v)))
        if tk is None:
            dtk = None
        if tv is None:
            dtv = None
        return dq, dk, dv, dtq, dtk, dtv, None, None


# The forward+JVP and its backward as registered torch ops: torch.compile traces
# each as one node (the autograd.Function above stays the differentiable
# wrapper), and selective activation checkpointing policies that keep outputs of
# ops whose name contains "flash_attn" (the reference's mm_only_policy,
# train/wan/rcm/utils/selective_activation_checkpoint.py:48-57) keep O, Ȯ and
# the row statistics instead of recomputing the forward.
@torch.library.custom_op("dmad::flash_attn_jvp_fwd", mutates_args=())
def flash_attn_jvp_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tq: torch.Tensor,
                       tk: Optional[torch.Tensor], tv: Optional[torch.Tensor],
                       sm_scale: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(O, Ȯ, LSE, mu) of the forward+JVP kernel; ``tk = tv = None`` means zero K, V tangents."""
    return jvp_attention_forward(q, k, v, tq, tk, tv, sm_scale)


@flash_attn_jvp_fwd.register_fake
def _(q, k, v, tq, tk, tv, sm_scale):
    B, H, Lq, _ = q.shape
    o = q.new_empty((B, H, Lq, v.shape[-1]))
    lse = q.new_empty((B, H, Lq), dtype=torch.float32)
    return o, torch.empty_like(o), lse, torch.empty_like(lse)


@torch.library.custom_op("dmad::flash_attn_jvp_bwd", mutates_args=())
def flash_attn_jvp_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tq: torch.Tensor,
                       tk: Optional[torch.Tensor], tv: Optional[torch.Tensor], o: torch.Tensor, to: torch.Tensor,
                       lse: torch.Tensor, mu: torch.Tensor, dout: torch.Tensor, dto: Optional[torch.Tensor],
                       sm_scale: float, tangent_grads: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                      torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV, dQ̇, dK̇, dV̇) of flash_attn_jvp_fwd. Without ``dto`` these are the dO-only
    gradients; the tangent gradients are computed when ``dto`` is given and ``tangent_grads``
    is set, else they are returned as 0-element tensors."""
    dq, dk, dv, dtq, dtk, dtv = jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, dout, dto, sm_scale,
                                                       tangent_grads)
    # one fresh 0-element tensor per absent gradient: outputs of a custom op may not alias
    return dq, dk, dv, *(q.new_empty((0,)) if g is None else g for g in (dtq, dtk, dtv))


@flash_attn_jvp_bwd.register_fake
def _(q, k, v, tq, tk, tv, o, to, lse, mu, dout, dto, sm_scale, tangent_grads):
    tg = dto is not None and tangent_grads
    # the kernels write contiguous gradients whatever the input strides
    grads = (q.new_empty(q.shape), q.new_empty(k.shape), q.new_empty(v.shape))
    return (*grads, *(q.new_empty(g.shape) if tg else q.new_empty((0,)) for g in grads))


attention = _attention.apply


# Plain attention as registered torch ops, so that graph tools see one op per
# pass: torch.compile traces it as a unit, and selective activation
# checkpointing policies that keep attention outputs by name (the reference's
# mm_only_policy saves any op whose name contains "flash_attn",
# train/wan/rcm/utils/selective_activation_checkpoint.py:48-57) save its output
# instead of recomputing the forward in the backward pass.
@torch.library.custom_op("dmad::flash_attn_fwd", mutates_args=())
def flash_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of softmax(sm_scale Q K^T) V for [B, H, L, D] tensors (gfx950 forward kernel)."""
    o, _, lse, _ = jvp_attention_forward(q, k, v, None, None, None, sm_scale)
    return o, lse


@flash_attn_fwd.register_fake
def _(q, k, v, sm_scale):
    B, H, Lq, _ = q.shape
    return q.new_empty((B, H, Lq, v.shape[-1])), q.new_empty((B, H, Lq), dtype=torch.float32)


@torch.library.custom_op("dmad::flash_attn_bwd", mutates_args=())
def flash_attn_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                   lse: torch.Tensor, sm_scale: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dO-only gradients (dQ, dK, dV) of flash_attn_fwd (the arithmetic the reference
    delegates to flash-attn, flash_attention_jvp_triton.py:540-578)."""
    dq, dk, dv, _, _, _ = jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, dout, None, sm_scale,
                                                 False)
    return dq, dk, dv


@flash_attn_bwd.register_fake
def _(dout, q, k, v, o, lse, sm_scale):
    return q.new_empty(q.shape), q.new_empty(k.shape), q.new_empty(v.shape)


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, sm_scale = inputs
    o, lse = output
    ctx.save_for_backward(q, k, v, o, lse)
    ctx.sm_scale = sm_scale


def _fwd_backward(ctx, dout, dlse):
    q, k, v, o, lse = ctx.saved_tensors
    assert q.shape[-1] == v.shape[-1], "Backward not supported with different headdim."
    dq, dk, dv = torch.ops.dmad.flash_attn_bwd(dout, q, k, v, o, lse, ctx.sm_scale)
    return dq, dk, dv, None


flash_attn_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup_context)


def plain_attention(q, k, v, sm_scale=None):
    """softmax(sm_scale * q k^T) v for [B, H, L, D] tensors (gfx950 kernels), with backward."""
    assert q.shape[:-2] == k.shape[:-2] and k.shape[:-2] == v.shape[:-2]
    assert k.shape[-2] == v.shape[-2] and q.shape[-1] == k.shape[-1]
    assert q.shape[-1] in _HEAD_DIMS and v.shape[-1] in _HEAD_DIMS
    if sm_scale is None:
        sm_scale = q.shape[-1] ** (-0.5)
    return torch.ops.dmad.flash_attn_fwd(q, k, v, float(sm_scale))[0]
