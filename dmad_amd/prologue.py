"""Fused attention-input prologue for gfx950: RMSNorm(+JVP) and RoPE-with-tangent.

In the reference the tensors handed to the JVP attention op are produced by two
separate steps, each a ``torch.func.jvp`` over float32 round trips:
  * ``WanRMSNorm._forward`` under ``torch.func.jvp`` inside
    ``WanSelfAttention._forward_jvp`` (train/wan/rcm/networks/wan2pt1_jvp.py:207-216,
    312-317), applied to the q and k Linear outputs and their tangents;
  * ``apply_rope_with_tangent`` (train/wan/rcm/utils/rope.py:106-114) inside
    ``MinimalA2AAttnOpWithT.forward`` (train/wan/rcm/utils/jvp_helper.py:180-196).
``rmsnorm_rope_with_tangent`` does both in one HIP kernel (one HBM read of the
Linear output and its tangent, one write of the rotated pair), with the
reference's rounding points. ``apply_rope_with_tangent`` is the rotation alone
(the reference function of that name), with a backward: the rotation's
transpose is the rotation by the negated angles, run on the same kernel.
Device work only: tensors off the GPU raise.
"""
from __future__ import annotations

import torch

from . import _native as nat


def rmsnorm_rope_with_tangent(x_with_t, weight, eps, freqs, num_heads):
    """((y, ty), weight [C], eps, freqs [L, D/2] or None, H) -> (q, q_dot) as [B, L, H, D].

    ``y`` is the [B, L, C] Linear output (C = H*D) and ``ty`` its tangent (or None
    for the primal only). The tangent output is detached, as both reference steps
    detach it (wan2pt1_jvp.py:212, jvp_helper.py:194).
    """
    y, ty = x_with_t
    if y.device.type != "cuda":
        raise RuntimeError("dmad_amd prologue runs on the GPU only (HIP kernel); got a tensor on " + str(y.device))
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (y, ty, weight)):
        raise RuntimeError("rmsnorm_rope_with_tangent has no backward: call it under torch.no_grad() "
                           "(the JVP evaluations it serves run without gradients)")
    B, L, C = y.shape
    if C % num_heads:
        raise ValueError(f"model dim {C} is not a multiple of num_heads {num_heads}")
    D = C // num_heads
    code = nat.dtype_code(y.dtype)
    if weight.dtype != y.dtype:
        weight = weight.to(y.dtype)
    y = y.reshape(B * L, C)
    if y.stride(-1) != 1 or y.stride(0) % 8 or y.data_ptr() % 16:
        y = y.contiguous()
    if ty is not None:
        ty = ty.reshape(B * L, C)
        if ty.stride() != y.stride() or ty.data_ptr() % 16:
            y, ty = y.contiguous(), ty.contiguous()
    weight = weight.contiguous()
    if freqs is not None:
        freqs = freqs.reshape(L, D // 2).to(device=y.device, dtype=torch.float32).contiguous()
    out = torch.empty((B * L, C), device=y.device, dtype=y.dtype)
    tout = torch.empty_like(out) if ty is not None else None
    nat.check(
        nat.lib().dmad_rmsnorm_rope_jvp(
            code, B * L, L, num_heads, D, nat.ptr(y), nat.ptr(ty), y.stride(0), nat.ptr(weight),
            nat.ctypes.cast(nat.ptr(freqs), nat._FP), float(eps), nat.ptr(out), nat.ptr(tout), out.stride(0),
            nat.stream_ptr(y.device),
        )
    )
    q = out.view(B, L, num_heads, D)
    return q, (None if tout is None else tout.view(B, L, num_heads, D).detach())


def _rope_launch(x, t_x, freqs):
    """Rotation of [B, S, H, D] x (and t_x) by freqs [S, D/2]; returns [B, S, H, D] outputs."""
    if x.device.type != "cuda":
        raise RuntimeError("dmad_amd RoPE runs on the GPU only (HIP kernel); got a tensor on " + str(x.device))
    B, S, H, D = x.shape
    code = nat.dtype_code(x.dtype)

    def rows(t):
        if t.stride(3) != 1 or t.stride(2) != D or t.stride(1) % 8 or t.data_ptr() % 16 or (B > 1 and t.stride(0) != S * t.stride(1)):
            t = t.contiguous()
        return t

    x = rows(x)
    if t_x is not None:
        t_x = rows(t_x)
        if t_x.stride() != x.stride():
            x, t_x = x.contiguous(), t_x.contiguous()
    f = freqs.reshape(S, D // 2).to(device=x.device, dtype=torch.float32).contiguous()
    out = torch.empty((B, S, H, D), device=x.device, dtype=x.dtype)
    tout = torch.empty_like(out) if t_x is not None else None
    nat.check(
        nat.lib().dmad_rmsnorm_rope_jvp(
            code, B * S, S, H, D, nat.ptr(x), nat.ptr(t_x), x.stride(1), nat.ptr(None),
            nat.ctypes.cast(nat.ptr(f), nat._FP), 0.0, nat.ptr(out), nat.ptr(tout), out.stride(1),
            nat.stream_ptr(x.device),
        )
    )
    return out, tout


class _RopeWithTangent(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, t_x, freqs):
        ctx.save_for_backward(freqs)
        return _rope_launch(x, t_x, freqs)

    @staticmethod
    def backward(ctx, g_out, g_tout):
        (freqs,) = ctx.saved_tensors
        neg = -freqs
        gx = gtx = None
        if g_out is not None and g_tout is not None and g_out.dtype == g_tout.dtype:
            gx, gtx = _rope_launch(g_out, g_tout, neg)
        else:
            if g_out is not None:
                gx = _rope_launch(g_out, None, neg)[0]
            if g_tout is not None:
                gtx = _rope_launch(g_tout, None, neg)[0]
        return gx, gtx, None


def apply_rope_with_tangent(x, t_x, freqs, fused: bool = False):
    """Interleaved rotary embedding of x [B, S, H, D] and of its tangent t_x by
    freqs [S, D/2] (train/wan/rcm/utils/rope.py:106-114, apply_rope :56-70):
    pairs (x[2i], x[2i+1]) rotated by freqs[s, i] in float32, cast back to the
    input type. ``freqs is None`` returns the inputs. ``fused`` is accepted for
    the reference's signature and ignored (one kernel either way). Differentiable:
    the gradient is the rotation by -freqs.
    """
    del fused
    if freqs is None:
        return x, t_x
    if t_x is None:
        return _RopeWithTangent.apply(x, None, freqs)[0], None
    return _RopeWithTangent.apply(x, t_x, freqs)
