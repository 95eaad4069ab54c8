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
reference's rounding points. Device work only: tensors off the GPU raise.
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
