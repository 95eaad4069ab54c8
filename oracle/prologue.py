"""CPU oracle for the attention-input prologue (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the checker.

What the reference does to a Linear output ``y`` ([B, L, C], C = H*D) and its
tangent ``ty`` before the JVP attention op, restated in plain PyTorch:

* ``rmsnorm_jvp``  -- ``WanRMSNorm._forward`` under ``torch.func.jvp``
  (train/wan/rcm/networks/wan2pt1_jvp.py:207-216): ``_norm(y.float())`` =
  ``x * rsqrt(mean(x^2) + eps)`` in float32, cast back to the input type
  (``type_as``), times the weight; the tangent goes through the same ops
  (wan2pt1_jvp.py:209-212 detaches it afterwards).
* ``rope_jvp``     -- ``apply_rope_with_tangent`` (train/wan/rcm/utils/rope.py:106-114):
  ``apply_rope(x, freqs, fused=False)`` under ``torch.func.jvp``; ``apply_rope``
  (rope.py:56-70) rotates interleaved pairs (x[2i], x[2i+1]) by ``freqs[l, i]``
  in float32 (``apply_rotary_emb_torch`` with ``interleaved=True``, rope.py:34-53)
  and casts back.
* ``rmsnorm_rope_jvp`` -- the two in sequence, as ``WanSelfAttention._forward_jvp``
  (wan2pt1_jvp.py:312-317) and ``MinimalA2AAttnOpWithT.forward``
  (train/wan/rcm/utils/jvp_helper.py:180-196) apply them to Q and K.

Pinned in tests/test_prologue.py by per-element float64 loops written from the
formulas (a sign error in the rotation fails them), central differences of the
tangent, the rotation's invariants (pair norms kept, zero angles = identity)
and linearity in the tangent.
"""
from __future__ import annotations

import torch


def rmsnorm(y: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``WanRMSNorm._forward``: norm in float32, cast to y's type, times the weight."""
    x = y.float() if y.dtype != torch.float64 else y
    n = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    return n.type_as(y) * weight


def rmsnorm_jvp(y, ty, weight, eps):
    return torch.func.jvp(lambda x: rmsnorm(x, weight, eps), (y,), (ty,))


def _rotate_half_interleaved(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x[..., ::2], x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(-2)


def apply_rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, L, H, D]; freqs [L, D/2]: interleaved rotation in float32, cast back."""
    _, L, _, D = x.shape
    f = freqs.view(L, D // 2)
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    cos = torch.cos(f).to(work).repeat_interleave(2, dim=-1)[:, None, :]
    sin = torch.sin(f).to(work).repeat_interleave(2, dim=-1)[:, None, :]
    xf = x.to(work)
    return (xf * cos + _rotate_half_interleaved(xf) * sin).to(x.dtype)


def rope_jvp(x, tx, freqs):
    return torch.func.jvp(lambda inp: apply_rope(inp, freqs), (x,), (tx,))


def rmsnorm_rope_jvp(y, ty, weight, eps, freqs, heads):
    """y, ty [B, L, C] -> rotated (q, q_dot) as [B, L, H, D]; freqs None skips RoPE."""
    B, L, C = y.shape
    q, tq = rmsnorm_jvp(y, ty, weight, eps)
    q, tq = q.view(B, L, heads, C // heads), tq.view(B, L, heads, C // heads)
    if freqs is None:
        return q, tq
    return rope_jvp(q, tq, freqs)
