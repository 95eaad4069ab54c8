"""Synthetic attention inputs with the value distribution of the Wan2.1 DiT.

Q and K are what ``WanSelfAttention._forward_jvp`` hands the attention op:
a Linear output RMS-normalised over the full model dim ``H*D`` (eps 1e-6,
unit weight; train/wan/rcm/networks/wan2pt1_jvp.py:192-216, 254-255) and
rotated by interleaved 3D RoPE with the t/h/w split of
``VideoRopePosition3DEmb`` (head_dim 128 -> 44/42/42, theta 10000,
wan2pt1_jvp.py:60-168; rotation as in train/wan/rcm/utils/rope.py:34-70).
The Linear outputs themselves are drawn N(0, 1); V ~ N(0, 1); tangents
~ N(0, 0.1^2); dO ~ N(0, 1); dOd ~ N(0, 0.1^2). Draw order: Q, K, V, Qd, Kd,
Vd, dO, dOd from one generator seeded with `seed`.

Tensors are returned as BSHD storage ``[B, L, H, D]`` viewed as BHSD
``[B, H, L, D]`` -- the layout the Wan callers pass to the op
(train/wan/rcm/utils/jvp_helper.py:52-66).
"""
from __future__ import annotations

import torch


def rope_freqs_3d(T: int, Hh: int, W: int, head_dim: int, device=None) -> torch.Tensor:
    """[T*Hh*W, head_dim/2] rotation angles, token order (t, h, w) row-major."""
    dim_h = head_dim // 6 * 2
    dim_w = dim_h
    dim_t = head_dim - 2 * dim_h
    sp = torch.arange(0, dim_h, 2, dtype=torch.float32, device=device)[: dim_h // 2] / dim_h
    tp = torch.arange(0, dim_t, 2, dtype=torch.float32, device=device)[: dim_t // 2] / dim_t
    h_f = 1.0 / (10000.0 ** sp)
    w_f = 1.0 / (10000.0 ** sp)
    t_f = 1.0 / (10000.0 ** tp)
    t_idx = torch.arange(T, device=device).repeat_interleave(Hh * W)
    h_idx = torch.arange(Hh, device=device).repeat_interleave(W).repeat(T)
    w_idx = torch.arange(W, device=device).repeat(Hh * T)
    return torch.cat(
        [t_idx.float()[:, None] * t_f[None], h_idx.float()[:, None] * h_f[None], w_idx.float()[:, None] * w_f[None]],
        dim=-1,
    )


def apply_rope_interleaved(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, L, H, D]; pairs (x[2i], x[2i+1]) rotated by freqs[l, i], in fp32."""
    B, L, H, D = x.shape
    cos = torch.cos(freqs).view(1, L, 1, D // 2)
    sin = torch.sin(freqs).view(1, L, 1, D // 2)
    xf = x.float()
    x0, x1 = xf[..., 0::2], xf[..., 1::2]
    out = torch.empty_like(xf)
    out[..., 0::2] = x0 * cos - x1 * sin
    out[..., 1::2] = x0 * sin + x1 * cos
    return out


def rms_norm_full_dim(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x [B, L, H, D] normalised over H*D per token (unit weight), fp32."""
    B, L, H, D = x.shape
    xf = x.float().reshape(B, L, H * D)
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return xf.reshape(B, L, H, D)


def make_inputs(B, H, Lq, Lk, D, dtype=torch.bfloat16, seed=0, device="cpu", grid=None, Dv=None,
                rope=True, with_grads=False, gen_device=None):
    """Returns dict of BHSD views over BSHD storage: q, k, v, tq, tk, tv (+ do, dto).

    grid = (T, Hh, W) with T*Hh*W == Lq == Lk selects 3D RoPE; rope=False (or no
    grid, or Lq != Lk) skips RMSNorm+RoPE and draws Q, K ~ N(0, 1) directly.
    The draws happen on `gen_device` (default: the CPU) and are moved to `device`.
    """
    Dv = D if Dv is None else Dv
    gdev = torch.device("cpu" if gen_device is None else gen_device)
    g = torch.Generator(device=gdev)
    g.manual_seed(seed)

    def draw(L, d, std=1.0):
        return torch.randn((B, L, H, d), generator=g, device=gdev, dtype=torch.float32) * std

    q, k, v = draw(Lq, D), draw(Lk, D), draw(Lk, Dv)
    tq, tk, tv = draw(Lq, D, 0.1), draw(Lk, D, 0.1), draw(Lk, Dv, 0.1)
    out = {}
    if rope and grid is not None and Lq == Lk and D == 128:
        T, Hh, W = grid
        assert T * Hh * W == Lq
        freqs = rope_freqs_3d(T, Hh, W, D, device=gdev)
        q = apply_rope_interleaved(rms_norm_full_dim(q).to(dtype), freqs)
        k = apply_rope_interleaved(rms_norm_full_dim(k).to(dtype), freqs)
    vals = {"q": q, "k": k, "v": v, "tq": tq, "tk": tk, "tv": tv}
    if with_grads:
        vals["do"] = draw(Lq, Dv)
        vals["dto"] = draw(Lq, Dv, 0.1)
    for name, x in vals.items():
        out[name] = x.to(dtype).to(device).transpose(1, 2)
    return out


WAN_CONFIGS = {
    # name: (B, H, Lq, Lk, D, rope grid)
    "plumbing": (1, 2, 256, 256, 64, None),
    "wan1.3b_self": (1, 12, 32760, 32760, 128, (21, 30, 52)),
    "wan1.3b_cross": (1, 12, 32760, 512, 128, None),
    "wan14b_self": (1, 40, 32760, 32760, 128, (21, 30, 52)),
    "wan14b_cross": (1, 40, 32760, 512, 128, None),
    "wan14b_720p_self": (1, 40, 75600, 75600, 128, (21, 45, 80)),
}
