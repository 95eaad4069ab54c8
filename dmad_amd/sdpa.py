"""Plain attention entry point of the non-JVP Wan models, on the gfx950 kernels.

Twin of ``attention`` in train/wan/rcm/utils/attention.py:120-167, which the
teacher, the fake-score network and the critics call (through
``FlexOrSdpaLocalAttention`` in dense mode, blockmask.py:354-355, and
wan2pt1.py:245, 281) and which picks FA3 / cuDNN / flash / efficient SDPA by
GPU generation. Here it is one path: the plain forward kernel and the dO-only
backward kernels, as the registered op ``dmad::flash_attn_fwd`` (so selective
activation checkpointing keeps its output).
"""
from __future__ import annotations

import torch

from .jvp_attention import plain_attention


def attention(q, k, v, dropout_p=0.0, softmax_scale=None, q_scale=None, causal=False, deterministic=False):
    """softmax(softmax_scale * q k^T) v for BSHD ``[B, S, H, D]`` tensors, returned BSHD contiguous.

    As the reference: q, k, v share one dtype, ``q_scale`` multiplies q first,
    ``softmax_scale=None`` means D^-1/2. The kernels are deterministic, so
    ``deterministic=True`` needs nothing more. bfloat16, float16 and float32
    inputs run on the gfx950 kernels (float32 on fp32 MFMAs, where the reference
    takes PyTorch's memory-efficient SDPA). Attention dropout and the causal
    mask are not provided by these kernels and raise ``NotImplementedError``
    (the Wan models call it with neither).
    """
    assert q.dtype == k.dtype and k.dtype == v.dtype
    del deterministic
    if dropout_p:
        raise NotImplementedError("attention dropout is not implemented by the gfx950 kernels")
    if causal:
        raise NotImplementedError("the causal mask is not implemented by the dense gfx950 kernels")
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise NotImplementedError(
            f"dtype {q.dtype} is not supported by the gfx950 kernels (bfloat16, float16 or float32)")
    if q_scale is not None:
        q = q * q_scale
    out = plain_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), softmax_scale)
    return out.transpose(1, 2).contiguous()
