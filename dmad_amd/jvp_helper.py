"""BSHD attention entry points of the Wan JVP network, on the gfx950 kernels.

Twins of train/wan/rcm/utils/jvp_helper.py:
  * ``torch_attention_op_withT`` (:52-66): takes (x, x_dot) pairs in
    ``[B, S, H, D]`` layout, calls the JVP op on ``.transpose(1, 2)`` views (no
    copy) and returns ``(o, o_dot.detach())`` in ``[B, S, H, D]``.
  * ``torch_attention_op`` (:305-308): plain attention in ``[B, S, H, D]``
    (the reference uses SDPA with its default scale D^-1/2).
"""
from __future__ import annotations

from typing import Tuple

import torch

from .jvp_attention import _attention, plain_attention

TensorWithT = Tuple[torch.Tensor, torch.Tensor]


def torch_attention_op_withT(q_B_S_H_D_withT: TensorWithT, k_B_S_H_D_withT: TensorWithT,
                             v_B_S_H_D_withT: TensorWithT, mask=None):
    q_B_S_H_D, t_q_B_S_H_D = q_B_S_H_D_withT
    k_B_S_H_D, t_k_B_S_H_D = k_B_S_H_D_withT
    v_B_S_H_D, t_v_B_S_H_D = v_B_S_H_D_withT
    result_B_H_S_D, t_result_B_H_S_D = _attention.apply(
        q_B_S_H_D.transpose(1, 2),
        k_B_S_H_D.transpose(1, 2),
        v_B_S_H_D.transpose(1, 2),
        t_q_B_S_H_D.transpose(1, 2),
        None if t_k_B_S_H_D is None else t_k_B_S_H_D.transpose(1, 2),
        None if t_v_B_S_H_D is None else t_v_B_S_H_D.transpose(1, 2),
        None,
        mask,
    )
    return result_B_H_S_D.transpose(1, 2), t_result_B_H_S_D.transpose(1, 2).detach()


def torch_attention_op(q_B_S_H_D, k_B_S_H_D, v_B_S_H_D):
    return plain_attention(q_B_S_H_D.transpose(1, 2), k_B_S_H_D.transpose(1, 2),
                           v_B_S_H_D.transpose(1, 2)).transpose(1, 2)
