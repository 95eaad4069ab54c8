"""BSHD attention entry points of the Wan JVP network, on the gfx950 kernels.

Twins of train/wan/rcm/utils/jvp_helper.py:
  * ``torch_attention_op_withT`` (:52-66): takes (x, x_dot) pairs in
    ``[B, S, H, D]`` layout, calls the JVP op on ``.transpose(1, 2)`` views (no
    copy) and returns ``(o, o_dot.detach())`` in ``[B, S, H, D]``.
  * ``torch_attention_op`` (:305-308): plain attention in ``[B, S, H, D]``
    (the reference uses SDPA with its default scale D^-1/2).
  * ``FlexOrSdpaLocalAttentionWithT`` (:213-269): the dense / block-sparse
    dispatcher of the JVP students, with its per-shape MagiMask cache.
  * ``MinimalA2AAttnOpWithT`` (:125-210): RoPE with tangent on q and k, then the
    local attention; the one-GPU branch (no all-to-all, no KV cache).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch
from torch import nn

from .jvp_attention import _attention, plain_attention
from .prologue import apply_rope_with_tangent
from .magimask import KERNEL_BLOCK_M, AttnMaskSpec, MagiMask, make_magi_ranges_full, prepare_magi_csr_and_tasks

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


def needs_block_mask(spec: Optional[AttnMaskSpec], Q: int, KV: int) -> bool:
    """False when the spec reduces to dense attention (jvp_helper.py:251-263):
    no mask, or a block-causal query block without sliding window whose keys all
    lie in blocks <= its own."""
    if spec is None or spec.mode == "none":
        return False
    if spec.mode == "block_causal" and int(spec.local_attn_blocks) == 0:
        pat, q_blk = spec.pattern, int(spec.q_block_offset)
        if Q == pat.get_block_tokens(q_blk) and KV <= pat.blocks_to_tokens(q_blk + 1):
            return False
    return True


class FlexOrSdpaLocalAttentionWithT(nn.Module):
    """Dense or block-sparse JVP attention on ``(x, x_dot)`` pairs in ``[B, S, H, D]``.

    ``forward(q_withT, k_withT, v_withT, attn_meta=None)``: with no mask (or one
    that covers every key, see ``needs_block_mask``) it calls the dense op;
    otherwise it builds (once per spec and shape) the MagiMask of the spec with
    the kernels' 128-query tiles and calls the block-sparse op. The block-sparse
    op is forward only, as in the reference.
    """

    def __init__(self, attn_T=torch_attention_op_withT):
        super().__init__()
        self.attn_T = attn_T
        self._cache: Dict[Tuple, MagiMask] = {}

    def get_magi_mask(self, spec: AttnMaskSpec, Q_real: int, KV_real: int, device,
                      BLOCK_M: int = KERNEL_BLOCK_M) -> MagiMask:
        device = torch.device(device)
        key = (spec.mode, spec.pattern, int(spec.local_attn_blocks), int(spec.sink_blocks), int(spec.q_block_offset),
               int(spec.clean_blocks), int(Q_real), int(KV_real), int(BLOCK_M), device.type, device.index)
        mask = self._cache.get(key)
        if mask is None:
            q_ranges, k_ranges = make_magi_ranges_full(spec, Q_real, KV_real, device)
            mask = prepare_magi_csr_and_tasks(q_ranges, k_ranges, Q_real, KV_real, BLOCK_M)
            self._cache[key] = mask
        return mask

    def clear_cache(self):
        self._cache.clear()

    def forward(self, q_withT, k_withT, v_withT, attn_meta: Optional[AttnMaskSpec] = None, **_ignored):
        q, k, v = q_withT[0], k_withT[0], v_withT[0]
        B, Q, H, D = q.shape
        KV = k.shape[1]
        assert k.shape == (B, KV, H, D) and v.shape == (B, KV, H, D)
        if not needs_block_mask(attn_meta, Q, KV):
            return self.attn_T(q_withT, k_withT, v_withT)
        mask = self.get_magi_mask(attn_meta, Q_real=Q, KV_real=KV, device=q.device)
        return self.attn_T(q_withT, k_withT, v_withT, mask)


@dataclass
class RopeCache:
    """Per-layer RoPE angles (train/wan/rcm/utils/rope.py:13-32): ``query_freqs`` and
    ``key_freqs`` [S, D/2]; with ``cached_k_rotated`` the keys arrive rotated except
    the current block's, rotated by ``current_key_freqs``."""

    query_freqs: Optional[torch.Tensor] = None
    key_freqs: Optional[torch.Tensor] = None
    current_key_freqs: Optional[torch.Tensor] = None
    use_fused: bool = True
    cached_k_rotated: bool = True


def _rotate(x_withT, freqs):
    x, tx = x_withT
    x, tx = apply_rope_with_tangent(x, tx, freqs)
    return x, (None if tx is None else tx.detach())


class MinimalA2AAttnOpWithT(nn.Module):
    """RoPE with tangent, then local JVP attention, on BSHD ``(x, x_dot)`` pairs
    (train/wan/rcm/utils/jvp_helper.py:125-210, one-GPU branch).

    ``forward(q_withT, k_withT, v_withT, *args, attn_ctx=None, **kwargs)``:
    ``attn_ctx.rope`` (a ``RopeCache``) gives the angles, applied as the
    reference does (:176-196): the current key block first when the cached keys
    are already rotated, then the query, and the whole key otherwise; rotated
    tangents are detached. The remaining arguments go to ``local_attn_T``
    (``FlexOrSdpaLocalAttentionWithT`` takes ``attn_meta``). Context parallelism
    (a process group of more than one rank) and the KV cache of streaming
    inference are not part of this one-GPU build and raise.
    """

    def __init__(self, local_attn_T=torch_attention_op_withT):
        super().__init__()
        self.local_attn_T = local_attn_T
        self.pg = None
        self.stream = None

    def set_context_parallel_group(self, process_group, ranks, stream):
        del ranks
        self.pg = process_group
        self.stream = stream

    def forward(self, query_withT, key_withT, value_withT, *args: Any, attn_ctx=None, **kwargs):
        if self.pg is not None and torch.distributed.get_world_size(self.pg) > 1:
            raise NotImplementedError("context parallelism (all-to-all over several GPUs) is not part of this build")
        cache = getattr(attn_ctx, "kv_cache", None) if attn_ctx is not None else None
        mode = getattr(attn_ctx, "mode", None)
        if cache is not None and getattr(mode, "name", mode) != "DISABLED":
            raise NotImplementedError("the KV cache of streaming inference is not part of this build")
        rope = attn_ctx.rope if attn_ctx is not None else None
        if rope is not None and rope.cached_k_rotated and rope.current_key_freqs is not None:
            key_withT = _rotate(key_withT, rope.current_key_freqs)
        if rope is not None and rope.query_freqs is not None:
            query_withT = _rotate(query_withT, rope.query_freqs)
            if not rope.cached_k_rotated:
                key_withT = _rotate(key_withT, rope.key_freqs)
        return self.local_attn_T(query_withT, key_withT, value_withT, *args, **kwargs)
