"""dmad_amd: MI355X (gfx950) flash-attention JVP path of DMAD / rCM.

Public surface (mirrors the reference module train/wan/rcm/utils/flash_attention_jvp_triton.py
and the attention helpers of train/wan/rcm/utils/jvp_helper.py):

* ``_attention`` / ``attention``    -- autograd op (q, k, v, tq, tk, tv, sm_scale, magi_mask) -> (o, to)
* ``torch_attention_op_withT``      -- BSHD (x, x_dot) pairs in, (o, o_dot.detach()) out
* ``torch_attention_op``            -- plain BSHD attention on the same kernels
* ``plain_attention``               -- plain BHSD attention with backward
* ``rmsnorm_rope_with_tangent``     -- fused RMSNorm(+JVP) and RoPE-with-tangent producing the op's q/k inputs
* ``magimask``                      -- block-sparse mask tables (MagiMask) for ``attention(..., magi_mask)``
* ``FlexOrSdpaLocalAttentionWithT`` -- dense / block-sparse dispatcher of the masked JVP students
* ``MinimalA2AAttnOpWithT``, ``RopeCache`` -- RoPE-with-tangent then local attention (one-GPU branch)
* ``apply_rope_with_tangent``       -- interleaved RoPE of a BSHD pair, differentiable
"""
from .jvp_attention import (  # noqa: F401
    _attention, attention, backward_mode, backward_score_budget, current_backward_mode, plain_attention,
    set_backward_mode, set_backward_score_budget, set_reference_backward,
)
from .jvp_helper import (  # noqa: F401
    FlexOrSdpaLocalAttentionWithT,
    MinimalA2AAttnOpWithT,
    RopeCache,
    torch_attention_op,
    torch_attention_op_withT,
)
from .prologue import apply_rope_with_tangent, rmsnorm_rope_with_tangent  # noqa: F401
from . import magimask  # noqa: F401
from .magimask import MagiMask, prepare_magi_csr_and_tasks  # noqa: F401
