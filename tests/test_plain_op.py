"""Plain attention as registered torch ops (dmad::flash_attn_fwd / flash_attn_bwd).

The reference's selective-activation-checkpointing policy saves an op's output
when its name contains "flash_attn" and recomputes everything else
(train/wan/rcm/utils/selective_activation_checkpoint.py:48-57, restated below
as `mm_only_policy`). Through the registered op the attention forward runs
once per step under that policy, and its gradients are the oracle's.
"""
import pytest
import torch
from torch.utils.checkpoint import CheckpointPolicy, checkpoint, create_selective_checkpoint_contexts

import dmad_amd  # noqa: F401  (registers the ops)
from oracle import attention as orc

SAVE = {torch.ops.aten.mm.default, torch.ops.aten.addmm.default}


def mm_only_policy(ctx, func, *args, **kwargs):
    name = str(func)
    keep = func in SAVE or "flash_attn" in name or "magi" in name
    return CheckpointPolicy.MUST_SAVE if keep else CheckpointPolicy.PREFER_RECOMPUTE


def test_ops_are_registered_with_flash_attn_names():
    assert "flash_attn" in str(torch.ops.dmad.flash_attn_fwd.default)
    assert "flash_attn" in str(torch.ops.dmad.flash_attn_bwd.default)
    assert mm_only_policy(None, torch.ops.dmad.flash_attn_fwd.default) == CheckpointPolicy.MUST_SAVE


def test_fake_tensor_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 3, 100, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 3, 70, 64, dtype=torch.bfloat16)
        v = torch.empty(2, 3, 70, 32, dtype=torch.bfloat16)
        o, lse = torch.ops.dmad.flash_attn_fwd(q, k, v, 0.125)
        assert o.shape == (2, 3, 100, 32) and o.dtype == torch.bfloat16
        assert lse.shape == (2, 3, 100) and lse.dtype == torch.float32


@pytest.mark.gpu
def test_selective_checkpointing_saves_the_attention_forward(gpu, monkeypatch):
    from dmad_amd import jvp_attention, torch_attention_op

    calls = {"fwd": 0}
    real = jvp_attention.jvp_attention_forward

    def counted(*a, **kw):
        calls["fwd"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(jvp_attention, "jvp_attention_forward", counted)
    g = torch.Generator().manual_seed(11)
    B, S, H, D = 1, 300, 2, 128
    xs = [(torch.randn((B, S, H, D), generator=g) * 0.5).to(torch.bfloat16) for _ in range(4)]
    w = torch.randn((D, D), generator=g) / D ** 0.5  # float32 projection (no bf16 batched products)
    q, k, v, do = (x.to(gpu) for x in xs)
    wq = w.to(gpu).requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)

    def block(q, k, v):
        return torch_attention_op((q.float() @ wq).to(torch.bfloat16), k, v)

    out = checkpoint(block, q, k, v, use_reentrant=False,
                     context_fn=lambda: create_selective_checkpoint_contexts(mm_only_policy))
    out.backward(do)
    torch.cuda.synchronize()
    assert calls["fwd"] == 1, calls  # saved, not recomputed in the backward
    # gradients against the oracle (through the projection of q)
    qp = (q.float() @ wq.detach()).to(torch.bfloat16)
    rq, rk, rv = orc.grads_dout_only(*(x.double().cpu().transpose(1, 2) for x in (qp, k.detach(), v.detach(), do)),
                                     sm_scale=D ** -0.5)
    assert orc.rel_l2(k.grad.transpose(1, 2), rk) <= 1e-2
    assert orc.rel_l2(v.grad.transpose(1, 2), rv) <= 1e-2
    ref_wq = torch.einsum("bshd,bshe->de", q.double().cpu(), rq.transpose(1, 2))
    assert orc.rel_l2(wq.grad, ref_wq) <= 1e-2


def test_sdpa_twin_refuses_what_the_kernels_lack():
    """dmad_amd.sdpa.attention (rcm/utils/attention.py:120-167): dropout, causal and
    float64 raise before anything reaches the GPU (float32 runs on the fp32 kernels)."""
    from dmad_amd.sdpa import attention

    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="dropout"):
        attention(q, q, q, dropout_p=0.1)
    with pytest.raises(NotImplementedError, match="causal"):
        attention(q, q, q, causal=True)
    with pytest.raises(NotImplementedError, match="float64"):
        attention(q.double(), q.double(), q.double())


@pytest.mark.gpu
def test_sdpa_twin_forward_and_backward(gpu):
    """BSHD in, BSHD contiguous out; q_scale and softmax_scale as the reference applies
    them; gradients through the registered op against the oracle."""
    from dmad_amd.sdpa import attention

    B, S, H, D = 2, 333, 3, 128
    g = torch.Generator().manual_seed(8)
    q, k, v, do = ((torch.randn(B, S, H, D, generator=g, dtype=torch.float64)).to(torch.bfloat16) for _ in range(4))
    leaves = [x.to(gpu).requires_grad_(True) for x in (q, k, v)]
    out = attention(*leaves, softmax_scale=0.1, q_scale=0.5, deterministic=True)
    assert out.shape == (B, S, H, D) and out.is_contiguous()
    out.backward(do.to(gpu))
    torch.cuda.synchronize()
    bhsd = lambda t: t.transpose(1, 2).double()  # noqa: E731
    qs = bhsd(q) * 0.5
    ref_o, _ = orc.math_attention(qs, bhsd(k), bhsd(v), 0.1)
    assert orc.rel_l2(bhsd(out.detach().cpu()), ref_o) < 1e-2
    rq, rk, rv = orc.grads_dout_only(qs, bhsd(k), bhsd(v), bhsd(do), 0.1)
    assert orc.rel_l2(bhsd(leaves[0].grad.cpu()), rq * 0.5) < 1e-2  # through q * q_scale
    assert orc.rel_l2(bhsd(leaves[1].grad.cpu()), rk) < 1e-2
    assert orc.rel_l2(bhsd(leaves[2].grad.cpu()), rv) < 1e-2
