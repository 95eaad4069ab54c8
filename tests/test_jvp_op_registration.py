"""The forward+JVP op and its backward as registered torch ops
(dmad::flash_attn_jvp_fwd / dmad::flash_attn_jvp_bwd) under the autograd
wrapper that replaces the reference's ``_attention``
(train/wan/rcm/utils/flash_attention_jvp_triton.py:450-582).

Graph tools see one node per pass: make_fx and torch.compile trace the two ops
(CPU: fake-tensor trace; GPU: compiled equals eager bit for bit), and the
reference's selective-checkpointing policy, which keeps the output of any op
whose name contains "flash_attn"
(train/wan/rcm/utils/selective_activation_checkpoint.py:48-57, restated as
`mm_only_policy` in test_plain_op.py), keeps O, Ȯ and the row statistics, so the
forward kernel runs once per step.
"""
import pytest
import torch
from torch.utils.checkpoint import CheckpointPolicy, checkpoint, create_selective_checkpoint_contexts

import dmad_amd  # noqa: F401  (registers the ops)
from dmad_amd.jvp_attention import attention
from oracle import attention as orc


def mm_only_policy(ctx, func, *args, **kwargs):
    name = str(func)
    keep = func in {torch.ops.aten.mm.default, torch.ops.aten.addmm.default} or "flash_attn" in name or "magi" in name
    return CheckpointPolicy.MUST_SAVE if keep else CheckpointPolicy.PREFER_RECOMPUTE


def _leaves(shape, n, seed, grad=True, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    xs = [(torch.randn(shape, generator=g, dtype=torch.float64) * s).to(torch.bfloat16)
          for s in (1.0, 1.0, 1.0, 0.1, 0.1, 0.1, 1.0, 0.1)[:n]]
    return [x.to(device).requires_grad_(grad and i < 6) for i, x in enumerate(xs)]


def test_op_names_match_the_checkpoint_policy():
    for op in (torch.ops.dmad.flash_attn_jvp_fwd.default, torch.ops.dmad.flash_attn_jvp_bwd.default):
        assert "flash_attn" in str(op)
        assert mm_only_policy(None, op) == CheckpointPolicy.MUST_SAVE


def test_fake_shapes_and_strides():
    """The fake implementations give the shapes, dtypes and (contiguous) strides the kernels write."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 100, 3, 64, dtype=torch.bfloat16).transpose(1, 2)  # BSHD storage viewed as BHSD
        k = torch.empty(2, 70, 3, 64, dtype=torch.bfloat16).transpose(1, 2)
        v = torch.empty(2, 70, 3, 32, dtype=torch.bfloat16).transpose(1, 2)
        o, to, lse, mu = torch.ops.dmad.flash_attn_jvp_fwd(q, k, v, q, None, None, 0.125)
        assert o.shape == to.shape == (2, 3, 100, 32) and o.is_contiguous() and o.dtype == torch.bfloat16
        assert lse.shape == mu.shape == (2, 3, 100) and lse.dtype == mu.dtype == torch.float32
        v = torch.empty(2, 70, 3, 64, dtype=torch.bfloat16).transpose(1, 2)
        o, to, lse, mu = torch.ops.dmad.flash_attn_jvp_fwd(q, k, v, q, k, v, 0.125)
        grads = torch.ops.dmad.flash_attn_jvp_bwd(q, k, v, q, k, v, o, to, lse, mu, o, None, 0.125, True)
        assert [tuple(g.shape) for g in grads] == [(2, 3, 100, 64), (2, 3, 70, 64), (2, 3, 70, 64), (0,), (0,), (0,)]
        assert all(g.is_contiguous() for g in grads)
        grads = torch.ops.dmad.flash_attn_jvp_bwd(q, k, v, q, None, None, o, to, lse, mu, o, to, 0.125, True)
        assert [tuple(g.shape) for g in grads[3:]] == [(2, 3, 100, 64), (2, 3, 70, 64), (2, 3, 70, 64)]
        grads = torch.ops.dmad.flash_attn_jvp_bwd(q, k, v, q, k, v, o, to, lse, mu, o, to, 0.125, False)
        assert [tuple(g.shape) for g in grads[3:]] == [(0,), (0,), (0,)]


@pytest.mark.parametrize("full", [False, True])
def test_fake_trace_has_one_node_per_pass(full):
    """make_fx over forward + torch.autograd.grad records exactly the two dmad ops."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def step(q, k, v, tq, tk, tv, do, dto):
        o, to = attention(q, k, v, tq, tk, tv)
        loss = (o.float() * do.float()).sum()
        if full:
            loss = loss + (to.float() * dto.float()).sum()
        return torch.autograd.grad(loss, (q, k, v, tq, tk, tv), allow_unused=True)

    gm = make_fx(step, tracing_mode="fake")(*_leaves((1, 2, 64, 32), 8, 0))
    ops = [n.target for n in gm.graph.nodes if n.op == "call_function" and "dmad" in str(n.target)]
    assert ops == [torch.ops.dmad.flash_attn_jvp_fwd.default, torch.ops.dmad.flash_attn_jvp_bwd.default]


@pytest.mark.gpu
@pytest.mark.parametrize("tangent_grad", [True, False])
def test_compiled_equals_eager(gpu, tangent_grad):
    """torch.compile (aot_eager: no generated kernels) traces the op without graph
    breaks and, the kernels being deterministic, reproduces eager bit for bit,
    gradients included: the full derivative when the tangents require grad, and
    the reference's dO-only backward (DMAD's case: `to` detached) when not."""
    import torch._dynamo

    torch._dynamo.reset()

    def fwd(q, k, v, tq, tk, tv):
        return attention(q, k, v, tq, tk, tv)

    def run(f):
        xs = _leaves((1, 2, 200, 128), 8, 3, device=gpu)
        if not tangent_grad:
            xs = [x.detach() if 3 <= i < 6 else x for i, x in enumerate(xs)]
        o, to = f(*xs[:6])
        loss = (o.float() * xs[6].float()).sum()
        if tangent_grad:
            loss = loss + (to.float() * xs[7].float()).sum()
        loss.backward()
        torch.cuda.synchronize()
        n = 6 if tangent_grad else 3
        return xs, (o.detach(), to.detach(), *(x.grad for x in xs[:n]))

    _, eager = run(fwd)
    xs, compiled = run(torch.compile(fwd, backend="aot_eager", fullgraph=True))
    names = ("o", "to", "dq", "dk", "dv", "dtq", "dtk", "dtv")
    for name, a, b in zip(names, eager, compiled):
        assert torch.equal(a, b), name
    x64 = [x.detach().double().cpu() for x in xs]
    ref = orc.grads_full(*x64) if tangent_grad else orc.grads_dout_only(x64[0], x64[1], x64[2], x64[6])
    for name, got, r in zip(names[2:], compiled[2:], ref):
        assert orc.rel_l2(got.cpu(), r) <= 1e-2, name


@pytest.mark.gpu
def test_selective_checkpointing_keeps_the_jvp_forward(gpu, monkeypatch):
    """Under the reference's mm_only policy the forward+JVP kernel runs once (saved,
    not recomputed in the backward) and the gradients equal the uncheckpointed ones."""
    from dmad_amd import jvp_attention

    calls = {"fwd": 0}
    real = jvp_attention.jvp_attention_forward

    def counted(*a, **kw):
        calls["fwd"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(jvp_attention, "jvp_attention_forward", counted)
    xs = _leaves((1, 2, 300, 128), 8, 5, device=gpu)
    do, dto = xs[6], xs[7]
    w = (torch.randn((128, 128), generator=torch.Generator().manual_seed(1)) / 128 ** 0.5).to(gpu)

    def block(q, k, v, tq, tk, tv):
        # float32 projection of q and its tangent (no bf16 batched products)
        return attention((q.float() @ w).to(torch.bfloat16), k, v, (tq.float() @ w).to(torch.bfloat16), tk, tv)

    def loss(o, to):
        return (o.float() * do.float()).sum() + (to.float() * dto.float()).sum()

    plain = torch.autograd.grad(loss(*block(*xs[:6])), xs[:6])
    calls["fwd"] = 0
    out = checkpoint(block, *xs[:6], use_reentrant=False,
                     context_fn=lambda: create_selective_checkpoint_contexts(mm_only_policy))
    sac = torch.autograd.grad(loss(*out), xs[:6])
    torch.cuda.synchronize()
    assert calls["fwd"] == 1, calls
    for name, a, b in zip(("dq", "dk", "dv", "dtq", "dtk", "dtv"), plain, sac):
        assert torch.equal(a, b), name
