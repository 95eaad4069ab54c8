"""Backward kernel parity on the GPU against the CPU oracle.

dO-only gradients (what the reference computes, flash_attention_jvp_triton.py:534-579)
at the shapes of the reference's `_test_fwd_bwd` (:585-624) and `_test_fwd_bwd_ca`
(:728-765), and the full derivative (cotangent of the tangent output included,
plus the tangent gradients) against oracle.grads_full, itself pinned against
autograd through torch.func.jvp.

Bar: relative L2 error <= 1e-2 on every gradient against the float64 oracle on
the same rounded inputs, no worse than 1.25x the reference backward's own error
(oracle.fa2_bwd_emulator, the FA2 numerics it calls) + 1e-4 for the dO-only
gradients, plus the reference tests' assert_close tolerances (atol 1e-2 / 2e-2,
rtol 2e-2) against the in-dtype naive oracle.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

REF_SA = [(1, 2, 1024, 1024, 64), (1, 2, 999, 999, 64)]
REF_CA = [(1, 2, 256, 1024, 128), (1, 2, 1024, 256, 128), (1, 2, 1024, 512, 64), (1, 2, 1000, 515, 64)]
DTYPES = [torch.bfloat16, torch.float16]


def _draw(g, shape, std, dtype):
    return (torch.randn(shape, generator=g, dtype=torch.float64) * std).to(dtype)


def _case(shape, dtype, seed=20, std=0.5, tstd=0.5):
    B, H, Lq, Lk, D = shape
    g = torch.Generator().manual_seed(seed)
    q, k, v = _draw(g, (B, H, Lq, D), std, dtype), _draw(g, (B, H, Lk, D), std, dtype), _draw(g, (B, H, Lk, D), std, dtype)
    tq, tk, tv = (_draw(g, (B, H, Lq, D), tstd, dtype), _draw(g, (B, H, Lk, D), tstd, dtype),
                  _draw(g, (B, H, Lk, D), tstd, dtype))
    do, dto = _draw(g, (B, H, Lq, D), 1.0, dtype), _draw(g, (B, H, Lq, D), 0.1, dtype)
    return q, k, v, tq, tk, tv, do, dto


def _grad_run(dev, xs, sm_scale, use_dto, tangent_grad):
    from dmad_amd import attention

    q, k, v, tq, tk, tv, do, dto = (x.to(dev) for x in xs)
    leaves = [q, k, v] + ([tq, tk, tv] if tangent_grad else [])
    leaves = [x.requires_grad_(True) for x in leaves]
    o, to = attention(q, k, v, tq, tk, tv, sm_scale)
    loss = (o.float() * do.float()).sum()
    if use_dto:
        loss = loss + (to.float() * dto.float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    return [None if x.grad is None else x.grad.cpu() for x in leaves]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", REF_SA + REF_CA)
def test_dout_only_backward(gpu, shape, dtype):
    print(f"case shape={shape} dtype={dtype}", flush=True)
    xs = _case(shape, dtype)
    dq, dk, dv = _grad_run(gpu, xs, 0.5, use_dto=False, tangent_grad=False)
    q, k, v, _, _, _, do, _ = (x.double() for x in xs)
    rq, rk, rv = orc.grads_dout_only(q, k, v, do, 0.5)
    errs = [orc.rel_l2(a, b) for a, b in zip((dq, dk, dv), (rq, rk, rv))]
    # the reference backward's own error: FA2 numerics emulated on the same inputs
    em = orc.fa2_bwd_emulator(xs[0], xs[1], xs[2], xs[6], 0.5, round_dtype=dtype)
    floor = [orc.rel_l2(a.to(dtype), b) for a, b in zip(em, (rq, rk, rv))]
    print("  rel-L2 dq %.2e dk %.2e dv %.2e" % tuple(errs), " FA2 floor dq %.2e dk %.2e dv %.2e" % tuple(floor))
    assert max(errs) <= 1e-2
    for e, f in zip(errs, floor):
        assert e <= 1.25 * f + 1e-4
    for a, b in zip((dq, dk, dv), (rq, rk, rv)):
        torch.testing.assert_close(a.double(), b, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_fwd_bwd_test_against_naive_in_dtype(gpu, dtype):
    """The reference's `_test_fwd_bwd` check: zero tangents, autograd of the in-dtype naive oracle."""
    shape = (1, 2, 999, 999, 64)
    q, k, v, _, _, _, do, _ = _case(shape, dtype)
    z = torch.zeros_like
    xs = (q, k, v, z(q), z(k), z(v), do, z(do))
    dq, dk, dv = _grad_run(gpu, xs, 0.5, use_dto=False, tangent_grad=False)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    ref_out = orc.naive_attention_in_dtype(*leaves, 0.5, dtype)
    ref_out.backward(do)
    rtol = 2e-2 if dtype == torch.bfloat16 else 0
    torch.testing.assert_close(leaves[0].grad, dq, atol=1e-2, rtol=rtol / 2)
    torch.testing.assert_close(leaves[1].grad, dk, atol=1e-2, rtol=rtol / 2)
    torch.testing.assert_close(leaves[2].grad, dv, atol=1e-2, rtol=rtol)


FULL_SHAPES = [(1, 2, 1024, 1024, 64), (1, 2, 999, 999, 128), (1, 2, 1000, 515, 64), (2, 3, 300, 700, 128),
               (1, 2, 256, 1024, 128)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FULL_SHAPES)
def test_full_backward_with_tangent_grads(gpu, shape, dtype):
    print(f"case shape={shape} dtype={dtype}", flush=True)
    xs = _case(shape, dtype, tstd=0.1)
    got = _grad_run(gpu, xs, shape[-1] ** -0.5, use_dto=True, tangent_grad=True)
    ref = orc.grads_full(*(x.double() for x in xs), sm_scale=shape[-1] ** -0.5)
    errs = [orc.rel_l2(a, b) for a, b in zip(got, ref)]
    print("  rel-L2 dq %.2e dk %.2e dv %.2e dtq %.2e dtk %.2e dtv %.2e" % tuple(errs))
    assert max(errs) <= 1e-2


@pytest.fixture
def backward_mode():
    """Sets dmad_amd's backward mode for one test and restores the default."""
    from dmad_amd import set_backward_mode

    yield set_backward_mode
    set_backward_mode("auto")


@pytest.mark.parametrize("shape", [(1, 2, 999, 999, 128), (1, 3, 200, 130, 64)])
def test_full_backward_without_tangent_grads(gpu, shape, backward_mode):
    """Mode "full": the cotangent of `to` reaches q, k, v although no tangent requires grad."""
    backward_mode("full")
    xs = _case(shape, torch.bfloat16, tstd=0.1)
    got = _grad_run(gpu, xs, None, use_dto=True, tangent_grad=False)
    ref = orc.grads_full(*(x.double() for x in xs), sm_scale=shape[-1] ** -0.5)[:3]
    errs = [orc.rel_l2(a, b) for a, b in zip(got, ref)]
    assert max(errs) <= 1e-2, errs


@pytest.mark.parametrize("mode,tangent_grad", [("auto", False), ("reference", False), ("reference", True)])
def test_reference_backward_ignores_dto(gpu, backward_mode, mode, tangent_grad):
    """The default without tangent grads, and mode "reference" always, give the reference's
    dO-only gradients (the cotangent of `to` is ignored, tangents get no gradient)."""
    backward_mode(mode)
    xs = _case((1, 2, 300, 300, 64), torch.bfloat16, tstd=0.1)
    got = _grad_run(gpu, xs, 0.5, use_dto=True, tangent_grad=tangent_grad)
    q, k, v, _, _, _, do, _ = (x.double() for x in xs)
    ref = orc.grads_dout_only(q, k, v, do, 0.5)
    assert max(orc.rel_l2(a, b) for a, b in zip(got[:3], ref)) <= 1e-2
    assert all(g is None for g in got[3:])  # tangents: no gradient, as the reference


@pytest.mark.parametrize("D", [16, 32, 256])
def test_dout_only_backward_other_head_dims(gpu, D):
    xs = _case((1, 2, 333, 200, D), torch.bfloat16)
    dq, dk, dv = _grad_run(gpu, xs, None, use_dto=False, tangent_grad=False)
    q, k, v, _, _, _, do, _ = (x.double() for x in xs)
    ref = orc.grads_dout_only(q, k, v, do, D ** -0.5)
    errs = [orc.rel_l2(a, b) for a, b in zip((dq, dk, dv), ref)]
    assert max(errs) <= 1e-2, errs


def test_plain_attention_backward_bshd(gpu):
    from dmad_amd import torch_attention_op

    B, S, H, D = 1, 517, 3, 128
    g = torch.Generator().manual_seed(1)
    xs = [_draw(g, (B, S, H, D), 1.0, torch.bfloat16) for _ in range(4)]
    q, k, v, do = (x.to(gpu) for x in xs)
    for x in (q, k, v):
        x.requires_grad_(True)
    o = torch_attention_op(q, k, v)
    o.backward(do)
    ref = orc.grads_dout_only(*(x.double().transpose(1, 2) for x in xs), sm_scale=D ** -0.5)
    for got, r in zip((q.grad, k.grad, v.grad), ref):
        assert orc.rel_l2(got.cpu().transpose(1, 2), r) <= 1e-2
