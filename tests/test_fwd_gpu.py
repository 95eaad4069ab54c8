"""Forward(+JVP) kernel parity on the GPU against the CPU oracle.

Shapes and value distributions are the reference's own op tests
(flash_attention_jvp_triton.py:627-658 `_test_jvp`, :768-803 `_test_jvp_ca`,
:585-624 `_test_fwd_bwd`, :728-765 `_test_fwd_bwd_ca`): N(0, 0.5^2) inputs,
seed 20, sm_scale 0.5, ragged lengths, Lq != Lk and Dqk != Dv.

Bar: relative L2 error <= 1e-2 against the float64 closed form on the same
rounded inputs, no worse than the reference kernel's own error (its numerics
emulated on the CPU, oracle.triton_fwd_emulator, BLOCK_N = 64) plus a small
margin, and the reference tests' own assert_close tolerances.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

REF_JVP = [(1, 2, 1024, 1024, 64, 64), (1, 2, 999, 999, 64, 64)]
REF_JVP_CA = [(1, 2, 256, 1024, 64, 128), (1, 2, 1000, 15, 128, 32), (1, 2, 512, 512, 16, 32),
              (1, 2, 515, 999, 16, 32)]
REF_FWD_CA = [(1, 2, 256, 1024, 128, 128), (1, 2, 1024, 256, 128, 128), (1, 2, 1024, 512, 64, 64),
              (1, 2, 1000, 515, 64, 64)]
DTYPES = [torch.bfloat16, torch.float16]


def _inputs(shape, dtype, seed=20, std=0.5, tstd=0.5):
    B, H, Lq, Lk, Dqk, Dv = shape
    g = torch.Generator().manual_seed(seed)

    def d(L, D, s):
        return (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * s).to(dtype)

    return d(Lq, Dqk, std), d(Lk, Dqk, std), d(Lk, Dv, std), d(Lq, Dqk, tstd), d(Lk, Dqk, tstd), d(Lk, Dv, tstd)


def _run(xs, dev, sm_scale):
    from dmad_amd import attention

    g = [x.to(dev) for x in xs]
    o, to = attention(*g, sm_scale)
    torch.cuda.synchronize()
    return o.cpu(), to.cpu()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", REF_JVP + REF_JVP_CA + REF_FWD_CA)
def test_jvp_forward_matches_oracle(gpu, shape, dtype):
    print(f"case shape={shape} dtype={dtype}", flush=True)
    xs = _inputs(shape, dtype)
    o, to = _run(xs, gpu, 0.5)
    ref_o, ref_to, _, _ = orc.jvp_closed_form(*(x.double() for x in xs), sm_scale=0.5)
    e_o, e_to = orc.rel_l2(o, ref_o), orc.rel_l2(to, ref_to)
    em_o, em_to, _ = orc.triton_fwd_emulator(*xs, sm_scale=0.5, block_n=64, round_dtype=dtype)
    f_o, f_to = orc.rel_l2(em_o.to(dtype), ref_o), orc.rel_l2(em_to.to(dtype), ref_to)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})")
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4
    atol = 2e-2 if dtype == torch.bfloat16 else 1e-2
    torch.testing.assert_close(o.double(), ref_o, atol=1e-2, rtol=0)
    torch.testing.assert_close(to.double(), ref_to, atol=atol, rtol=1e-2)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_jvp_test_against_naive_in_dtype(gpu, dtype):
    """The reference's `_test_jvp` check verbatim: jvp of the in-dtype naive oracle."""
    xs = _inputs((1, 2, 1024, 1024, 64, 64), dtype)
    fn = lambda q, k, v: orc.naive_attention_in_dtype(q, k, v, 0.5, dtype)  # noqa: E731
    _, ref_to = torch.func.jvp(fn, tuple(xs[:3]), tuple(xs[3:]))
    _, to = _run(xs, gpu, 0.5)
    torch.testing.assert_close(ref_to.to(dtype), to, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("shape", [(1, 2, 999, 999, 64, 64), (2, 3, 300, 77, 128, 128), (1, 1, 64, 64, 256, 256),
                                   (1, 2, 100, 200, 32, 16), (1, 1, 130, 1, 64, 64)])
def test_lse_and_mu(gpu, shape):
    from dmad_amd.jvp_attention import jvp_attention_forward

    xs = _inputs(shape, torch.bfloat16, seed=3)
    g = [x.to(gpu) for x in xs]
    o, to, lse, mu = jvp_attention_forward(*g, sm_scale=shape[4] ** -0.5)
    ref_o, ref_to, ref_lse, ref_mu = orc.jvp_closed_form(*(x.double() for x in xs), sm_scale=shape[4] ** -0.5)
    assert (lse.cpu().double() - ref_lse).abs().max() < 2e-3
    assert orc.rel_l2(mu.cpu(), ref_mu) < 1e-2
    assert orc.rel_l2(o.cpu(), ref_o) < 1e-2 and orc.rel_l2(to.cpu(), ref_to) < 1e-2


@pytest.mark.parametrize("shape", [(1, 2, 999, 999, 64, 64), (1, 3, 1000, 515, 128, 128), (1, 2, 64, 15, 16, 32)])
def test_plain_forward(gpu, shape):
    from dmad_amd.jvp_attention import jvp_attention_forward

    q, k, v, *_ = _inputs(shape, torch.bfloat16, seed=4)
    o, to, lse, mu = jvp_attention_forward(q.to(gpu), k.to(gpu), v.to(gpu), None, None, None, sm_scale=0.3)
    assert to is None and mu is None
    ref_o, ref_lse = orc.math_attention(q.double(), k.double(), v.double(), 0.3)
    assert orc.rel_l2(o.cpu(), ref_o) < 1e-2
    assert (lse.cpu().double() - ref_lse).abs().max() < 2e-3


@pytest.mark.parametrize("Lk", [512, 4100])  # the two-workgroups-per-CU kernel, then the one-per-CU kernel
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kv_tangent_zero_fast_path(gpu, dtype, Lk):
    """tk = tv = None against zero tangents through the general path: O bit for bit. In fp16
    the fast path forms the same H~ = P~ (s Sd), so Od matches too; in bf16 it leaves the
    softmax scale out of H~ (and applies it to C~ and r in the epilogue), so Od differs by the
    rounding of H~, and must be as close to the float64 oracle as the general path's."""
    from dmad_amd import attention

    xs = _inputs((1, 2, 700, Lk, 128, 128), dtype, seed=5)
    q, k, v, tq, tk, tv = (x.to(gpu) for x in xs)
    o1, to1 = attention(q, k, v, tq, None, None)
    o2, to2 = attention(q, k, v, tq, torch.zeros_like(tk), torch.zeros_like(tv))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    if dtype == torch.float16:
        assert orc.rel_l2(to1, to2) < 1e-6
    else:
        zk, zv = torch.zeros_like(xs[4]), torch.zeros_like(xs[5])
        _, ref_to, _, _ = orc.jvp_closed_form(*(x.double() for x in (xs[0], xs[1], xs[2], xs[3], zk, zv)))
        e_fast, e_gen = orc.rel_l2(to1.cpu(), ref_to), orc.rel_l2(to2.cpu(), ref_to)
        assert orc.rel_l2(to1, to2) < 1e-2
        assert e_fast <= 1.1 * e_gen + 1e-4, (e_fast, e_gen)


def test_bshd_views_and_helper(gpu):
    """Wan layout: [B, S, H, D] storage, BHSD views with row stride H*D."""
    from dmad_amd import torch_attention_op_withT

    B, S, H, D = 2, 333, 5, 128
    g = torch.Generator().manual_seed(9)
    xs = [(torch.randn((B, S, H, D), generator=g, dtype=torch.float64) * 0.5).to(torch.bfloat16) for _ in range(6)]
    q, k, v, tq, tk, tv = (x.to(gpu) for x in xs)
    o, to = torch_attention_op_withT((q, tq), (k, tk), (v, tv))
    assert o.shape == (B, S, H, D) and not to.requires_grad
    ref_o, ref_to, _, _ = orc.jvp_closed_form(*(x.double().transpose(1, 2) for x in xs))
    assert orc.rel_l2(o.cpu().transpose(1, 2), ref_o) < 1e-2
    assert orc.rel_l2(to.cpu().transpose(1, 2), ref_to) < 1e-2


def test_non_unit_head_stride_is_copied(gpu):
    from dmad_amd import attention

    xs = _inputs((1, 2, 200, 300, 64, 64), torch.bfloat16, seed=6)
    # [B,H,D,L] storage viewed as [B,H,L,D]: stride_d != 1
    g = [x.transpose(-1, -2).contiguous().to(gpu).transpose(-1, -2) for x in xs]
    o, to = attention(*g)
    ref_o, ref_to, _, _ = orc.jvp_closed_form(*(x.double() for x in xs))
    assert orc.rel_l2(o.cpu(), ref_o) < 1e-2 and orc.rel_l2(to.cpu(), ref_to) < 1e-2


def test_tangent_linearity_and_zero(gpu):
    from dmad_amd import attention

    xs = _inputs((1, 2, 512, 512, 128, 128), torch.bfloat16, seed=7)
    q, k, v, tq, tk, tv = (x.to(gpu) for x in xs)
    _, t0 = attention(q, k, v, torch.zeros_like(tq), torch.zeros_like(tk), torch.zeros_like(tv))
    assert torch.count_nonzero(t0) == 0
    _, t1 = attention(q, k, v, tq, tk, tv)
    _, t2 = attention(q, k, v, 2 * tq, 2 * tk, 2 * tv)  # exact in bf16
    assert orc.rel_l2(t2.float(), 2 * t1.float()) < 1e-2
