"""Pins the CPU oracle (oracle/attention.py) before it is used as the checker.

Each oracle function is checked against something independent of its own
formula: brute-force loops, autodiff (forward and reverse mode), float64
central differences, and exact invariants of attention. A deliberately wrong
variant of the closed form is checked to fail, so the checks have teeth.
"""
import math

import pytest
import torch

from oracle import attention as orc

def _rand(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64) * std


def _inputs(B=1, H=2, Lq=7, Lk=5, D=4, Dv=None, seed=0, tstd=0.5):
    Dv = D if Dv is None else Dv
    q, k, v = _rand((B, H, Lq, D), seed), _rand((B, H, Lk, D), seed + 1), _rand((B, H, Lk, Dv), seed + 2)
    tq, tk, tv = (_rand((B, H, Lq, D), seed + 3, tstd), _rand((B, H, Lk, D), seed + 4, tstd),
                  _rand((B, H, Lk, Dv), seed + 5, tstd))
    return q, k, v, tq, tk, tv


def test_math_attention_brute_force():
    q, k, v, *_ = _inputs(Lq=3, Lk=4, D=2, Dv=3)
    s = 0.7
    o, lse = orc.math_attention(q, k, v, s)
    for b in range(1):
        for h in range(2):
            for i in range(3):
                sc = [s * sum(q[b, h, i, d] * k[b, h, j, d] for d in range(2)) for j in range(4)]
                mx = max(sc)
                den = sum(math.exp(x - mx) for x in sc)
                assert abs(float(lse[b, h, i]) - (mx + math.log(den))) < 1e-12
                for e in range(3):
                    ref = sum(math.exp(sc[j] - mx) / den * float(v[b, h, j, e]) for j in range(4))
                    assert abs(float(o[b, h, i, e]) - ref) < 1e-12


def test_lse_bounds_and_single_key():
    q, k, v, *_ = _inputs(Lq=9, Lk=6, D=8)
    _, lse = orc.math_attention(q, k, v, 0.3)
    smax = (torch.matmul(q, k.transpose(-1, -2)) * 0.3).amax(-1)
    assert torch.all(lse >= smax - 1e-12)
    assert torch.all(lse <= smax + math.log(6) + 1e-12)
    q, k, v, tq, tk, tv = _inputs(Lq=5, Lk=1, D=8)
    o, to, _, _ = orc.jvp_closed_form(q, k, v, tq, tk, tv)
    assert torch.allclose(o, v.expand_as(o))
    assert torch.allclose(to, tv.expand_as(to))


@pytest.mark.parametrize("shape", [(1, 2, 33, 17, 8, 8), (2, 3, 16, 40, 16, 4), (1, 1, 5, 5, 32, 64)])
def test_closed_form_matches_autodiff(shape):
    B, H, Lq, Lk, D, Dv = shape
    args = _inputs(B, H, Lq, Lk, D, Dv, seed=3)
    o, to, _, _ = orc.jvp_closed_form(*args, sm_scale=0.4)
    o_ad, to_ad = orc.jvp_attention_autodiff(*args, sm_scale=0.4)
    assert torch.allclose(o, o_ad, atol=1e-13, rtol=0)
    assert torch.allclose(to, to_ad, atol=1e-13, rtol=0)


def test_closed_form_matches_central_difference():
    q, k, v, tq, tk, tv = _inputs(Lq=6, Lk=9, D=8, seed=11)
    eps = 1e-6
    plus = orc.math_attention(q + eps * tq, k + eps * tk, v + eps * tv, 0.5)[0]
    minus = orc.math_attention(q - eps * tq, k - eps * tk, v - eps * tv, 0.5)[0]
    fd = (plus - minus) / (2 * eps)
    _, to, _, _ = orc.jvp_closed_form(q, k, v, tq, tk, tv, 0.5)
    assert torch.allclose(to, fd, atol=1e-8, rtol=0)


def test_wrong_closed_form_is_caught():
    """A plausible slip (dropping the -mu centring) must fail the autodiff check."""
    q, k, v, tq, tk, tv = _inputs(Lq=6, Lk=9, D=8, seed=12)
    s = 0.5
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    P = torch.softmax(S, -1)
    Sd = (torch.matmul(tq, k.transpose(-1, -2)) + torch.matmul(q, tk.transpose(-1, -2))) * s
    wrong = torch.matmul(P, tv) + torch.matmul(P * Sd, v)
    _, to_ad = orc.jvp_attention_autodiff(q, k, v, tq, tk, tv, s)
    assert not torch.allclose(wrong, to_ad, atol=1e-6)


def test_jvp_invariants():
    q, k, v, tq, tk, tv = _inputs(Lq=10, Lk=12, D=8, seed=5)
    s = 0.35
    z = torch.zeros_like
    # zero tangents
    _, to, _, _ = orc.jvp_closed_form(q, k, v, z(tq), z(tk), z(tv), s)
    assert torch.all(to == 0)
    # linearity in the tangents (jointly)
    _, t1, _, _ = orc.jvp_closed_form(q, k, v, tq, tk, tv, s)
    _, t2, _, _ = orc.jvp_closed_form(q, k, v, 3 * tq, 3 * tk, 3 * tv, s)
    assert torch.allclose(t2, 3 * t1, atol=1e-12)
    # Vd-only tangent: Od = attention(Q, K, Vd)
    _, to, _, _ = orc.jvp_closed_form(q, k, v, z(tq), z(tk), tv, s)
    assert torch.allclose(to, orc.math_attention(q, k, tv, s)[0], atol=1e-13)
    # joint key permutation leaves everything invariant
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(0))
    a = orc.jvp_closed_form(q, k, v, tq, tk, tv, s)
    b = orc.jvp_closed_form(q, k[..., perm, :], v[..., perm, :], tq, tk[..., perm, :], tv[..., perm, :], s)
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=1e-12)
    # Qd = c Q with Kd = 0: Sd = c S (temperature derivative)
    c = 0.7
    o, to, _, mu = orc.jvp_closed_form(q, k, v, c * q, z(tk), z(tv), s)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    P = torch.softmax(S, -1)
    assert torch.allclose(mu, c * (P * S).sum(-1), atol=1e-12)


def test_grads_dout_only_match_autograd():
    q, k, v, *_ = _inputs(Lq=11, Lk=7, D=8, seed=7)
    do = _rand((1, 2, 11, 8), 99)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    o = orc.math_attention(*leaves, 0.6)[0]
    ref = torch.autograd.grad((o * do).sum(), leaves)
    got = orc.grads_dout_only(q, k, v, do, 0.6)
    for x, y in zip(got, ref):
        assert torch.allclose(x, y, atol=1e-13)


@pytest.mark.parametrize("shape", [(1, 2, 9, 13, 8, 8), (1, 1, 16, 4, 4, 4)])
def test_grads_full_match_autograd_and_finite_differences(shape):
    B, H, Lq, Lk, D, Dv = shape
    args = _inputs(B, H, Lq, Lk, D, Dv, seed=21)
    do, dto = _rand((B, H, Lq, Dv), 31), _rand((B, H, Lq, Dv), 32, 0.1)
    got = orc.grads_full(*args, do, dto, sm_scale=0.45)
    ref = orc.grads_full_autodiff(*args, do, dto, sm_scale=0.45)
    for x, y in zip(got, ref):
        assert torch.allclose(x, y, atol=1e-13)

    # directional finite difference of L = <dO, O> + <dOd, Od>
    def loss(a):
        o, to, _, _ = orc.jvp_closed_form(*a, sm_scale=0.45)
        return float((o * do).sum() + (to * dto).sum())

    dirs = [_rand(x.shape, 40 + i) for i, x in enumerate(args)]
    eps = 1e-6
    fd = (loss([x + eps * d for x, d in zip(args, dirs)]) - loss([x - eps * d for x, d in zip(args, dirs)])) / (2 * eps)
    an = sum(float((g * d).sum()) for g, d in zip(got, dirs))
    assert abs(fd - an) < 1e-6 * max(1.0, abs(an))


def test_dout_only_grads_are_full_grads_without_dto():
    args = _inputs(Lq=8, Lk=8, D=8, seed=50)
    do = _rand((1, 2, 8, 8), 51)
    full = orc.grads_full(*args, do, torch.zeros_like(do), sm_scale=0.5)
    a = orc.grads_dout_only(*args[:3], do, sm_scale=0.5)
    for x, y in zip(a, full[:3]):
        assert torch.allclose(x, y, atol=1e-13)
    for g in full[3:]:
        assert torch.all(g == 0)


@pytest.mark.parametrize("block_n", [16, 32, 64, 128])
def test_triton_emulator_exact_without_rounding(block_n):
    args = _inputs(Lq=20, Lk=150, D=16, seed=60)
    o, to, lse = orc.triton_fwd_emulator(*args, sm_scale=0.3, block_n=block_n, round_dtype=None)
    ro, rto, rlse, _ = orc.jvp_closed_form(*args, sm_scale=0.3)
    assert torch.allclose(o, ro, atol=1e-12)
    assert torch.allclose(to, rto, atol=1e-12)
    assert torch.allclose(lse, rlse, atol=1e-12)


def test_triton_emulator_bf16_within_reference_tolerance():
    # reference _test_jvp shape (1, 2, 999, 64), N(0, 0.5^2) inputs, sm_scale 0.5
    g = torch.Generator().manual_seed(20)
    xs = [(torch.randn((1, 2, 999, 64), generator=g, dtype=torch.float64) * 0.5).to(torch.bfloat16) for _ in range(6)]
    o, to, _ = orc.triton_fwd_emulator(*xs, sm_scale=0.5, block_n=64)
    ref_o, ref_to = orc.jvp_attention_autodiff(*(x.double() for x in xs), sm_scale=0.5)
    torch.testing.assert_close(o.to(torch.bfloat16).double(), ref_o, atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(to.to(torch.bfloat16).double(), ref_to, atol=2e-2, rtol=1e-2)
    assert orc.rel_l2(o, ref_o) < 1e-2 and orc.rel_l2(to, ref_to) < 1e-2


def test_naive_in_dtype_reduces_to_math_attention():
    q, k, v, *_ = _inputs(Lq=12, Lk=9, D=8, seed=70)
    a = orc.naive_attention_in_dtype(q, k, v, 0.5, torch.float64)
    b = orc.math_attention(q, k, v, 0.5)[0]
    assert torch.allclose(a, b, atol=1e-13)


def test_rows_subset_matches_full():
    args = _inputs(Lq=30, Lk=40, D=8, seed=80)
    full = orc.jvp_closed_form(*args, sm_scale=0.5)
    rows = [0, 7, 29]
    sub = orc.jvp_rows(*args, rows=rows, sm_scale=0.5)
    for x, y in zip(full, sub):
        assert torch.allclose(x[..., rows, :] if x.dim() == 4 else x[..., rows], y, atol=1e-13)


@pytest.mark.parametrize("shape", [(1, 2, 40, 40, 16), (2, 1, 33, 17, 32)])
def test_fa2_bwd_emulator_exact_without_rounding(shape):
    B, H, Lq, Lk, D = shape
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (torch.randn(B, H, L, D, generator=g, dtype=torch.float64) for L in (Lq, Lk, Lk, Lq))
    got = orc.fa2_bwd_emulator(q, k, v, do, 0.3, round_dtype=None)
    ref = orc.grads_dout_only(q, k, v, do, 0.3)
    for a, b in zip(got, ref):
        assert torch.allclose(a, b, atol=1e-12, rtol=0)


def test_fa2_bwd_emulator_bf16_within_reference_tolerance():
    g = torch.Generator().manual_seed(20)
    q, k, v, do = ((torch.randn(1, 2, 256, 64, generator=g, dtype=torch.float64) * sd).to(torch.bfloat16)
                   for sd in (0.5, 0.5, 0.5, 1.0))
    got = orc.fa2_bwd_emulator(q, k, v, do, 0.5)
    ref = orc.grads_dout_only(*(x.double() for x in (q, k, v, do)), 0.5)
    for a, b in zip(got, ref):
        e = orc.rel_l2(a.to(torch.bfloat16), b)
        assert 1e-4 < e < 1e-2  # rounding shows, and stays within the reference tests' bar
