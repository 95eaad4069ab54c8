"""Fused RMSNorm(+JVP) + RoPE-with-tangent prologue.

CPU: the oracle (oracle/prologue.py) is pinned by per-element float64 loops
written from the formulas, by central differences of its tangent, and by the
rotation's invariants; a sign error planted in the rotation fails the loops.
GPU: the HIP kernel against the oracle on the same bf16 inputs at the Wan
shapes. Bar: the reference's rounding points are reproduced, so outputs differ
from the oracle only where float32 reductions or sin/cos differ in the last
bit: relative L2 <= 2e-3 and at most 2 bf16 ulps (relative 2^-7) per element.
"""
import math

import pytest
import torch

from dmad_amd.workload import rope_freqs_3d
from oracle import prologue as orp


def _loops(y, ty, w, eps, freqs, H):
    """Per-element float64 restatement (no intermediate rounding)."""
    B, L, C = y.shape
    D = C // H
    q = torch.zeros(B, L, H, D, dtype=torch.float64)
    tq = torch.zeros_like(q)
    for b in range(B):
        for l in range(L):
            row, trow = y[b, l].tolist(), ty[b, l].tolist()
            m = sum(v * v for v in row) / C
            md = sum(2 * a * t for a, t in zip(row, trow)) / C
            r = 1.0 / math.sqrt(m + eps)
            rd = -0.5 * r ** 3 * md
            n = [row[c] * r * w[c] for c in range(C)]
            nd = [(trow[c] * r + row[c] * rd) * w[c] for c in range(C)]
            for h in range(H):
                for i in range(D // 2):
                    a = float(freqs[l, i]) if freqs is not None else 0.0
                    cs, sn = math.cos(a), math.sin(a)
                    e, o = h * D + 2 * i, h * D + 2 * i + 1
                    q[b, l, h, 2 * i] = n[e] * cs - n[o] * sn
                    q[b, l, h, 2 * i + 1] = n[o] * cs + n[e] * sn
                    tq[b, l, h, 2 * i] = nd[e] * cs - nd[o] * sn
                    tq[b, l, h, 2 * i + 1] = nd[o] * cs + nd[e] * sn
    return q, tq


def _small(seed=0, B=2, L=6, H=3, D=8, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    C = H * D
    y = torch.randn(B, L, C, generator=g, dtype=torch.float64).to(dtype)
    ty = (torch.randn(B, L, C, generator=g, dtype=torch.float64) * 0.1).to(dtype)
    w = (1 + 0.1 * torch.randn(C, generator=g, dtype=torch.float64)).to(dtype)
    freqs = torch.rand(L, D // 2, generator=g, dtype=torch.float64) * 6.0
    return y, ty, w, freqs, H


def test_oracle_matches_elementwise_loops():
    y, ty, w, freqs, H = _small()
    q, tq = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, freqs, H)
    rq, rtq = _loops(y, ty, w, 1e-6, freqs, H)
    assert torch.allclose(q, rq, rtol=1e-12, atol=1e-12) and torch.allclose(tq, rtq, rtol=1e-12, atol=1e-12)


def test_planted_rotation_sign_error_fails_the_loops():
    y, ty, w, freqs, H = _small(seed=1)
    q, _ = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, -freqs, H)  # rotating the wrong way
    rq, _ = _loops(y, ty, w, 1e-6, freqs, H)
    assert not torch.allclose(q, rq, rtol=1e-6, atol=1e-6)


def test_oracle_tangent_is_the_derivative():
    y, ty, w, freqs, H = _small(seed=2)
    _, tq = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, freqs, H)
    h = 1e-6
    qp, _ = orp.rmsnorm_rope_jvp(y + h * ty, ty, w, 1e-6, freqs, H)
    qm, _ = orp.rmsnorm_rope_jvp(y - h * ty, ty, w, 1e-6, freqs, H)
    assert torch.allclose((qp - qm) / (2 * h), tq, rtol=1e-6, atol=1e-8)


def test_rotation_invariants():
    y, ty, w, freqs, H = _small(seed=3)
    q0, tq0 = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, None, H)
    q, tq = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, freqs, H)
    # pair norms are kept; zero angles are the identity; the tangent is linear
    pn = lambda x: x.view(*x.shape[:-1], -1, 2).pow(2).sum(-1)  # noqa: E731
    assert torch.allclose(pn(q), pn(q0)) and torch.allclose(pn(tq), pn(tq0))
    qz, tqz = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, torch.zeros_like(freqs), H)
    assert torch.allclose(qz, q0) and torch.allclose(tqz, tq0)
    _, tq2 = orp.rmsnorm_rope_jvp(y, 3 * ty, w, 1e-6, freqs, H)
    assert torch.allclose(tq2, 3 * tq)


def test_oracle_rounding_points_in_bf16():
    """In bf16 the oracle rounds after the norm, after the weight and after the rotation."""
    y, ty, w, freqs, H = _small(seed=4, dtype=torch.bfloat16)
    q, tq = orp.rmsnorm_rope_jvp(y, ty, w, 1e-6, freqs, H)
    assert q.dtype == torch.bfloat16 and tq.dtype == torch.bfloat16
    rq, rtq = _loops(y.double(), ty.double(), w.double(), 1e-6, freqs, H)
    assert (q.double() - rq).abs().max() <= 2 ** -6 * rq.abs().max()


def _bf16_ulp_ratio(a, b):
    """max |a - b| in bf16 ulps of |b| (2^-7 relative), with a floor of one ulp of
    1/2 the rms (where the rotation cancels, the output is far below its terms)."""
    a, b = a.double(), b.double()
    ulp = (torch.maximum(b.abs(), 0.5 * b.pow(2).mean().sqrt())) * 2.0 ** -7
    return float(((a - b).abs() / ulp).max())


WAN = [(1, 32760, 12, 128, (21, 30, 52)), (1, 32760, 40, 128, (21, 30, 52)), (2, 512, 40, 128, None)]


@pytest.mark.gpu
@pytest.mark.parametrize("B,L,H,D,grid", WAN)
def test_kernel_matches_oracle(gpu, B, L, H, D, grid):
    from dmad_amd import rmsnorm_rope_with_tangent

    print(f"case prologue B={B} L={L} H={H} D={D} rope={grid is not None}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(0)
    C = H * D
    y = torch.randn(B, L, C, generator=g, device=gpu).to(torch.bfloat16)
    ty = (torch.randn(B, L, C, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(C, generator=g, device=gpu)).to(torch.bfloat16)
    freqs = rope_freqs_3d(*grid, D, device=gpu) if grid is not None else None
    q, tq = rmsnorm_rope_with_tangent((y, ty), w, 1e-6, freqs, H)
    torch.cuda.synchronize()
    rows = slice(0, 4096)  # the oracle on the CPU over the first 4096 tokens
    ry, rty = y[:, rows].cpu(), ty[:, rows].cpu()
    rf = freqs[rows].cpu() if freqs is not None else None
    rq, rtq = orp.rmsnorm_rope_jvp(ry, rty, w.cpu(), 1e-6, rf, H)
    gq, gtq = q[:, rows].cpu(), tq[:, rows].cpu()
    for got, ref, name in ((gq, rq, "q"), (gtq, rtq, "q_dot")):
        rel = float((got.double() - ref.double()).norm() / ref.double().norm())
        ulps = _bf16_ulp_ratio(got, ref)
        same = float((got == ref).double().mean())
        print(f"  {name}: rel-L2 {rel:.2e}  max {ulps:.2f} ulp  identical {100 * same:.2f}%")
        assert rel <= 2e-3 and ulps <= 2.0, name


@pytest.mark.gpu
def test_kernel_primal_only_and_no_rope(gpu):
    from dmad_amd import rmsnorm_rope_with_tangent

    g = torch.Generator(device=gpu).manual_seed(1)
    y = torch.randn(2, 100, 3 * 64, generator=g, device=gpu).to(torch.bfloat16)
    w = torch.ones(192, device=gpu, dtype=torch.bfloat16)
    q, tq = rmsnorm_rope_with_tangent((y, None), w, 1e-6, None, 3)
    torch.cuda.synchronize()
    assert tq is None
    rq = orp.rmsnorm(y.cpu(), w.cpu(), 1e-6).view(2, 100, 3, 64)
    assert _bf16_ulp_ratio(q.cpu(), rq) <= 2.0
