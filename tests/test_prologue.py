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
@pytest.mark.parametrize("B,L,H,D", [(1, 300, 8, 96), (2, 70, 20, 40), (1, 50, 30, 24), (1, 40, 11, 112)])
def test_kernel_matches_oracle_odd_head_dims(gpu, B, L, H, D):
    """Head dims whose 16-byte chunk count D/8 does not divide the 64 lanes of a wave
    (a lane's chunks then sit at different positions inside their heads, so each
    chunk needs its own rotation angles), at model dims C = H*D above 512 so that
    every lane holds more than one chunk."""
    from dmad_amd import apply_rope_with_tangent, rmsnorm_rope_with_tangent

    print(f"case prologue odd head dim B={B} L={L} H={H} D={D}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(D)
    C = H * D
    y = torch.randn(B, L, C, generator=g, device=gpu).to(torch.bfloat16)
    ty = (torch.randn(B, L, C, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(C, generator=g, device=gpu)).to(torch.bfloat16)
    freqs = torch.rand(L, D // 2, generator=g, device=gpu) * 40
    q, tq = rmsnorm_rope_with_tangent((y, ty), w, 1e-6, freqs, H)
    x = y.view(B, L, H, D)
    out, tout = apply_rope_with_tangent(x, ty.view(B, L, H, D), freqs)
    torch.cuda.synchronize()
    rq, rtq = orp.rmsnorm_rope_jvp(y.cpu(), ty.cpu(), w.cpu(), 1e-6, freqs.cpu(), H)
    ro, rto = orp.rope_jvp(x.cpu(), ty.view(B, L, H, D).cpu(), freqs.cpu())
    for got, ref, name in ((q, rq, "q"), (tq, rtq, "q_dot"), (out, ro, "rope"), (tout, rto, "rope_dot")):
        ulps = _bf16_ulp_ratio(got.cpu(), ref)
        print(f"  {name}: max {ulps:.2f} ulp")
        assert ulps <= 2.0, name


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


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 32760, 12, 128), (2, 300, 3, 64)])
def test_rope_only_matches_oracle_and_backward(gpu, shape):
    """apply_rope_with_tangent (the rotation alone, rope.py:106-114): outputs against the
    oracle's apply_rope / its jvp, and the backward against autograd of the oracle."""
    from dmad_amd import apply_rope_with_tangent

    B, S, H, D = shape
    g = torch.Generator(device=gpu).manual_seed(2)
    x = torch.randn(B, S, H, D, generator=g, device=gpu).to(torch.bfloat16)
    tx = (torch.randn(B, S, H, D, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    freqs = rope_freqs_3d(21, 30, 52, D, device=gpu) if S == 32760 else torch.rand(S, D // 2, generator=g, device=gpu) * 40
    out, tout = apply_rope_with_tangent(x, tx, freqs)
    torch.cuda.synchronize()
    rows = slice(0, min(S, 4096))
    rx, rtx, rf = x[:, rows].cpu(), tx[:, rows].cpu(), freqs[rows].cpu()
    ro, rto = orp.rope_jvp(rx, rtx, rf)
    for got, ref, name in ((out[:, rows].cpu(), ro, "out"), (tout[:, rows].cpu(), rto, "t_out")):
        ulps = _bf16_ulp_ratio(got, ref)
        print(f"  {name}: max {ulps:.2f} ulp")
        assert ulps <= 2.0, name
    # backward: rotation by -freqs, against autograd through the oracle's apply_rope
    xs = x[:, rows].detach().clone().requires_grad_(True)
    txs = tx[:, rows].detach().clone().requires_grad_(True)
    o2, to2 = apply_rope_with_tangent(xs, txs, freqs[rows])
    go = torch.randn_like(o2)
    gto = torch.randn_like(to2)
    ((o2.float() * go.float()).sum() + (to2.float() * gto.float()).sum()).backward()
    torch.cuda.synchronize()
    cx = rx.clone().requires_grad_(True)
    orp.apply_rope(cx, rf).float().mul(go.cpu().float()).sum().backward()
    ctx_ = rtx.clone().requires_grad_(True)
    orp.apply_rope(ctx_, rf).float().mul(gto.cpu().float()).sum().backward()
    for got, ref, name in ((xs.grad.cpu(), cx.grad, "grad x"), (txs.grad.cpu(), ctx_.grad, "grad t_x")):
        ulps = _bf16_ulp_ratio(got, ref)
        print(f"  {name}: max {ulps:.2f} ulp")
        assert ulps <= 2.0, name


@pytest.mark.gpu
def test_fused_prologue_refuses_gradients(gpu):
    from dmad_amd import rmsnorm_rope_with_tangent

    y = torch.randn(1, 8, 128, device=gpu, dtype=torch.bfloat16, requires_grad=True)
    w = torch.ones(128, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no backward"):
        rmsnorm_rope_with_tangent((y, None), w, 1e-6, None, 1)
    with torch.no_grad():
        rmsnorm_rope_with_tangent((y, None), w, 1e-6, None, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("cached_k_rotated", [False, True])
def test_a2a_op_one_gpu_with_rope(gpu, cached_k_rotated):
    """MinimalA2AAttnOpWithT (jvp_helper.py:125-210, one GPU): RoPE with tangent on q
    (and k), then the JVP attention, against the oracle's rope_jvp followed by the
    attention closed form."""
    from types import SimpleNamespace

    from dmad_amd import MinimalA2AAttnOpWithT, RopeCache
    from oracle import attention as orc

    B, S, H, D = 1, 700, 2, 128
    g = torch.Generator(device=gpu).manual_seed(3)
    r = lambda sd: (torch.randn(B, S, H, D, generator=g, device=gpu) * sd).to(torch.bfloat16)  # noqa: E731
    q, k, v, tq, tk, tv = r(1.0), r(1.0), r(1.0), r(0.1), r(0.1), r(0.1)
    fq = torch.rand(S, D // 2, generator=g, device=gpu) * 30
    fk = torch.rand(S, D // 2, generator=g, device=gpu) * 30
    if cached_k_rotated:
        rope = RopeCache(query_freqs=fq, current_key_freqs=fk, cached_k_rotated=True)
    else:
        rope = RopeCache(query_freqs=fq, key_freqs=fk, cached_k_rotated=False)
    op = MinimalA2AAttnOpWithT()
    with torch.no_grad():
        o, to = op((q, tq), (k, tk), (v, tv), attn_ctx=SimpleNamespace(rope=rope, kv_cache=None))
    torch.cuda.synchronize()
    qr, tqr = orp.rope_jvp(q.cpu(), tq.cpu(), fq.cpu())
    kr, tkr = orp.rope_jvp(k.cpu(), tk.cpu(), fk.cpu())
    bhsd = lambda t: t.transpose(1, 2).double()  # noqa: E731
    ro, rto, _, _ = orc.jvp_closed_form(bhsd(qr), bhsd(kr), bhsd(v.cpu()), bhsd(tqr), bhsd(tkr), bhsd(tv.cpu()))
    assert orc.rel_l2(o.transpose(1, 2).cpu(), ro) < 1e-2
    assert orc.rel_l2(to.transpose(1, 2).cpu(), rto) < 1e-2
    with pytest.raises(NotImplementedError):
        op((q, tq), (k, tk), (v, tv), attn_ctx=SimpleNamespace(rope=rope, kv_cache=object(), mode="APPEND"))
