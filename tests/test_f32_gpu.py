"""fp32 operands on the fp32 MFMA kernels (attn_f32.h).

The reference's forward accepts float32 q, k, v and tangents (no dtype assert
in _attention.forward, flash_attention_jvp_triton.py:463-499; the Triton dots
then take fp32 operands), and rcm/utils/attention.py:120-167 sends float32 to
PyTorch's memory-efficient SDPA, forward and backward. Here: the forward in the
three dense modes and the block-sparse one at every head dim (Dqk != Dv too),
ragged lengths and BSHD-strided views, and the dO-only backward, all against the
float64 oracle on the same fp32 inputs.

Bar: relative L2 <= 1e-5 on O, Od and the gradients, LSE and mu to 1e-5 absolute
(fp32 products and sums over at most a few thousand terms; the reference's own
fp32 forward is no more exact than this, its dots may even round to TF32).
"""
import math
import warnings

import pytest
import torch

from dmad_amd import magimask as mm
from oracle import attention as orc
from oracle import magi as om

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _draw(g, B, H, L, D, std, bshd):
    if bshd:
        return (torch.randn((B, L, H, D), generator=g, dtype=torch.float64) * std).float().transpose(1, 2)
    return (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * std).float()


FWD = [
    # B, H, Lq, Lk, Dqk, Dv, BSHD view
    (1, 2, 256, 256, 64, 64, False),  # the reference's CPU plumbing shape
    (2, 3, 999, 515, 128, 128, True),
    (1, 2, 77, 1000, 16, 16, False),
    (1, 2, 300, 129, 32, 32, True),
    (1, 1, 200, 333, 256, 256, False),
    (2, 2, 130, 97, 64, 128, False),
    (1, 2, 150, 260, 128, 256, True),
    (1, 2, 100, 64, 256, 64, False),
    (1, 1, 1, 1, 128, 128, False),
]


@pytest.mark.parametrize("mode", ["jvp", "qonly", "plain"])
@pytest.mark.parametrize("B,H,Lq,Lk,Dqk,Dv,bshd", FWD)
def test_forward_matches_oracle(gpu, B, H, Lq, Lk, Dqk, Dv, bshd, mode):
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case f32 fwd B={B} H={H} Lq={Lq} Lk={Lk} Dqk={Dqk} Dv={Dv} bshd={bshd} {mode}", flush=True)
    g = torch.Generator().manual_seed(Lq * 7 + Lk)
    q, k, v = _draw(g, B, H, Lq, Dqk, 1.0, bshd), _draw(g, B, H, Lk, Dqk, 1.0, bshd), _draw(g, B, H, Lk, Dv, 1.0, bshd)
    tq, tk, tv = _draw(g, B, H, Lq, Dqk, 0.1, bshd), _draw(g, B, H, Lk, Dqk, 0.1, bshd), _draw(g, B, H, Lk, Dv, 0.1, bshd)
    if mode == "qonly":
        tk, tv = torch.zeros_like(k), torch.zeros_like(v)
    s = Dqk ** -0.5
    dev = lambda x: x.to(gpu)  # noqa: E731
    o, to, lse, mu = jvp_attention_forward(dev(q), dev(k), dev(v), None if mode == "plain" else dev(tq),
                                           None if mode != "jvp" else dev(tk), None if mode != "jvp" else dev(tv), s)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and o.is_contiguous()
    ro, rto, rlse, rmu = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, tk, tv)), sm_scale=s)
    e_o = orc.rel_l2(o.cpu(), ro)
    assert e_o <= TOL, e_o
    assert float((lse.cpu().double() - rlse).abs().max()) <= TOL
    if mode != "plain":
        e_to = orc.rel_l2(to.cpu(), rto)
        assert e_to <= TOL, e_to
        assert float((mu.cpu().double() - rmu).abs().max()) <= TOL


BWD = [
    # B, H, Lq, Lk, D, BSHD view
    (1, 2, 256, 256, 64, False),
    (2, 3, 333, 515, 128, True),
    (1, 2, 200, 77, 16, False),
    (1, 2, 130, 300, 32, True),
    (1, 1, 150, 190, 256, False),
    (1, 2, 1, 40, 128, False),
]


@pytest.mark.parametrize("B,H,Lq,Lk,D,bshd", BWD)
def test_dout_only_backward_matches_oracle(gpu, B, H, Lq, Lk, D, bshd):
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    print(f"case f32 bwd B={B} H={H} Lq={Lq} Lk={Lk} D={D} bshd={bshd}", flush=True)
    g = torch.Generator().manual_seed(Lq + 3 * Lk + D)
    q, k, v, do = (_draw(g, B, H, L, D, 1.0, bshd) for L in (Lq, Lk, Lk, Lq))
    s = D ** -0.5
    qd, kd, vd, dod = (x.to(gpu) for x in (q, k, v, do))
    o, _, lse, _ = jvp_attention_forward(qd, kd, vd, None, None, None, s)
    dq, dk, dv, *_ = jvp_attention_backward(qd, kd, vd, None, None, None, o, None, lse, None, dod, None, s, False)
    torch.cuda.synchronize()
    rq, rk, rv = orc.grads_dout_only(q.double(), k.double(), v.double(), do.double(), sm_scale=s)
    for name, a, r in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        e = orc.rel_l2(a.cpu(), r)
        assert e <= TOL, (name, e)


def test_autograd_op_fp32(gpu):
    """_attention.apply on fp32: O, Od and the dO-only gradients of q, k, v; a tangent
    that requires grad gets None with a one-time warning in mode "auto" (the full
    derivative takes bf16/fp16), and mode "full" raises before any work."""
    import dmad_amd.jvp_attention as ja

    B, H, L, D = 2, 2, 200, 64
    g = torch.Generator().manual_seed(3)
    q, k, v, tq, tk, tv, do = (_draw(g, B, H, L, D, 1.0 if i < 3 or i == 6 else 0.1, False) for i in range(7))
    leaves = [x.to(gpu).requires_grad_(True) for x in (q, k, v)]
    o, to = ja.attention(*leaves, tq.to(gpu), tk.to(gpu), tv.to(gpu))
    o.backward(do.to(gpu))
    torch.cuda.synchronize()
    ro, rto, _, _ = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, tk, tv)))
    assert orc.rel_l2(o.detach().cpu(), ro) <= TOL and orc.rel_l2(to.detach().cpu(), rto) <= TOL
    for x, r in zip(leaves, orc.grads_dout_only(q.double(), k.double(), v.double(), do.double())):
        assert orc.rel_l2(x.grad.cpu(), r) <= TOL

    ja._warned_full_fallback = False
    tql = tq.to(gpu).requires_grad_(True)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        o, to = ja.attention(*(x.detach().requires_grad_(True) for x in leaves), tql, tk.to(gpu), tv.to(gpu))
    assert any("bfloat16 and float16" in str(x.message) for x in w)
    (o.sum() + to.sum()).backward()
    assert tql.grad is None
    ja.set_backward_mode("full")
    try:
        with pytest.raises(NotImplementedError, match="bfloat16 and float16"):
            ja.attention(*(x.detach().requires_grad_(True) for x in leaves), tql, tk.to(gpu), tv.to(gpu))
    finally:
        ja.set_backward_mode("auto")


def test_sdpa_twin_fp32(gpu):
    """rcm/utils/attention.py:120-167's entry point with float32 BSHD inputs: forward and
    backward on the fp32 kernels, against the float64 oracle."""
    from dmad_amd.sdpa import attention

    B, S, H, D = 1, 257, 3, 128
    g = torch.Generator().manual_seed(11)
    q, k, v, do = (torch.randn(B, S, H, D, generator=g, dtype=torch.float64).float() for _ in range(4))
    leaves = [x.to(gpu).requires_grad_(True) for x in (q, k, v)]
    out = attention(*leaves, softmax_scale=0.1, q_scale=0.5)
    out.backward(do.to(gpu))
    torch.cuda.synchronize()
    bhsd = lambda t: t.transpose(1, 2).double()  # noqa: E731
    qs = bhsd(q) * 0.5
    ro = orc.math_attention(qs, bhsd(k), bhsd(v), sm_scale=0.1)[0]
    assert orc.rel_l2(out.detach().cpu().transpose(1, 2), ro) <= TOL
    rq, rk, rv = orc.grads_dout_only(qs, bhsd(k), bhsd(v), bhsd(do), sm_scale=0.1)
    assert orc.rel_l2(leaves[0].grad.cpu().transpose(1, 2), rq * 0.5) <= TOL
    assert orc.rel_l2(leaves[1].grad.cpu().transpose(1, 2), rk) <= TOL
    assert orc.rel_l2(leaves[2].grad.cpu().transpose(1, 2), rv) <= TOL


MAGI = [
    # mode, frame tokens, blocks, window, sink, Dqk, Dv, tangent-free K/V
    ("block_causal", 16, 5, 0, 0, 64, 64, False),
    ("block_causal", 40, 4, 2, 1, 128, 128, True),
    ("teacher_forcing", 24, 3, 0, 0, 128, 128, False),
    ("teacher_forcing", 16, 6, 3, 1, 32, 256, False),
    # 256-wide Q, K: two 64-row workgroups per 128-query task, all of V in each
    ("block_causal", 24, 4, 2, 1, 256, 256, False),
    ("teacher_forcing", 20, 3, 0, 0, 256, 128, True),
]


@pytest.mark.parametrize("case", MAGI)
def test_block_sparse_forward_matches_oracle(gpu, case):
    from dmad_amd import attention

    mode, ft, nb, local, sink, dqk, dv, qonly = case
    print(f"case f32 magi {case}", flush=True)
    pat = mm.BlockPattern(frame_tokens=ft, first_chunk_frames=1, chunk_frames=1)
    if mode == "block_causal":
        Q = KV = pat.blocks_to_tokens(nb)
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, local_attn_blocks=local, sink_blocks=sink)
        allow = om.allowed_mask(mode, ft, Q, KV, 1, 1, local_attn_blocks=local, sink_blocks=sink)
    else:
        Q = KV = 2 * pat.blocks_to_tokens(nb)
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, clean_blocks=nb, local_attn_blocks=local, sink_blocks=sink)
        allow = om.allowed_mask(mode, ft, Q, KV, 1, 1, local_attn_blocks=local, sink_blocks=sink, clean_blocks=nb,
                                as_range_builder=True)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=64)
    g = torch.Generator().manual_seed(ft + nb)
    B, H = 2, 2
    q, k, v = _draw(g, B, H, Q, dqk, 1.0, False), _draw(g, B, H, KV, dqk, 1.0, False), _draw(g, B, H, KV, dv, 1.0, False)
    tq, tk, tv = _draw(g, B, H, Q, dqk, 0.1, False), _draw(g, B, H, KV, dqk, 0.1, False), _draw(g, B, H, KV, dv, 0.1, False)
    if qonly:
        tk, tv = torch.zeros_like(k), torch.zeros_like(v)
    s = dqk ** -0.5
    o, to = attention(q.to(gpu), k.to(gpu), v.to(gpu), tq.to(gpu), None if qonly else tk.to(gpu),
                      None if qonly else tv.to(gpu), s, mask)
    torch.cuda.synchronize()
    ro, rto, _, _ = om.masked_jvp(q, k, v, tq, tk, tv, allow, s)
    assert orc.rel_l2(o.cpu(), ro) <= TOL and orc.rel_l2(to.cpu(), rto) <= TOL


def test_block_sparse_hand_made_tables(gpu):
    """A group without keys gets O = Od = 0, LSE = -inf, mu = 0; rows no task covers
    stay untouched; ranges reaching outside the sequences are clipped (fp32, 256-wide V
    so both column chunks of a query tile take part)."""
    from dmad_amd import _native as nat

    Lq, Lk, D, Dv = 333, 240, 64, 256
    g = torch.Generator().manual_seed(13)
    q, k, tq, tk = (_draw(g, 1, 2, L, D, s, False) for L, s in ((Lq, 1.0), (Lk, 1.0), (Lq, 0.1), (Lk, 0.1)))
    v, tv = _draw(g, 1, 2, Lk, Dv, 1.0, False), _draw(g, 1, 2, Lk, Dv, 0.1, False)
    q_ranges = [[0, 100], [100, 230], [230, 300]]
    k_ranges = [[-20, 50], [90, 95], [250, 400], [10, 20], [200, 1000]]
    qk_map = [0, 2, 3, 5]
    tasks = [(0, 0), (1, 0), (1, 1), (2, 1), (2, 2)]
    S = 7.0
    xs = [x.to(gpu) for x in (q, k, v, tq, tk, tv)]
    i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=gpu).contiguous()  # noqa: E731
    qr, kr, qm = i32(q_ranges), i32(k_ranges), i32(qk_map)
    tg, tt = i32([t[0] for t in tasks]), i32([t[1] for t in tasks])
    o = torch.full((1, 2, Lq, Dv), S, device=gpu)
    to = torch.full_like(o, S)
    lse = torch.full((1, 2, Lq), S, device=gpu)
    mu = torch.full_like(lse, S)
    nat.check(nat.lib().dmad_attn_jvp_fwd_magi(
        nat.DMAD_F32, nat.DMAD_FWD_JVP, 1, 2, Lq, Lk, D, Dv,
        *(nat.ptr(x) for x in xs), nat.strides4(xs[0]), nat.strides4(xs[1]), nat.strides4(xs[2]),
        nat.ptr(o), nat.ptr(to), nat.strides4(o), nat.ptr(lse), nat.ptr(mu), 0.125,
        nat.ptr(qr), nat.ptr(kr), nat.ptr(qm), 3, 5, nat.ptr(tg), nat.ptr(tt), len(tasks), 128, None, 0,
        nat.stream_ptr(gpu)))
    torch.cuda.synchronize()
    o, to, lse, mu = o.cpu(), to.cpu(), lse.cpu(), mu.cpu()
    allow = torch.zeros(Lq, Lk, dtype=torch.bool)
    allow[0:100, 0:50] = True
    allow[0:100, 90:95] = True
    allow[230:300, 10:20] = True
    allow[230:300, 200:240] = True
    ro, rto, rlse, rmu = om.masked_jvp(q, k, v, tq, tk, tv, allow, 0.125)
    for a in (slice(0, 100), slice(230, 300)):
        assert orc.rel_l2(o[..., a, :], ro[..., a, :]) <= TOL
        assert orc.rel_l2(to[..., a, :], rto[..., a, :]) <= TOL
        assert float((lse[..., a].double() - rlse[..., a]).abs().max()) <= TOL
    assert (o[..., 100:230, :] == 0).all() and (to[..., 100:230, :] == 0).all()
    assert (lse[..., 100:230] == -math.inf).all() and (mu[..., 100:230] == 0).all()
    assert (o[..., 300:, :] == S).all() and (lse[..., 300:] == S).all()


def _random_cases(n, seed):
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(len(xs), (1,), generator=g))]

    out = []
    for i in range(n):
        D = pick([16, 32, 64, 128, 256])
        lmax = 700 if D == 256 else 1500
        out.append(dict(B=pick([1, 2]), H=pick([1, 3]), Lq=int(torch.randint(1, lmax, (1,), generator=g)),
                        Lk=int(torch.randint(1, lmax, (1,), generator=g)), D=D, bshd=pick([False, True]),
                        seed=500 + i))
    return out


@pytest.mark.parametrize("c", _random_cases(16, 77), ids=lambda c: "B{B}H{H}q{Lq}k{Lk}D{D}".format(**c))
def test_random_shapes_fp32(gpu, c):
    """Seeded sweep over batch, heads, ragged lengths, head dims and layouts: forward+JVP
    and the dO-only backward against float64."""
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    print(f"case f32 random {c}", flush=True)
    B, H, Lq, Lk, D, bshd = c["B"], c["H"], c["Lq"], c["Lk"], c["D"], c["bshd"]
    g = torch.Generator().manual_seed(c["seed"])
    q, k, v, do = (_draw(g, B, H, L, D, 1.0, bshd) for L in (Lq, Lk, Lk, Lq))
    tq, tk, tv = (_draw(g, B, H, L, D, 0.1, bshd) for L in (Lq, Lk, Lk))
    s = D ** -0.5
    d = [x.to(gpu) for x in (q, k, v, tq, tk, tv, do)]
    o, to, lse, mu = jvp_attention_forward(*d[:6], s)
    dq, dk, dv, *_ = jvp_attention_backward(d[0], d[1], d[2], None, None, None, o, None, lse, None, d[6], None, s,
                                            False)
    torch.cuda.synchronize()
    x64 = [x.double() for x in (q, k, v, tq, tk, tv, do)]
    ro, rto, rlse, _ = orc.jvp_closed_form(*x64[:6], sm_scale=s)
    rq, rk, rv = orc.grads_dout_only(x64[0], x64[1], x64[2], x64[6], sm_scale=s)
    for name, a, r in (("o", o, ro), ("to", to, rto), ("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        e = orc.rel_l2(a.cpu(), r)
        assert e <= TOL, (name, e)
    assert float((lse.cpu().double() - rlse).abs().max()) <= TOL
