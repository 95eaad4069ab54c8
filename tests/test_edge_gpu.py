"""Edge cases of the dense op on the GPU against the float64 oracle: single
queries and keys, lengths just off the 32/64/128 tile grids, logits large
enough that the online softmax rescales on almost every tile, inputs with no
query rows, and a seeded sweep of random shapes, head dims, dtypes and
layouts (BHSD contiguous or BSHD views, as the Wan callers pass them), and
bitwise-equal repeat runs (no atomics, fixed reduction order).

Bar: rel-L2 <= 1e-2 on O, Ȯ and every gradient (the reference's own tests
use atol/rtol 1e-2), with an absolute bound where the exact value is zero.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _draw(g, shape, std, dtype, bshd):
    B, H, L, D = shape
    if bshd:  # [B, L, H, D] storage viewed as [B, H, L, D]
        x = torch.randn((B, L, H, D), generator=g, dtype=torch.float64) * std
        return x.to(dtype).transpose(1, 2)
    return (torch.randn(shape, generator=g, dtype=torch.float64) * std).to(dtype)


def _case(B, H, Lq, Lk, D, dtype=torch.bfloat16, seed=0, std=1.0, tstd=0.1, bshd=False):
    g = torch.Generator().manual_seed(seed)
    q = _draw(g, (B, H, Lq, D), std, dtype, bshd)
    k = _draw(g, (B, H, Lk, D), std, dtype, bshd)
    v = _draw(g, (B, H, Lk, D), 1.0, dtype, bshd)
    tq = _draw(g, (B, H, Lq, D), tstd, dtype, bshd)
    tk = _draw(g, (B, H, Lk, D), tstd, dtype, bshd)
    tv = _draw(g, (B, H, Lk, D), tstd, dtype, bshd)
    do = _draw(g, (B, H, Lq, D), 1.0, dtype, bshd)
    dto = _draw(g, (B, H, Lq, D), 0.1, dtype, bshd)
    return q, k, v, tq, tk, tv, do, dto


def _gpu_run(dev, xs, full):
    """(o, to) and the gradients of <o, dO> (+ <to, dȮ> when full) through the op."""
    from dmad_amd import attention

    q, k, v, tq, tk, tv, do, dto = (x.to(dev) for x in xs)
    leaves = [q, k, v] + ([tq, tk, tv] if full else [])
    for x in leaves:
        x.requires_grad_(True)
    o, to = attention(q, k, v, tq, tk, tv)
    loss = (o.float() * do.float()).sum()
    if full:
        loss = loss + (to.float() * dto.float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    return [o.detach().cpu(), to.detach().cpu()] + [x.grad.cpu() for x in leaves]


def _check(xs, got, full, tol=1e-2):
    x64 = [x.double() for x in xs]
    D = xs[0].shape[-1]
    ro, rto, _, _ = orc.jvp_closed_form(*x64[:6], sm_scale=D ** -0.5)
    if full:
        rg = orc.grads_full(*x64, sm_scale=D ** -0.5)
    else:
        rg = orc.grads_dout_only(x64[0], x64[1], x64[2], x64[6], D ** -0.5)
    names = ("o", "to", "dq", "dk", "dv", "dtq", "dtk", "dtv")
    errs = {}
    for name, a, r in zip(names, got, [ro, rto, *rg]):
        assert a.shape == r.shape, (name, a.shape, r.shape)
        if float(r.abs().max()) == 0.0:
            errs[name] = float(a.double().abs().max())  # exact zero: absolute error
        else:
            errs[name] = orc.rel_l2(a, r)
    print("  errors " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


# 16 and 32: the generic and pipelined passes (keys beyond Lk unmasked in the dK/dV
# passes, the 32-wide dK/dV pass's statistics in 32-query tiles)
@pytest.mark.parametrize("D", [128, 64, 32, 16])
@pytest.mark.parametrize("Lq,Lk", [(1, 1), (1, 257), (257, 1), (33, 31), (129, 95), (64, 128)])
@pytest.mark.parametrize("full", [False, True])
def test_tiny_and_off_grid_lengths(gpu, D, Lq, Lk, full):
    print(f"case Lq={Lq} Lk={Lk} D={D} full={full}", flush=True)
    xs = _case(2, 3, Lq, Lk, D, seed=Lq * 1000 + Lk)
    _check(xs, _gpu_run(gpu, xs, full), full)


@pytest.mark.parametrize("D", [128, 64])
def test_large_logits(gpu, D):
    """Q, K ~ N(0, 4^2): scaled logits of standard deviation ~16, so the running row
    maximum moves on most key tiles and P is close to one-hot. The errors grow
    (the bf16 rounding of P and H~ no longer averages out) and stay within 1.25x
    of the reference kernels' own: the forward emulator (BLOCK_N 64) for O, Ȯ and
    the FA2 emulator for the dO-only gradients, all rounded to bf16."""
    print(f"case large logits D={D}", flush=True)
    xs = _case(1, 2, 300, 300, D, seed=3, std=4.0)
    _check(xs, _gpu_run(gpu, xs, True), True)
    got = _gpu_run(gpu, xs, False)
    x64 = [x.double() for x in xs]
    s = D ** -0.5
    ref = list(orc.jvp_closed_form(*x64[:6], sm_scale=s)[:2]) + list(orc.grads_dout_only(x64[0], x64[1], x64[2], x64[6], s))
    emu = list(orc.triton_fwd_emulator(*xs[:6], sm_scale=s, block_n=64)[:2]) + list(
        orc.fa2_bwd_emulator(xs[0], xs[1], xs[2], xs[6], s))
    for name, a, e, r in zip(("o", "to", "dq", "dk", "dv"), got, emu, ref):
        err, floor = orc.rel_l2(a, r), orc.rel_l2(e.to(torch.bfloat16), r)
        print(f"  {name}: {err:.2e} (reference kernel {floor:.2e})", flush=True)
        assert err <= 1.25 * floor + 1e-4, (name, err, floor)


def test_single_key_has_exact_zero_score_gradients(gpu):
    """One key: P = 1, so O = V, Ȯ = V̇ and dQ = dK = 0 (up to summation order)."""
    xs = _case(1, 2, 77, 1, 128, seed=9)
    got = _gpu_run(gpu, xs, False)
    v, tv = xs[2].float(), xs[5].float()
    assert torch.equal(got[0].float(), v.expand(-1, -1, 77, -1))
    torch.testing.assert_close(got[1].float(), tv.expand(-1, -1, 77, -1), atol=1e-2, rtol=1e-2)
    assert float(got[2].abs().max()) < 1e-2 and float(got[3].abs().max()) < 1e-2


def test_no_query_rows(gpu):
    """Lq = 0: empty outputs and dQ, zero dK, dV (and tangent gradients); B = 0: all empty."""
    from dmad_amd import attention

    for B, Lq in ((1, 0), (0, 5)):
        print(f"case B={B} Lq={Lq}", flush=True)
        q, k, v, tq, tk, tv = (torch.randn(s, device=gpu, dtype=torch.bfloat16).requires_grad_(True)
                               for s in [(B, 2, Lq, 64), (B, 2, 9, 64), (B, 2, 9, 64)] * 2)
        o, to = attention(q, k, v, tq, tk, tv)
        assert o.shape == (B, 2, Lq, 64) and to.shape == (B, 2, Lq, 64)
        (o.float().sum() + to.float().sum()).backward()
        torch.cuda.synchronize()
        assert q.grad.shape == q.shape and tq.grad.shape == tq.shape
        for x in (k, v, tk, tv):
            assert x.grad.shape == x.shape and float(x.grad.abs().sum()) == 0.0


def _random_cases(n, seed):
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(len(xs), (1,), generator=g))]

    out = []
    for i in range(n):
        D = pick([16, 32, 64, 128, 256])
        lmax = 1500 if D == 256 else 2500
        out.append(dict(B=pick([1, 2]), H=pick([1, 3, 4]), Lq=int(torch.randint(1, lmax, (1,), generator=g)),
                        Lk=int(torch.randint(1, lmax, (1,), generator=g)), D=D,
                        dtype=pick([torch.bfloat16, torch.float16]), bshd=pick([False, True]),
                        full=pick([False, True]) and D <= 128, seed=100 + i))  # full backward: D <= 128
    return out


@pytest.mark.parametrize("c", _random_cases(40, 2024), ids=lambda c: "B{B}H{H}q{Lq}k{Lk}D{D}".format(**c))
def test_random_shapes(gpu, c):
    print(f"case {c}", flush=True)
    xs = _case(c["B"], c["H"], c["Lq"], c["Lk"], c["D"], dtype=c["dtype"], seed=c["seed"], bshd=c["bshd"])
    _check(xs, _gpu_run(gpu, xs, c["full"]), c["full"])


@pytest.mark.parametrize("D", [128, 64])
def test_repeat_runs_are_bitwise_equal(gpu, D):
    """No kernel uses atomics and every reduction has a fixed order: two runs of the
    forward and of both backward modes on the same inputs agree bit for bit, and
    so does the block-sparse forward."""
    from dmad_amd import attention
    from dmad_amd import magimask as mm

    print(f"case repeat D={D}", flush=True)
    xs = _case(1, 4, 2100, 2100, D, seed=31)
    for full in (False, True):
        a, b = _gpu_run(gpu, xs, full), _gpu_run(gpu, xs, full)
        for name, x, y in zip(("o", "to", "dq", "dk", "dv", "dtq", "dtk", "dtv"), a, b):
            assert torch.equal(x, y), (full, name)
    pat = mm.BlockPattern(frame_tokens=300, first_chunk_frames=1, chunk_frames=2)
    spec = mm.AttnMaskSpec(mode="block_causal", pattern=pat, local_attn_blocks=2, sink_blocks=1)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=2100, KV_real=2100, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=2100, KV_real=2100)
    g = [x.to(gpu) for x in xs[:6]]
    r1, r2 = attention(*g, None, mask), attention(*g, None, mask)
    torch.cuda.synchronize()
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])


@pytest.mark.parametrize("dtype_code", [0, 1])
def test_mfma_probe_runs(gpu, dtype_code):
    """The ceiling probe the benchmark times (dmad_probe_mfma): a short launch on two
    workgroups finishes and writes one finite float per thread."""
    from dmad_amd import _native as nat

    sink = torch.full((2 * 256,), float("nan"), device=gpu)
    nat.check(nat.lib().dmad_probe_mfma(dtype_code, 2, 512, nat.ptr(sink), nat.stream_ptr(gpu)))
    torch.cuda.synchronize()
    assert torch.isfinite(sink).all()
