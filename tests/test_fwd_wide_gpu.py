"""Dense 256-wide heads on the row-reading forward kernel (attn_fwd32_kernel, D = 256).

In the JVP modes each query tile runs two workgroups, one per 128-column chunk of V (and
Vd, O, Od), each computing the full 256-wide scores; with Kd, Vd the ring has three stages
and the main loop six steps per pass. The plain forward keeps all 256 columns in one
workgroup (512-byte V rows). Checked here against the float64 oracle with the forward tests'
bar (relative L2 <= 1e-2 and no worse than 1.25x the emulated reference kernel + 1e-4, LSE
within 2e-3, mu within 1e-2 relative):
  * key counts giving every remainder of the six-step loop (1-6 tiles left) and partial
    last tiles, ragged query counts, all three modes, bf16 and fp16;
  * BSHD-strided operands (rows H*D apart) as the Wan callers pass them;
  * logits rising along the keys, so the running max moves at every step and the
    accumulators (in AGPRs in the JVP mode, rescaled one block at a time) are rescaled
    each time.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

D = 256


def _draw(g, B, H, L, std, dtype):
    return (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * std).to(dtype)


def _check(o, to, lse, mu, xs, s, dtype, mode):
    q, k, v, tq, tk, tv = xs
    if mode == "plain":
        ro, rlse = orc.math_attention(q.double(), k.double(), v.double(), s)
        assert orc.rel_l2(o, ro) <= 1e-2
        assert float((lse.double() - rlse).abs().max()) <= 2e-3
        return
    zk = torch.zeros_like(k) if tk is None else tk
    zv = torch.zeros_like(v) if tv is None else tv
    ro, rto, rlse, rmu = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, zk, zv)), sm_scale=s)
    em_o, em_to, _ = orc.triton_fwd_emulator(q, k, v, tq, zk, zv, sm_scale=s, block_n=64, round_dtype=dtype)
    e_o, e_to = orc.rel_l2(o, ro), orc.rel_l2(to, rto)
    f_o, f_to = orc.rel_l2(em_o.to(dtype), ro), orc.rel_l2(em_to.to(dtype), rto)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})", flush=True)
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4
    assert float((lse.double() - rlse).abs().max()) <= 2e-3
    assert orc.rel_l2(mu, rmu) <= 1e-2


def _run(gpu, xs, s, mode):
    from dmad_amd.jvp_attention import jvp_attention_forward

    q, k, v, tq, tk, tv = (None if x is None else x.to(gpu) for x in xs)
    if mode == "plain":
        tq = tk = tv = None
    elif mode == "qonly":
        tk = tv = None
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    torch.cuda.synchronize()
    return (o.cpu(), None if to is None else to.cpu(), lse.cpu(), None if mu is None else mu.cpu())


def test_plan_is_the_row_kernel():
    from dmad_amd import _native as nat

    for mode in (nat.DMAD_FWD_PLAIN, nat.DMAD_FWD_JVP, nat.DMAD_FWD_JVP_KV_TANGENT_ZERO):
        p = nat.fwd_plan(nat.DMAD_BF16, mode, 1, 2, 300, 600, D, D)
        chunks = 1 if mode == nat.DMAD_FWD_PLAIN else 2
        assert (p["kernel"], p["chunks"], p["transposed_copies"]) == ("attn_fwd32_kernel", chunks, 0)


# (Lq, Lk): 32-key tiles 1, 2, 3, 4, 5, 6, 7 (one pass and 1 left), 11 (5 left), 13 (1 left)
SHAPES = [(129, 17), (300, 64), (77, 70), (256, 128), (300, 150), (1, 190), (200, 200), (130, 330), (300, 385)]


@pytest.mark.parametrize("mode", ["jvp", "qonly", "plain"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Lq,Lk", SHAPES)
def test_wide_row_kernel_matches_oracle(gpu, Lq, Lk, dtype, mode):
    print(f"case D=256 Lq={Lq} Lk={Lk} {dtype} {mode}", flush=True)
    B, H = 1, 2
    g = torch.Generator().manual_seed(Lq * 1000 + Lk)
    xs = (_draw(g, B, H, Lq, 0.5, dtype), _draw(g, B, H, Lk, 0.5, dtype), _draw(g, B, H, Lk, 0.5, dtype),
          _draw(g, B, H, Lq, 0.5, dtype), _draw(g, B, H, Lk, 0.5, dtype), _draw(g, B, H, Lk, 0.5, dtype))
    if mode == "qonly":
        xs = xs[:4] + (None, None)
    s = D ** -0.5
    o, to, lse, mu = _run(gpu, xs, s, mode)
    _check(o, to, lse, mu, xs, s, dtype, mode)


@pytest.mark.parametrize("mode", ["jvp", "qonly"])
def test_wide_bshd_strides(gpu, mode):
    """Operands as (B, L, H, D) storage viewed as (B, H, L, D): rows H*D elements apart."""
    print(f"case D=256 BSHD {mode}", flush=True)
    B, H, Lq, Lk, dtype = 2, 3, 200, 250, torch.bfloat16
    g = torch.Generator().manual_seed(7)

    def bshd(L, std):
        x = (torch.randn((B, L, H, D), generator=g, dtype=torch.float64) * std).to(dtype)
        return x.transpose(1, 2)

    xs = (bshd(Lq, 0.5), bshd(Lk, 0.5), bshd(Lk, 0.5), bshd(Lq, 0.3), bshd(Lk, 0.3), bshd(Lk, 0.3))
    if mode == "qonly":
        xs = xs[:4] + (None, None)
    s = D ** -0.5
    o, to, lse, mu = _run(gpu, xs, s, mode)
    _check(o, to, lse, mu, tuple(None if x is None else x.contiguous() for x in xs), s, dtype, mode)


def _growing_logits(g, B, H, Lq, Lk, dtype, rise):
    """Q, K whose logits rise along the keys by about `rise` (log2 units) per 32-key tile."""
    u = torch.randn(D, generator=g, dtype=torch.float64)
    u = u / u.norm()
    qa = 1.0 + 0.5 * torch.rand((B, H, Lq, 1), generator=g, dtype=torch.float64)
    q = qa * u * D ** 0.25 + 0.3 * torch.randn((B, H, Lq, D), generator=g, dtype=torch.float64)
    step = rise / 32 / 1.4426950408889634
    ramp = torch.arange(Lk, dtype=torch.float64).view(1, 1, Lk, 1) * step
    k = ramp * u * D ** 0.25 + 0.3 * torch.randn((B, H, Lk, D), generator=g, dtype=torch.float64)
    return q.to(dtype), k.to(dtype)


@pytest.mark.parametrize("mode", ["jvp", "qonly"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_rescale_at_every_step(gpu, dtype, mode):
    print(f"case D=256 rescale every step {dtype} {mode}", flush=True)
    B, H, Lq, Lk, rise = 1, 2, 200, 400, 10.0
    g = torch.Generator().manual_seed(11)
    q, k = _growing_logits(g, B, H, Lq, Lk, dtype, rise)
    v = _draw(g, B, H, Lk, 1.0, dtype)
    tq = _draw(g, B, H, Lq, 0.1, dtype)
    tk, tv = (_draw(g, B, H, Lk, 0.1, dtype), _draw(g, B, H, Lk, 0.1, dtype)) if mode == "jvp" else (None, None)
    s = D ** -0.5
    o, to, lse, _ = _run(gpu, (q, k, v, tq, tk, tv), s, mode)
    zk, zv = (torch.zeros_like(k), torch.zeros_like(v)) if tk is None else (tk, tv)
    ro, rto, rlse, _ = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, zk, zv)), sm_scale=s)
    em_o, em_to, _ = orc.triton_fwd_emulator(q, k, v, tq, zk, zv, sm_scale=s, block_n=32, round_dtype=dtype)
    e_o, f_o = orc.rel_l2(o, ro), orc.rel_l2(em_o.to(dtype), ro)
    e_to, f_to = orc.rel_l2(to, rto), orc.rel_l2(em_to.to(dtype), rto)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})", flush=True)
    assert e_o <= 1e-2 and e_o <= 1.25 * f_o + 1e-4, (e_o, f_o)
    # a softmax this concentrated makes Od = C~/l - mu O cancel: the contract is the reference kernel's error
    assert e_to <= 1.25 * f_to + 1e-4, (e_to, f_to)
    assert float((lse.double() - rlse).abs().max()) <= 2e-3 * max(1.0, float(rlse.abs().max()))
    # the logits really did rise across the tiles
    assert float(rlse.mean()) > rise * (Lk // 32 - 2) / 1.4426950408889634 / 2


def _oracle_head(q, k, v, tq, tk, tv, h, s, chunk=2048):
    """Oracle (O, Od, LSE, mu) of head h, float32 on the device, chunked over query rows (rows are independent)."""
    f = lambda x: x[0, h].float().contiguous()  # noqa: E731
    kh, vh = f(k), f(v)
    tkh = torch.zeros_like(kh) if tk is None else f(tk)
    tvh = torch.zeros_like(vh) if tv is None else f(tv)
    qh, tqh = f(q), f(tq)
    outs = [[], [], [], []]
    for c in range(0, qh.shape[0], chunk):
        for o, r in zip(outs, orc.jvp_closed_form(qh[c:c + chunk], kh, vh, tqh[c:c + chunk], tkh, tvh, sm_scale=s)):
            o.append(r)
    return [torch.cat(o, 0) for o in outs]


@pytest.mark.parametrize("H,L,mode", [(3, 16384, "jvp"), (1, 32768, "jvp"), (2, 16384, "qonly")])
def test_wide_row_kernel_long_sequences(gpu, H, L, mode):
    """128 query tiles per head (work items dealt contiguously per XCD) and 256 (head-major order):
    every row of two heads against the oracle in float32 on the GPU, sampled rows against float64."""
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case D=256 long H={H} L={L} {mode}", flush=True)
    dtype = torch.bfloat16
    g = torch.Generator(device=gpu).manual_seed(L + H)
    r = lambda std: (torch.randn((1, H, L, D), device=gpu, generator=g) * std).to(dtype)  # noqa: E731
    q, k, v, tq = r(1.0), r(1.0), r(1.0), r(0.1)
    tk, tv = (r(0.1), r(0.1)) if mode == "jvp" else (None, None)
    s = D ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    torch.cuda.synchronize()
    for h in sorted({0, H - 1}):
        ro, rto, rlse, rmu = _oracle_head(q, k, v, tq, tk, tv, h, s)
        e_o, e_to, e_mu = orc.rel_l2(o[0, h], ro), orc.rel_l2(to[0, h], rto), orc.rel_l2(mu[0, h], rmu)
        dl = float((lse[0, h] - rlse).abs().max())
        print(f"  head {h}: rel-L2 O {e_o:.2e} Od {e_to:.2e} mu {e_mu:.2e} max|dLSE| {dl:.2e}", flush=True)
        assert max(e_o, e_to, e_mu) <= 1e-2 and dl <= 2e-3
    rows = torch.tensor([0, 1, 127, 128, L // 2, L - 129, L - 1], device=gpu)
    h = H - 1
    sub = lambda x: None if x is None else x[:, h:h + 1].cpu()  # noqa: E731
    qs, tqs = q[:, h:h + 1, rows].cpu(), tq[:, h:h + 1, rows].cpu()
    kh, vh, tkh, tvh = sub(k), sub(v), sub(tk), sub(tv)
    tkh = torch.zeros_like(kh) if tkh is None else tkh
    tvh = torch.zeros_like(vh) if tvh is None else tvh
    ref_o, ref_to, _, _ = orc.jvp_closed_form(*(x.double() for x in (qs, kh, vh, tqs, tkh, tvh)), sm_scale=s)
    assert orc.rel_l2(o[:, h:h + 1, rows].cpu(), ref_o) <= 1e-2
    assert orc.rel_l2(to[:, h:h + 1, rows].cpu(), ref_to) <= 1e-2
