"""Parity at the Wan2.1 shapes the benchmark runs (L = 32760 and 75600).

The oracle's own float code (oracle.attention) evaluates whole heads here, in
float32 on the GPU and chunked over query rows: every row of O, Od, LSE, mu and
dQ depends only on its own query row, and dK, dV are sums of per-chunk
contributions, so the chunked evaluation is the same mathematics. Sampled rows
are also checked against the float64 oracle and the emulated reference-kernel
error on the CPU, and the backward against identities that hold at any size:
  sum_j dV_j = sum_i dO_i             (rows of P sum to one)
  sum_j dK_j = 0                      (rows of dS sum to zero)
  sum_i <dQ_i, Q_i> = sum_j <dK_j, K_j>   (S depends on Q K^T only).

Bar: relative L2 <= 1e-2 on O, Od and every gradient (bf16 kernels against the
float oracle on the same rounded inputs), |LSE - LSE_ref| <= 2e-3, and no worse
than 1.25x the emulated reference kernels + 1e-4 (the Triton forward's numerics,
and the FA2 backward's for dQ, dK, dV).
"""
import pytest
import torch

from dmad_amd.workload import make_inputs
from oracle import attention as orc

pytestmark = pytest.mark.gpu

CHUNK = 2048


def _head(x, h):
    """Head h of a BHSD view as a contiguous float32 [L, D] tensor."""
    return x[0, h].float().contiguous()


def oracle_fwd_head(q, k, v, tq, tk, tv, h, sm_scale):
    """Oracle (O, Od, LSE, mu) of head h, float32 on the inputs' device, query-chunked."""
    kh, vh = _head(k, h), _head(v, h)
    tkh = torch.zeros_like(kh) if tk is None else _head(tk, h)
    tvh = torch.zeros_like(vh) if tv is None else _head(tv, h)
    qh, tqh = _head(q, h), _head(tq, h)
    outs = [[], [], [], []]
    for c in range(0, qh.shape[0], CHUNK):
        res = orc.jvp_closed_form(qh[c:c + CHUNK], kh, vh, tqh[c:c + CHUNK], tkh, tvh, sm_scale=sm_scale)
        for o, r in zip(outs, res):
            o.append(r)
    return [torch.cat(o, 0) for o in outs]


def oracle_bwd_head(q, k, v, do, h, sm_scale):
    """Oracle dO-only (dQ, dK, dV) of head h, float32, query-chunked."""
    qh, kh, vh, doh = _head(q, h), _head(k, h), _head(v, h), _head(do, h)
    dqs, dk, dv = [], torch.zeros_like(kh), torch.zeros_like(vh)
    for c in range(0, qh.shape[0], CHUNK):
        dq_c, dk_c, dv_c = orc.grads_dout_only(qh[c:c + CHUNK], kh, vh, doh[c:c + CHUNK], sm_scale=sm_scale)
        dqs.append(dq_c)
        dk += dk_c
        dv += dv_c
    return torch.cat(dqs, 0), dk, dv


def oracle_full_bwd_head(x, h, sm_scale, tangents=True):
    """Oracle full derivative (dQ, dK, dV, dQd, dKd, dVd) of head h (oracle.grads_full),
    float32, query-chunked: every row statistic (LSE, mu, rho, D') is row-local,
    dQ, dQd are row-local and dK, dV, dKd, dVd are sums over query rows."""
    qh, kh, vh, tqh = (_head(x[n], h) for n in ("q", "k", "v", "tq"))
    tkh = _head(x["tk"], h) if tangents else torch.zeros_like(kh)
    tvh = _head(x["tv"], h) if tangents else torch.zeros_like(vh)
    doh, dtoh = _head(x["do"], h), _head(x["dto"], h)
    rows = [[], []]
    cols = [torch.zeros_like(kh), torch.zeros_like(vh), torch.zeros_like(kh), torch.zeros_like(vh)]
    for c in range(0, qh.shape[0], CHUNK):
        sl = slice(c, c + CHUNK)
        dq, dk, dv, dtq, dtk, dtv = orc.grads_full(qh[sl], kh, vh, tqh[sl], tkh, tvh, doh[sl], dtoh[sl],
                                                   sm_scale=sm_scale)
        rows[0].append(dq)
        rows[1].append(dtq)
        for acc, part in zip(cols, (dk, dv, dtk, dtv)):
            acc += part
    dq, dtq = torch.cat(rows[0], 0), torch.cat(rows[1], 0)
    return dq, cols[0], cols[1], dtq, cols[2], cols[3]


def fa2_floor_head(q, k, v, do, h, sm_scale):
    """The reference backward's numerics (oracle.fa2_bwd_emulator, bf16 rounding of P
    and dS) for head h, float32, query-chunked the same way."""
    qh, kh, vh, doh = _head(q, h), _head(k, h), _head(v, h), _head(do, h)
    dqs, dk, dv = [], torch.zeros_like(kh), torch.zeros_like(vh)
    for c in range(0, qh.shape[0], CHUNK):
        dq_c, dk_c, dv_c = orc.fa2_bwd_emulator(qh[c:c + CHUNK], kh, vh, doh[c:c + CHUNK], sm_scale=sm_scale,
                                                round_dtype=q.dtype)
        dqs.append(dq_c)
        dk += dk_c
        dv += dv_c
    return torch.cat(dqs, 0), dk, dv


def _rel(a, b):
    return float(torch.linalg.vector_norm((a.float() - b.float()).double()) / torch.linalg.vector_norm(b.double()))


def _check_fwd(o, to, lse, mu, q, k, v, tq, tk, tv, heads, sm_scale):
    for h in heads:
        ro, rto, rlse, rmu = oracle_fwd_head(q, k, v, tq, tk, tv, h, sm_scale)
        e = {"o": _rel(o[0, h], ro), "to": _rel(to[0, h], rto), "mu": _rel(mu[0, h], rmu)}
        dl = float((lse[0, h] - rlse).abs().max())
        print(f"  head {h}: rel-L2 O {e['o']:.2e} Od {e['to']:.2e} mu {e['mu']:.2e}  max|dLSE| {dl:.2e}", flush=True)
        assert max(e.values()) <= 1e-2, e
        assert dl <= 2e-3


def _check_rows_against_cpu(o, to, q, k, v, tq, tk, tv, h, rows, sm_scale):
    """Sampled rows against the float64 oracle and the emulated reference kernel (CPU)."""
    sel = torch.as_tensor(rows, device=q.device)
    qs, tqs = q[:, h:h + 1, sel].cpu(), tq[:, h:h + 1, sel].cpu()
    kh, vh = k[:, h:h + 1].cpu(), v[:, h:h + 1].cpu()
    tkh = torch.zeros_like(kh) if tk is None else tk[:, h:h + 1].cpu()
    tvh = torch.zeros_like(vh) if tv is None else tv[:, h:h + 1].cpu()
    ref_o, ref_to, _, _ = orc.jvp_closed_form(*(x.double() for x in (qs, kh, vh, tqs, tkh, tvh)), sm_scale=sm_scale)
    got_o, got_to = o[:, h:h + 1, sel].cpu(), to[:, h:h + 1, sel].cpu()
    em_o, em_to, _ = orc.triton_fwd_emulator(qs, kh, vh, tqs, tkh, tvh, sm_scale=sm_scale, block_n=64,
                                             round_dtype=torch.bfloat16)
    e_o, e_to = orc.rel_l2(got_o, ref_o), orc.rel_l2(got_to, ref_to)
    f_o, f_to = orc.rel_l2(em_o.to(torch.bfloat16), ref_o), orc.rel_l2(em_to.to(torch.bfloat16), ref_to)
    print(f"  head {h} sampled rows: O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})",
          flush=True)
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4


def _check_bwd(dq, dk, dv, q, k, v, do, heads, sm_scale):
    for h in heads:
        rq, rk, rv = oracle_bwd_head(q, k, v, do, h, sm_scale)
        e = {"dq": _rel(dq[0, h], rq), "dk": _rel(dk[0, h], rk), "dv": _rel(dv[0, h], rv)}
        fq, fk, fv = fa2_floor_head(q, k, v, do, h, sm_scale)
        f = {"dq": _rel(fq.to(dq.dtype), rq), "dk": _rel(fk.to(dq.dtype), rk), "dv": _rel(fv.to(dq.dtype), rv)}
        print(f"  head {h}: rel-L2 dQ {e['dq']:.2e} dK {e['dk']:.2e} dV {e['dv']:.2e}  "
              f"(FA2 floor {f['dq']:.2e} {f['dk']:.2e} {f['dv']:.2e})", flush=True)
        assert max(e.values()) <= 1e-2, e
        for n in e:
            assert e[n] <= 1.25 * f[n] + 1e-4, (n, e[n], f[n])
    # identities over every head, in float64
    L = k.shape[2]
    sv = dv.double().sum(2)
    sdo = do.double().sum(2)
    rms_dv = dv.double().pow(2).mean(dim=(2, 3)).sqrt()[..., None]
    r_v = float(((sv - sdo).abs() / (rms_dv * L ** 0.5)).max())
    sk = dk.double().sum(2)
    rms_dk = dk.double().pow(2).mean(dim=(2, 3)).sqrt()[..., None]
    r_k = float((sk.abs() / (rms_dk * L ** 0.5)).max())
    qq = (dq.double() * q.double()).sum(dim=(2, 3))
    kk = (dk.double() * k.double()).sum(dim=(2, 3))
    scale = (dq.double().pow(2).sum(dim=(2, 3)) * q.double().pow(2).sum(dim=(2, 3))).sqrt()
    r_qk = float(((qq - kk).abs() / scale).max())
    print(f"  identities (all heads): sum dV - sum dO {r_v:.2e}  sum dK {r_k:.2e}  <dQ,Q> - <dK,K> {r_qk:.2e}",
          flush=True)
    assert r_v <= 2e-2 and r_k <= 2e-2 and r_qk <= 2e-2


def _check_bwd_full(grads, x, heads, sm_scale, tangents=True):
    """The full derivative against the chunked oracle on `heads`; on every head the
    identities that hold for it at any size:
      sum_j dV_j = sum_i dO_i, sum_j dVd_j = sum_i dOd_i  (rows of P sum to one,
          rows of Pd = P*(Sd - mu) to zero),
      sum_j dK_j = 0, sum_j dKd_j = 0  (rows of dS and dSd sum to zero),
      <dQ,Q> + <dQd,Qd> = <dK,K> + <dKd,Kd>  ((Q, Qd, K, Kd) -> (aQ, aQd, K/a, Kd/a)
          leaves S and Sd unchanged)."""
    names = ("dq", "dk", "dv", "dtq", "dtk", "dtv")
    for h in heads:
        ref = oracle_full_bwd_head(x, h, sm_scale, tangents=tangents)
        e = {n: _rel(g[0, h], r) for n, g, r in zip(names, grads, ref)}
        print(f"  head {h}: rel-L2 " + " ".join(f"{n} {v:.2e}" for n, v in e.items()), flush=True)
        assert max(e.values()) <= 1e-2, e
    dq, dk, dv, dtq, dtk, dtv = (g.double() for g in grads)
    q, k, tq = x["q"].double(), x["k"].double(), x["tq"].double()
    tk = x["tk"].double() if tangents else torch.zeros_like(k)
    L = k.shape[2]

    def col_sum_err(g, target):
        rms = g.pow(2).mean(dim=(2, 3)).sqrt()[..., None]
        return float(((g.sum(2) - target).abs() / (rms * L ** 0.5)).max())

    r = {"sum dV - sum dO": col_sum_err(dv, x["do"].double().sum(2)),
         "sum dVd - sum dOd": col_sum_err(dtv, x["dto"].double().sum(2)),
         "sum dK": col_sum_err(dk, 0.0), "sum dKd": col_sum_err(dtk, 0.0)}
    lhs = (dq * q).sum(dim=(2, 3)) + (dtq * tq).sum(dim=(2, 3))
    rhs = (dk * k).sum(dim=(2, 3)) + (dtk * tk).sum(dim=(2, 3))
    scale = (dq.pow(2).sum(dim=(2, 3)) * q.pow(2).sum(dim=(2, 3))).sqrt()
    r["<dQ,Q>+<dQd,Qd> - <dK,K>-<dKd,Kd>"] = float(((lhs - rhs).abs() / scale).max())
    print("  identities (all heads): " + "  ".join(f"{n} {v:.2e}" for n, v in r.items()), flush=True)
    assert max(r.values()) <= 2e-2, r


def _run(x, tangents=True, backward=False):
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    q, k, v = x["q"], x["k"], x["v"]
    tq = x["tq"]
    tk, tv = (x["tk"], x["tv"]) if tangents else (None, None)
    s = q.shape[-1] ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    grads = None
    if backward:
        grads = jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, x["do"], None, s, False)[:3]
    torch.cuda.synchronize()
    return (o, to, lse, mu), grads, s


def test_wan13b_self_attention_full_size(gpu):
    """Wan2.1-1.3B self-attention: B=1, H=12, L=32760 (21x30x52 latent), RMSNorm + 3D RoPE Q/K."""
    print("case wan1.3b self fwd+JVP+bwd", flush=True)
    x = make_inputs(1, 12, 32760, 32760, 128, seed=0, device=gpu, grid=(21, 30, 52), with_grads=True, gen_device=gpu)
    (o, to, lse, mu), (dq, dk, dv), s = _run(x, backward=True)
    args = (x["q"], x["k"], x["v"], x["tq"], x["tk"], x["tv"])
    _check_fwd(o, to, lse, mu, *args, heads=(0, 11), sm_scale=s)
    g = torch.Generator().manual_seed(5)
    rows = sorted(set(torch.randint(0, 32760, (96,), generator=g).tolist()) | {0, 32759})
    _check_rows_against_cpu(o, to, *args, h=5, rows=rows, sm_scale=s)
    _check_bwd(dq, dk, dv, x["q"], x["k"], x["v"], x["do"], heads=(0, 11), sm_scale=s)


def test_wan13b_self_attention_full_derivative_full_size(gpu):
    """BASELINE config 3 at its size: the 1.3B self-attention (H=12, L=32760, RMSNorm + 3D
    RoPE Q/K) with both cotangents, dO ~ N(0,1) and dOd ~ N(0,0.1^2), and every input
    requiring grad: the full derivative dQ, dK, dV, dQd, dKd, dVd."""
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    print("case wan1.3b self fwd+JVP+full bwd", flush=True)
    x = make_inputs(1, 12, 32760, 32760, 128, seed=0, device=gpu, grid=(21, 30, 52), with_grads=True, gen_device=gpu)
    q, k, v, tq, tk, tv = (x[n] for n in ("q", "k", "v", "tq", "tk", "tv"))
    s = 128 ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    grads = jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, x["do"], x["dto"], s, True)
    torch.cuda.synchronize()
    assert all(g is not None for g in grads)
    _check_bwd_full(grads, x, heads=(0, 11), sm_scale=s)


def test_wan13b_cross_attention_full_size(gpu):
    """The 1.3B text cross-attention of config 3: H=12, 32760 queries over 512 keys,
    Kd = Vd = 0 (wan2pt1_jvp.py:366-372); forward+JVP, then the full derivative with
    dO and dOd (the gradients of the zero K, V tangents included)."""
    from dmad_amd.jvp_attention import jvp_attention_backward

    print("case wan1.3b cross fwd+JVP+full bwd", flush=True)
    x = make_inputs(1, 12, 32760, 512, 128, seed=4, device=gpu, with_grads=True, gen_device=gpu)
    (o, to, lse, mu), _, s = _run(x, tangents=False)
    _check_fwd(o, to, lse, mu, x["q"], x["k"], x["v"], x["tq"], None, None, heads=(0, 11), sm_scale=s)
    grads = jvp_attention_backward(x["q"], x["k"], x["v"], x["tq"], None, None, o, to, lse, mu, x["do"], x["dto"],
                                   s, True)
    torch.cuda.synchronize()
    _check_bwd_full(grads, x, heads=(0, 7), sm_scale=s, tangents=False)


def test_wan14b_cross_attention_full_size(gpu):
    """Wan2.1-14B text cross-attention: H=40, 32760 queries over 512 keys, Kd = Vd = 0, on
    the tensors the benchmark times (the CPU generator seeded 1)."""
    print("case wan14b cross fwd+JVP (benchmark inputs)", flush=True)
    x = make_inputs(1, 40, 32760, 512, 128, seed=1, device=gpu)
    (o, to, lse, mu), _, s = _run(x, tangents=False)
    _check_fwd(o, to, lse, mu, x["q"], x["k"], x["v"], x["tq"], None, None, heads=(0, 17, 39), sm_scale=s)


def test_wan14b_720p_self_attention_full_size(gpu):
    """Wan2.1-14B at 720p, the grid config 5 runs: B=1, H=40, L=75600 (21x45x80 latent);
    two heads against the oracle, the backward identities on all 40."""
    print("case wan14b 720p self fwd+JVP+bwd (H=40)", flush=True)
    x = make_inputs(1, 40, 75600, 75600, 128, seed=2, device=gpu, grid=(21, 45, 80), with_grads=True, gen_device=gpu)
    (o, to, lse, mu), (dq, dk, dv), s = _run(x, backward=True)
    args = (x["q"], x["k"], x["v"], x["tq"], x["tk"], x["tv"])
    _check_fwd(o, to, lse, mu, *args, heads=(1, 39), sm_scale=s)
    _check_rows_against_cpu(o, to, *args, h=0, rows=[0, 1, 4097, 37800, 75598, 75599], sm_scale=s)
    _check_bwd(dq, dk, dv, x["q"], x["k"], x["v"], x["do"], heads=(0, 26), sm_scale=s)


@pytest.fixture(scope="module")
def bench_inputs(gpu):
    """The exact tensors the benchmark step times: B=1, H=40, L=32760, D=128, bf16, drawn on
    the CPU generator seeded 0 in the order Q, K, V, Qd, Kd, Vd, dO, dOd, Q and K
    RMS-normalised and rotated with 3D RoPE over the 21x30x52 latent grid."""
    print("drawing the benchmark inputs on the CPU generator", flush=True)
    x = make_inputs(1, 40, 32760, 32760, 128, seed=0, device=gpu, grid=(21, 30, 52), with_grads=True)
    yield x
    del x
    torch.cuda.empty_cache()


def test_wan14b_self_attention_bench_shape(gpu, bench_inputs):
    """The benchmark workload on the benchmark's own inputs (H=40, L=32760): forward+JVP and
    the dO-only backward, two heads against the oracle, the identities on all 40."""
    print("case wan14b self fwd+JVP+bwd (benchmark inputs)", flush=True)
    x = bench_inputs
    (o, to, lse, mu), (dq, dk, dv), s = _run(x, backward=True)
    args = (x["q"], x["k"], x["v"], x["tq"], x["tk"], x["tv"])
    _check_fwd(o, to, lse, mu, *args, heads=(0, 39), sm_scale=s)
    _check_rows_against_cpu(o, to, *args, h=21, rows=[0, 1, 2047, 16380, 32758, 32759], sm_scale=s)
    _check_bwd(dq, dk, dv, x["q"], x["k"], x["v"], x["do"], heads=(20, 39), sm_scale=s)


def test_wan14b_self_attention_full_derivative_bench_inputs(gpu, bench_inputs):
    """The full derivative (all six gradients, as the benchmark's full-derivative field
    times it) at the 14B head count on the benchmark's inputs: two heads against the
    oracle, the identities on all 40."""
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    print("case wan14b self fwd+JVP+full bwd (benchmark inputs)", flush=True)
    x = bench_inputs
    q, k, v, tq, tk, tv = (x[n] for n in ("q", "k", "v", "tq", "tk", "tv"))
    s = 128 ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    grads = jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, x["do"], x["dto"], s, True)
    torch.cuda.synchronize()
    assert all(g is not None for g in grads)
    _check_bwd_full(grads, x, heads=(7, 33), sm_scale=s)
