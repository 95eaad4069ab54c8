"""Non-finite inputs: a NaN or an Inf stays inside its (batch, head) slice.

The rCM sCM step drops a sample whose teacher output or tangent is non-finite
with a per-sample mask (train/wan/rcm/models/t2v_model_distill_rcm.py:596-609),
which relies on a NaN in one sample's q, k, v or tangent reaching that sample's
O / Od and on no other sample being touched. Contract checked here, for one
poisoned element in sample 1, head 0:
  * every other (batch, head) slice of O, Od, LSE, mu and of the dO-only
    gradients is bitwise equal to the clean run (they are separate workgroups);
  * in the poisoned slice, O and Od are non-finite exactly where the float64
    math attention (oracle.attention) on the same inputs is non-finite (IEEE
    propagation: a NaN score poisons its row, +Inf scores give Inf - Inf, -Inf
    scores drop the key), dQ, dK, dV are non-finite at least there, and where
    both are finite they agree to the usual rel-L2 <= 1e-2;
  * a poisoned tangent leaves O, LSE and the dO-only gradients bitwise unchanged.
bf16 on the 128-, 64- and 256-wide kernels (at 256: two forward workgroups per query tile, one
per 128-column chunk of V), fp32 on the fp32 kernels.
"""
import math

import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

B, H, L = 3, 2, 300
ROW_Q, ROW_K, COL = 37, 123, 5


def _inputs(D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    r = lambda sd: (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * sd).to(dtype)  # noqa: E731
    return {"q": r(1.0), "k": r(1.0), "v": r(1.0), "tq": r(0.1), "tk": r(0.1), "tv": r(0.1), "do": r(1.0)}


def _run(x, dev):
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    g = {n: t.to(dev) for n, t in x.items()}
    s = g["q"].shape[-1] ** -0.5
    o, to, lse, mu = jvp_attention_forward(g["q"], g["k"], g["v"], g["tq"], g["tk"], g["tv"], s)
    dq, dk, dv = jvp_attention_backward(g["q"], g["k"], g["v"], None, None, None, o, None, lse, None, g["do"], None,
                                        s, False)[:3]
    torch.cuda.synchronize()
    return {n: t.cpu() for n, t in (("o", o), ("to", to), ("lse", lse), ("mu", mu), ("dq", dq), ("dk", dk),
                                     ("dv", dv))}


def _oracle(x):
    """float64 (O, Od, dQ, dK, dV) of sample 1, head 0."""
    sl = {n: t[1:2, 0:1].double() for n, t in x.items()}
    o, to, _, _ = orc.jvp_closed_form(sl["q"], sl["k"], sl["v"], sl["tq"], sl["tk"], sl["tv"])
    dq, dk, dv = orc.grads_dout_only(sl["q"], sl["k"], sl["v"], sl["do"])
    return {"o": o, "to": to, "dq": dq, "dk": dk, "dv": dv}


def _poison(x, where, val):
    y = {n: t.clone() for n, t in x.items()}
    row = ROW_K if where in ("k", "v") else ROW_Q
    y[where][1, 0, row, COL] = val
    return y


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.bfloat16), (256, torch.bfloat16),
                                     (128, torch.float32), (32, torch.float32)])
@pytest.mark.parametrize("where", ["q", "k", "v", "tq"])
@pytest.mark.parametrize("val", [math.nan, math.inf])
def test_nonfinite_input_stays_in_its_slice(gpu, D, dtype, where, val):
    print(f"case nonfinite D={D} {dtype} {where}={val}", flush=True)
    x = _inputs(D, seed=D, dtype=dtype)
    clean = _run(x, gpu)
    y = _poison(x, where, val)
    got = _run(y, gpu)
    # untouched slices: bitwise equal to the clean run
    for name, t in got.items():
        for b in range(B):
            for h in range(H):
                if (b, h) == (1, 0):
                    continue
                assert torch.equal(t[b, h], clean[name][b, h]), (name, b, h)
    if where == "tq":
        # the tangent feeds Od and mu only
        for name in ("o", "lse", "dq", "dk", "dv"):
            assert torch.equal(got[name][1, 0], clean[name][1, 0]), name
    ref = _oracle(y)
    n_bad = {}
    for name, r in ref.items():
        gv, rv = got[name][1, 0].double(), r[0, 0]
        fin_g, fin_r = torch.isfinite(gv), torch.isfinite(rv)
        n_bad[name] = int((~fin_r).sum())
        if name in ("o", "to"):
            assert torch.equal(fin_g, fin_r), (name, int((~fin_g).sum()), int((~fin_r).sum()))
        else:
            # The backward recomputes P from the stored LSE. A row holding a +Inf
            # score has LSE = m + log2(l) = NaN (as the reference kernel's), where
            # math's logsumexp is +Inf, so the gradients may be non-finite in more
            # places than the math's -- but never finite where the math is not.
            assert not (fin_g & ~fin_r).any(), (name, int((~fin_g).sum()), int((~fin_r).sum()))
        both = fin_g & fin_r
        if both.any():
            err = orc.rel_l2(gv[both], rv[both])
            assert err <= 1e-2, (name, err)
    print(f"  non-finite entries (kernel = float64 math): {n_bad}", flush=True)
    # the poisoned element reaches the outputs it feeds
    assert n_bad["to"] > 0
    if where != "tq":
        assert n_bad["o"] > 0 and n_bad["dk"] > 0
    if where in ("q", "k"):  # dV = P^T dO does not involve V
        assert n_bad["dv"] > 0


@pytest.mark.parametrize("where", ["q", "k", "v", "tq"])
@pytest.mark.parametrize("val", [math.nan, math.inf])
def test_nonfinite_kv_tangent_free_forward(gpu, where, val):
    """The same contract for the K, V tangent-free forward (Kd = Vd = 0, 128-wide heads, short key
    sequences: the two-workgroups-per-CU kernel): O, Od, LSE and mu of the other slices bitwise
    clean, the poisoned slice non-finite exactly where float64 math is."""
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case nonfinite kv-tangent-free {where}={val}", flush=True)
    x = _inputs(128, seed=11, dtype=torch.bfloat16)

    def run(inp):
        g = {n: t.to(gpu) for n, t in inp.items()}
        o, to, lse, mu = jvp_attention_forward(g["q"], g["k"], g["v"], g["tq"], None, None, 128 ** -0.5)
        torch.cuda.synchronize()
        return {"o": o.cpu(), "to": to.cpu(), "lse": lse.cpu(), "mu": mu.cpu()}

    clean = run(x)
    y = _poison(x, where, val)
    got = run(y)
    for name, t in got.items():
        for b in range(B):
            for h in range(H):
                if (b, h) != (1, 0):
                    assert torch.equal(t[b, h], clean[name][b, h]), (name, b, h)
    if where == "tq":
        for name in ("o", "lse"):
            assert torch.equal(got[name][1, 0], clean[name][1, 0]), name
    sl = {n: t[1:2, 0:1].double() for n, t in y.items()}
    zk, zv = torch.zeros_like(sl["k"]), torch.zeros_like(sl["v"])
    ro, rto, _, _ = orc.jvp_closed_form(sl["q"], sl["k"], sl["v"], sl["tq"], zk, zv)
    for name, r in (("o", ro), ("to", rto)):
        gv, rv = got[name][1, 0].double(), r[0, 0]
        fin_g, fin_r = torch.isfinite(gv), torch.isfinite(rv)
        assert torch.equal(fin_g, fin_r), (name, int((~fin_g).sum()), int((~fin_r).sum()))
        both = fin_g & fin_r
        if both.any():
            assert orc.rel_l2(gv[both], rv[both]) <= 1e-2, name
        if name == "to" or where != "tq":
            assert (~fin_r).any(), name
