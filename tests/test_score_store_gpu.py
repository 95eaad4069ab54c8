"""Backward on stored score gradients (128-wide bf16/fp16 heads).

The key pass also writes the dS (full derivative: and dSd) tiles it computes,
and the query pass (attn_bwd_dq_sc_kernel) reads them back instead of
recomputing S and dP. Checked on the same inputs against the recomputing passes
(score budget 0): dK, dV (dKd, dVd) bit for bit, since the key pass's arithmetic
is unchanged, and dQ (dQd) to rounding (the query pass sums the same bf16/fp16
products in the same key order). Each case runs with every (b, h) slice in one
launch pair and with one slice per pair (the chunked launch), and two cases go
against the float64 oracle. The reference has no such path: its backward is
flash-attn's (flash_attention_jvp_triton.py:534-579), which recomputes.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

SHAPES = [(1, 2, 64, 64), (1, 3, 200, 200), (2, 2, 1000, 1000), (1, 2, 300, 700), (1, 1, 777, 129),
          (1, 2, 4100, 4100), (1, 2, 129, 1000)]
DTYPES = [torch.bfloat16, torch.float16]


@pytest.fixture
def budget(monkeypatch):
    """Sets the stored-score budget for one test (the dO-only backward's length threshold and
    the minimum workgroups per launch pair lifted, so that short sequences and one-slice pairs
    take the path too) and restores the process default."""
    import dmad_amd
    from dmad_amd import jvp_attention as ja

    monkeypatch.setattr(ja, "_SCORE_MIN_LEN_DOUT_ONLY", 0)
    monkeypatch.setattr(ja, "_SCORE_MIN_KEY_WORKGROUPS", 0)
    old = dmad_amd.backward_score_budget()
    yield dmad_amd.set_backward_score_budget
    dmad_amd.set_backward_score_budget(old)


def _inputs(dev, B, H, Lq, Lk, dtype, seed=5, bshd=False):
    g = torch.Generator().manual_seed(seed)

    def r(L, std):
        x = (torch.randn((B, L, H, 128) if bshd else (B, H, L, 128), generator=g) * std).to(dtype).to(dev)
        return x.transpose(1, 2) if bshd else x

    q, k, v = r(Lq, 0.5), r(Lk, 0.5), r(Lk, 0.5)
    tq, tk, tv = r(Lq, 0.1), r(Lk, 0.1), r(Lk, 0.1)
    do, dto = r(Lq, 1.0), r(Lq, 0.1)
    return q, k, v, tq, tk, tv, do, dto


def _backward(xs, full, nbytes, budget):
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    q, k, v, tq, tk, tv, do, dto = xs
    s = 128 ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    budget(nbytes)
    out = jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, do, dto if full else None, s, full)
    torch.cuda.synchronize()
    return [None if x is None else x.cpu() for x in out]


def _plan_slices(xs, full, nbytes):
    from dmad_amd import _native as nat
    from dmad_amd import jvp_attention as ja

    q, k = xs[0], xs[1]
    B, H, Lq, D = q.shape
    code = nat.dtype_code(q.dtype)
    base = nat.bwd_workspace_bytes_of(code, (2 if full else 0), B, H, Lq, k.shape[2], D)
    old = ja.backward_score_budget()
    ja.set_backward_score_budget(nbytes)
    try:
        extra = ja._score_bytes(code, full, B, H, Lq, k.shape[2], D)
    finally:
        ja.set_backward_score_budget(old)
    assert extra > 0
    pl = nat.bwd_plan(code, B, H, Lq, k.shape[2], D, full=full, tangent_grads=full, workspace_bytes=base + extra)
    return pl["score_slices"], pl


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("full", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_stored_scores_match_recomputing_passes(gpu, budget, shape, full, dtype):
    B, H, Lq, Lk = shape
    print(f"case shape={shape} full={full} dtype={dtype}", flush=True)
    xs = _inputs(gpu, B, H, Lq, Lk, dtype)
    from dmad_amd import _native as nat

    one = nat.bwd_score_bytes(nat.dtype_code(dtype), full, Lq, Lk, 128)
    assert one > 0
    ref = _backward(xs, full, 0, budget)
    for nbytes, want_slices in ((1 << 62, B * H), (one, 1)):
        slices, pl = _plan_slices(xs, full, nbytes)
        assert slices == want_slices and pl["kernel2"] == "attn_bwd_dq_sc_kernel"
        got = _backward(xs, full, nbytes, budget)
        for name, a, b in zip(("dq", "dk", "dv", "dtq", "dtk", "dtv"), got, ref):
            if b is None:
                assert a is None
                continue
            assert torch.isfinite(a).all(), name
            if name in ("dk", "dv", "dtk", "dtv"):
                assert torch.equal(a, b), f"{name} differs with {slices} slice(s) per pair"
            else:
                e = orc.rel_l2(a.double(), b.double())
                print(f"  {name} slices={slices} rel-L2 vs recompute {e:.2e}")
                assert e <= 2e-3, (name, slices, e)


def test_stored_scores_bshd_views(gpu, budget):
    """Wan's [B, L, H, D] layout seen as [B, H, L, D] views (row stride H*D)."""
    xs = _inputs(gpu, 2, 3, 520, 520, torch.bfloat16, bshd=True)
    assert xs[0].stride()[2] == 3 * 128
    for full in (False, True):
        ref = _backward(xs, full, 0, budget)
        got = _backward(xs, full, 1 << 62, budget)
        for a, b in zip(got, ref):
            if b is not None:
                assert orc.rel_l2(a.double(), b.double()) <= 2e-3


@pytest.mark.parametrize("full", [False, True])
def test_stored_scores_against_oracle(gpu, budget, full):
    """The stored-score gradients against the float64 oracle (dO-only or all six)."""
    B, H, Lq, Lk = 1, 2, 999, 1031
    xs = _inputs(gpu, B, H, Lq, Lk, torch.bfloat16, seed=11)
    got = _backward(xs, full, 1 << 62, budget)
    x64 = [x.cpu().double() for x in xs]
    s = 128 ** -0.5
    if full:
        ref = orc.grads_full(*x64, sm_scale=s)
    else:
        q, k, v, _, _, _, do, _ = x64
        ref = orc.grads_dout_only(q, k, v, do, s)
    errs = [orc.rel_l2(a.double(), b) for a, b in zip(got, ref)]
    print("  rel-L2", " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= 1e-2
