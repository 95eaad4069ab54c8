"""dO-only backward of 256-wide heads: the generic dK/dV pass (on transposed Q, dO copies)
and the row-reading dQ pass (attn_bwd_dq_tr_kernel at D = 256: K, V read as 512-byte
rows, K^T formed on the LDS read, Q and dO held in AGPRs; no K^T copy).

Bar, as for the other backward tests: relative L2 <= 1e-2 on dQ, dK, dV against the
float64 oracle (oracle.grads_dout_only) on the same rounded inputs, and no worse than
1.25x the reference backward's own error (oracle.fa2_bwd_emulator, FA2 numerics) + 1e-4:
  * key counts leaving every remainder of the dQ pass's four-step loop (1-4 tiles left)
    and partial last tiles, ragged query counts, bf16 and fp16;
  * BSHD-strided operands;
  * 8192 tokens (64 query tiles per head): every dQ row of one head against the oracle
    in float32 on the GPU, and the identities sum_j dV_j = sum_i dO_i (rows of P sum to
    one) and sum_j dK_j = 0 (rows of dS sum to zero) on every head.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

D = 256


def _draw(g, shape, std, dtype):
    return (torch.randn(shape, generator=g, dtype=torch.float64) * std).to(dtype)


def _grads(gpu, q, k, v, do, s):
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    q, k, v, do = (x.to(gpu) for x in (q, k, v, do))
    o, _, lse, _ = jvp_attention_forward(q, k, v, None, None, None, s)
    dq, dk, dv, *_ = jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)
    torch.cuda.synchronize()
    return dq, dk, dv


def test_plan_uses_the_row_dq_pass():
    from dmad_amd import _native as nat

    b = nat.bwd_plan(nat.DMAD_BF16, 1, 2, 1000, 1000, D)
    assert (b["kernel"], b["kernel2"], b["transposed_copies"]) == ("attn_bwd_kernel", "attn_bwd_dq_tr_kernel", 2)


# (Lq, Lk): 32-key tiles 1 (partial), 2, 3 (partial), 4, 5 (one pass, 1 left), 7 (3 left), 32 (4 left)
SHAPES = [(129, 17), (300, 64), (77, 70), (256, 128), (1, 150), (200, 200), (333, 1000)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Lq,Lk", SHAPES)
def test_wide_backward_matches_oracle(gpu, Lq, Lk, dtype):
    print(f"case bwd D=256 Lq={Lq} Lk={Lk} {dtype}", flush=True)
    g = torch.Generator().manual_seed(Lq * 7 + Lk)
    B, H = 1, 2
    q, k, v = _draw(g, (B, H, Lq, D), 0.5, dtype), _draw(g, (B, H, Lk, D), 0.5, dtype), _draw(g, (B, H, Lk, D), 0.5, dtype)
    do = _draw(g, (B, H, Lq, D), 1.0, dtype)
    s = D ** -0.5
    got = [x.cpu() for x in _grads(gpu, q, k, v, do, s)]
    ref = orc.grads_dout_only(q.double(), k.double(), v.double(), do.double(), s)
    em = orc.fa2_bwd_emulator(q, k, v, do, s, round_dtype=dtype)
    errs = [orc.rel_l2(a, b) for a, b in zip(got, ref)]
    floor = [orc.rel_l2(a.to(dtype), b) for a, b in zip(em, ref)]
    print("  rel-L2 dq %.2e dk %.2e dv %.2e" % tuple(errs), " FA2 floor dq %.2e dk %.2e dv %.2e" % tuple(floor),
          flush=True)
    assert max(errs) <= 1e-2
    for e, f in zip(errs, floor):
        assert e <= 1.25 * f + 1e-4


def test_wide_backward_bshd_strides(gpu):
    print("case bwd D=256 BSHD", flush=True)
    g = torch.Generator().manual_seed(5)
    B, H, Lq, Lk, dtype = 2, 3, 200, 250, torch.bfloat16

    def bshd(L, std):
        return _draw(g, (B, L, H, D), std, dtype).transpose(1, 2)

    q, k, v, do = bshd(Lq, 0.5), bshd(Lk, 0.5), bshd(Lk, 0.5), bshd(Lq, 1.0)
    s = D ** -0.5
    got = [x.cpu() for x in _grads(gpu, q, k, v, do, s)]
    ref = orc.grads_dout_only(*(x.double().contiguous() for x in (q, k, v, do)), s)
    errs = [orc.rel_l2(a, b) for a, b in zip(got, ref)]
    print("  rel-L2 dq %.2e dk %.2e dv %.2e" % tuple(errs), flush=True)
    assert max(errs) <= 1e-2


def test_wide_backward_long_sequence(gpu):
    print("case bwd D=256 L=8192", flush=True)
    B, H, L, dtype = 1, 3, 8192, torch.bfloat16
    g = torch.Generator(device=gpu).manual_seed(9)
    r = lambda std: (torch.randn((B, H, L, D), device=gpu, generator=g) * std).to(dtype)  # noqa: E731
    q, k, v, do = r(1.0), r(1.0), r(1.0), r(1.0)
    s = D ** -0.5
    dq, dk, dv = _grads(gpu, q, k, v, do, s)
    # every dQ row of head 1 (dQ rows depend on their own query only): float32 oracle in query chunks
    h = 1
    f = lambda x: x[0, h].float()  # noqa: E731
    ref_dq = torch.cat([orc.grads_dout_only(f(q)[c:c + 2048], f(k), f(v), f(do)[c:c + 2048], s)[0]
                        for c in range(0, L, 2048)], 0)
    e = orc.rel_l2(dq[0, h].float(), ref_dq)
    print(f"  head {h}: rel-L2 dQ {e:.2e}", flush=True)
    assert e <= 1e-2
    # identities on every head
    for hh in range(H):
        sv, so = dv[0, hh].double().sum(0), do[0, hh].double().sum(0)
        assert float((sv - so).norm() / so.norm()) <= 1e-2
        sk = dk[0, hh].double().sum(0)
        assert float(sk.norm() / dk[0, hh].double().norm()) <= 1e-2
