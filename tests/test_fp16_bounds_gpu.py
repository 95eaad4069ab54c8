"""fp16 forward: the lazy rescale keeps P~ <= 1, so H~ = P~ s Sd overflows no sooner than the reference's.

The fp16 kernels let the running max m lag a row's true max by up to 2^4 (log2 units) and form
P~ = exp2(x - m - 4). Built here: each query's largest logit sits in an early key tile, and a later
tile holds a key 3 log2 units above it whose tangent logit s*Sd is 2e4. The reference kernel
(`_attn_fwd`, flash_attention_jvp_triton.py:150-223: exact running max, P~ <= 1) forms H~ = 2e4
there, finite in fp16; a kernel with P~ = exp2(x - m) would reach 2^3 * 2e4 = 1.6e5 and overflow to
inf. Checked for the full JVP mode (Kd given) and the K, V tangent-free mode (two workgroups per CU),
at head dims served by the row kernels (64, 128) and the 32-key generic forward (32): every output
finite, and as close to float64 math as the emulated fp16 reference kernel is.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _inputs(D, mode, seed=7):
    g = torch.Generator().manual_seed(seed)
    B, H, Lq, Lk = 1, 2, 200, 700
    j1, js = 40, 333  # the early max key (tile 1) and the later, higher one (tile 10)
    s = D ** -0.5
    c = s * 1.4426950408889634  # log2 units per unit of q.k
    u = torch.randn(D, generator=g, dtype=torch.float64)
    u = u / u.norm() * D ** 0.5  # |u|^2 = D
    q = u + 0.05 * torch.randn((B, H, Lq, D), generator=g, dtype=torch.float64)
    k = 0.3 * torch.randn((B, H, Lk, D), generator=g, dtype=torch.float64)
    k[:, :, j1] = (10.0 / c / D) * u  # log2 logit ~10
    k[:, :, js] = (13.0 / c / D) * u  # ~13: 3 above the max the row has seen
    v = torch.randn((B, H, Lk, D), generator=g, dtype=torch.float64)
    v[:, :, js] *= 1e-3  # keeps Od within fp16's range
    tq = torch.zeros_like(q)
    tk = torch.zeros_like(k)
    tv = torch.zeros_like(v)
    if mode == "jvp":
        tk[:, :, js] = (2e4 / s / D) * u  # s Sd ~ 2e4 at key js only
    else:
        # Sd = s Qd K^T: 2e4 at key js (10/13 of it at key j1)
        tq = ((2e4 / s) / float(k[0, 0, js] @ u)) * u.expand_as(q).clone()
    f16 = lambda x: x.to(torch.float16)  # noqa: E731
    return [f16(x) for x in (q, k, v, tq, tk, tv)], s


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("mode", ["jvp", "qonly"])
def test_fp16_tangent_logits_near_overflow(gpu, D, mode):
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case fp16 bounds D={D} {mode}", flush=True)
    (q, k, v, tq, tk, tv), s = _inputs(D, mode)
    args = [x.to(gpu) for x in (q, k, v, tq)]
    kd, vd = (tk.to(gpu), tv.to(gpu)) if mode == "jvp" else (None, None)
    o, to, lse, mu = jvp_attention_forward(*args, kd, vd, s)
    torch.cuda.synchronize()
    o, to, lse, mu = o.cpu(), to.cpu(), lse.cpu(), mu.cpu()
    for name, x in (("o", o), ("to", to), ("lse", lse), ("mu", mu)):
        assert torch.isfinite(x).all(), name
    ro, rto, rlse, rmu = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, tk, tv)), sm_scale=s)
    em_o, em_to, _ = orc.triton_fwd_emulator(q, k, v, tq, tk, tv, sm_scale=s, block_n=32, round_dtype=torch.float16)
    assert torch.isfinite(em_o).all() and torch.isfinite(em_to).all()  # the reference kernel stays finite
    assert float(rmu.abs().max()) > 1e4  # the tangent logits really are that large
    e_o, f_o = orc.rel_l2(o, ro), orc.rel_l2(em_o.to(torch.float16), ro)
    e_to, f_to = orc.rel_l2(to, rto), orc.rel_l2(em_to.to(torch.float16), rto)
    print(f"  rel-L2 O {e_o:.2e} (reference kernel {f_o:.2e}), Od {e_to:.2e} ({f_to:.2e})")
    assert e_o <= 1e-2 and e_o <= 1.25 * f_o + 1e-4, (e_o, f_o)
    assert e_to <= 1e-2 and e_to <= 1.25 * f_to + 1e-4, (e_to, f_to)
    assert orc.rel_l2(mu, rmu) <= 1e-3
    assert float((lse.double() - rlse).abs().max()) <= 2e-3 * max(1.0, float(rlse.abs().max()))
