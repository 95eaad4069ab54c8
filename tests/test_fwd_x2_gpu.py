"""The K, V tangent-free forward of 128-wide heads at two workgroups per CU (attn_fwd32_x2_kernel).

K, V tangent-free forwards of 128-wide heads (the Wan text cross-attention, Lk = 512) with at
most 64 key tiles (2048 keys) run on a kernel that reads Qd from LDS and fits two workgroups per
CU; longer key sequences, 64-wide heads and the plain forward run the one-workgroup-per-CU
kernel (the last four cases of the table below).

Checked against the float64 oracle on the same rounded inputs (rel-L2 <= 1e-2 and no worse than
1.25x the emulated reference kernel + 1e-4, LSE to 2e-3), and for tile independence: a head's
outputs are bitwise the same whether it runs alone or among 40 heads whose workgroups share the
CUs with it.
"""
import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _draw(g, B, H, L, D, std, dtype):
    return (torch.randn((B, L, H, D), generator=g, dtype=torch.float64) * std).to(dtype).transpose(1, 2)


def _run(dev, q, k, v, tq, mode):
    from dmad_amd.jvp_attention import jvp_attention_forward

    s = q.shape[-1] ** -0.5
    o, to, lse, mu = jvp_attention_forward(q.to(dev), k.to(dev), v.to(dev), None if mode == "plain" else tq.to(dev),
                                           None, None, s)
    torch.cuda.synchronize()
    return o.cpu(), (None if to is None else to.cpu()), lse.cpu(), (None if mu is None else mu.cpu())


CASES = [
    # B, H, Lq, Lk, D, dtype, mode
    (2, 3, 1000, 128, 128, torch.bfloat16, "qonly"),  # 4 key tiles; fewer workgroups than CUs
    (3, 5, 777, 500, 128, torch.float16, "qonly"),    # 16 tiles, the last one partial
    (1, 4, 129, 1024, 128, torch.bfloat16, "qonly"),  # 32 tiles, a partial query tile
    (1, 40, 300, 97, 128, torch.bfloat16, "qonly"),   # 4 tiles, the last one partial
    (1, 2, 200, 33, 128, torch.bfloat16, "qonly"),    # the second tile holds one key
    (2, 2, 333, 2048, 128, torch.float16, "qonly"),   # 64 tiles, the largest count on this kernel
    (1, 2, 300, 97, 64, torch.float16, "plain"),      # one-workgroup-per-CU kernels from here on
    (1, 4, 129, 2048, 64, torch.bfloat16, "qonly"),
    (2, 2, 555, 512, 128, torch.bfloat16, "plain"),
    (1, 3, 64, 8192, 128, torch.bfloat16, "qonly"),
]


@pytest.mark.parametrize("B,H,Lq,Lk,D,dtype,mode", CASES)
def test_kv_tangent_free_forward_matches_oracle(gpu, B, H, Lq, Lk, D, dtype, mode):
    print(f"case kv-tangent-free fwd B={B} H={H} Lq={Lq} Lk={Lk} D={D} {dtype} {mode}", flush=True)
    g = torch.Generator().manual_seed(Lq + Lk)
    q, k, v = _draw(g, B, H, Lq, D, 1.0, dtype), _draw(g, B, H, Lk, D, 1.0, dtype), _draw(g, B, H, Lk, D, 1.0, dtype)
    tq = _draw(g, B, H, Lq, D, 0.1, dtype)
    o, to, lse, mu = _run(gpu, q, k, v, tq, mode)
    zk, zv = torch.zeros_like(k), torch.zeros_like(v)
    ro, rto, rlse, rmu = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, zk, zv)))
    em_o, em_to, _ = orc.triton_fwd_emulator(q, k, v, tq, zk, zv, block_n=32, round_dtype=dtype)
    e_o, f_o = orc.rel_l2(o, ro), orc.rel_l2(em_o.to(dtype), ro)
    assert e_o <= 1e-2 and e_o <= 1.25 * f_o + 1e-4, (e_o, f_o)
    assert float((lse.double() - rlse).abs().max()) <= 2e-3
    if mode == "qonly":
        e_to, f_to = orc.rel_l2(to, rto), orc.rel_l2(em_to.to(dtype), rto)
        assert e_to <= 1e-2 and e_to <= 1.25 * f_to + 1e-4, (e_to, f_to)
        assert orc.rel_l2(mu, rmu) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_heads_are_independent(gpu, dtype):
    """40 heads (two workgroups of different heads or tiles share each CU) against each head
    run alone: bitwise equal."""
    print(f"case x2 head independence {dtype}", flush=True)
    B, H, Lq, Lk, D = 1, 40, 4000, 512, 128
    g = torch.Generator().manual_seed(7)
    q, k, v = _draw(g, B, H, Lq, D, 1.0, dtype), _draw(g, B, H, Lk, D, 1.0, dtype), _draw(g, B, H, Lk, D, 1.0, dtype)
    tq = _draw(g, B, H, Lq, D, 0.1, dtype)
    many = _run(gpu, q, k, v, tq, "qonly")
    for h in (0, 17, 39):
        one = _run(gpu, q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], tq[:, h:h + 1], "qonly")
        for a, b in zip(many, one):
            assert torch.equal(a[:, h:h + 1], b), h


def _growing_logits(g, B, H, Lq, Lk, D, dtype, rise):
    """Q, K whose logits rise with the key index by about `rise` (log2 units) per 32-key tile, so the
    running max moves past the lazy-rescale slack at every step and the accumulators are rescaled
    each time; plus some row-to-row variation."""
    u = torch.randn(D, generator=g, dtype=torch.float64)
    u = u / u.norm()
    qa = 1.0 + 0.5 * torch.rand((B, H, Lq, 1), generator=g, dtype=torch.float64)
    q = qa * u * D ** 0.25 + 0.3 * torch.randn((B, H, Lq, D), generator=g, dtype=torch.float64)
    step = rise / 32 / 1.4426950408889634  # natural-log units of the logit per key
    ramp = torch.arange(Lk, dtype=torch.float64).view(1, 1, Lk, 1) * step
    k = ramp * u * D ** 0.25 + 0.3 * torch.randn((B, H, Lk, D), generator=g, dtype=torch.float64)
    to = lambda x: x.to(dtype).transpose(1, 2).contiguous().transpose(1, 2)  # noqa: E731  (BSHD-like strides)
    return to(q.transpose(1, 2).contiguous().transpose(1, 2)), to(k.transpose(1, 2).contiguous().transpose(1, 2))


@pytest.mark.parametrize("Lk,D,mode,rise", [(512, 128, "qonly", 12.0), (1000, 128, "qonly", 9.0),
                                            (2100, 128, "qonly", 9.0), (700, 64, "qonly", 12.0),
                                            (900, 128, "jvp", 10.0), (640, 64, "jvp", 10.0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rescale_at_every_step(gpu, Lk, D, mode, rise, dtype):
    """Logits rising along the keys: every tile moves the running max beyond the slack (2^8 for
    bf16, 2^4 for fp16), exercising the accumulator rescale on each kernel (two-workgroups-per-CU for
    Kd = Vd = 0 up to 2048 keys, the row kernels otherwise)."""
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case rescale every step Lk={Lk} D={D} {mode} {dtype}", flush=True)
    B, H, Lq = 1, 3, 300
    g = torch.Generator().manual_seed(Lk + D)
    q, k = _growing_logits(g, B, H, Lq, Lk, D, dtype, rise)
    v = _draw(g, B, H, Lk, D, 1.0, dtype)
    tq = _draw(g, B, H, Lq, D, 0.1, dtype)
    tk = _draw(g, B, H, Lk, D, 0.1, dtype) if mode == "jvp" else None
    tv = _draw(g, B, H, Lk, D, 0.1, dtype) if mode == "jvp" else None
    s = D ** -0.5
    o, to, lse, mu = jvp_attention_forward(q.to(gpu), k.to(gpu), v.to(gpu), tq.to(gpu),
                                           None if tk is None else tk.to(gpu), None if tv is None else tv.to(gpu), s)
    torch.cuda.synchronize()
    o, to, lse = o.cpu(), to.cpu(), lse.cpu()
    zk, zv = (torch.zeros_like(k), torch.zeros_like(v)) if tk is None else (tk, tv)
    ro, rto, rlse, _ = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, zk, zv)))
    em_o, em_to, _ = orc.triton_fwd_emulator(q, k, v, tq, zk, zv, block_n=32, round_dtype=dtype)
    e_o, f_o = orc.rel_l2(o, ro), orc.rel_l2(em_o.to(dtype), ro)
    e_to, f_to = orc.rel_l2(to, rto), orc.rel_l2(em_to.to(dtype), rto)
    assert e_o <= 1e-2 and e_o <= 1.25 * f_o + 1e-4, (e_o, f_o)
    # With the softmax this concentrated, Od = C~/l - mu O cancels almost entirely and both the
    # emulated reference kernel and this one sit far from float64 math (~25% at 512 keys); the
    # contract is the reference kernel's own error.
    assert e_to <= 1.25 * f_to + 1e-4, (e_to, f_to)
    assert float((lse.double() - rlse).abs().max()) <= 2e-3 * max(1.0, float(rlse.abs().max()))
    # the softmax is concentrated on the last keys: the logits really did rise across the tiles
    assert float(rlse.mean()) > rise * (Lk // 32 - 2) / 1.4426950408889634 / 2
