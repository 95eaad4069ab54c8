"""The persistent forward for short key sequences (attn_fwd32_persist_kernel).

K, V tangent-free forwards of 128-wide heads (the Wan text cross-attention,
Lk = 512) whose key-tile count (32 keys a tile) is a multiple of 4, up to 32
tiles, run on a kernel whose workgroups loop over (batch*head, query tile)
items with the key ring running on across items, the next item's Q prefetched
into LDS and the finished item's O leaving through LDS as whole rows. The other
cases of the table below run the per-tile kernel, whose O now also leaves
through LDS as whole rows.

Checked against the float64 oracle on the same rounded inputs (rel-L2 <= 1e-2
and no worse than 1.25x the emulated reference kernel + 1e-4, LSE to 2e-3), and
for item independence: a head's outputs are bitwise the same whether its
workgroup ran one item or many (the transition between items -- accumulator
reset, prefetched Q, the ring's stage order -- leaves no trace).
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
    (2, 3, 1000, 128, 128, torch.bfloat16, "qonly"),  # 4 key tiles; fewer items than workgroup slots
    (3, 5, 777, 500, 128, torch.float16, "qonly"),    # 16 tiles, the last one partial
    (1, 4, 129, 1024, 128, torch.bfloat16, "qonly"),  # 32 tiles, the largest count on the persistent kernel
    (1, 40, 300, 97, 128, torch.bfloat16, "qonly"),   # 4 tiles, 120 items
    (1, 2, 300, 97, 64, torch.float16, "plain"),      # per-tile kernels from here on
    (1, 4, 129, 2048, 64, torch.bfloat16, "qonly"),
    (2, 2, 555, 512, 128, torch.bfloat16, "plain"),
    (1, 3, 64, 8192, 128, torch.bfloat16, "qonly"),
]


@pytest.mark.parametrize("B,H,Lq,Lk,D,dtype,mode", CASES)
def test_persistent_forward_matches_oracle(gpu, B, H, Lq, Lk, D, dtype, mode):
    print(f"case persistent fwd B={B} H={H} Lq={Lq} Lk={Lk} D={D} {dtype} {mode}", flush=True)
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


@pytest.mark.parametrize("D,mode", [(128, "qonly")])
def test_persistent_items_are_independent(gpu, D, mode):
    """40 heads (a workgroup runs up to 40 items, crossing heads) against each head run
    alone (one item per workgroup): bitwise equal."""
    print(f"case persistent item independence D={D} {mode}", flush=True)
    B, H, Lq, Lk = 1, 40, 4000, 512
    g = torch.Generator().manual_seed(D)
    q, k, v = _draw(g, B, H, Lq, D, 1.0, torch.bfloat16), _draw(g, B, H, Lk, D, 1.0, torch.bfloat16), \
        _draw(g, B, H, Lk, D, 1.0, torch.bfloat16)
    tq = _draw(g, B, H, Lq, D, 0.1, torch.bfloat16)
    many = _run(gpu, q, k, v, tq, mode)
    for h in (0, 17, 39):
        one = _run(gpu, q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], tq[:, h:h + 1], mode)
        for a, b in zip(many, one):
            if a is not None:
                assert torch.equal(a[:, h:h + 1], b), h
