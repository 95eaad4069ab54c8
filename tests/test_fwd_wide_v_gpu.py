"""Forward of 256-wide V heads (and 256-wide Q/K) on the generic kernels.

In the JVP modes the O~ and C~ accumulators of 256 V columns do not fit next
to Q, Qd and the score tiles, so these launches run attn_fwd_simple_kernel on
128-column halves of V, two workgroups per query tile each recomputing the
scores (fwd_generic_uses_halves); the block-sparse forward does the same.
Checked against the float64 oracle with the forward tests' bar (relative L2
<= 1e-2 and no worse than 1.25x the emulated reference kernel + 1e-4), and the
LSE and mu, which only the first half stores.
"""
import pytest
import torch

from dmad_amd import magimask as mm
from oracle import attention as orc
from oracle import magi as om

pytestmark = pytest.mark.gpu


def _inputs(B, H, Lq, Lk, Dqk, Dv, dtype, seed):
    g = torch.Generator().manual_seed(seed)

    def d(L, D, s):
        return (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * s).to(dtype)

    return d(Lq, Dqk, 0.5), d(Lk, Dqk, 0.5), d(Lk, Dv, 0.5), d(Lq, Dqk, 0.5), d(Lk, Dqk, 0.5), d(Lk, Dv, 0.5)


CASES = [
    # B, H, Lq, Lk, Dqk, Dv, dtype
    (2, 2, 300, 257, 16, 256, torch.bfloat16),
    (1, 2, 129, 333, 32, 256, torch.float16),
    (1, 3, 200, 100, 64, 256, torch.bfloat16),
    (2, 1, 257, 300, 128, 256, torch.float16),
    (1, 2, 300, 190, 256, 256, torch.bfloat16),
    (1, 2, 140, 77, 256, 128, torch.float16),
]


@pytest.mark.parametrize("qonly", [False, True])
@pytest.mark.parametrize("B,H,Lq,Lk,Dqk,Dv,dtype", CASES)
def test_wide_v_forward_matches_oracle(gpu, B, H, Lq, Lk, Dqk, Dv, dtype, qonly):
    from dmad_amd.jvp_attention import jvp_attention_forward

    print(f"case wide V B={B} H={H} Lq={Lq} Lk={Lk} Dqk={Dqk} Dv={Dv} {dtype} qonly={qonly}", flush=True)
    xs = list(_inputs(B, H, Lq, Lk, Dqk, Dv, dtype, seed=Lq + Dqk))
    if qonly:
        xs[4], xs[5] = torch.zeros_like(xs[4]), torch.zeros_like(xs[5])
    s = Dqk ** -0.5
    g = [x.to(gpu) for x in xs]
    o, to, lse, mu = jvp_attention_forward(g[0], g[1], g[2], g[3], None if qonly else g[4], None if qonly else g[5], s)
    torch.cuda.synchronize()
    ro, rto, rlse, rmu = orc.jvp_closed_form(*(x.double() for x in xs), sm_scale=s)
    em_o, em_to, _ = orc.triton_fwd_emulator(*xs, sm_scale=s, block_n=64, round_dtype=dtype)
    e_o, e_to = orc.rel_l2(o.cpu(), ro), orc.rel_l2(to.cpu(), rto)
    f_o, f_to = orc.rel_l2(em_o.to(dtype), ro), orc.rel_l2(em_to.to(dtype), rto)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})", flush=True)
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4
    assert float((lse.cpu().double() - rlse).abs().max()) <= 2e-3
    assert orc.rel_l2(mu.cpu(), rmu) <= 1e-2


@pytest.mark.parametrize("dqk", [64, 256])
def test_wide_v_block_sparse(gpu, dqk):
    """Block-causal mask (window 2, sink 1) with a 256-wide V: both halves of every task."""
    from dmad_amd import attention

    print(f"case wide V block-sparse Dqk={dqk}", flush=True)
    ft, nb = 24, 5
    pat = mm.BlockPattern(frame_tokens=ft, first_chunk_frames=1, chunk_frames=1)
    Q = KV = pat.blocks_to_tokens(nb)
    spec = mm.AttnMaskSpec(mode="block_causal", pattern=pat, local_attn_blocks=2, sink_blocks=1)
    allow = om.allowed_mask("block_causal", ft, Q, KV, 1, 1, local_attn_blocks=2, sink_blocks=1)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    xs = _inputs(1, 2, Q, KV, dqk, 256, torch.bfloat16, seed=dqk)
    s = dqk ** -0.5
    o, to = attention(*(x.to(gpu) for x in xs), s, mask)
    torch.cuda.synchronize()
    ro, rto, _, _ = om.masked_jvp(*xs, allow, s)
    e_o, e_to = orc.rel_l2(o.cpu(), ro), orc.rel_l2(to.cpu(), rto)
    eo, eto, _ = om.magi_fwd_emulator(*xs, mask.q_unique.cpu(), mask.k_flat.cpu(), mask.qk_map.cpu(), s,
                                      block_n=64, round_dtype=torch.bfloat16)
    f_o, f_to = orc.rel_l2(eo.to(torch.bfloat16), ro), orc.rel_l2(eto.to(torch.bfloat16), rto)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})", flush=True)
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4
