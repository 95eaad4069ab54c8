"""Block-sparse (MagiMask) forward+JVP on the GPU against the CPU oracle.

Cases: the reference's own test_jvp_magi grid (flash_attention_jvp_triton.py:
910-930: block_causal / teacher_forcing, frame_tokens 8-32, head dims 64/64
and 64/128, fp16 and bf16, masks built with BLOCK_M = 64, plus the sliding
window + sink case), 128-wide heads (the production kernel's block-sparse
variant) with block edges off the 32-key and 128-query grids, batch and heads
> 1, the zero-K/V-tangent mode, hand-made tables (a group without keys, ranges
reaching outside the sequences, rows no task covers), a seeded sweep of
schedules (frame and block sizes, windows, sinks, query block offsets) and
seeded masks given as raw overlapping rectangles.

Bar: relative L2 <= 1e-2 against the float64 masked closed form, no worse than
the reference kernel's numerics (oracle.magi.magi_fwd_emulator, BLOCK_N 64) plus
a small margin, and the reference test's assert_close tolerances.
"""
import ctypes
import math

import pytest
import torch

from dmad_amd import magimask as mm
from oracle import attention as orc
from oracle import magi as om

pytestmark = pytest.mark.gpu


def _spec(mode, ft, nb, first=1, chunk=1, local=0, sink=0, q_bo=0):
    pat = mm.BlockPattern(frame_tokens=ft, first_chunk_frames=first, chunk_frames=chunk)
    if mode == "block_causal":
        KV = pat.blocks_to_tokens(q_bo + nb)
        Q = KV - pat.blocks_to_tokens(q_bo) if q_bo else KV
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, q_block_offset=q_bo, local_attn_blocks=local, sink_blocks=sink)
        allow = om.allowed_mask(mode, ft, Q, KV, first, chunk, q_block_offset=q_bo, local_attn_blocks=local,
                                sink_blocks=sink)
    else:
        Q = KV = 2 * pat.blocks_to_tokens(nb)
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, clean_blocks=nb, local_attn_blocks=local, sink_blocks=sink)
        allow = om.allowed_mask(mode, ft, Q, KV, first, chunk, local_attn_blocks=local, sink_blocks=sink,
                                clean_blocks=nb, as_range_builder=True)
    return spec, Q, KV, allow


def _inputs(B, H, Q, KV, dqk, dv, dtype, seed=42):
    g = torch.Generator().manual_seed(seed)

    def d(L, D):
        return (torch.randn((B, H, L, D), generator=g, dtype=torch.float64) * 0.5).to(dtype)

    return d(Q, dqk), d(KV, dqk), d(KV, dv), d(Q, dqk), d(KV, dqk), d(KV, dv)


def _check(xs, dev, mask, allow, sm_scale, dtype, tol_ref=True):
    from dmad_amd import attention

    g = [x.to(dev) for x in xs]
    o, to = attention(*g, sm_scale, mask)
    torch.cuda.synchronize()
    o, to = o.cpu(), to.cpu()
    ro, rto, _, _ = om.masked_jvp(*xs, allow, sm_scale)
    e_o, e_to = orc.rel_l2(o, ro), orc.rel_l2(to, rto)
    eo, eto, _ = om.magi_fwd_emulator(*xs, mask.q_unique.cpu(), mask.k_flat.cpu(), mask.qk_map.cpu(), sm_scale,
                                      block_n=64, round_dtype=dtype)
    f_o, f_to = orc.rel_l2(eo.to(dtype), ro), orc.rel_l2(eto.to(dtype), rto)
    print(f"  rel-L2 O {e_o:.2e} (ref kernel {f_o:.2e})  Od {e_to:.2e} (ref kernel {f_to:.2e})", flush=True)
    assert e_o <= 1e-2 and e_to <= 1e-2
    assert e_o <= 1.25 * f_o + 1e-4 and e_to <= 1.25 * f_to + 1e-4
    if tol_ref:
        atol = 2e-2 if dtype == torch.bfloat16 else 1e-2
        torch.testing.assert_close(o.double(), ro, atol=atol, rtol=1e-2)
        torch.testing.assert_close(to.double(), rto, atol=atol, rtol=1e-2)
    return o, to


REF_SHAPES = [(1, 2, 16, 4, 64, 64), (1, 2, 32, 3, 64, 64), (1, 2, 8, 5, 64, 128)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", REF_SHAPES)
@pytest.mark.parametrize("mode", ["block_causal", "teacher_forcing"])
def test_reference_magi_cases(gpu, mode, shape, dtype):
    B, H, ft, nb, dqk, dv = shape
    print(f"case mode={mode} shape={shape} dtype={dtype}", flush=True)
    spec, Q, KV, allow = _spec(mode, ft, nb)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=64)
    _check(_inputs(B, H, Q, KV, dqk, dv, dtype), gpu, mask, allow, dqk ** -0.5, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", ["block_causal", "teacher_forcing"])
def test_reference_magi_sliding_window(gpu, mode, dtype):
    print(f"case mode={mode} window 3 sink 1 dtype={dtype}", flush=True)
    spec, Q, KV, allow = _spec(mode, 16, 6, local=3, sink=1)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=64)
    _check(_inputs(1, 2, Q, KV, 64, 64, dtype), gpu, mask, allow, 64 ** -0.5, dtype)


# 128-wide heads: block edges at multiples of 40 / 52 / 77 tokens, off the
# 32-key tiles and the 128-query tiles
WIDE = [
    ("block_causal", 40, 5, 1, 2, 0, 0, 2, 3),
    ("block_causal", 52, 6, 1, 3, 3, 1, 1, 2),
    ("teacher_forcing", 77, 3, 1, 1, 0, 0, 1, 2),
    ("teacher_forcing", 40, 4, 1, 2, 2, 1, 2, 1),
]


# D = 256: the row-reading kernel in two 128-column chunks of V per task
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", WIDE)
def test_wide_heads(gpu, case, dtype, D):
    mode, ft, nb, first, chunk, local, sink, B, H = case
    print(f"case {case} dtype={dtype} D={D}", flush=True)
    spec, Q, KV, allow = _spec(mode, ft, nb, first, chunk, local, sink)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    _check(_inputs(B, H, Q, KV, D, D, dtype, seed=7), gpu, mask, allow, D ** -0.5, dtype)


def _sweep(n, seed):
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(len(xs), (1,), generator=g))]

    def rint(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    out = []
    for i in range(n):
        mode = pick(["block_causal", "teacher_forcing"])
        out.append(dict(mode=mode, ft=rint(3, 48), nb=rint(2, 5), first=rint(1, 2), chunk=rint(1, 3),
                        local=pick([0, 0, 1, 2, 3]), sink=rint(0, 2),
                        q_bo=pick([0, 1, 2]) if mode == "block_causal" else 0, B=rint(1, 2), H=rint(1, 3),
                        dims=pick([(128, 128), (64, 64), (64, 128)]), block_m=pick([64, 128]),
                        dtype=pick([torch.bfloat16, torch.float16]), seed=300 + i))
    return out


@pytest.mark.parametrize("c", _sweep(12, 77), ids=lambda c: "{mode}-ft{ft}-nb{nb}-bo{q_bo}-d{dims[0]}".format(**c))
def test_pattern_sweep(gpu, c):
    """Seeded schedules: frame sizes off every tile grid, 1-2 frame first blocks,
    1-3 frame blocks, windows and sinks, a query block offset (block-causal
    queries that start past the first blocks), tables built at BLOCK_M 64 or 128.
    The mask comes from the oracle's allowed_mask (with the range builder's rule
    for a 1-block teacher-forcing window), not from the range tables."""
    print(f"case {c}", flush=True)
    dqk, dv = c["dims"]
    spec, Q, KV, allow = _spec(c["mode"], c["ft"], c["nb"], c["first"], c["chunk"], c["local"], c["sink"], c["q_bo"])
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=c["block_m"])
    xs = _inputs(c["B"], c["H"], Q, KV, dqk, dv, c["dtype"], seed=c["seed"])
    _check(xs, gpu, mask, allow, dqk ** -0.5, c["dtype"])


@pytest.mark.parametrize("seed", range(8))
def test_random_rectangles(gpu, seed):
    """Masks given as raw rectangles: query groups of random lengths, each with
    1-4 key ranges that overlap, touch or reach outside [0, KV), rows shuffled;
    the expected mask is painted from the raw rectangles."""
    g = torch.Generator().manual_seed(500 + seed)
    Q, KV = (int(x) for x in torch.randint(40, 600, (2,), generator=g))
    D = (128, 64)[seed % 2]
    dtype = (torch.bfloat16, torch.float16)[(seed // 2) % 2]
    print(f"case seed={seed} Q={Q} KV={KV} D={D} dtype={dtype}", flush=True)
    qr, kr, allow = om.random_rectangles(seed, Q, KV)
    mask = mm.prepare_magi_csr_and_tasks(qr.to(gpu), kr.to(gpu), Q_real=Q, KV_real=KV)
    xs = _inputs(1 + seed % 2, 2, Q, KV, D, D, dtype, seed=600 + seed)
    _check(xs, gpu, mask, allow, D ** -0.5, dtype)


@pytest.mark.parametrize("dims", [(128, 128), (64, 64), (128, 32)])
def test_kv_tangent_zero_mode(gpu, dims):
    from dmad_amd import attention

    dqk, dv = dims
    spec, Q, KV, allow = _spec("block_causal", 40, 4, chunk=2)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    xs = _inputs(1, 2, Q, KV, dqk, dv, torch.bfloat16, seed=9)
    q, k, v, tq, _, _ = (x.to(gpu) for x in xs)
    o1, to1 = attention(q, k, v, tq, None, None, None, mask)
    o2, to2 = attention(q, k, v, tq, torch.zeros_like(k), torch.zeros_like(v), None, mask)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    if dqk != dv:  # the generic kernel forms the same H~ = P~ (s Sd) in both modes
        assert orc.rel_l2(to1, to2) < 1e-6
    else:  # bf16 K, V tangent-free mode: H~ = P~ Sd, the scale applied in the epilogue
        zk, zv = torch.zeros_like(xs[4]), torch.zeros_like(xs[5])
        _, rto, _, _ = om.masked_jvp(xs[0], xs[1], xs[2], xs[3], zk, zv, allow, dqk ** -0.5)
        e_fast, e_gen = orc.rel_l2(to1.cpu(), rto), orc.rel_l2(to2.cpu(), rto)
        assert orc.rel_l2(to1, to2) < 1e-2
        assert e_fast <= 1.1 * e_gen + 1e-4, (e_fast, e_gen)


def test_lse_and_mu(gpu):
    from dmad_amd.jvp_attention import jvp_attention_forward_magi

    spec, Q, KV, allow = _spec("teacher_forcing", 40, 3, chunk=2, local=2, sink=1)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    xs = _inputs(1, 3, Q, KV, 128, 128, torch.bfloat16, seed=11)
    o, to, lse, mu = jvp_attention_forward_magi(*(x.to(gpu) for x in xs), 0.09, mask)
    ro, rto, rlse, rmu = om.masked_jvp(*xs, allow, 0.09)
    assert (lse.cpu().double() - rlse).abs().max() < 2e-3
    assert orc.rel_l2(mu.cpu(), rmu) < 1e-2
    assert orc.rel_l2(o.cpu(), ro) < 1e-2 and orc.rel_l2(to.cpu(), rto) < 1e-2


def _call_tables(gpu, xs, q_ranges, k_ranges, qk_map, tasks, sentinel):
    """Direct C-ABI call with hand-made tables; outputs pre-filled with `sentinel`."""
    from dmad_amd import _native as nat

    q, k, v, tq, tk, tv = (x.to(gpu) for x in xs)
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=gpu).contiguous()  # noqa: E731
    qr, kr, qm = i32(q_ranges), i32(k_ranges), i32(qk_map)
    tg, tt = i32([t[0] for t in tasks]), i32([t[1] for t in tasks])
    o = torch.full((B, H, Lq, D), sentinel, device=gpu, dtype=q.dtype)
    to = torch.full_like(o, sentinel)
    lse = torch.full((B, H, Lq), sentinel, device=gpu, dtype=torch.float32)
    mu = torch.full_like(lse, sentinel)
    ws = torch.empty(1 << 20, device=gpu, dtype=torch.uint8)
    nat.check(nat.lib().dmad_attn_jvp_fwd_magi(
        nat.dtype_code(q.dtype), nat.DMAD_FWD_JVP, B, H, Lq, Lk, D, D,
        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(tq), nat.ptr(tk), nat.ptr(tv),
        nat.strides4(q), nat.strides4(k), nat.strides4(v), nat.ptr(o), nat.ptr(to), nat.strides4(o),
        nat.ptr(lse), nat.ptr(mu), 0.125, nat.ptr(qr), nat.ptr(kr), nat.ptr(qm), len(q_ranges), len(k_ranges),
        nat.ptr(tg), nat.ptr(tt), len(tasks), 128, nat.ptr(ws), ws.numel(), nat.stream_ptr(gpu)))
    torch.cuda.synchronize()
    return o.cpu(), to.cpu(), lse.cpu(), mu.cpu()


@pytest.mark.parametrize("D", [128, 64, 256])
def test_hand_made_tables(gpu, D):
    """Group 0 [0, 100): keys [-20, 50) and [90, 95) (clipped at 0);
    group 1 [100, 230): keys [250, 400) entirely past Lk = 240 -> no keys;
    group 2 [230, 300): keys [10, 20) and [200, 1000) (clipped at Lk);
    rows [300, 333) belong to no task and must stay untouched."""
    Lq, Lk = 333, 240
    xs = _inputs(1, 2, Lq, Lk, D, D, torch.bfloat16, seed=13)
    q_ranges = [[0, 100], [100, 230], [230, 300]]
    k_ranges = [[-20, 50], [90, 95], [250, 400], [10, 20], [200, 1000]]
    qk_map = [0, 2, 3, 5]
    tasks = [(0, 0), (1, 0), (1, 1), (2, 1), (2, 2)]
    S = 7.0
    o, to, lse, mu = _call_tables(gpu, xs, q_ranges, k_ranges, qk_map, tasks, S)
    allow = torch.zeros(Lq, Lk, dtype=torch.bool)
    allow[0:100, 0:50] = True
    allow[0:100, 90:95] = True
    allow[230:300, 10:20] = True
    allow[230:300, 200:240] = True
    ro, rto, rlse, rmu = om.masked_jvp(*xs, allow, 0.125)
    for a, b in ((slice(0, 100), None), (slice(230, 300), None)):
        assert orc.rel_l2(o[..., a, :], ro[..., a, :]) < 1e-2
        assert orc.rel_l2(to[..., a, :], rto[..., a, :]) < 1e-2
        assert (lse[..., a].double() - rlse[..., a]).abs().max() < 2e-3
    # the group without keys: zeros and -inf, as the reference's epilogue gives
    assert (o[..., 100:230, :] == 0).all() and (to[..., 100:230, :] == 0).all()
    assert (lse[..., 100:230] == -math.inf).all() and (mu[..., 100:230] == 0).all()
    # rows no task covers keep what was there
    assert (o[..., 300:, :] == S).all() and (to[..., 300:, :] == S).all()
    assert (lse[..., 300:] == S).all() and (mu[..., 300:] == S).all()


def test_grad_raises(gpu):
    from dmad_amd import attention

    spec, Q, KV, _ = _spec("block_causal", 16, 3)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    q, k, v, tq, tk, tv = (x.to(gpu) for x in _inputs(1, 1, Q, KV, 64, 64, torch.bfloat16))
    with pytest.raises(RuntimeError, match="MagiMask"):
        attention(q.requires_grad_(), k, v, tq, tk, tv, None, mask)
    with pytest.raises(RuntimeError, match="MagiMask"):
        attention(q.detach(), k, v, tq.requires_grad_(), tk, tv, None, mask)


def test_wan_block_causal_full_width(gpu):
    """A Wan-shaped causal student: 1560-token frames, a 1-frame first block and
    4-frame blocks (3 blocks, Q = KV = 14040), 128-wide heads; rows at every block
    edge and a random sample checked against the oracle."""
    from dmad_amd import attention

    ft, nb = 1560, 3
    spec, Q, KV, allow = _spec("block_causal", ft, nb, first=1, chunk=4)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=gpu)
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    xs = _inputs(1, 2, Q, KV, 128, 128, torch.bfloat16, seed=21)
    o, to = attention(*(x.to(gpu) for x in xs), None, mask)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(0)
    edges = [0, 1, ft - 1, ft, ft + 1, 5 * ft - 1, 5 * ft, Q - 1]
    rows = sorted(set(edges + torch.randint(0, Q, (40,), generator=g).tolist()))
    ro, rto, _, _ = om.masked_jvp_rows(*xs, allow, rows, 128 ** -0.5)
    idx = torch.tensor(rows)
    assert orc.rel_l2(o.cpu()[..., idx, :], ro) < 1e-2
    assert orc.rel_l2(to.cpu()[..., idx, :], rto) < 1e-2


def test_dispatcher(gpu):
    """FlexOrSdpaLocalAttentionWithT on BSHD pairs: no mask -> the dense op; a
    block-causal spec -> the block-sparse op, equal to the oracle's masked JVP."""
    from dmad_amd import FlexOrSdpaLocalAttentionWithT, torch_attention_op_withT

    mod = FlexOrSdpaLocalAttentionWithT()
    spec, Q, KV, allow = _spec("block_causal", 40, 4, chunk=2)
    xs = _inputs(1, 2, Q, KV, 128, 128, torch.bfloat16, seed=17)
    bshd = [x.to(gpu).transpose(1, 2) for x in xs]  # BSHD views, as the Wan callers pass
    pairs = [(bshd[0], bshd[3]), (bshd[1], bshd[4]), (bshd[2], bshd[5])]
    o_d, to_d = mod(*pairs)
    o_r, to_r = torch_attention_op_withT(*pairs)
    o_m, to_m = mod(*pairs, attn_meta=spec)
    torch.cuda.synchronize()
    assert torch.equal(o_d, o_r) and torch.equal(to_d, to_r)
    ro, rto, _, _ = om.masked_jvp(*xs, allow, 128 ** -0.5)
    assert orc.rel_l2(o_m.transpose(1, 2).cpu(), ro) < 1e-2
    assert orc.rel_l2(to_m.transpose(1, 2).cpu(), rto) < 1e-2
    assert not to_m.requires_grad
