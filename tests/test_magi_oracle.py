"""The block-sparse oracle and the host-side mask tables, on the CPU.

* ``oracle.magi.allowed_mask`` against hand-written matrices of small block
  schedules (a wrong block index, an off-by-one in the window or the sink, or a
  missing diagonal fails one of them).
* The range tables built by ``dmad_amd.magimask`` (the reference's
  magimask.py:10-283 restated) describe exactly ``allowed_mask`` for a sweep
  of schedules, the cross-check the reference's own test_jvp_magi relies on
  (flash_attention_jvp_triton.py:871-907).
* ``masked_jvp`` against autodiff of masked math attention, the dense closed
  form, per-row brute force and the empty-row rule.
* ``magi_fwd_emulator`` (the reference kernel's tile walk) equals
  ``masked_jvp`` in float64 without rounding for several BLOCK_N.
"""
import math

import numpy as np
import pytest
import torch

from dmad_amd import magimask as mm
from oracle import attention as orc
from oracle import magi as om


def _t(rows):
    return torch.tensor(rows, dtype=torch.bool)


def test_allowed_mask_block_causal_by_hand():
    # one token per frame, one frame per block: plain causal
    assert torch.equal(om.allowed_mask("block_causal", 1, 4, 4), torch.tril(torch.ones(4, 4, dtype=torch.bool)))
    # two tokens per frame: block lower triangle, full inside a block
    exp = _t([[1, 1, 0, 0, 0, 0], [1, 1, 0, 0, 0, 0], [1, 1, 1, 1, 0, 0], [1, 1, 1, 1, 0, 0],
              [1, 1, 1, 1, 1, 1], [1, 1, 1, 1, 1, 1]])
    assert torch.equal(om.allowed_mask("block_causal", 2, 6, 6), exp)
    # first block 2 frames, then 1-frame blocks (frame_tokens 1): blocks {0,1},{2},{3}
    exp = _t([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 0], [1, 1, 1, 1]])
    assert torch.equal(om.allowed_mask("block_causal", 1, 4, 4, first_chunk_frames=2), exp)
    # window of 2 blocks (the query's and one before)
    exp = _t([[1, 0, 0, 0, 0], [1, 1, 0, 0, 0], [0, 1, 1, 0, 0], [0, 0, 1, 1, 0], [0, 0, 0, 1, 1]])
    assert torch.equal(om.allowed_mask("block_causal", 1, 5, 5, local_attn_blocks=2), exp)
    # the same window plus a one-block sink
    exp = _t([[1, 0, 0, 0, 0], [1, 1, 0, 0, 0], [1, 1, 1, 0, 0], [1, 0, 1, 1, 0], [1, 0, 0, 1, 1]])
    assert torch.equal(om.allowed_mask("block_causal", 1, 5, 5, local_attn_blocks=2, sink_blocks=1), exp)
    # queries start at block 2 of the schedule (cache offset): keys of blocks 0..2 for query block 0
    exp = _t([[1, 1, 1, 0], [1, 1, 1, 1]])
    assert torch.equal(om.allowed_mask("block_causal", 1, 2, 4, q_block_offset=2), exp)


def test_allowed_mask_teacher_forcing_by_hand():
    # clean tokens 0,1 (blocks 0,1), noisy tokens 2,3 (blocks 0,1)
    exp = _t([[1, 0, 0, 0], [1, 1, 0, 0], [0, 0, 1, 0], [1, 0, 0, 1]])
    assert torch.equal(om.allowed_mask("teacher_forcing", 1, 4, 4, clean_blocks=2), exp)
    # three clean blocks, window 2, sink 1
    got = om.allowed_mask("teacher_forcing", 1, 6, 6, clean_blocks=3, local_attn_blocks=2, sink_blocks=1)
    exp = _t([[1, 0, 0, 0, 0, 0],
              [1, 1, 0, 0, 0, 0],
              [1, 1, 1, 0, 0, 0],
              [0, 0, 0, 1, 0, 0],
              [1, 0, 0, 0, 1, 0],
              [1, 1, 0, 0, 0, 1]])
    assert torch.equal(got, exp)


def _spec_mask(mode, ft, nb, first=1, chunk=1, local=0, sink=0, q_bo=0):
    pat = mm.BlockPattern(frame_tokens=ft, first_chunk_frames=first, chunk_frames=chunk)
    if mode == "block_causal":
        KV = pat.blocks_to_tokens(q_bo + nb)
        Q = KV - pat.blocks_to_tokens(q_bo) if q_bo else KV
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, q_block_offset=q_bo, local_attn_blocks=local, sink_blocks=sink)
        ref = om.allowed_mask(mode, ft, Q, KV, first, chunk, q_block_offset=q_bo, local_attn_blocks=local,
                              sink_blocks=sink)
    else:
        Q = KV = 2 * pat.blocks_to_tokens(nb)
        spec = mm.AttnMaskSpec(mode=mode, pattern=pat, clean_blocks=nb, local_attn_blocks=local, sink_blocks=sink)
        ref = om.allowed_mask(mode, ft, Q, KV, first, chunk, local_attn_blocks=local, sink_blocks=sink,
                              clean_blocks=nb, as_range_builder=True)
    return spec, Q, KV, ref


SWEEP = [
    (mode, ft, nb, first, chunk, local, sink)
    for mode in ("block_causal", "teacher_forcing")
    for ft, nb, first, chunk in ((1, 5, 1, 1), (3, 4, 1, 2), (5, 3, 2, 1), (16, 4, 1, 1), (7, 6, 1, 3))
    for local, sink in ((0, 0), (3, 1), (2, 0), (2, 2), (1, 0), (1, 1), (1, 2))
]


@pytest.mark.parametrize("mode,ft,nb,first,chunk,local,sink", SWEEP)
@pytest.mark.parametrize("block_m", [64, 128])
def test_tables_describe_the_mask(mode, ft, nb, first, chunk, local, sink, block_m):
    spec, Q, KV, ref = _spec_mask(mode, ft, nb, first, chunk, local, sink)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=block_m)
    dense = mm.csr_to_dense(mask.q_unique, mask.k_flat, mask.qk_map, Q, KV)
    if mode == "teacher_forcing":
        # the reference's boolean oracle ORs in the diagonal, which the noisy
        # block's own rectangle and the causal clean rectangles already hold
        assert torch.equal(dense | torch.eye(Q, KV, dtype=torch.bool), dense)
    assert torch.equal(dense, ref)
    # CSR invariants: groups partition [0, Q), ranges per group sorted, disjoint, non-touching
    qu = mask.q_unique.numpy()
    assert qu[0, 0] == 0 and qu[-1, 1] == Q and (qu[1:, 0] == qu[:-1, 1]).all()
    qm, kf = mask.qk_map.numpy(), mask.k_flat.numpy()
    for g in range(mask.G):
        segs = kf[qm[g]:qm[g + 1]]
        assert len(segs) >= 1 and (segs[:, 1] > segs[:, 0]).all()
        assert (segs[1:, 0] > segs[:-1, 1]).all()
    # tasks: exactly the (group, tile) pairs that intersect, in group order
    exp = [(g, t) for g in range(mask.G) for t in range(Q // block_m + 1)
           if max(qu[g, 0], t * block_m) < min(qu[g, 1], (t + 1) * block_m)]
    assert list(zip(mask.task_group.tolist(), mask.task_qtile.tolist())) == exp
    assert mask.T == len(exp) and mask.BLOCK_M == block_m


def test_block_causal_with_query_offset():
    spec, Q, KV, ref = _spec_mask("block_causal", 4, 3, first=1, chunk=2, q_bo=2)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    assert torch.equal(mm.csr_to_dense(mask.q_unique, mask.k_flat, mask.qk_map, Q, KV), ref)


@pytest.mark.parametrize("first,chunk,sink", [(1, 1, 1), (2, 1, 2), (1, 2, 1), (1, 3, 3)])
def test_one_block_window_noisy_sink(first, chunk, sink):
    """Teacher forcing with a 1-block window and a sink: the reference's test mask
    and its range builder differ by exactly the rectangles noisy block i (i >= 1)
    x clean keys [0, end of block min(sink, i)), which only the test mask grants."""
    ft, nb = 3, 4
    pat = mm.BlockPattern(frame_tokens=ft, first_chunk_frames=first, chunk_frames=chunk)
    clean = pat.blocks_to_tokens(nb)
    Q = KV = 2 * clean
    kw = dict(local_attn_blocks=1, sink_blocks=sink, clean_blocks=nb)
    test_mask = om.allowed_mask("teacher_forcing", ft, Q, KV, first, chunk, **kw)
    builder = om.allowed_mask("teacher_forcing", ft, Q, KV, first, chunk, as_range_builder=True, **kw)
    expect = torch.zeros(Q, KV, dtype=torch.bool)
    for i in range(1, nb):
        q0, q1 = clean + pat.blocks_to_tokens(i), clean + pat.blocks_to_tokens(i + 1)
        expect[q0:q1, :pat.blocks_to_tokens(min(sink, i))] = True
    assert torch.equal(test_mask & ~builder, expect) and not (builder & ~test_mask).any()
    spec = mm.AttnMaskSpec(mode="teacher_forcing", pattern=pat, **kw)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
    assert torch.equal(mm.csr_to_dense(mask.q_unique, mask.k_flat, mask.qk_map, Q, KV), builder)


def test_merge_clips_sorts_and_merges():
    qr = torch.tensor([[5, 9], [0, 5], [5, 9], [0, 5], [5, 9], [0, 5]], dtype=torch.int32)
    kr = torch.tensor([[8, 12], [-3, 2], [0, 3], [2, 4], [3, 5], [20, 30]], dtype=torch.int32)
    q2, k2 = mm.merge_k_ranges(qr, kr, KV_real=10)
    assert q2.tolist() == [[0, 5], [5, 9], [5, 9]]
    assert k2.tolist() == [[0, 4], [0, 5], [8, 10]]
    qu, kf, qm = mm.group_q_ranges_csr(q2, k2)
    assert qu.tolist() == [[0, 5], [5, 9]] and qm.tolist() == [0, 1, 3]
    with pytest.raises(AssertionError):
        mm.merge_k_ranges(torch.tensor([[0, 4]]), torch.tensor([[12, 14]]), KV_real=10)
    with pytest.raises(AssertionError):
        mm.prepare_magi_csr_and_tasks(torch.tensor([[0, 4], [5, 8]]), torch.tensor([[0, 1], [0, 1]]), 8, 8)


@pytest.mark.parametrize("seed", range(24))
def test_random_rectangles_build_their_mask(seed):
    """Random overlapping / touching / out-of-range key ranges: the generator's mask
    is the element-wise union of the raw rectangles, and the CSR tables the builder
    makes from the shuffled rows describe exactly that mask."""
    g = np.random.default_rng(1000 + seed)
    Q, KV = int(g.integers(1, 300)), int(g.integers(1, 300))
    qr, kr, allow = om.random_rectangles(seed, Q, KV)
    qi, kj = np.arange(Q)[None, :, None], np.arange(KV)[None, None, :]
    q0, q1 = qr[:, 0].numpy()[:, None, None], qr[:, 1].numpy()[:, None, None]
    k0, k1 = kr[:, 0].numpy()[:, None, None], kr[:, 1].numpy()[:, None, None]
    member = ((qi >= q0) & (qi < q1) & (kj >= k0) & (kj < k1)).any(0)
    assert np.array_equal(allow.numpy(), member)
    assert allow.any(1).all()  # every query row has a key
    for block_m in (64, 128):
        mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV, BLOCK_M=block_m)
        assert torch.equal(mm.csr_to_dense(mask.q_unique, mask.k_flat, mask.qk_map, Q, KV), allow)
        qm, kf = mask.qk_map.numpy(), mask.k_flat.numpy()
        for grp in range(mask.G):
            segs = kf[qm[grp]:qm[grp + 1]]
            assert (segs[:, 0] >= 0).all() and (segs[:, 1] <= KV).all() and (segs[1:, 0] > segs[:-1, 1]).all()


def test_tasks_for_kernel_rebuilds_other_block_m():
    spec, Q, KV, _ = _spec_mask("block_causal", 40, 5, chunk=2)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    m64 = mm.prepare_magi_csr_and_tasks(qr, kr, Q, KV, BLOCK_M=64)
    m128 = mm.prepare_magi_csr_and_tasks(qr, kr, Q, KV, BLOCK_M=128)
    tg, tq, T = mm.tasks_for_kernel(m64, Q, torch.device("cpu"))
    assert T == m128.T and torch.equal(tg, m128.task_group) and torch.equal(tq, m128.task_qtile)
    assert mm.tasks_for_kernel(m64, Q, torch.device("cpu"))[0] is tg  # cached per mask object


def _rand(shape, seed, dtype=torch.float64):
    B, H, Lq, Lk, Dqk, Dv = shape
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=dtype) * 0.5  # noqa: E731
    return (r(B, H, Lq, Dqk), r(B, H, Lk, Dqk), r(B, H, Lk, Dv), r(B, H, Lq, Dqk), r(B, H, Lk, Dqk), r(B, H, Lk, Dv))


def _masked_autodiff(q, k, v, tq, tk, tv, allow, s):
    def f(a, b, c):
        S = torch.matmul(a, b.transpose(-1, -2)) * s
        S = S.masked_fill(~allow, -math.inf)
        return torch.matmul(torch.softmax(S, -1), c)
    return torch.func.jvp(f, (q, k, v), (tq, tk, tv))


def test_masked_jvp_matches_autodiff():
    xs = _rand((2, 2, 24, 24, 16, 8), 1)
    allow = om.allowed_mask("teacher_forcing", 3, 24, 24, chunk_frames=1, clean_blocks=4, local_attn_blocks=2)
    o, to, lse, mu = om.masked_jvp(*xs, allow, 0.4)
    ro, rto = _masked_autodiff(*xs, allow, 0.4)
    assert torch.allclose(o, ro, atol=1e-12) and torch.allclose(to, rto, atol=1e-12)


def test_masked_jvp_all_allowed_is_dense():
    xs = _rand((1, 2, 17, 29, 16, 16), 2)
    o, to, lse, mu = om.masked_jvp(*xs, torch.ones(17, 29, dtype=torch.bool), 0.3)
    ro, rto, rlse, rmu = orc.jvp_closed_form(*xs, sm_scale=0.3)
    for a, b in ((o, ro), (to, rto), (lse, rlse), (mu, rmu)):
        assert torch.allclose(a, b, atol=1e-12)


def test_masked_jvp_brute_force_rows_and_empty_rows():
    q, k, v, tq, tk, tv = _rand((1, 1, 5, 6, 4, 3), 3)
    allow = _t([[1, 0, 1, 0, 0, 0], [0, 0, 0, 0, 0, 0], [1, 1, 1, 1, 1, 1], [0, 0, 0, 0, 0, 1], [0, 1, 0, 1, 0, 1]])
    o, to, lse, mu = om.masked_jvp(q, k, v, tq, tk, tv, allow, 0.7)
    for i in range(5):
        keys = [j for j in range(6) if allow[i, j]]
        if not keys:
            assert lse[0, 0, i] == -math.inf and mu[0, 0, i] == 0
            assert (o[0, 0, i] == 0).all() and (to[0, 0, i] == 0).all()
            continue
        sc = [0.7 * float(q[0, 0, i] @ k[0, 0, j]) for j in keys]
        sd = [0.7 * float(tq[0, 0, i] @ k[0, 0, j] + q[0, 0, i] @ tk[0, 0, j]) for j in keys]
        mx = max(sc)
        e = [math.exp(x - mx) for x in sc]
        z = sum(e)
        p = [x / z for x in e]
        m = sum(pi * di for pi, di in zip(p, sd))
        ro = sum(pi * v[0, 0, j] for pi, j in zip(p, keys))
        rto = sum(pi * tv[0, 0, j] + pi * (di - m) * v[0, 0, j] for pi, di, j in zip(p, sd, keys))
        assert abs(float(lse[0, 0, i]) - (mx + math.log(z))) < 1e-12 and abs(float(mu[0, 0, i]) - m) < 1e-12
        assert torch.allclose(o[0, 0, i], ro, atol=1e-12) and torch.allclose(to[0, 0, i], rto, atol=1e-12)


@pytest.mark.parametrize("block_n", [16, 32, 64])
@pytest.mark.parametrize("mode", ["block_causal", "teacher_forcing"])
def test_emulator_without_rounding_is_the_masked_closed_form(block_n, mode):
    spec, Q, KV, allow = _spec_mask(mode, 7, 4, chunk=2, local=2, sink=1)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q, KV)
    xs = _rand((1, 2, Q, KV, 16, 8), 4)
    eo, eto, else_ = om.magi_fwd_emulator(*xs, mask.q_unique, mask.k_flat, mask.qk_map, 0.5, block_n=block_n,
                                         round_dtype=None)
    o, to, lse, _ = om.masked_jvp(*xs, allow, 0.5)
    assert torch.allclose(eo, o, atol=1e-12) and torch.allclose(eto, to, atol=1e-12)
    assert torch.allclose(else_, lse, atol=1e-12)


def test_emulator_bf16_within_reference_tolerance():
    spec, Q, KV, allow = _spec_mask("block_causal", 16, 4)
    qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device="cpu")
    mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q, KV, BLOCK_M=64)
    xs = [x.to(torch.bfloat16) for x in _rand((1, 2, Q, KV, 64, 64), 42)]
    eo, eto, _ = om.magi_fwd_emulator(*xs, mask.q_unique, mask.k_flat, mask.qk_map, 64 ** -0.5)
    o, to, _, _ = om.masked_jvp(*xs, allow, 64 ** -0.5)
    torch.testing.assert_close(eo.to(torch.bfloat16).double(), o, atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(eto.to(torch.bfloat16).double(), to, atol=2e-2, rtol=1e-2)


def test_dispatcher_decision_and_cache():
    """FlexOrSdpaLocalAttentionWithT's dense/masked decision (jvp_helper.py:251-263) and its mask cache."""
    from dmad_amd.jvp_helper import FlexOrSdpaLocalAttentionWithT, needs_block_mask

    pat = mm.BlockPattern(frame_tokens=16, first_chunk_frames=1, chunk_frames=2)
    assert not needs_block_mask(None, 64, 64)
    assert not needs_block_mask(mm.AttnMaskSpec(mode="none"), 64, 64)
    # one query block (block 1 = 32 tokens) over keys of blocks 0..1 (48 tokens): dense
    one = mm.AttnMaskSpec(mode="block_causal", pattern=pat, q_block_offset=1)
    assert not needs_block_mask(one, 32, 48)
    assert needs_block_mask(one, 32, 49) and needs_block_mask(one, 64, 48)
    # a sliding window always needs the mask
    assert needs_block_mask(mm.AttnMaskSpec(mode="block_causal", pattern=pat, q_block_offset=1, local_attn_blocks=1),
                            32, 48)
    assert needs_block_mask(mm.AttnMaskSpec(mode="teacher_forcing", pattern=pat, clean_blocks=2), 96, 96)
    mod = FlexOrSdpaLocalAttentionWithT()
    spec = mm.AttnMaskSpec(mode="block_causal", pattern=pat)
    a = mod.get_magi_mask(spec, 80, 80, "cpu")
    assert mod.get_magi_mask(spec, 80, 80, "cpu") is a and a.BLOCK_M == 128
    assert mod.get_magi_mask(spec, 48, 48, "cpu") is not a
    mod.clear_cache()
    assert mod.get_magi_mask(spec, 80, 80, "cpu") is not a
