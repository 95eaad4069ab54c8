"""The per-shape launch table (dmad_attn_fwd_plan / dmad_attn_bwd_plan), on the CPU.

The reference autotunes its Triton forward over 48 configs keyed on (SEQ_LEN_Q,
SEQ_LEN_KV, HEAD_DIM_QK, HEAD_DIM_V) (train/wan/rcm/utils/flash_attention_jvp_triton.py:98-107).
The library instead picks from a fixed table keyed on the dtype, the mode, the mask, Lq, Lk and
the head dims; the entry points launch what the plan query reports (one function decides both).
These tests pin the table: the Wan shapes, the reference's harness and test shapes, every head
dim, fp32, the block-sparse forward, the backward passes, the workspace sizes (equal to the
workspace queries) and the argument checks.
"""
import pytest
import torch

from dmad_amd import _native as nat

BF16, F16, F32 = nat.DMAD_BF16, nat.DMAD_F16, nat.DMAD_F32
PLAIN, JVP, QONLY = nat.DMAD_FWD_PLAIN, nat.DMAD_FWD_JVP, nat.DMAD_FWD_JVP_KV_TANGENT_ZERO


def test_wan_shapes():
    # 14B self-attention: row-reading 32-query-wave kernel, head-major order (256 tiles per head), no workspace
    p = nat.fwd_plan(BF16, JVP, 1, 40, 32760, 32760, 128, 128)
    assert (p["kernel"], p["grid"], p["xcd_order"], p["chunks"], p["workspace_bytes"]) == \
        ("attn_fwd32_kernel", 256 * 40, 0, 1, 0)
    # text cross-attention (512 keys, Kd = Vd = 0), 14B and 1.3B: two workgroups per CU
    for H in (40, 12):
        p = nat.fwd_plan(BF16, QONLY, 1, H, 32760, 512, 128, 128)
        assert (p["kernel"], p["grid"], p["transposed_copies"]) == ("attn_fwd32_x2_kernel", 256 * H, 0)
    # 720p: 591 tiles per head
    p = nat.fwd_plan(BF16, JVP, 1, 40, 75600, 75600, 128, 128)
    assert (p["kernel"], p["grid"], p["xcd_order"]) == ("attn_fwd32_kernel", 591 * 40, 0)


@pytest.mark.parametrize("Lk,kernel", [(1, "attn_fwd32_x2_kernel"), (2048, "attn_fwd32_x2_kernel"),
                                       (2049, "attn_fwd32_kernel"), (32760, "attn_fwd32_kernel")])
def test_short_key_kernel_is_keyed_on_lk(Lk, kernel):
    """Kd = Vd = 0 with 128-wide heads: at most 64 key tiles run two workgroups per CU."""
    for dt in (BF16, F16):
        assert nat.fwd_plan(dt, QONLY, 1, 40, 32760, Lk, 128, 128)["kernel"] == kernel
    # the other modes and head dims never take it
    assert nat.fwd_plan(BF16, JVP, 1, 40, 32760, Lk, 128, 128)["kernel"] == "attn_fwd32_kernel"
    assert nat.fwd_plan(BF16, PLAIN, 1, 40, 32760, Lk, 128, 128)["kernel"] == "attn_fwd32_kernel"
    assert nat.fwd_plan(BF16, QONLY, 1, 40, 32760, Lk, 64, 64)["kernel"] == "attn_fwd32_kernel"


@pytest.mark.parametrize("L,xcd", [(1024, 1), (4096, 1), (16384, 1), (32640, 1), (32768, 0)])
@pytest.mark.parametrize("D", [64, 128])
def test_block_order_is_keyed_on_query_tiles(L, xcd, D):
    """The reference harness shape (B=4, H=32): fewer than 256 query tiles per head deal each
    XCD a contiguous range of work items; from 256 on the order is head-major."""
    p = nat.fwd_plan(F16, JVP, 4, 32, L, L, D, D)
    assert (p["kernel"], p["grid"], p["xcd_order"]) == ("attn_fwd32_kernel", (L + 127) // 128 * 128, xcd)
    b = nat.bwd_plan(F16, 4, 32, L, L, D)
    assert (b["kernel"], b["kernel2"]) == ("attn_bwd_kv_tr_kernel", "attn_bwd_dq_tr_kernel")
    assert (b["xcd_order"], b["xcd_order2"]) == (xcd, xcd)


@pytest.mark.parametrize("D,kernel,chunks", [(16, "attn_fwd_simple_kernel", 1), (32, "attn_fwd_kernel", 1)])
def test_generic_head_dims(D, kernel, chunks):
    """Head dims the row-reading kernels do not take run on transposed copies of V (and Vd)."""
    p = nat.fwd_plan(F16, JVP, 4, 32, 4096, 4096, D, D)
    assert (p["kernel"], p["chunks"], p["transposed_copies"]) == (kernel, chunks, 2)
    assert p["grid"] == 32 * 128 * chunks
    assert p["workspace_bytes"] == nat.fwd_workspace_bytes(JVP, 4, 32, 4096, D, D) > 0
    assert nat.fwd_plan(F16, PLAIN, 4, 32, 4096, 4096, D, D)["transposed_copies"] == 1


@pytest.mark.parametrize("mode", [PLAIN, JVP, QONLY])
@pytest.mark.parametrize("dt", [BF16, F16])
def test_wide_heads_on_the_row_kernel(mode, dt):
    """256-wide heads, dense and block-sparse: the row-reading kernel (JVP modes: one workgroup
    per 128-column chunk of V, per query tile or task), V read in place (no workspace)."""
    p = nat.fwd_plan(dt, mode, 4, 32, 4096, 4096, 256, 256)
    chunks = 1 if mode == PLAIN else 2  # the plain forward keeps all 256 columns in one workgroup
    assert (p["kernel"], p["chunks"], p["transposed_copies"], p["workspace_bytes"]) == \
        ("attn_fwd32_kernel", chunks, 0, 0)
    assert p["grid"] == (4096 // 128) * 4 * 32 * chunks  # query tiles x B x H x chunks
    assert nat.fwd_workspace_bytes(mode, 4, 32, 4096, 256, 256) == 0
    if mode != PLAIN:
        pm = nat.fwd_plan(dt, mode, 1, 2, 1000, 1000, 256, 256, magi_tasks=20)
        assert (pm["kernel"], pm["chunks"], pm["grid"], pm["transposed_copies"], pm["workspace_bytes"]) == \
            ("attn_fwd32_kernel", 2, 20 * 2 * 2, 0, 0)
    # mixed widths stay on the generic kernels
    assert nat.fwd_plan(dt, mode, 1, 2, 1000, 1000, 128, 256)["kernel"] != "attn_fwd32_kernel"
    assert nat.fwd_plan(dt, mode, 1, 2, 1000, 1000, 256, 128)["kernel"] != "attn_fwd32_kernel"


def test_mixed_head_dims():
    # Dqk != Dv: the reference's _test_jvp_ca shapes
    p = nat.fwd_plan(F16, JVP, 1, 2, 1024, 512, 128, 64)
    assert p["transposed_copies"] == 2 and p["kernel"] != "attn_fwd32_kernel"
    assert nat.fwd_plan(F16, JVP, 1, 2, 1024, 512, 64, 64)["kernel"] == "attn_fwd32_kernel"


def test_block_sparse_forward():
    for D, kernel in ((128, "attn_fwd32_kernel"), (64, "attn_fwd32_kernel"), (32, "attn_fwd_simple_kernel")):
        p = nat.fwd_plan(BF16, JVP, 1, 40, 24960, 32760, D, D, magi_tasks=198)
        assert (p["kernel"], p["grid"], p["xcd_order"]) == (kernel, 198 * 40, 1)
    # Kd = Vd = 0 with a mask stays on the block-sparse kernel
    assert nat.fwd_plan(BF16, QONLY, 1, 40, 24960, 512, 128, 128, magi_tasks=198)["kernel"] == "attn_fwd32_kernel"
    with pytest.raises(ValueError):
        nat.fwd_plan(BF16, PLAIN, 1, 40, 24960, 512, 128, 128, magi_tasks=198)


# (Dqk, Dv, V chunks, query rows per workgroup): 256-wide Q, K in the JVP modes run
# four waves of 16 queries (one per SIMD) with all of V in one workgroup
@pytest.mark.parametrize("Dqk,Dv,chunks,bm", [(64, 64, 1, 128), (128, 128, 1, 128), (256, 256, 1, 64),
                                              (256, 128, 1, 64), (128, 256, 2, 128), (16, 32, 1, 128)])
def test_fp32_forward(Dqk, Dv, chunks, bm):
    for mode in (JVP, QONLY):
        p = nat.fwd_plan(F32, mode, 4, 32, 4096, 4096, Dqk, Dv)
        assert (p["kernel"], p["chunks"], p["grid"], p["transposed_copies"], p["workspace_bytes"]) == \
            ("attn_f32_fwd_kernel", chunks, (4096 // bm) * 128 * chunks, 0, 0)
    # the plain forward takes all of V (up to 256 columns) in one workgroup at every Q, K width
    p = nat.fwd_plan(F32, PLAIN, 4, 32, 4096, 4096, Dqk, Dv)
    assert (p["chunks"], p["grid"]) == (1, 32 * 128)
    # block-sparse: 128-query tasks, each 128 // bm workgroups
    m = nat.fwd_plan(F32, JVP, 1, 40, 24960, 32760, Dqk, Dv, magi_tasks=198)
    assert (m["chunks"], m["grid"]) == (chunks, 198 * (128 // bm) * 40 * chunks)


def test_backward_passes():
    # dO-only, 64- and 128-wide heads: row-reading passes, statistics only
    for D in (64, 128):
        b = nat.bwd_plan(BF16, 1, 40, 32760, 32760, D)
        assert (b["kernel"], b["kernel2"], b["kernel3"], b["kernel4"]) == \
            ("attn_bwd_kv_tr_kernel", "attn_bwd_dq_tr_kernel", None, None)
        assert (b["grid"], b["grid2"], b["transposed_copies"]) == (256 * 40, 256 * 40, 0)
    # the full derivative of 128-wide heads (its query pass gives dQd)
    b = nat.bwd_plan(BF16, 1, 40, 32760, 32760, 128, full=True, tangent_grads=True)
    assert (b["kernel"], b["kernel2"], b["kernel3"], b["kernel4"]) == \
        ("attn_bwd_kv_full_kernel", "attn_bwd_dq_full_kernel", "attn_bwd_kv_tr_kernel", None)
    assert b["transposed_copies"] == 0
    # the full derivative of the other head dims: generic passes on six transposed copies
    b = nat.bwd_plan(F16, 1, 2, 1024, 1024, 64, full=True, tangent_grads=True)
    assert (b["kernel"], b["kernel2"], b["kernel3"], b["kernel4"]) == \
        ("attn_bwd_kernel", "attn_bwd_dq_kernel", "attn_bwd_kv_tr_kernel", "attn_bwd_dq_tr_kernel")
    assert b["transposed_copies"] == 6
    # dO-only for the generic head dims: Q^T, dO^T and K^T copies (K^T only for a generic dQ pass)
    assert nat.bwd_plan(F16, 4, 32, 4096, 4096, 32)["kernel"] == "attn_bwd_kv_pipe_kernel"
    assert nat.bwd_plan(F16, 4, 32, 4096, 4096, 32)["kernel2"] == "attn_bwd_dq_pipe_kernel"
    b = nat.bwd_plan(F16, 4, 32, 4096, 4096, 16)
    assert (b["kernel"], b["kernel2"], b["transposed_copies"]) == ("attn_bwd_kernel", "attn_bwd_dq_kernel", 3)
    # 256: generic dK/dV pass on Q^T, dO^T copies; the dQ pass reads K row-major
    b = nat.bwd_plan(F16, 4, 32, 4096, 4096, 256)
    assert (b["kernel"], b["kernel2"], b["transposed_copies"]) == ("attn_bwd_kernel", "attn_bwd_dq_tr_kernel", 2)
    assert b["workspace_bytes"] == nat.bwd_workspace_bytes(0, 4, 32, 4096, 4096, 256)
    # fp32 (dO only): 64-key / 64-query workgroups at D = 256, 128 otherwise
    b = nat.bwd_plan(F32, 4, 32, 4096, 4096, 256)
    assert (b["kernel"], b["kernel2"], b["grid"], b["grid2"]) == \
        ("attn_f32_bwd_kv_kernel", "attn_f32_bwd_dq_kernel", 64 * 128, 64 * 128)
    assert nat.bwd_plan(F32, 4, 32, 4096, 4096, 128)["grid"] == 32 * 128


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_fp32_backward_workspace_is_the_statistics(D):
    # fp32 passes read Q, dO, K in place: the workspace holds only the log2 LSE and D per
    # query row, [B*H][round_up(Lq, 64)] floats each (4 MiB at B=4, H=32, L=4096)
    b = nat.bwd_plan(F32, 4, 32, 4096, 4096, D)
    assert (b["workspace_bytes"], b["transposed_copies"]) == (4 * 32 * 4096 * 2 * 4, 0)
    assert nat.bwd_plan(F32, 1, 3, 999, 515, D)["workspace_bytes"] == (3 * 1024 * 8 + 255) // 256 * 256
    # the dtype-free query bounds it (it sizes bf16/fp16 operands)
    assert b["workspace_bytes"] <= nat.bwd_workspace_bytes(0, 4, 32, 4096, 4096, D)


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("Lq,Lk", [(999, 515), (32760, 512), (1, 1)])
def test_workspace_matches_the_queries(D, Lq, Lk):
    for mode in (PLAIN, JVP, QONLY):
        # the query covers every forward entry; the dense row kernel at D = 256 needs none of it
        want = 0 if D == 256 else nat.fwd_workspace_bytes(mode, 2, 3, Lk, D, D)
        assert nat.fwd_plan(BF16, mode, 2, 3, Lq, Lk, D, D)["workspace_bytes"] == want
    fulls = ((0, False), (1, False), (2, True)) if D <= 128 else ((0, False),)
    for full, tg in fulls:
        assert nat.bwd_plan(BF16, 2, 3, Lq, Lk, D, full=full > 0, tangent_grads=tg)["workspace_bytes"] == \
            nat.bwd_workspace_bytes(full, 2, 3, Lq, Lk, D)


def test_argument_checks():
    with pytest.raises(ValueError):
        nat.fwd_plan(BF16, JVP, 1, 2, 64, 64, 96, 96)  # head dim outside {16, 32, 64, 128, 256}
    with pytest.raises(ValueError):
        nat.fwd_plan(BF16, 7, 1, 2, 64, 64, 64, 64)
    with pytest.raises(ValueError):
        nat.fwd_plan(BF16, JVP, -1, 2, 64, 64, 64, 64)
    with pytest.raises(NotImplementedError):
        nat.fwd_plan(9, JVP, 1, 2, 64, 64, 64, 64)
    with pytest.raises(NotImplementedError):
        nat.bwd_plan(BF16, 1, 2, 64, 64, 256, full=True)
    with pytest.raises(NotImplementedError):
        nat.bwd_plan(F32, 1, 2, 64, 64, 64, full=True)
    with pytest.raises(ValueError):
        nat.bwd_plan(BF16, 1, 2, 64, 64, 64, tangent_grads=True)


def test_stored_score_sizes():
    """Bytes per (b, h) slice of stored score gradients: dS (and dSd) in bf16/fp16 over Lq
    rounded up to 128 queries and the key pass's 128-key tiles, one strip per 128-query block
    padded by 20 KiB; none for other head dims and fp32."""
    def size(lq, lk, nt):
        strip = (lk + 127) // 128 * 128 * 128 * 2 * nt + 20480
        return -(-((lq + 127) // 128 * strip) // 256) * 256

    gib = 1 << 30
    for dt in (BF16, F16):
        assert nat.bwd_score_bytes(dt, False, 32760, 32760, 128) == size(32760, 32760, 1) == 2 * gib + 256 * 20480
        assert nat.bwd_score_bytes(dt, True, 32760, 32760, 128) == size(32760, 32760, 2) == 4 * gib + 256 * 20480
        assert nat.bwd_score_bytes(dt, False, 1, 1, 128) == 128 * 128 * 2 + 20480
        assert nat.bwd_score_bytes(dt, True, 300, 700, 128) == size(300, 700, 2) == 384 * 768 * 2 * 2 + 3 * 20480
    assert nat.bwd_score_bytes(F32, False, 4096, 4096, 128) == 0
    for D in (16, 32, 64, 256):
        assert nat.bwd_score_bytes(BF16, False, 4096, 4096, D) == 0


@pytest.mark.parametrize("full", [False, True])
def test_stored_score_plan_follows_the_workspace(full):
    """dmad_attn_bwd_plan_ws: whole score slices beyond the minimum workspace select the
    stored-score passes, as many (b, h) slices per launch pair as fit (at most B*H)."""
    B, H, L = 1, 40, 32760
    base = nat.bwd_plan(BF16, B, H, L, L, 128, full=full, tangent_grads=full)
    one = nat.bwd_score_bytes(BF16, full, L, L, 128)
    p = nat.bwd_plan(BF16, B, H, L, L, 128, full=full, tangent_grads=full,
                     workspace_bytes=base["workspace_bytes"] + 3 * one + one // 2)
    assert p["score_slices"] == 3
    assert p["kernel"] == ("attn_bwd_kv_full_kernel<store>" if full else "attn_bwd_kv_tr_kernel<store>")
    assert p["kernel2"] == "attn_bwd_dq_sc_kernel"
    assert (p["grid"], p["grid2"]) == (3 * 256, 3 * 128)  # two 128-query blocks per query-pass workgroup
    assert p["workspace_bytes"] == base["workspace_bytes"] + 3 * one
    # with tangent gradients the tangent key pass runs in every pair, on the stored dSd
    assert p["kernel3"] == ("attn_bwd_kv_tr_kernel<load>" if full else None)
    # the minimum workspace, or less than one slice beyond it, keeps the recomputing passes
    for extra in (0, one - 256):
        q = nat.bwd_plan(BF16, B, H, L, L, 128, full=full, tangent_grads=full,
                         workspace_bytes=base["workspace_bytes"] + extra)
        assert q["score_slices"] == 0 and q["kernel2"] == base["kernel2"]
    # more room than B*H slices: all of them in one pair
    p = nat.bwd_plan(BF16, B, H, L, L, 128, full=full, tangent_grads=full,
                     workspace_bytes=base["workspace_bytes"] + 100 * one)
    assert p["score_slices"] == 40
    # no stored-score path for fp32 or other head dims
    for dt, D in ((F32, 128), (BF16, 64)):
        if dt == F32 and full:
            continue
        q = nat.bwd_plan(dt, B, H, L, L, D, full=full, tangent_grads=full, workspace_bytes=1 << 50)
        assert q["score_slices"] == 0


def test_python_score_budget():
    """The op's workspace: whole slices within the process budget (0 turns the path off)."""
    from dmad_amd import jvp_attention as ja

    one = nat.bwd_score_bytes(BF16, False, 32760, 32760, 128)
    old = ja.backward_score_budget()
    try:
        ja.set_backward_score_budget(18 << 30)
        assert ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 128) == 8 * one
        assert ja._score_bytes(BF16, True, 1, 40, 32760, 32760, 128) == \
            4 * nat.bwd_score_bytes(BF16, True, 32760, 32760, 128)
        # 7 slices fit in 16 GiB, but pairs of 7 leave the query pass's last round half
        # empty (896 workgroups); pairs of 6 fill it (768, and a last pair of 4: 512)
        ja.set_backward_score_budget(16 << 30)
        assert ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 128) == 6 * one
        assert ja._score_slices(40, 8, 32760, 32760) == 8
        ja.set_backward_score_budget(0)
        assert ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 128) == 0
        ja.set_backward_score_budget(one - 1)
        assert ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 128) == 0
        ja.set_backward_score_budget(1 << 50)
        assert ja._score_bytes(BF16, True, 2, 3, 300, 300, 128) == 6 * nat.bwd_score_bytes(BF16, True, 300, 300, 128)
        # the dO-only backward keeps the recomputing passes below 2048 queries or keys
        assert ja._score_bytes(BF16, False, 2, 3, 300, 300, 128) == 0
        assert ja._score_bytes(BF16, False, 1, 2, 4096, 2047, 128) == 0
        assert ja._score_bytes(BF16, False, 1, 2, 2048, 2048, 128) == 2 * nat.bwd_score_bytes(BF16, False, 2048, 2048, 128)
        assert ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 64) == 0
        # a pair of fewer than B*H slices keeps at least four key-pass workgroups per CU
        one720 = nat.bwd_score_bytes(BF16, False, 75600, 75600, 128)
        ja.set_backward_score_budget(18 << 30)  # one 11.4 GB slice: 591 workgroups per pair
        assert ja._score_bytes(BF16, False, 1, 40, 75600, 75600, 128) == 0
        ja.set_backward_score_budget(2 * one720)  # 1182 workgroups per pair
        assert ja._score_bytes(BF16, False, 1, 40, 75600, 75600, 128) == 2 * one720
        ja.set_backward_score_budget(one720)  # one slice, but it is all of them
        assert ja._score_bytes(BF16, False, 1, 1, 75600, 75600, 128) == one720
        with pytest.raises(ValueError):
            ja.set_backward_score_budget(-1)
    finally:
        ja.set_backward_score_budget(old)


def test_backward_workspace_falls_back_to_the_minimum(monkeypatch):
    """The stored score gradients are a speed-up: when the device cannot hold them the
    backward takes its minimum workspace (the recomputing query pass); a failure to
    allocate the minimum itself is not hidden."""
    from dmad_amd import jvp_attention as ja

    base = nat.bwd_workspace_bytes_of(BF16, 0, 1, 40, 32760, 32760, 128)
    extra = ja._score_bytes(BF16, False, 1, 40, 32760, 32760, 128)
    assert extra > 0
    asked = []

    def fake_workspace(nbytes, device, limit=base):
        asked.append(nbytes)
        if nbytes > limit:
            raise torch.cuda.OutOfMemoryError("no room")
        return 1 << 20, nbytes, object()

    monkeypatch.setattr(ja.nat, "workspace", fake_workspace)
    ptr, size, owner = ja._backward_workspace(BF16, 0, 1, 40, 32760, 32760, 128, "cpu")
    assert asked == [base + extra, base] and size == base
    # with room for both, one allocation of the whole
    asked.clear()
    monkeypatch.setattr(ja.nat, "workspace", lambda n, d: fake_workspace(n, d, limit=1 << 50))
    assert ja._backward_workspace(BF16, 0, 1, 40, 32760, 32760, 128, "cpu")[1] == base + extra
    assert asked == [base + extra]
    # the minimum itself failing propagates
    monkeypatch.setattr(ja.nat, "workspace", lambda n, d: fake_workspace(n, d, limit=0))
    with pytest.raises(torch.cuda.OutOfMemoryError):
        ja._backward_workspace(BF16, 0, 1, 40, 32760, 32760, 128, "cpu")
