"""The C-ABI library loads, exports every symbol include/dmad_attn.h declares,
and rejects bad arguments before touching the GPU (no kernel launch here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dmad_attn.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(dmad_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def nat():
    from dmad_amd import _native

    return _native


def test_header_and_binding_agree(nat):
    assert _declared() == sorted(nat.SIGNATURES)


def test_library_exports_every_declared_symbol(nat):
    lib = nat.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.dmad_abi_version() == 2


def _strides(*v):
    return (ctypes.c_int64 * 4)(*v)


def _fwd(nat, **over):
    args = dict(dtype=0, mode=1, B=1, H=2, Lq=64, Lk=64, Dqk=64, Dv=64, q=256, k=256, v=256, tq=256, tk=256,
                tv=256, qs=_strides(8192, 4096, 64, 1), ks=_strides(8192, 4096, 64, 1),
                vs=_strides(8192, 4096, 64, 1), o=256, to=256, os=_strides(8192, 4096, 64, 1), lse=256, mu=256,
                scale=0.125, ws=256, wsb=1 << 30, stream=0)
    args.update(over)
    a = args
    return nat.lib().dmad_attn_jvp_fwd(
        a["dtype"], a["mode"], a["B"], a["H"], a["Lq"], a["Lk"], a["Dqk"], a["Dv"],
        ctypes.c_void_p(a["q"]), ctypes.c_void_p(a["k"]), ctypes.c_void_p(a["v"]), ctypes.c_void_p(a["tq"]),
        ctypes.c_void_p(a["tk"]), ctypes.c_void_p(a["tv"]), a["qs"], a["ks"], a["vs"],
        ctypes.c_void_p(a["o"]), ctypes.c_void_p(a["to"]), a["os"], ctypes.c_void_p(a["lse"]),
        ctypes.c_void_p(a["mu"]), a["scale"], ctypes.c_void_p(a["ws"]), a["wsb"], ctypes.c_void_p(a["stream"]))


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(Dqk=48), 2, "head dims"),
        (dict(Dv=512), 2, "head dims"),
        (dict(dtype=7), 2, "dtype"),
        (dict(mode=9), 1, "mode"),
        (dict(scale=0.0), 2, "sm_scale"),
        (dict(Lk=0), 1, "Lk"),
        (dict(q=0), 1, "q: null"),
        (dict(tk=0), 1, "tk: null"),
        (dict(qs=_strides(8192, 4096, 64, 2)), 1, "stride of the head dim"),
        (dict(ks=_strides(8192, 4096, 60, 1)), 1, "multiples of 8"),
        (dict(v=258), 1, "aligned"),
        (dict(mu=0), 1, "mu"),
        (dict(wsb=16, Dqk=32, Dv=32), 3, "workspace"),  # 32-wide heads read a transposed copy of V
        (dict(ws=0, Dqk=32, Dv=32), 3, "workspace"),
        (dict(Lq=1 << 22, qs=_strides(0, 0, 4096, 1)), 2, "2 GiB"),
        # fp32 operands: rows 16-byte aligned means strides in multiples of 4 elements
        (dict(dtype=2, ks=_strides(8192, 4096, 62, 1)), 1, "multiples of 4"),
        (dict(dtype=2, Lq=1 << 21, qs=_strides(0, 0, 256, 1)), 2, "2 GiB"),
    ],
)
def test_fwd_rejects_bad_arguments(nat, over, code, needle):
    assert _fwd(nat, **over) == code
    assert needle in nat.lib().dmad_last_error().decode()


def test_fwd_empty_problem_is_a_no_op(nat):
    assert _fwd(nat, Lq=0) == 0
    assert _fwd(nat, B=0) == 0


def test_kv_tangent_zero_mode_does_not_need_kv_tangents(nat):
    # mode 2 never reads tk/tv: null is accepted up to the workspace check
    assert _fwd(nat, mode=2, tk=0, tv=0, wsb=16, Dqk=32, Dv=32) == 3


def test_workspace_query(nat):
    n = ctypes.c_size_t(0)
    q = nat.lib().dmad_attn_fwd_workspace_bytes
    # 64-, 128- and 256-wide heads read V in place: no workspace
    for d in (64, 128, 256):
        for mode in (0, 1, 2):
            assert q(mode, 1, 40, 32760, d, d, ctypes.byref(n)) == 0 and n.value == 0
    # other head dims (or Dqk != Dv): transposed, key-padded copies of V (and Vd in the full JVP mode)
    assert q(1, 1, 40, 32760, 64, 128, ctypes.byref(n)) == 0
    assert n.value == 2 * 40 * 128 * 32768 * 2
    assert q(0, 1, 40, 32760, 128, 256, ctypes.byref(n)) == 0
    assert n.value == 40 * 256 * 32768 * 2
    assert q(0, 1, 1, 10, 16, 16, ctypes.byref(n)) == 0
    assert n.value == 32 * 64 * 2  # Dv < 32 pads to 32 rows, keys pad to 64
    assert q(0, 1, 1, 10, 48, 64, ctypes.byref(n)) == 1  # bad head dim


def test_kernel_event_hook_validates(nat):
    lib = nat.lib()
    assert lib.dmad_set_kernel_events(None, 0) == 0
    assert lib.dmad_set_kernel_events(None, 2) == 1
    arr = (ctypes.c_void_p * 3)(None, None, None)
    assert lib.dmad_set_kernel_events(arr, 3) == 1
    arr = (ctypes.c_void_p * 258)()
    assert lib.dmad_set_kernel_events(arr, 258) == 1  # at most 256 events
    assert lib.dmad_set_kernel_events(arr, 256) == 0
    assert lib.dmad_set_kernel_events(None, 0) == 0


def _pro(nat, **over):
    a = dict(dtype=0, rows=64, L=32, H=2, D=64, y=256, ty=256, ys=128, w=256, freqs=256, eps=1e-6, out=256, tout=256,
             os=128, stream=0)
    a.update(over)
    return nat.lib().dmad_rmsnorm_rope_jvp(
        a["dtype"], a["rows"], a["L"], a["H"], a["D"], ctypes.c_void_p(a["y"]), ctypes.c_void_p(a["ty"]), a["ys"],
        ctypes.c_void_p(a["w"]), ctypes.cast(ctypes.c_void_p(a["freqs"]), ctypes.POINTER(ctypes.c_float)), a["eps"],
        ctypes.c_void_p(a["out"]), ctypes.c_void_p(a["tout"]), a["os"], ctypes.c_void_p(a["stream"]))


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(dtype=5), 2, "dtype"),
        (dict(D=12), 2, "multiple of 8"),
        (dict(D=1024), 2, "multiple of 8"),
        (dict(H=100, D=128), 2, "exceeds"),
        (dict(tout=0), 1, "both"),
        (dict(y=0), 1, "null"),
        (dict(w=0, freqs=0), 1, "nothing to do"),
        (dict(out=264), 1, "aligned"),
        (dict(ys=100), 1, "strides"),
        (dict(os=64), 1, "strides"),
        (dict(rows=48), 1, "multiple of L"),
        (dict(eps=-1.0), 1, "eps"),
    ],
)
def test_prologue_rejects_bad_arguments(nat, over, code, needle):
    assert _pro(nat, **over) == code
    assert needle in nat.lib().dmad_last_error().decode()


def test_prologue_empty_is_a_no_op(nat):
    assert _pro(nat, rows=0) == 0


def _magi(nat, **over):
    a = dict(dtype=0, mode=1, B=1, H=2, Lq=64, Lk=64, Dqk=128, Dv=128, q=256, k=256, v=256, tq=256, tk=256,
             tv=256, qs=_strides(16384, 8192, 128, 1), ks=_strides(16384, 8192, 128, 1),
             vs=_strides(16384, 8192, 128, 1), o=256, to=256, os=_strides(16384, 8192, 128, 1), lse=256, mu=256,
             scale=0.125, qr=256, kr=256, qm=256, G=1, R=1, tg=256, tq_=256, T=1, bm=128, ws=256, wsb=1 << 30,
             stream=0)
    a.update(over)
    P = ctypes.c_void_p
    return nat.lib().dmad_attn_jvp_fwd_magi(
        a["dtype"], a["mode"], a["B"], a["H"], a["Lq"], a["Lk"], a["Dqk"], a["Dv"],
        P(a["q"]), P(a["k"]), P(a["v"]), P(a["tq"]), P(a["tk"]), P(a["tv"]), a["qs"], a["ks"], a["vs"],
        P(a["o"]), P(a["to"]), a["os"], P(a["lse"]), P(a["mu"]), a["scale"],
        P(a["qr"]), P(a["kr"]), P(a["qm"]), a["G"], a["R"], P(a["tg"]), P(a["tq_"]), a["T"], a["bm"],
        P(a["ws"]), a["wsb"], P(a["stream"]))


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(bm=64), 2, "128-query tiles"),
        (dict(G=0), 1, "table sizes"),
        (dict(T=-1), 1, "table sizes"),
        (dict(qr=0), 1, "null"),
        (dict(qm=0), 1, "null"),
        (dict(kr=0), 1, "null"),
        (dict(tg=0), 1, "null"),
        (dict(mode=0), 2, "JVP modes"),
        (dict(Dqk=48), 2, "head dims"),
        (dict(tk=0), 1, "tk: null"),
        (dict(wsb=16, Dqk=32, Dv=32), 3, "workspace"),
    ],
)
def test_magi_fwd_rejects_bad_arguments(nat, over, code, needle):
    assert _magi(nat, **over) == code
    assert needle in nat.lib().dmad_last_error().decode()


def test_magi_fwd_without_tasks_is_a_no_op(nat):
    assert _magi(nat, T=0, tg=0, tq_=0) == 0
    assert _magi(nat, R=0, kr=0, T=0) == 0


def _bwd(nat, **over):
    st = _strides(8192, 4096, 64, 1)
    args = dict(dtype=0, B=1, H=2, Lq=64, Lk=64, D=64, q=256, k=256, v=256, tq=0, tk=0, tv=0, qs=st, ks=st, vs=st,
                o=256, to=0, os=st, lse=256, mu=0, do=256, dto=0, dos=st, dq=256, dk=256, dv=256, dtq=0, dtk=0,
                dtv=0, dqs=st, dks=st, dvs=st, scale=0.125, ws=256, wsb=1 << 30, stream=0)
    args.update(over)
    a = args
    p = ctypes.c_void_p
    return nat.lib().dmad_attn_jvp_bwd(
        a["dtype"], a["B"], a["H"], a["Lq"], a["Lk"], a["D"], p(a["q"]), p(a["k"]), p(a["v"]), p(a["tq"]),
        p(a["tk"]), p(a["tv"]), a["qs"], a["ks"], a["vs"], p(a["o"]), p(a["to"]), a["os"], p(a["lse"]), p(a["mu"]),
        p(a["do"]), p(a["dto"]), a["dos"], p(a["dq"]), p(a["dk"]), p(a["dv"]), p(a["dtq"]), p(a["dtk"]), p(a["dtv"]),
        a["dqs"], a["dks"], a["dvs"], a["scale"], p(a["ws"]), a["wsb"], p(a["stream"]))


_FULL = dict(tq=256, tk=256, tv=256, to=256, mu=256, dto=256)


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(dtype=7), 2, "dtype"),
        (dict(D=48), 2, "head dim"),
        (dict(scale=-1.0), 2, "sm_scale"),
        (dict(Lq=-1), 1, "negative"),
        (dict(dtq=256, dtk=256, dtv=256), 1, "need the cotangent dto"),
        (dict(_FULL, dtq=256, dtk=256), 1, "all set or all null"),
        (dict(_FULL, D=256), 2, "up to 128"),
        (dict(Lk=0), 1, "Lk must be"),
        (dict(Lq=0), 1, "Lq must be"),
        (dict(q=0), 1, "q: null"),
        (dict(dk=0), 1, "dk: null"),
        (dict(dqs=_strides(8192, 4096, 64, 2)), 1, "stride of the head dim"),
        (dict(lse=0), 1, "lse"),
        (dict(_FULL, mu=0), 1, "mu"),
        (dict(_FULL, tk=0), 1, "tk: null"),
        (dict(_FULL, dtq=256, dtk=256, dtv=0), 1, "all set or all null"),
        (dict(wsb=16), 3, "workspace"),
        (dict(ws=272), 1, "256-byte"),
        (dict(_FULL, dtype=2), 2, "bf16 or fp16"),  # fp32: dO-only gradients
        (dict(dtype=2, dos=_strides(8192, 4096, 66, 1)), 1, "multiples of 4"),
    ],
)
def test_bwd_rejects_bad_arguments(nat, over, code, needle):
    """dmad_attn_jvp_bwd checks its arguments before any launch; bad ones return the
    documented status with a message naming the problem."""
    assert _bwd(nat, **over) == code
    assert needle in nat.lib().dmad_last_error().decode()


def test_bwd_workspace_query(nat):
    n = ctypes.c_size_t(0)
    q = nat.lib().dmad_attn_bwd_workspace_bytes
    stats = 40 * 32768 * 2 * 4  # lse2 and D per (head, padded query row)
    # dO-only, 64- and 128-wide heads: the kernels read rows, only the statistics
    for d in (64, 128):
        assert q(0, 1, 40, 32760, 32760, d, ctypes.byref(n)) == 0 and n.value == stats
    # 32-wide heads read transposed copies of Q, dO and K
    copy = 40 * 32 * 32768 * 2
    assert q(0, 1, 40, 32760, 32760, 32, ctypes.byref(n)) == 0 and n.value == 3 * copy + stats
    # the full derivative of 128-wide heads reads rows: four statistics per row
    # (lse2, D', mu, rho), and two more (lse2, rho) for the tangent gradients
    assert q(1, 1, 40, 32760, 32760, 128, ctypes.byref(n)) == 0 and n.value == 2 * stats
    assert q(2, 1, 40, 32760, 32760, 128, ctypes.byref(n)) == 0 and n.value == 3 * stats
    # other head dims: Q, dO, Qd, dOd, K, Kd copies as well
    copy = 40 * 64 * 32768 * 2
    stats64 = 40 * 32768 * 2 * 4
    assert q(1, 1, 40, 32760, 32760, 64, ctypes.byref(n)) == 0 and n.value == 6 * copy + 2 * stats64


def test_bwd_empty_problem_is_a_no_op(nat):
    assert _bwd(nat, B=0) == 0
    assert _bwd(nat, H=0) == 0
    assert _bwd(nat, Lq=0, Lk=0) == 0


def _bwd_noalloc(nat, **over):
    st = _strides(8192, 4096, 64, 1)
    args = dict(dtype=0, B=1, H=2, Lq=64, Lk=64, D=64, q=256, k=256, v=256, tq=0, tk=0, tv=0, qs=st, ks=st, vs=st,
                o=256, to=0, os=st, lse=256, mu=0, do=256, dto=0, dos=st, dq=256, dk=256, dv=256, dtq=0, dtk=0,
                dtv=0, dqs=st, dks=st, dvs=st, scale=0.125, stream=0)
    args.update(over)
    a = args
    p = ctypes.c_void_p
    return nat.lib().dmad_attn_jvp_bwd_noalloc(
        a["dtype"], a["B"], a["H"], a["Lq"], a["Lk"], a["D"], p(a["q"]), p(a["k"]), p(a["v"]), p(a["tq"]),
        p(a["tk"]), p(a["tv"]), a["qs"], a["ks"], a["vs"], p(a["o"]), p(a["to"]), a["os"], p(a["lse"]), p(a["mu"]),
        p(a["do"]), p(a["dto"]), a["dos"], p(a["dq"]), p(a["dk"]), p(a["dv"]), p(a["dtq"]), p(a["dtk"]), p(a["dtv"]),
        a["dqs"], a["dks"], a["dvs"], a["scale"], p(a["stream"]))


def test_bwd_noalloc_rejects_problems_beyond_its_scratch(nat):
    """The allocation-free backward refuses, before any HIP call, a problem whose
    workspace exceeds its 64 MiB static scratch: here the full derivative with
    tangent gradients at the Wan2.1-14B 720p shape (24 bytes of statistics per
    (head, query row): 72.6 MB)."""
    st = _strides(75600 * 40 * 128, 128, 40 * 128, 1)
    rc = _bwd_noalloc(nat, **_FULL, dtq=256, dtk=256, dtv=256, B=1, H=40, Lq=75600, Lk=75600, D=128, qs=st, ks=st,
                      vs=st, os=st, dos=st, dqs=st, dks=st, dvs=st)
    assert rc == 2
    assert "static scratch" in nat.lib().dmad_last_error().decode()
    n = ctypes.c_size_t(0)
    assert nat.lib().dmad_attn_bwd_workspace_bytes(2, 1, 40, 75600, 75600, 128, ctypes.byref(n)) == 0
    assert n.value > nat.BWD_SCRATCH_BYTES
    # without the tangent gradients the same problem fits
    assert nat.lib().dmad_attn_bwd_workspace_bytes(1, 1, 40, 75600, 75600, 128, ctypes.byref(n)) == 0
    assert n.value <= nat.BWD_SCRATCH_BYTES


def test_bwd_noalloc_sizes_fp32_by_its_statistics(nat):
    """fp32 operands need only the per-row statistics (B=1, H=32, L=2048: 512 KiB), so the
    size gate of the allocation-free backward passes a 256-wide fp32 problem that the
    bf16 sizing (transposed Q, dO copies) would refuse. Without a GPU the call then stops
    at the device lookup, never at the scratch size."""
    st = _strides(32 * 2048 * 256, 2048 * 256, 256, 1)
    rc = _bwd_noalloc(nat, dtype=2, B=1, H=32, Lq=2048, Lk=2048, D=256, qs=st, ks=st, vs=st, os=st, dos=st, dqs=st,
                      dks=st, dvs=st)
    assert "static scratch" not in nat.lib().dmad_last_error().decode()
    assert rc in (0, 4)
    assert nat.bwd_plan(nat.DMAD_F32, 1, 32, 2048, 2048, 256)["workspace_bytes"] == 32 * 2048 * 8
    assert nat.bwd_workspace_bytes(0, 1, 32, 2048, 2048, 256) > nat.BWD_SCRATCH_BYTES


@pytest.mark.parametrize("over,code,needle", [(dict(dtype=7), 2, "dtype"), (dict(q=0), 1, "q: null"),
                                              (dict(D=48), 2, "head dim")])
def test_bwd_noalloc_rejects_bad_arguments(nat, over, code, needle):
    assert _bwd_noalloc(nat, **over) == code
    assert needle in nat.lib().dmad_last_error().decode()


def test_bwd_noalloc_empty_problem_is_a_no_op(nat):
    assert _bwd_noalloc(nat, B=0) == 0


@pytest.mark.parametrize("args,code,needle", [((7, 1, 256), 2, "bf16 or fp16"), ((0, 0, 256), 1, "blocks"),
                                              ((0, 1, 100), 1, "multiple of 256"), ((1, 1, 0), 1, "multiple")])
def test_mfma_probe_rejects_bad_arguments(nat, args, code, needle):
    assert nat.lib().dmad_probe_mfma(*args, ctypes.c_void_p(256), ctypes.c_void_p(0)) == code
    assert needle in nat.lib().dmad_last_error().decode()
    assert nat.lib().dmad_probe_mfma(0, 1, 256, ctypes.c_void_p(0), ctypes.c_void_p(0)) == 1
