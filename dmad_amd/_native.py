"""ctypes binding of ``libdmad_attn.so`` (C ABI declared in ``include/dmad_attn.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded (both name it ``libamdhip64.so.7``); streams and device
pointers then mean the same thing on both sides. There is no fallback: if the
library is missing, every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
import functools
import os

import torch  # noqa: F401  (loads the HIP runtime the library must share)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdmad_attn.so")

DMAD_OK = 0
DMAD_ERR_INVALID = 1
DMAD_ERR_UNSUPPORTED = 2
DMAD_ERR_WORKSPACE = 3
DMAD_ERR_HIP = 4

DMAD_BF16 = 0
DMAD_F16 = 1
DMAD_F32 = 2

DMAD_FWD_PLAIN = 0
DMAD_FWD_JVP = 1
DMAD_FWD_JVP_KV_TANGENT_ZERO = 2



class Plan(ctypes.Structure):
    """``dmad_plan``: the kernels a call runs, their grids, block order, column chunks,
    transposed copies and workspace (see dmad_attn_fwd_plan / dmad_attn_bwd_plan)."""

    _fields_ = [
        ("kernel", ctypes.c_char_p),
        ("kernel2", ctypes.c_char_p),
        ("kernel3", ctypes.c_char_p),
        ("kernel4", ctypes.c_char_p),
        ("grid", ctypes.c_int64),
        ("grid2", ctypes.c_int64),
        ("xcd_order", ctypes.c_int32),
        ("xcd_order2", ctypes.c_int32),
        ("chunks", ctypes.c_int32),
        ("transposed_copies", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_int64),
        ("score_slices", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        out = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            out[name] = v.decode() if isinstance(v, bytes) else v
        return out


# Every function the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I64P = ctypes.POINTER(ctypes.c_int64)
_FP = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.c_size_t
_SZP = ctypes.POINTER(ctypes.c_size_t)
_INT = ctypes.c_int
_F = ctypes.c_float

SIGNATURES = {
    "dmad_abi_version": (_INT, []),
    "dmad_last_error": (ctypes.c_char_p, []),
    "dmad_attn_fwd_workspace_bytes": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64, _SZP]),
    "dmad_attn_jvp_fwd": (_INT, [_INT, _INT, _I64, _I64, _I64, _I64, _I64, _I64,
                                 _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                 _P, _P, _I64P, _P, _P, _F, _P, _SZ, _P]),
    "dmad_attn_jvp_fwd_magi": (_INT, [_INT, _INT, _I64, _I64, _I64, _I64, _I64, _I64,
                                      _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                      _P, _P, _I64P, _P, _P, _F,
                                      _P, _P, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _SZ, _P]),
    "dmad_attn_fwd": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P,
                             _I64P, _I64P, _I64P, _P, _I64P, _P, _F, _P, _SZ, _P]),
    "dmad_set_kernel_events": (_INT, [ctypes.POINTER(ctypes.c_void_p), _INT]),
    "dmad_probe_mfma": (_INT, [_INT, _I64, _I64, _P, _P]),
    "dmad_rmsnorm_rope_jvp": (_INT, [_INT, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _FP, _F, _P, _P, _I64, _P]),
    "dmad_attn_bwd_workspace_bytes": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64, _SZP]),
    "dmad_attn_fwd_plan": (_INT, [_INT, _INT, _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.POINTER(Plan)]),
    "dmad_attn_bwd_plan": (_INT, [_INT, _INT, _INT, _I64, _I64, _I64, _I64, _I64, ctypes.POINTER(Plan)]),
    "dmad_attn_bwd_plan_ws": (_INT, [_INT, _INT, _INT, _I64, _I64, _I64, _I64, _I64, _SZ, ctypes.POINTER(Plan)]),
    "dmad_attn_bwd_score_bytes": (_INT, [_INT, _INT, _I64, _I64, _I64, _SZP]),
    "dmad_attn_jvp_bwd": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64,
                                 _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                 _P, _P, _I64P, _P, _P, _P, _P, _I64P,
                                 _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                 _F, _P, _SZ, _P]),
    "dmad_attn_jvp_bwd_noalloc": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64,
                                         _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                         _P, _P, _I64P, _P, _P, _P, _P, _I64P,
                                         _P, _P, _P, _P, _P, _P, _I64P, _I64P, _I64P,
                                         _F, _P]),
}

# Bytes of the static device scratch of dmad_attn_jvp_bwd_noalloc (DMAD_BWD_SCRATCH_BYTES).
BWD_SCRATCH_BYTES = 64 << 20


class DmadError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[dmad status {code}] {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: the gfx950 HIP kernels are required "
                "(build with `python -m dmad_amd.build`)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(code: int) -> None:
    if code != DMAD_OK:
        msg = lib().dmad_last_error().decode(errors="replace")
        if code == DMAD_ERR_INVALID:
            raise ValueError(f"[dmad status {code}] {msg}")
        if code == DMAD_ERR_UNSUPPORTED:
            raise NotImplementedError(f"[dmad status {code}] {msg}")
        raise DmadError(code, msg)


# The helpers below sit on every call's host path, which the GPU waits on when a
# call follows a synchronisation (tens of microseconds against a 0.12 ms
# forward at 1024 tokens): plain ints go to ctypes as c_void_p, stride arrays
# are made once per stride tuple, and the workspace sizes (pure functions of
# the shape) are asked once per shape.
_strides_cache: dict = {}


def strides4(t: torch.Tensor):
    st = t.stride()
    arr = _strides_cache.get(st)
    if arr is None:
        if len(_strides_cache) > 4096:
            _strides_cache.clear()
        arr = _strides_cache[st] = (ctypes.c_int64 * 4)(*st)
    return arr


def ptr(t):
    """Device address of ``t`` (None -> NULL) as an int, which ctypes passes as c_void_p."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """The current HIP stream of ``device`` (what torch launches on) as an int."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


@functools.lru_cache(maxsize=1024)
def fwd_workspace_bytes(mode: int, B: int, H: int, Lk: int, Dqk: int, Dv: int) -> int:
    n = ctypes.c_size_t(0)
    check(lib().dmad_attn_fwd_workspace_bytes(mode, B, H, Lk, Dqk, Dv, ctypes.byref(n)))
    return int(n.value)


@functools.lru_cache(maxsize=1024)
def bwd_workspace_bytes(mode: int, B: int, H: int, Lq: int, Lk: int, D: int) -> int:
    n = ctypes.c_size_t(0)
    check(lib().dmad_attn_bwd_workspace_bytes(mode, B, H, Lq, Lk, D, ctypes.byref(n)))
    return int(n.value)


def fwd_plan(dtype: int, mode: int, B: int, H: int, Lq: int, Lk: int, Dqk: int, Dv: int,
             magi_tasks: int = -1) -> dict:
    """The launch plan of a forward call (no GPU needed): kernel, grid, block order, column
    chunks, transposed copies, workspace. ``magi_tasks`` >= 0 for the block-sparse forward."""
    pl = Plan()
    check(lib().dmad_attn_fwd_plan(dtype, mode, magi_tasks, B, H, Lq, Lk, Dqk, Dv, ctypes.byref(pl)))
    return pl.as_dict()


def bwd_plan(dtype: int, B: int, H: int, Lq: int, Lk: int, D: int, full: bool = False,
             tangent_grads: bool = False, workspace_bytes: int | None = None) -> dict:
    """The launch plan of a backward call (no GPU needed): the key and query passes (and the
    tangent passes), their grids and block order, transposed copies, workspace. With
    ``workspace_bytes`` the plan of a call given that much workspace (``score_slices`` > 0:
    the stored-score passes)."""
    pl = Plan()
    if workspace_bytes is None:
        check(lib().dmad_attn_bwd_plan(dtype, int(full), int(tangent_grads), B, H, Lq, Lk, D, ctypes.byref(pl)))
    else:
        check(lib().dmad_attn_bwd_plan_ws(dtype, int(full), int(tangent_grads), B, H, Lq, Lk, D,
                                          int(workspace_bytes), ctypes.byref(pl)))
    return pl.as_dict()


@functools.lru_cache(maxsize=1024)
def bwd_score_bytes(dtype: int, full: bool, Lq: int, Lk: int, D: int) -> int:
    """Bytes of stored score gradients per (b, h) slice (0 where the path does not exist)."""
    n = ctypes.c_size_t(0)
    check(lib().dmad_attn_bwd_score_bytes(dtype, int(full), Lq, Lk, D, ctypes.byref(n)))
    return int(n.value)


@functools.lru_cache(maxsize=1024)
def bwd_workspace_bytes_of(dtype: int, mode: int, B: int, H: int, Lq: int, Lk: int, D: int) -> int:
    """Workspace of a backward whose operands have dtype code ``dtype`` (``mode`` as in
    ``bwd_workspace_bytes``): fp32 operands need only the per-row statistics."""
    return int(bwd_plan(dtype, B, H, Lq, Lk, D, full=mode > 0, tangent_grads=mode == 2)["workspace_bytes"])


def workspace(nbytes: int, device: torch.device):
    """(pointer, size) of a fresh workspace of ``nbytes`` (NULL, 0 when none is needed) and the
    tensor that owns it, which the caller keeps alive until the launch is queued."""
    if nbytes == 0:
        return None, 0, None
    ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
    return ws.data_ptr(), nbytes, ws


class KernelTimer:
    """Times the main kernels of the next library calls with HIP events.

    Use as a context manager around one call: `timer.ms[i]` is then the
    duration of its i-th main kernel (see dmad_set_kernel_events).
    """

    def __init__(self, nkernels: int):
        self.n = nkernels
        self.events = []
        self.ms = []

    def __enter__(self):
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * self.n)]
        for e in self.events:  # torch creates the HIP event on first record
            e.record()
        arr = (ctypes.c_void_p * len(self.events))(*[e.cuda_event for e in self.events])
        check(lib().dmad_set_kernel_events(arr, len(self.events)))
        return self

    def __exit__(self, *exc):
        check(lib().dmad_set_kernel_events(None, 0))
        return False

    def elapsed(self):
        """Per-kernel milliseconds (synchronises on the events)."""
        return [self.events[2 * i].elapsed_time(self.events[2 * i + 1]) for i in range(self.n)]


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return DMAD_BF16
    if dtype == torch.float16:
        return DMAD_F16
    if dtype == torch.float32:
        return DMAD_F32
    raise NotImplementedError(
        f"dtype {dtype} is not supported by the gfx950 kernels (bfloat16, float16 or float32 operands)"
    )
