"""Build recipe for ``libdmad_attn.so``: the gfx950 HIP kernels and the C ABI.

Every kernel instantiation unit is compiled by ``hipcc`` in parallel, then the
objects are linked into one shared library next to this file. The library
needs nothing from PyTorch; Python reaches it through ``ctypes``
(``dmad_amd._native``).

Usage: ``python -m dmad_amd.build`` (or ``dmad_amd.build.build()``).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libdmad_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"
HEAD_DIMS = (16, 32, 64, 128, 256)


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


# Packed fp32 VALU instructions are switched off for all device code. No kernel
# branches on a NaN test, so fmaxf needs no operand canonicalisation; a NaN or
# an Inf in the inputs still reaches every output row it touches and no other
# (batch, head) slice (tests/test_nonfinite_gpu.py holds that contract).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fno-honor-nans",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-I", CSRC,
    "-I", INCLUDE,
]


def units():
    """(source, object name, extra flags) for every compilation unit."""
    out = [("capi.hip", "capi", []), ("aux.hip", "aux", []), ("prologue.hip", "prologue", []),
           ("probe.hip", "probe", [])]
    for t, tname in ((0, "bf16"), (1, "f16")):
        out.append(("fwd32_inst.hip", f"fwd32_{tname}", [f"-DDMAD_T={t}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
        out.append(("bwd_dq_inst.hip", f"bwd_dq_{tname}", [f"-DDMAD_T={t}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
        out.append(("bwd_kv_inst.hip", f"bwd_kv_{tname}", [f"-DDMAD_T={t}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
        out.append(("bwd_full_inst.hip", f"bwd_full_{tname}", [f"-DDMAD_T={t}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
        for d in HEAD_DIMS:
            out.append(("fwd_inst.hip", f"fwd_{tname}_d{d}", [f"-DDMAD_T={t}", f"-DDMAD_D={d}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
            if os.path.exists(os.path.join(CSRC, "bwd_inst.hip")):
                out.append(("bwd_inst.hip", f"bwd_{tname}_d{d}", [f"-DDMAD_T={t}", f"-DDMAD_D={d}", "-mllvm", "-amdgpu-mfma-vgpr-form"]))
    for d in HEAD_DIMS:
        out.append(("f32_inst.hip", f"f32_d{d}", [f"-DDMAD_D={d}"]))
    return out


def _compile(hipcc: str, src: str, obj: str, extra: list[str], verbose: bool) -> None:
    cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} {extra}:\n{res.stdout}\n{res.stderr}")


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile all units and link ``libdmad_attn.so``; returns its path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    todo = units()
    jobs = jobs or min(len(todo), max(1, (os.cpu_count() or 4)))
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for src, name, extra in todo:
            obj = os.path.join(BUILD_DIR, name + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, hipcc, src, obj, extra, verbose))
        for f in futs:
            f.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
