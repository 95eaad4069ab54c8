#!/usr/bin/env python3
"""Benchmark of the flash-attention JVP path on one MI355X.

One step = one Wan2.1-14B DiT layer's attention work on the JVP path, in the layer's order
(self-attention, then text cross-attention, forward; then the self-attention backward):
  * self-attention forward + JVP     B=1, H=40, L=32760, D=128, bf16   (12 L^2 D H flop)
  * text cross-attention forward + JVP, Lq=32760 over 512 keys, Kd=Vd=0  (8 Lq Lk D H flop)
  * self-attention backward, dO only (what the reference computes)       (10 L^2 D H flop)
Inputs are resident in HBM before timing starts (synthetic, seeded: Q, K RMS-normalised
over H*D and rotated by 3D RoPE on the 21x30x52 latent grid, V ~ N(0,1), tangents
~ N(0, 0.1^2), dO ~ N(0,1)).

Prints one JSON line: value = algorithmic TFLOP/s of the whole step (flops as above,
exp/softmax work not counted, the convention of flash_attention_jvp_triton.py:716-724),
plus a roofline record for the dominant kernel timed live with HIP events, and a
CPU baseline (the oracle's float32 PyTorch math path on the host cores, on a bounded
sample, extrapolated).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 flop/clk/CU
PEAK_F32_TFLOPS = 157.3  # 256 CU x 2.4 GHz x 256 dense fp32 MFMA flop/clk/CU
ROOT = os.path.dirname(os.path.abspath(__file__))


# Board power / clock sampler, run as a separate process started before this
# process touches the GPU (amd-smi reads the driver, not HIP).
_SAMPLER = r'''
import re, subprocess, sys, time
out = open(sys.argv[1], "w", buffering=1)
while True:
    t = time.time()
    try:
        txt = subprocess.run(["amd-smi", "metric", "-p", "-c"], capture_output=True, text=True, timeout=5).stdout
    except Exception:
        txt = ""
    pw = re.search(r"SOCKET_POWER: (\d+)", txt)
    clk = [int(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK: (\d+) MHz", txt)]
    if pw and clk:
        out.write(f"{t:.3f} {pw.group(1)} {sum(clk) / len(clk):.0f}\n")
    time.sleep(0.05)
'''


def _start_power_sampler(path):
    import subprocess

    return subprocess.Popen([sys.executable, "-c", _SAMPLER, path], stdout=subprocess.DEVNULL,
                            stderr=subprocess.DEVNULL)


def _power_summary(path, t0, t1):
    rows = []
    for line in open(path):
        t, w, c = line.split()
        if t0 <= float(t) <= t1:
            rows.append((float(w), float(c)))
    if not rows:
        return {"samples": 0}
    return {"samples": len(rows), "avg_W": round(sum(r[0] for r in rows) / len(rows), 1),
            "max_W": max(r[0] for r in rows), "avg_gfx_MHz": round(sum(r[1] for r in rows) / len(rows)),
            "source": "amd-smi metric -p -c (SOCKET_POWER, mean GFX CLK over the XCDs)"}


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--heads", type=int, default=40, help="attention heads (14B: 40, 1.3B: 12)")
    ap.add_argument("--seq", type=int, default=32760)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample time")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-full-bwd", dest="full_bwd", action="store_false",
                    help="skip timing the full-derivative backward (extra field)")
    ap.add_argument("--no-prologue", dest="prologue", action="store_false",
                    help="skip timing the fused RMSNorm+RoPE prologue (extra field)")
    ap.add_argument("--power", action="store_true",
                    help="also sample board power and GFX clock over the forward and backward alone (extra field)")
    ap.add_argument("--no-clock", dest="clock", action="store_false",
                    help="do not sample the GFX clock and board power during the timed steps")
    ap.add_argument("--no-plain", dest="plain", action="store_false",
                    help="skip timing plain attention forward + backward (extra field)")
    ap.add_argument("--no-magi", dest="magi", action="store_false",
                    help="skip timing the block-sparse forward on the causal-student masks (extra field)")
    ap.add_argument("--harness", action="store_true",
                    help="also time the reference perf harness configuration (B=4, H=32, D=64 and 128, fp16), "
                         "and the same at head dims 16, 32 and 256")
    ap.add_argument("--harness-dims", default="16,32,64,128,256",
                    help="head dims the --harness timing covers (comma-separated; default all five)")
    ap.add_argument("--no-ceiling", dest="ceiling", action="store_false",
                    help="skip the MFMA ceiling probe after the timed steps (extra field)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after timing, run one elementwise kernel that reads and writes this many MiB "
                         "(a known-size reference for HBM byte counters under a profiler)")
    return ap.parse_args()


def _traffic_from_profiles(name):
    """HBM bytes per launch of `name` from a committed rocprofv3 counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def _cpu_model():
    """CPU model name as lscpu reports it (None if unavailable)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return None


def cpu_baseline(x, H, seconds):
    """Oracle float32 math path on the host: torch.func.jvp for (O, Od), autograd for dQ/dK/dV.

    Runs on the benchmark's own inputs (head 0 of the same seeded tensors, copied
    to the host): 2048-row query chunks at full Lk until `seconds` of work are
    done; FLOP/s are extrapolated linearly (the work is linear in rows and heads).
    """
    import torch

    sys.path.insert(0, ROOT)
    from oracle.attention import math_attention

    h0 = {n: x[n][0, 0].float().cpu()[None, None] for n in ("q", "k", "v", "tq", "tk", "tv", "do")}
    L, D = h0["k"].shape[-2], h0["k"].shape[-1]
    k, v, tk, tv = h0["k"], h0["v"], h0["tk"], h0["tv"]
    rows, done, t = 2048, 0, 0.0
    s = D ** -0.5
    while t < seconds:
        r0 = done % L
        q, tq, do = (h0[n][..., r0:r0 + rows, :] for n in ("q", "tq", "do"))
        t0 = time.perf_counter()
        fn = lambda a, b, c: math_attention(a, b, c, s)[0]  # noqa: E731
        torch.func.jvp(fn, (q, k, v), (tq, tk, tv))
        leaves = [y.clone().requires_grad_(True) for y in (q, k, v)]
        o = math_attention(*leaves, s)[0]
        torch.autograd.grad(o, leaves, do)
        t += time.perf_counter() - t0
        done += q.shape[-2]
    flops = 22.0 * done * L * D
    return {
        "value": round(flops / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": f"head 0 of the benchmark inputs: {done} query rows x {L} keys, D={D}, fp32 torch.func.jvp "
                  f"+ autograd (fwd+JVP+dO-only bwd) in {t:.1f} s on {torch.get_num_threads()} threads; "
                  f"extrapolates to {H * L / done * t / 60:.0f} min for the {H}-head layer",
    }


def prologue_timing(H, L, D, grid, dev):
    """q and k prologues of one layer: [1, L, H*D] Linear outputs and tangents -> rotated BSHD pairs."""
    import torch

    from dmad_amd import _native, rmsnorm_rope_with_tangent
    from dmad_amd.workload import rope_freqs_3d

    C = H * D
    g = torch.Generator(device=dev).manual_seed(3)
    ys = [torch.randn(1, L, C, generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    w = torch.ones(C, device=dev, dtype=torch.bfloat16)
    freqs = rope_freqs_3d(*grid, D, device=dev) if grid is not None else None
    for _ in range(2):
        rmsnorm_rope_with_tangent((ys[0], ys[1]), w, 1e-6, freqs, H)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        tq, tk = _native.KernelTimer(1), _native.KernelTimer(1)
        with tq:
            rmsnorm_rope_with_tangent((ys[0], ys[1]), w, 1e-6, freqs, H)
        with tk:
            rmsnorm_rope_with_tangent((ys[2], ys[3]), w, 1e-6, freqs, H)
        torch.cuda.synchronize()
        best = min(best, tq.elapsed()[0] + tk.elapsed()[0])
    # algorithmic bytes per call: y, ty read and q, q_dot written (bf16), weight and angles
    per_call = 4 * L * C * 2 + C * 2 + (L * D // 2 * 4 if grid is not None else 0)
    gbs = 2 * per_call / (best * 1e-3) / 1e9
    return {"kernel": "rmsnorm_rope_kernel<bf16,10,jvp,rope,norm>", "ms_q_and_k": round(best, 4),
            "bytes_per_call": per_call, "achieved_GBps": round(gbs, 1), "hbm_peak_GBps": 8000.0,
            "frac": round(gbs / 8000.0, 4)}


def plain_timing(q, k, v, do, dev):
    """Plain attention (no tangents) forward and dO-only backward at the step's
    shape: the op DMAD's critics and student gradients train through
    (dmad::flash_attn_fwd / flash_attn_bwd). Flops: 4 and 10 units of H*L^2*D."""
    import torch

    from dmad_amd import _native
    from dmad_amd.jvp_attention import backward_plan, jvp_attention_backward, jvp_attention_forward

    s = q.shape[-1] ** -0.5
    o, _, lse, _ = jvp_attention_forward(q, k, v, None, None, None, s)
    jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)
    torch.cuda.synchronize()
    B, H, L, D = q.shape
    bplan = backward_plan(q.dtype, B, H, L, L, D)
    best_f = best_b = float("inf")
    for _ in range(3):
        tf, tb = _native.KernelTimer(1), _native.KernelTimer(2 * bplan["pairs"])
        with tf:
            o, _, lse, _ = jvp_attention_forward(q, k, v, None, None, None, s)
        with tb:
            jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)
        torch.cuda.synchronize()
        best_f = min(best_f, tf.elapsed()[0])
        best_b = min(best_b, sum(tb.elapsed()))
    unit = B * H * L * L * D
    tfs = 14.0 * unit / ((best_f + best_b) * 1e-3) / 1e12
    return {"kernels": f"attn_fwd32_kernel<bf16,plain> + {bplan['kernel']} + {bplan['kernel2']}",
            "ms_fwd": round(best_f, 3), "ms_bwd": round(best_b, 3),
            "fwd_pct_peak": round(100 * 4.0 * unit / (best_f * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
            "TFLOPs_fwd_bwd": round(tfs, 1), "pct_peak_fwd_bwd": round(100 * tfs / PEAK_BF16_TFLOPS, 2)}


def full_bwd_timing(q, k, v, tq, tk, tv, do, dto):
    """The full-derivative backward (the cotangent dOd of the tangent output included)
    at the step's shape: gradients of q, k, v only, and all six gradients (the
    tangents' too). Whole library calls (statistics and passes), best of 3.
    Algorithmic flops: 24 and 30 units of H*L^2*D (12 and 15 GEMMs of 2*L^2*D)."""
    import torch

    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    s = q.shape[-1] ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    B, H, L, D = q.shape
    unit = B * H * L * L * D
    from dmad_amd.jvp_attention import backward_plan

    bplan = backward_plan(q.dtype, B, H, L, L, D, full=True, tangent_grads=True)
    res = {"kernels": f"bwd_prep_kernel + {bplan['kernel']} + {bplan['kernel2']} "
                      f"[+ {bplan['kernel3']} for the tangents' dK, dV]",
           "score_slices_per_pair": bplan["score_slices"]}
    for tg, units, name in ((False, 24.0, "dq_dk_dv"), (True, 30.0, "all_six")):
        jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, do, dto, s, tg)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, do, dto, s, tg)
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
        tfs = units * unit / (best * 1e-3) / 1e12
        res[f"ms_{name}"] = round(best, 3)
        res[f"pct_peak_{name}"] = round(100 * tfs / PEAK_BF16_TFLOPS, 2)
    return res


def _do_bench(fn, flush, rep_ms=100.0, warmup_ms=25.0):
    """Mean and minimum time (ms) of fn() the way triton.testing.do_bench measures it (the
    reference harness's timer, flash_attention_jvp_triton.py:703): before each timed call
    the L2 (and the 256 MB memory-side cache) is flushed by zeroing a 256 MB buffer, which also
    gives the host time to queue the call, then HIP events bracket the call; about 25 ms of
    warm-up calls and 100 ms of timed calls, at least 3 and at most 1000."""
    import torch

    for _ in range(3):  # first calls (lazy code-object loads, allocator growth) stay out of the estimate
        flush.zero_()
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(5):
        flush.zero_()
        fn()
    b.record()
    torch.cuda.synchronize()
    est = a.elapsed_time(b) / 5
    for _ in range(max(1, int(warmup_ms / est))):
        fn()
    n = max(3, min(1000, int(rep_ms / est)))
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for s, e in ev:
        flush.zero_()
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    ts = [s.elapsed_time(e) for s, e in ev]
    return sum(ts) / n, min(ts), n


def harness_timing(dev, D=64, lengths=(1024, 2048, 4096, 8192, 16384), dtype=None, as_reference=False):
    """The configuration of the reference's own perf_report harness
    (flash_attention_jvp_triton.py:662-725): B=4, H=32, fp16, L = 1024..16384,
    forward+JVP and its backward, with the harness's flop convention (12 and 10
    units of B*H*L^2*D). The reference publishes no result for it. With
    dtype=float32 the same on the fp32 kernels, against the fp32 MFMA peak.

    Timed as the harness times its op (triton.testing.do_bench, see _do_bench):
    whole library calls (statistics, transposed copies and kernels) with the L2
    flushed before each, the mean reported (and the minimum beside it).

    By default Q, K, V, the tangents and dO are N(0,1) and sm_scale = D^-0.5.
    as_reference=True takes the harness's own values (:686-698): Q, K, V, dO
    ~ N(0,1), zero tangent tensors (the full six-GEMM forward still runs) and
    sm_scale = 1.3, whose logits are about 10x larger, so the online softmax
    raises its running maximum, and rescales, far more often."""
    import torch

    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    dtype = torch.float16 if dtype is None else dtype
    peak = PEAK_F32_TFLOPS if dtype == torch.float32 else PEAK_BF16_TFLOPS
    B, H = 4, 32
    flush = torch.empty(256 * 1024 * 1024, dtype=torch.int8, device=dev)
    rows = []
    for L in lengths:
        g = torch.Generator(device=dev).manual_seed(0)
        q, k, v, tq, tk, tv, do = (torch.randn((B, H, L, D), device=dev, dtype=dtype, generator=g)
                                   for _ in range(7))
        s = D ** -0.5
        if as_reference:
            tq, tk, tv = (torch.zeros_like(x) for x in (q, k, v))
            s = 1.3
        o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
        mean_f, min_f, n_f = _do_bench(lambda: jvp_attention_forward(q, k, v, tq, tk, tv, s), flush)
        mean_b, min_b, n_b = _do_bench(
            lambda: jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, do, None, s, False), flush)
        unit = B * H * L * L * D
        tf_f, tf_b = 12.0 * unit / (mean_f * 1e-3) / 1e12, 10.0 * unit / (mean_b * 1e-3) / 1e12
        rows.append({"L": L, "ms_fwd_jvp": round(mean_f, 3), "ms_fwd_jvp_min": round(min_f, 3),
                     "fwd_jvp_TFLOPs": round(tf_f, 1), "fwd_pct_peak": round(100 * tf_f / peak, 1),
                     "ms_bwd": round(mean_b, 3), "ms_bwd_min": round(min_b, 3), "bwd_TFLOPs": round(tf_b, 1),
                     "bwd_pct_peak": round(100 * tf_b / peak, 1), "calls": [n_f, n_b]})
        del q, k, v, tq, tk, tv, do, o, to, lse, mu
    del flush
    return {"B": 4, "H": 32, "D": D, "dtype": "fp32" if dtype == torch.float32 else "fp16", "peak_TFLOPs": peak,
            "sm_scale": 1.3 if as_reference else "D^-0.5", "tangents": "zeros" if as_reference else "N(0,1)",
            "timer": "do_bench protocol: 256 MB flush before each call, mean (and min) over ~100 ms of calls",
            "rows": rows}


def mfma_ceiling(dev, kernel_tflops):
    """The board's practical MFMA rate, measured right after the timed steps: the
    library's probe kernel (dmad_probe_mfma) runs back-to-back bf16 32x32x16 MFMAs,
    one workgroup of four waves per CU, about 3.5 ms per launch, under the same
    power limit as the attention kernels. Reported with each main kernel's rate as
    a fraction of it."""
    import torch

    from dmad_amd import _native

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    per_wave = 256 * 750  # 192000 MFMAs: ~3.3 ms at 1.86 GHz
    sink = torch.empty(cus * 256, device=dev, dtype=torch.float32)
    stream = _native.stream_ptr(dev)
    lib = _native.lib()
    for _ in range(3):
        _native.check(lib.dmad_probe_mfma(_native.DMAD_BF16, cus, per_wave, _native.ptr(sink), stream))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    e0.record()
    for _ in range(reps):
        _native.check(lib.dmad_probe_mfma(_native.DMAD_BF16, cus, per_wave, _native.ptr(sink), stream))
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    tflops = cus * 4 * per_wave * 32768.0 / (ms * 1e-3) / 1e12
    return {"kernel": "mfma_probe_kernel<bf16>", "cus": cus, "ms_per_launch": round(ms, 3),
            "TFLOPs": round(tflops, 1), "pct_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
            "kernels_pct_of_ceiling": {n: round(100 * t / tflops, 1) for n, t in kernel_tflops.items()}}


def magi_timing(H, D, dev):
    """Block-sparse forward+JVP on two Wan2.1-14B causal-student masks (1560-token
    frames, a 1-frame first block, 4-frame blocks, window of 3 blocks, 1 sink
    block): block-causal streaming with 16 query frames over 21 key frames
    (query block offset 2), and teacher forcing on the packed 2 x 21-frame
    sequence. Flops count only the allowed (query, key) pairs."""
    import torch

    from dmad_amd import _native
    from dmad_amd import magimask as mm
    from dmad_amd.jvp_attention import jvp_attention_forward_magi

    pat = mm.BlockPattern(frame_tokens=1560, first_chunk_frames=1, chunk_frames=4)
    cases = {
        "block_causal": (mm.AttnMaskSpec(mode="block_causal", pattern=pat, q_block_offset=2, local_attn_blocks=3,
                                         sink_blocks=1), 1560 * 16, 1560 * 21),
        "teacher_forcing": (mm.AttnMaskSpec(mode="teacher_forcing", pattern=pat, clean_blocks=6,
                                            local_attn_blocks=3, sink_blocks=1), 1560 * 42, 1560 * 42),
    }
    res = {}
    g = torch.Generator(device=dev).manual_seed(5)
    for name, (spec, Q, KV) in cases.items():
        qr, kr = mm.make_magi_ranges_full(spec, Q_real=Q, KV_real=KV, device=dev)
        mask = mm.prepare_magi_csr_and_tasks(qr, kr, Q_real=Q, KV_real=KV)
        qu, kf, qm = mask.q_unique.cpu().tolist(), mask.k_flat.cpu().tolist(), mask.qk_map.cpu().tolist()
        pairs = sum((qu[i][1] - qu[i][0]) * sum(kf[r][1] - kf[r][0] for r in range(qm[i], qm[i + 1]))
                    for i in range(len(qu)))
        r = lambda L: torch.randn(1, L, H, D, generator=g, device=dev).to(torch.bfloat16).transpose(1, 2)  # noqa: E731
        q, tq, k, tk, v, tv = r(Q), r(Q), r(KV), r(KV), r(KV), r(KV)
        for _ in range(2):
            jvp_attention_forward_magi(q, k, v, tq, tk, tv, D ** -0.5, mask)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            t = _native.KernelTimer(1)
            with t:
                jvp_attention_forward_magi(q, k, v, tq, tk, tv, D ** -0.5, mask)
            torch.cuda.synchronize()
            best = min(best, t.elapsed()[0])
        flops = 12.0 * H * D * pairs
        tfs = flops / (best * 1e-3) / 1e12
        res[name] = {"Q": Q, "KV": KV, "density": round(pairs / (Q * KV), 4), "tasks": mask.T,
                     "ms": round(best, 3), "TFLOPs": round(tfs, 1),
                     "pct_peak": round(100 * tfs / PEAK_BF16_TFLOPS, 2)}
        del q, tq, k, tk, v, tv
    res["kernel"] = "attn_fwd32_kernel<bf16,jvp,magi>"
    return res


def main():
    args = _args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the attention of one device "
              "(no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    sampler = None
    if args.power or args.clock:  # before any GPU use in this process
        import tempfile

        power_file = tempfile.NamedTemporaryFile(prefix="dmad_power_", suffix=".txt", delete=False).name
        sampler = _start_power_sampler(power_file)

    import torch

    sys.path.insert(0, ROOT)
    from dmad_amd import _native
    from dmad_amd.jvp_attention import backward_plan, jvp_attention_backward, jvp_attention_forward
    from dmad_amd.workload import make_inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    H, L, D, LKX = args.heads, args.seq, 128, 512
    grid = (21, 30, 52) if L == 32760 else ((21, 45, 80) if L == 75600 else None)
    # one CPU generator seeded 0, draws in the order Q, K, V, Qd, Kd, Vd, dO, dOd (reproducible on any host)
    x = make_inputs(1, H, L, L, D, dtype=torch.bfloat16, seed=0, device=dev, grid=grid, with_grads=True)
    q, k, v, tq, tk, tv, do = (x[n] for n in ("q", "k", "v", "tq", "tk", "tv", "do"))
    xc = make_inputs(1, H, L, LKX, D, dtype=torch.bfloat16, seed=1, device=dev)
    kc, vc = xc["k"], xc["v"]
    s = D ** -0.5
    lib = _native.lib()

    f_fwd = 12.0 * H * L * L * D
    f_bwd = 10.0 * H * L * L * D
    f_cross = 8.0 * H * L * LKX * D
    f_step = f_fwd + f_bwd + f_cross

    # the dO-only backward's passes: with stored score gradients the key and query
    # passes run once per group of (b, h) slices ("pairs"), timed pair by pair
    bplan = backward_plan(torch.bfloat16, 1, H, L, L, D)
    timers = []

    def step(record):
        if record:
            tf, tb, tc = _native.KernelTimer(1), _native.KernelTimer(2 * bplan["pairs"]), _native.KernelTimer(1)
            timers.append((tf, tb, tc))
            with tf:
                o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
            with tc:
                jvp_attention_forward(q, kc, vc, tq, None, None, s)
            with tb:
                jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)
        else:
            o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
            jvp_attention_forward(q, kc, vc, tq, None, None, s)
            jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    w0 = time.time()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step(True)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    w1 = time.time()
    ms_step = e0.elapsed_time(e1) / args.steps
    k_ms = {"fwd": 0.0, "bwd_dkdv": 0.0, "bwd_dq": 0.0, "cross": 0.0}
    for tf, tb, tc in timers:
        k_ms["fwd"] += tf.elapsed()[0] / len(timers)
        b = tb.elapsed()
        k_ms["bwd_dkdv"] += sum(b[0::2]) / len(timers)
        k_ms["bwd_dq"] += sum(b[1::2]) / len(timers)
        k_ms["cross"] += tc.elapsed()[0] / len(timers)
    value = f_step / (ms_step * 1e-3) / 1e12

    # algorithmic flops of each main kernel (GEMM flops it must do: the recomputing dQ
    # pass counts its S and dP recomputation, the stored-score one only dQ = s dS K)
    sc = bplan["score_slices"] > 0
    k_flops = {"fwd": f_fwd, "bwd_dkdv": 8.0 * H * L * L * D, "bwd_dq": (2.0 if sc else 6.0) * H * L * L * D,
               "cross": f_cross}
    k_names = {"fwd": "attn_fwd32_kernel<bf16,jvp>",
               "bwd_dkdv": "attn_bwd_kv_tr_kernel<bf16,128,store>" if sc else "attn_bwd_kv_tr_kernel<bf16,128>",
               "bwd_dq": "attn_bwd_dq_sc_kernel<bf16,1>" if sc else "attn_bwd_dq_tr_kernel<bf16,128>",
               "cross": "attn_fwd32_x2_kernel<bf16>"}
    dom = max(k_ms, key=k_ms.get)
    dom_flops, dom_name = k_flops[dom], k_names[dom]
    achieved = dom_flops / (k_ms[dom] * 1e-3) / 1e12
    out = {
        "metric": "attn fwd+JVP+bwd TFLOP/s & %MFMA peak; ms/layer at Wan2.1-14B L=32760",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: one CPU torch.Generator seeded 0, drawn in the order Q, K, V, Qd, Kd, Vd, dO, dOd as "
                "float32 and cast to bf16 (Q, K: N(0,1) RMS-normalised over H*D and 3D-RoPE rotated; V, dO ~ N(0,1); "
                "tangents, dOd ~ N(0,0.1^2)); cross-attention keys from a second generator seeded 1",
        "config": {
            "workload": f"Wan2.1 self-attn fwd+JVP+bwd(dO-only) + text cross-attn fwd+JVP, one layer",
            "B": 1, "H": H, "L": L, "D": D, "cross_keys": LKX,
            "step_tflop": round(f_step / 1e12, 3),
        },
        "pct_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "ms_self_fwd_jvp_kernel": round(k_ms["fwd"], 3),
        "ms_self_bwd_dkdv_kernel": round(k_ms["bwd_dkdv"], 3),
        "ms_self_bwd_dq_kernel": round(k_ms["bwd_dq"], 3),
        "ms_cross_fwd_jvp_kernel": round(k_ms["cross"], 4),
        "bwd_kernels": {"dkdv": k_names["bwd_dkdv"], "dq": k_names["bwd_dq"], "pairs": bplan["pairs"],
                        "score_slices_per_pair": bplan["score_slices"]},
        "kernel_pct_peak": {n: round(100 * k_flops[n] / (k_ms[n] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)
                            for n in k_ms},
        # the whole dO-only backward (both passes, every launch pair) on the reference's 10 units
        "bwd_pct_peak": round(100 * f_bwd / ((k_ms["bwd_dkdv"] + k_ms["bwd_dq"]) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "roofline": {
            "kernel": dom_name,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": _traffic_from_profiles(dom_name),
        },
        "wall_s_timed": round(wall, 3),
    }
    if sc:
        # the stored-score query pass streams the dS tiles from HBM once: its bound is HBM
        sc_bytes = H * _native.bwd_score_bytes(_native.DMAD_BF16, False, L, L, D)
        tbs = sc_bytes / (k_ms["bwd_dq"] * 1e-3) / 1e12
        out["bwd_dq_hbm"] = {"bytes_read": sc_bytes, "achieved_TBps": round(tbs, 3), "peak_TBps": 8.0,
                             "frac": round(tbs / 8.0, 4)}
    if sampler is not None and not args.power:
        # mean GFX clock and board power over the timed steps: the board runs at its power
        # limit, so the clock (not only the kernels) sets the step time. amd-smi gives about
        # one reading per 0.1 s and its power reading trails a change of load, so the window
        # skips its first 0.5 s and is continued with the same step, untimed, until it spans 3 s.
        extra = 0
        while time.time() - w0 < 3.0:
            step(False)
            torch.cuda.synchronize()
            extra += 1
        w2 = time.time()
        time.sleep(0.3)
        sampler.terminate()
        sampler.wait()
        out["clock_timed"] = _power_summary(power_file, w0 + 0.5, w2)
        out["clock_timed"].update({"window_s": round(w2 - w0 - 0.5, 2), "untimed_steps_after": extra})
        os.unlink(power_file)
    if sampler is not None and args.power:
        # then each main pass alone for ~3 s, so each gets its own power/clock window
        def phase(fn):
            a = time.time()
            while time.time() - a < 3.0:
                for _ in range(4):
                    fn()
                torch.cuda.synchronize()
            return a, time.time()

        windows = {"step": (w0, w1)}
        o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
        windows["fwd_jvp"] = phase(lambda: jvp_attention_forward(q, k, v, tq, tk, tv, s))
        windows["bwd_dout_only"] = phase(
            lambda: jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False))
        time.sleep(0.3)
        sampler.terminate()
        sampler.wait()
        # skip the first 0.5 s of each window: the clock settles after a change of load
        out["power"] = {name: _power_summary(power_file, a + 0.5, b) for name, (a, b) in windows.items()}
        os.unlink(power_file)
    if args.ceiling:
        out["mfma_ceiling"] = mfma_ceiling(dev, {n: k_flops[n] / (k_ms[n] * 1e-3) / 1e12 for n in k_ms})
    if args.full_bwd:
        out["full_derivative_bwd"] = full_bwd_timing(q, k, v, tq, tk, tv, do, x["dto"])
    # fused RMSNorm(+JVP) + RoPE prologue that produces q and k for this layer,
    # timed after the step (HBM-bound; not part of the step or its flops)
    if args.prologue:
        out["prologue_rmsnorm_rope_jvp"] = prologue_timing(H, L, D, grid, dev)
    if args.plain:
        out["plain_attn_fwd_bwd"] = plain_timing(q, k, v, do, dev)
    if args.magi:
        out["magi_fwd_jvp"] = magi_timing(H, D, dev)
    if args.harness:
        dims = {int(d) for d in args.harness_dims.split(",") if d}
        out["reference_harness"] = [harness_timing(dev, D=d) for d in (64, 128) if d in dims]
        # the harness's own inputs: sm_scale = 1.3, zero tangents (:686-698)
        out["reference_harness_as_written"] = [harness_timing(dev, D=d, as_reference=True) for d in (64, 128)
                                               if d in dims]
        # the other head dims the reference accepts (:471-472): 16 and 32 on the generic kernels, 256 on the
        # row-reading forward, the generic dK/dV pass and the row-reading dQ pass
        out["other_head_dims"] = [harness_timing(dev, D=d, lengths=(1024, 4096, 16384)) for d in (16, 32, 256)
                                  if d in dims]
        out["fp32_harness"] = [harness_timing(dev, D=d, lengths=(1024, 4096, 16384), dtype=torch.float32)
                               for d in (64, 128) if d in dims]
    if args.calibration_copy_mib:
        n = args.calibration_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)  # reads n*4 bytes, writes n*4 bytes
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(x, H, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
