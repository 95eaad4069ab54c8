"""bench.py host logic on the CPU: the one-GPU rule, the committed traffic
figure it reports, and the power summary of its sampler (no GPU work)."""
import importlib.util
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_exits_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_traffic_figure_comes_from_the_committed_counters():
    bench = _bench()
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        table = json.load(f)
    name = "attn_fwd32_kernel<bf16,jvp>"
    assert bench._traffic_from_profiles(name) == table[name] > 0
    assert bench._traffic_from_profiles("no such kernel") is None


def test_power_summary_keeps_the_timed_window(tmp_path):
    bench = _bench()
    p = tmp_path / "power.txt"
    p.write_text("10.0 1300 1800\n11.0 1350 1700\n12.0 1340 1750\n13.0 900 2100\n")
    s = bench._power_summary(str(p), 10.5, 12.5)
    assert s["samples"] == 2 and s["avg_W"] == 1345.0 and s["max_W"] == 1350.0 and s["avg_gfx_MHz"] == 1725
    assert bench._power_summary(str(p), 20.0, 30.0) == {"samples": 0}
