"""bench.py end to end on the GPU at a short setting: one JSON line with the
contract's keys, a roofline entry for a kernel the step runs, the
cold-cache step, the peak forward activation memory, a CPU baseline, and a
config-5 train step whose loss is finite and falls."""
import json
import math
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*extra):
    cmd = [sys.executable, os.path.join(REPO, "bench.py"), "--steps", "3", "--warmup", "1", "--ramp-seconds", "0.05",
           "--cold-reps", "3", "--cpu-seconds", "1", *extra]
    print("running", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=REPO)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [l for l in p.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, p.stdout
    return json.loads(lines[0])


def check_roofline(roof, step_kernels):
    assert roof["kernel"] in step_kernels and roof["bound"] in ("hbm", "mfma")
    assert roof["unit"] == ("GB/s" if roof["bound"] == "hbm" else "TFLOP/s")
    assert 0 < roof["frac"] < 1 and roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], rel=1e-3)


def test_bench_json_line(cuda_device):
    r = run_bench("--train-steps", "6", "--no-extra-configs", "--no-ref-sweep")
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "cold",
                "peak_fwd_activation_mb"):
        assert key in r, key
    assert r["n_gpus"] == 1 and r["steps"] == 3 and r["warmup"] == 1 and r["dtype"] == "bf16"
    assert r["config"]["workload"] == "c2_model_bf16"
    assert r["value"] > 0 and r["ms_per_step"] > 0
    check_roofline(r["roofline"], r["step_kernels"])
    assert r["cold"]["step_us_median"] > 0 and r["cold"]["reps"] == 3
    # the op-level step runs the same kernels plus Python dispatch and allocation
    assert r["op_step_us"] >= 0.9 * r["ms_per_step"] * 1e3
    assert r["op_graph_step_us"] is not None and r["op_graph_step_us"] > 0
    # the C++ harness times the same step through the C ABI without Python
    nh = r["native_harness"]
    assert "error" not in nh, nh
    assert nh["workload"] == "c2_model_bf16" and nh["steps"] == 3 and nh["cold"]["reps"] == 3
    assert 0.5 < nh["step_us"] / (r["ms_per_step"] * 1e3) < 2.0
    # the forward keeps out (B,H,N,D bf16) and L (B,H,N fp32) for backward
    expect = (32 * 8 * 516 * 64 * 2 + 32 * 8 * 516 * 4) / 2 ** 20
    assert r["peak_fwd_activation_mb"] == pytest.approx(expect, rel=0.05)
    cpu = r["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] >= 1 and cpu["kind"] in ("port", "reference") and cpu["sample"]
    ts = r["train_step"]
    assert ts["value"] > 0
    assert math.isfinite(ts["loss_first"]) and math.isfinite(ts["loss_last"])
    # random init over a vocab of 8192: ~ln(8192) = 9.01 at the start, and the
    # steps on the repeated batch lower it
    assert abs(ts["loss_first"] - math.log(8192)) < 1.0
    assert ts["loss_last"] < ts["loss_first"]
    assert r["decode"]["value"] > 0


def test_bench_extra_configs(cuda_device):
    """The C3 and C4 objects (GPU only) carry a step time, per-kernel times
    and a roofline entry on their dominant kernel."""
    r = run_bench("--no-train-step", "--no-decode", "--no-cpu-baseline", "--no-ref-sweep")
    for key, wname in (("c3", "c3_long_bf16"), ("c4", "c4_nonsoftmax_bf16")):
        c = r[key]
        assert c["config"]["workload"] == wname
        assert c["step_us"] > 0 and c["tflops"] > 0 and c["cold"]["step_us_median"] > 0
        assert c["op_step_us"] >= 0.9 * c["step_us"]
        assert c["roofline"]["bound"] == "mfma"
        check_roofline(c["roofline"], c["step_kernels"])
    # the C++ harness (C ABI, no Python) times the same C3 step
    nh = r["c3"]["native_harness"]
    assert "error" not in nh, nh
    assert 0.8 < nh["step_us"] / r["c3"]["step_us"] < 1.25
