"""bench.py host logic: compulsory bytes per kernel and the roofline bound
(no GPU needed)."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402
from rbf_attention_amd import workloads as wl  # noqa: E402


def test_algorithmic_bytes_c2():
    w = wl.CONFIGS["c2_model_bf16"]
    t = 32 * 8 * 516 * 64 * 2  # one (B,H,N,D) bf16 tensor
    v = 32 * 8 * 516 * 4  # one (B,H,N) fp32 vector
    assert bench.algorithmic_bytes(w, "fwd") == 4 * t + v
    assert bench.algorithmic_bytes(w, "bwd_dq") == 6 * t + 3 * v
    assert bench.algorithmic_bytes(w, "bwd_dkdv") == 6 * t + 2 * v
    # one-launch backward: q, k, v, dO, o, L in; dq, dk, dv, Delta out
    assert bench.algorithmic_bytes(w, "bwd") == 8 * t + 2 * v


def test_algorithmic_bytes_non_softmax():
    w = wl.CONFIGS["c4_nonsoftmax_bf16"]
    t = w.B * w.H * w.N * w.D * 2
    v = 4 * w.B * w.H * w.N
    assert bench.algorithmic_bytes(w, "fwd") == 4 * t
    assert bench.algorithmic_bytes(w, "bwd_dq") == 5 * t + v
    assert bench.algorithmic_bytes(w, "bwd_dkdv") == 6 * t + v
    assert bench.algorithmic_bytes(w, "bwd") == 7 * t + v


def test_roofline_bound_follows_intensity():
    c2 = wl.CONFIGS["c2_model_bf16"]
    flops = 8.0 * c2.D * c2.visible_pairs() * c2.B * c2.H
    r = bench.roofline(c2, "bwd_dkdv", flops, 50e-6, 2500.0)
    # 8*64 flop per pair over ~102 MB: ~171 flop/B, below the 312.5 ridge
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["achieved"] == pytest.approx(bench.algorithmic_bytes(c2, "bwd_dkdv") / 50e-6 / 1e9, rel=1e-3)
    assert r["frac"] == pytest.approx(r["achieved"] / 8000.0, rel=1e-3)
    assert r["ai_flop_per_byte"] < r["ridge_flop_per_byte"] == 312.5

    c3 = wl.CONFIGS["c3_long_bf16"]
    flops3 = 8.0 * c3.D * c3.visible_pairs() * c3.B * c3.H
    r3 = bench.roofline(c3, "bwd_dkdv", flops3, 2.5e-3, 2500.0)
    assert r3["bound"] == "mfma" and r3["unit"] == "TFLOP/s"
    assert r3["achieved"] == pytest.approx(flops3 / 2.5e-3 / 1e12, rel=1e-3)


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert p.returncode != 0
    assert "one GPU" in (p.stdout + p.stderr)
