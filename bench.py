"""Benchmark of the fused RBF attention hot path on one MI355X.

A step is one forward + backward of the benchmark's model-shaped
configuration (c2_model_bf16: B=32, H=8, N=512+4 registers, D=64, bf16,
causal) on synthetic seeded inputs resident in HBM, called through the C ABI
(rbf_attn_fwd, rbf_attn_bwd) on torch's current stream.  The backward is one
kernel where every head fits one work-group (the dQ pass, then the dK/dV
pass, of each head; c2) and two otherwise (dQ(+Delta), then dK/dV; c3, c4).
Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--quick]

Timing protocol
  * Before the W warmup steps the step runs for --ramp-seconds (default 0.4 s)
    untimed, so that the timed steps see the GPU's steady clocks: in a fresh
    process the first ~100 C2 steps ran up to 9 % slower.  The reference's own
    benchmark does the same through triton.testing.do_bench, whose warm-up is
    25 ms of calls (rbf_attention.py:1877, 1888).
  * `value` / `ms_per_step`: exactly K back-to-back steps between two HIP
    events on the launch stream (warm caches: the step's ~205 MB working set
    stays in the 256 MB MALL between steps).
  * `kernel_us`: each kernel of the step in an event-timed loop of its own,
    run right after the step loop (clocks still at their steady state), of
    at least 200 launches and 0.2 s; the roofline entry is computed from the
    dominant one.  `kernel_sum_us` is the sum over the step's kernels, which
    should match `step_us` (the kernels of a step run back to back).
  * `cold`: the protocol of the reference's do_bench (a cache-evicting write
    before every rep; rbf_attention.py:1877, 1888): the median over >= 20
    reps of one step timed alone after a 512 MiB write that evicts L2 and
    MALL (outside the events); likewise the forward alone, the backward alone
    from the saved forward outputs, and each kernel of the step.  `value` is
    the warm step: in a model the attention's inputs are written by the
    projections just before it (and dO by the layer above), so they arrive
    in the cache hierarchy as they do in back-to-back steps.
  * `native_harness`: the same step timed by rbf_attn_bench, a C++ program
    that calls the C ABI directly (no Python), in a child process, with the
    same protocol (ramp, warm-up, K steps between events, cold reps).
  * `op_step_us`: the same step through the torch ops instead of the C ABI
    (run_triton_rbf / run_triton_non_softmax_rbf forward, then backward through
    their autograd): Python dispatch and the outputs, L and gradients from
    torch's caching allocator on top of the same kernels.  `op_graph_step_us`:
    those op-level steps captured ten to a graph and replayed (per step).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "RBF-attn fwd+bwd TFLOP/s and % bf16 MFMA peak; train-step tokens/s"
PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp32": 157.3}  # MI355X dense MFMA
HBM_GBS = 8000.0
FLUSH_MIB = 512  # > the 256 MB MALL + 8 x 4 MB L2

# The reference's own benchmark sweep (rbf_attention.py:1768-1771, 1819-1911:
# fp16, B=4, H=8, D=64, causal, torch.compile'd op, do_bench) and the values
# its only published figure shows (outputs/attention_profiling_results.png,
# read off the plot, +-3 %; the GPU is not recorded).
REF_SWEEP = {"B": 4, "H": 8, "D": 64, "dtype": "fp16", "N": (1024, 2048, 4096, 8192)}
REF_PUBLISHED = {
    1024: {"fwd_ms": 0.13, "bwd_ms": 0.35, "peak_mb": 4.2},
    2048: {"fwd_ms": 0.38, "bwd_ms": 1.07, "peak_mb": 8.3},
    4096: {"fwd_ms": 1.28, "bwd_ms": 3.78, "peak_mb": 16.5},
    8192: {"fwd_ms": 4.67, "bwd_ms": 14.25, "peak_mb": 33.0},
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_args(_lib, w, bufs, variant):
    a = _lib.Args()
    a.abi_version = _lib.ABI_VERSION
    a.variant = variant
    a.dtype = _lib.DTYPE_CODES[w.torch_dtype]
    a.B, a.H, a.N, a.D = w.B, w.H, w.N, w.D
    a.causal = 1 if w.causal else 0
    a.num_prefix = 0
    a.gamma = w.sm_scale
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(bufs[f]))
    a.lse = bufs["lse"].data_ptr()
    a.delta = bufs["delta"].data_ptr()
    return a


def cpu_baseline(w, target_s: float):
    """The reference math path (oracle/math_path.py) on the host CPU, on a
    bounded sample of the workload: the first B' batch rows (all of them when
    one pass fits in a third of the time budget), repeated for about
    target_s seconds."""
    import torch

    from oracle import math_path
    from rbf_attention_amd import workloads as wl

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def one(sample):
        q, k, v, do = wl.make_inputs(sample)
        t0 = time.perf_counter()
        math_path.fwd_bwd(q, k, v, do, sample.sm_scale, softmax=w.softmax, is_causal=w.causal)
        return time.perf_counter() - t0, (q, k, v, do)

    sample = w.with_(B=1)
    first, _ = one(sample)  # warm-up and size probe
    b = max(1, min(w.B, int((target_s / 3.0) / max(first, 1e-4))))
    sample = w.with_(B=b)
    _, (q, k, v, do) = one(sample)
    times = []
    t_end = time.perf_counter() + target_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        math_path.fwd_bwd(q, k, v, do, sample.sm_scale, softmax=w.softmax, is_causal=w.causal)
        times.append(time.perf_counter() - t0)
    reps = len(times)
    med = statistics.median(times)
    return {
        "value": round(sample.flops_fwd_bwd() / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"reference math path restated in torch fp32 on CPU (augmented-dimension SDPA + autograd, "
            f"test_equivalence.py:9-33), fwd+bwd of B={sample.B} of {w.B} (H={w.H}, N={w.N}, D={w.D}); "
            f"median of {reps} reps = {med * 1e3:.1f} ms ({sum(times):.1f} s of CPU work) after a warm-up"
        ),
    }


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload`, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.json,
    calibrated on a copy kernel of known size); None if not profiled."""
    path = os.path.join(REPO, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None


def algorithmic_bytes(w, kernel: str) -> float:
    """Compulsory HBM bytes of one launch: every input read once, every
    output written once (element tensors (B,H,N,D), fp32 (B,H,N) vectors).
    fwd: q, k, v -> o (+ L); dQ: q, k, v, dO (+ o, L) -> dq, Delta (or the
    non-softmax norm offsets); dK/dV: q, k, v, dO, L (+ Delta) -> dk, dv;
    bwd (both passes in one kernel): q, k, v, dO (+ o, L) -> dq, dk, dv,
    Delta (or the norm offsets)."""
    esz = {"bf16": 2, "fp16": 2, "fp32": 4}[w.dtype]
    t = w.B * w.H * w.N * w.D * esz
    vec = 4 * w.B * w.H * w.N
    if kernel == "fwd":
        return 4 * t + (vec if w.softmax else 0)
    if kernel == "bwd":
        return (8 * t + 2 * vec) if w.softmax else (7 * t + vec)
    if kernel == "bwd_dq":
        return (6 * t + 3 * vec) if w.softmax else (5 * t + vec)
    return (6 * t + 2 * vec) if w.softmax else (6 * t + vec)


def roofline(w, kernel: str, flops: float, seconds: float, peak_tflops: float):
    """Roofline entry of one kernel.  The bound is the lower roof at the
    kernel's arithmetic intensity (attributed flops / compulsory bytes): HBM
    below the ridge (peak flops / 8 TB/s), MFMA above it."""
    nbytes = algorithmic_bytes(w, kernel)
    ai = flops / nbytes
    ridge = peak_tflops * 1e12 / (HBM_GBS * 1e9)
    if ai < ridge:
        achieved, peak, unit, bound = nbytes / seconds / 1e9, HBM_GBS, "GB/s", "hbm"
    else:
        achieved, peak, unit, bound = flops / seconds / 1e12, peak_tflops, "TFLOP/s", "mfma"
    return {
        "kernel": kernel,
        "bound": bound,
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 5),
        "traffic": measured_traffic(w.name, kernel),
        "algorithmic_bytes": nbytes,
        "flops": flops,
        "ai_flop_per_byte": round(ai, 1),
        "ridge_flop_per_byte": round(ridge, 1),
        "mfma_frac": round(flops / seconds / 1e12 / peak_tflops, 5),
    }


class Timer:
    """HIP-event timing on one stream, and an L2/MALL flush buffer."""

    def __init__(self, torch, dev, stream):
        self.torch, self.dev, self.stream = torch, dev, stream
        self._flush = None

    def kernel_loop(self, fn, min_s: float = 0.2, min_n: int = 200) -> float:
        """Mean ms of back-to-back calls of one kernel: at least min_n calls
        and min_s seconds, after a short loop that also estimates the count."""
        est = self.loop(fn, 20)
        n = max(min_n, int(math.ceil(min_s / max(est * 1e-3, 1e-7))))
        return self.loop(fn, min(n, 20000))

    def loop(self, fn, n: int) -> float:
        """Mean ms of n back-to-back calls between two events."""
        torch = self.torch
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(self.stream)
        for _ in range(n):
            fn()
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def flush(self):
        if self._flush is None:
            self._flush = self.torch.empty(FLUSH_MIB << 18, device=self.dev, dtype=self.torch.float32)
        self._flush.fill_(1.0)

    def cold(self, fn, reps: int, pre=None) -> list:
        """ms of single calls, each after a cache-evicting write (and pre(),
        e.g. resetting gradients), both outside the events."""
        torch = self.torch
        out = []
        for _ in range(reps):
            if pre is not None:
                pre()
            self.flush()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            fn()
            e1.record(self.stream)
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1))
        return out

    def ramp(self, fn, seconds: float) -> int:
        """Runs fn untimed for about `seconds` (clock ramp); returns the count."""
        n, t_end = 0, time.perf_counter() + seconds
        while time.perf_counter() < t_end:
            for _ in range(8):
                fn()
            n += 8
            self.torch.cuda.synchronize()
        return n


def setup_workload(w, dev):
    import torch

    from rbf_attention_amd import _lib
    from rbf_attention_amd import workloads as wl

    q, k, v, do = (t.to(dev) for t in wl.make_inputs(w))
    bufs = {"q": q, "k": k, "v": v, "dout": do}
    for f in ("o", "dq", "dk", "dv"):
        bufs[f] = torch.empty_like(q)
    bufs["lse"] = torch.empty((w.B, w.H, w.N), device=dev, dtype=torch.float32)
    bufs["delta"] = torch.empty_like(bufs["lse"])
    variant = _lib.SOFTMAX if w.softmax else _lib.NON_SOFTMAX
    return bufs, make_args(_lib, w, bufs, variant)


GRAPH_STEPS = 10  # steps per captured HIP graph (graph_step_us)


def measure_workload(w, dev, timer, steps: int, warmup: int, ramp_s: float, cold_reps: int, graph: bool,
                     kernel_s: float = 0.2, kernel_n: int = 200):
    """Step, per-kernel and cold-cache timings of one workload through the C
    ABI; returns (result dict, step ms)."""
    import torch

    from rbf_attention_amd import _lib

    bufs, a = setup_workload(w, dev)
    sp = timer.stream.cuda_stream

    def fwd():
        _lib.call("rbf_attn_fwd", a, sp)

    def bwd():
        _lib.call("rbf_attn_bwd", a, sp)

    def stage(s):
        return lambda: _lib.call("rbf_attn_bwd_stage", a, sp, s)

    def step():
        fwd()
        bwd()

    ramp_n = timer.ramp(step, ramp_s)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ms_step = timer.loop(step, steps)
    wall = time.perf_counter() - wall0
    log(f"{w.name}: step {ms_step * 1e3:.2f} us over {steps} steps (ramp {ramp_n} steps, wall {wall:.3f} s)")

    # Per-kernel averages, each kernel in a loop of its own (events between
    # single launches add their own cost to every launch), right after the
    # step loop while the clocks are at their steady state.  With a
    # one-launch backward its two stages are timed too, for reference.
    bwd_launches = _lib.bwd_kernels(a)
    step_kernels = ("fwd", "bwd") if bwd_launches == 1 else ("fwd", "bwd_dq", "bwd_dkdv")
    calls = {"fwd": fwd, "bwd": bwd, "bwd_dq": stage(1), "bwd_dkdv": stage(2)}
    timed_kernels = step_kernels + (("bwd_dq", "bwd_dkdv") if bwd_launches == 1 else ())
    kern_ms = {kname: timer.kernel_loop(calls[kname], kernel_s, kernel_n) for kname in timed_kernels}
    for kname, t in kern_ms.items():
        log(f"  {kname}: {t * 1e3:.2f} us/launch" + ("" if kname in step_kernels else " (stage alone)"))
    kern_sum = sum(kern_ms[kk] for kk in step_kernels)
    log(f"  sum of the step's kernels {kern_sum * 1e3:.2f} us against the step's {ms_step * 1e3:.2f} us")

    # Cold caches: every rep after a cache-evicting write.  The backward alone
    # reads the outputs the last forward saved (O, L), as in training.
    cold = timer.cold(step, cold_reps)
    cold_med = statistics.median(cold)
    log(f"  cold step (after a {FLUSH_MIB} MiB write): median {cold_med * 1e3:.2f} us of {cold_reps}")
    cold_fwd = statistics.median(timer.cold(fwd, cold_reps))
    step()
    cold_bwd = statistics.median(timer.cold(bwd, cold_reps))
    cold_kern = {kname: statistics.median(timer.cold(calls[kname], cold_reps)) for kname in timed_kernels}
    log(f"  cold fwd {cold_fwd * 1e3:.2f} us, cold bwd {cold_bwd * 1e3:.2f} us, per kernel "
        + ", ".join(f"{kk} {t * 1e3:.2f}" for kk, t in cold_kern.items()))

    ms_graph = None
    if graph:
        # GRAPH_STEPS steps captured in one HIP graph and replayed; reported
        # per step, beside the eager step, not as it.  Several steps per
        # graph separate the graph launch's own cost from the time added
        # between kernel nodes.
        def cur_step():
            s = torch.cuda.current_stream(dev).cuda_stream
            _lib.call("rbf_attn_fwd", a, s)
            _lib.call("rbf_attn_bwd", a, s)

        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(GRAPH_STEPS):
                    cur_step()
            g.replay()
            ms_graph = timer.loop(g.replay, max(1, steps // GRAPH_STEPS)) / GRAPH_STEPS
            log(f"  graph step: {ms_graph * 1e3:.2f} us ({GRAPH_STEPS} steps per graph)")
        except RuntimeError as e:  # reported as null; the eager measurement stands
            log(f"  graph step: capture failed ({e})")

    # The same step through the torch ops (the rbf_attn_v5 / rbf_attn_amd ops
    # and their autograd): Python dispatch, output, L and gradient tensors
    # from torch's caching allocator, then the same kernels.
    import rbf_attention_amd as ra

    op_fn = ra.run_triton_rbf if w.softmax else ra.run_triton_non_softmax_rbf
    oq, ok_, ov = (bufs[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v"))

    def op_step():
        oq.grad = ok_.grad = ov.grad = None
        op_fn(oq, ok_, ov, w.causal, sm_scale=w.sm_scale).backward(bufs["dout"])

    with torch.cuda.stream(timer.stream):
        for _ in range(max(3, warmup // 10)):
            op_step()
        ms_op = timer.loop(op_step, steps)
    log(f"  op-level step (torch ops + autograd): {ms_op * 1e3:.2f} us")
    ms_op_graph = None
    if graph:
        # The op-level steps captured in one graph (outputs and gradients from
        # the graph's pool): the host cost of dispatch and autograd is paid
        # once, at capture.
        try:
            og = torch.cuda.CUDAGraph()
            oq.grad = ok_.grad = ov.grad = None
            with torch.cuda.graph(og):
                for _ in range(GRAPH_STEPS):
                    op_step()
            og.replay()
            ms_op_graph = timer.loop(og.replay, max(1, steps // GRAPH_STEPS)) / GRAPH_STEPS
            log(f"  op-level graph step: {ms_op_graph * 1e3:.2f} us ({GRAPH_STEPS} steps per graph)")
            del og
        except RuntimeError as e:  # reported as null; the eager measurements stand
            log(f"  op-level graph step: capture failed ({e})")
    del oq, ok_, ov

    P = w.visible_pairs() * w.B * w.H
    per_pair = {"fwd": 4.0, "bwd_dq": 2.0, "bwd_dkdv": 8.0, "bwd": 10.0}  # algorithmic flop/pair/D per kernel
    total = w.flops_fwd_bwd()
    peak = PEAK_TFLOPS[w.dtype]
    dom = max(step_kernels, key=kern_ms.get)
    tflops = total / (ms_step * 1e-3) / 1e12
    res = {
        "step_us": round(ms_step * 1e3, 3),
        "tflops": round(tflops, 3),
        "pct_of_bf16_peak": round(100.0 * tflops / peak, 3),
        "cold": {
            "step_us_median": round(cold_med * 1e3, 3),
            "tflops": round(total / (cold_med * 1e-3) / 1e12, 3),
            "fwd_us_median": round(cold_fwd * 1e3, 3),
            "bwd_us_median": round(cold_bwd * 1e3, 3),
            "kernel_us_median": {kk: round(t * 1e3, 3) for kk, t in cold_kern.items()},
            "reps": cold_reps,
            "flush": f"{FLUSH_MIB} MiB write before each rep, outside the events",
        },
        "graph_step_us": round(ms_graph * 1e3, 3) if ms_graph is not None else None,
        "op_step_us": round(ms_op * 1e3, 3),
        "op_graph_step_us": round(ms_op_graph * 1e3, 3) if ms_op_graph is not None else None,
        "kernel_us": {kk: round(t * 1e3, 3) for kk, t in kern_ms.items()},
        "kernel_sum_us": round(kern_sum * 1e3, 3),
        "step_kernels": list(step_kernels),
        "roofline": roofline(w, dom, per_pair[dom] * w.D * P, kern_ms[dom] * 1e-3, peak),
        "config": {
            "workload": w.name, "B": w.B, "H": w.H, "N": w.N, "D": w.D, "dtype": w.dtype, "causal": w.causal,
            "softmax": w.softmax, "gamma": w.sm_scale, "flops_per_step": total,
        },
    }
    del bufs
    return res, ms_step


def peak_fwd_mb(dev, w) -> float:
    """Peak memory the forward op allocates with autograd recording (its
    saved output and L), as rbf_attention.py:1809-1816 measures it."""
    import torch

    import rbf_attention_amd as ra
    from rbf_attention_amd import workloads as wl

    q, k, v, _ = (t.to(dev).requires_grad_(True) for t in wl.make_inputs(w))
    fn = ra.run_triton_rbf if w.softmax else ra.run_triton_non_softmax_rbf
    out = fn(q, k, v, w.causal)  # first call outside the probe (library load)
    del out
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    out = fn(q, k, v, w.causal)
    peak = (torch.cuda.max_memory_allocated(dev) - base) / (1024 * 1024)
    del out
    return round(peak, 3)


def reference_sweep(dev, timer, reps: int):
    """The reference's own benchmark (rbf_attention.py:1819-1911) on our op:
    fp16 B=4 H=8 D=64 causal, N = 1024..8192, gamma = 1/sqrt(D) through
    run_triton_rbf (the rbf_attn_v5 ops and their autograd).  Like
    triton.testing.do_bench: each rep is timed alone after a cache-evicting
    write, gradients reset to None outside the events, mean over reps;
    bwd = (fwd + bwd) - fwd (rbf_attention.py:1891)."""
    import torch

    import rbf_attention_amd as ra

    c = REF_SWEEP
    out = {"config": dict(c, N=list(c["N"]), causal=True, gamma="1/sqrt(D)", op="run_triton_rbf",
                          timing=f"mean of {reps} reps, each after a {FLUSH_MIB} MiB write"), "rows": []}
    for n in c["N"]:
        g = torch.Generator().manual_seed(0)
        shape = (c["B"], c["H"], n, c["D"])
        q, k, v, do = (torch.randn(shape, generator=g).to(torch.float16).to(dev) for _ in range(4))
        for t in (q, k, v):
            t.requires_grad_(True)

        def fwd():
            with torch.no_grad():
                ra.run_triton_rbf(q, k, v, True)

        def fwd_bwd():
            o = ra.run_triton_rbf(q, k, v, True)
            o.backward(do)

        def reset():
            q.grad = k.grad = v.grad = None

        for _ in range(3):
            reset()
            fwd_bwd()
        timer.ramp(fwd, 0.05)
        f_ms = statistics.fmean(timer.cold(fwd, reps))
        fb_ms = statistics.fmean(timer.cold(fwd_bwd, reps, pre=reset))
        reset()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        o = ra.run_triton_rbf(q, k, v, True)
        peak = (torch.cuda.max_memory_allocated(dev) - base) / (1024 * 1024)
        del o
        flops = 2.0 * c["B"] * c["H"] * n * n * c["D"]  # the figure's FA convention: causal fwd
        pub = REF_PUBLISHED[n]
        row = {
            "N": n,
            "fwd_ms": round(f_ms, 4),
            "bwd_ms": round(fb_ms - f_ms, 4),
            "peak_fwd_mb": round(peak, 2),
            "fwd_tflops_fa": round(flops / (f_ms * 1e-3) / 1e12, 1),
            "bwd_tflops_fa": round(2.5 * flops / ((fb_ms - f_ms) * 1e-3) / 1e12, 1),
            "published": pub,
            "speedup_vs_published": {"fwd": round(pub["fwd_ms"] / f_ms, 2), "bwd": round(pub["bwd_ms"] / (fb_ms - f_ms), 2)},
        }
        out["rows"].append(row)
        log(f"  ref sweep N={n}: fwd {row['fwd_ms']} ms, bwd {row['bwd_ms']} ms, peak {row['peak_fwd_mb']} MB "
            f"(published {pub})")
        del q, k, v, do
    return out


def train_step_bench(dev, steps: int, warmup: int):
    """Benchmark config 5: one next-token training step (bf16 autocast fwd,
    bwd, AdamW) of the 8-layer d512 RBF transformer on synthetic tokens,
    with the HIP attention kernels.  Returns a dict for the JSON line."""
    import torch

    from rbf_attention_amd import model as M

    cfg = M.ModelConfig()
    batch, seq = 32, 512
    torch.manual_seed(0)
    model = M.CausalLM(cfg).to(dev)
    tr = M.Trainer(model)
    tokens = M.synthetic_tokens(batch, seq, cfg.vocab_size, device=dev)
    first = tr.step(tokens)
    for _ in range(max(0, warmup - 1)):
        tr.step(tokens)
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        last = tr.step(tokens)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {
        "metric": "train-step tokens/s",
        "value": round(batch * seq / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms, 4),
        "steps": steps,
        "warmup": warmup,
        "dtype": "bf16 autocast",
        "loss_first": round(float(first), 4),
        "loss_last": round(float(last), 4),
        "attention_tflop_per_step": round(M.attention_flops_per_step(cfg, batch, seq) / 1e12, 4),
        "config": {
            "workload": "c5_train_step",
            "layers": cfg.num_layers,
            "d_model": cfg.d_model,
            "heads": cfg.num_heads,
            "registers": cfg.num_registers,
            "vocab": cfg.vocab_size,
            "tied_embeddings": cfg.tie_embeddings,
            "batch": batch,
            "seq_len": seq,
            "optimizer": "AdamW",
            "params": M.gpt_param_count(model),
        },
    }


DECODE_WORKLOAD = {"B": 8, "H": 16, "T": 1, "L": 16384, "D": 128}


def decode_bench(dev, iters: int):
    """KV-cache decode (the build's rbf_attn_decode; no reference counterpart):
    one new token per (batch, head) against a 16K-token bf16 cache.  HBM-bound:
    the algorithmic bytes are the K and V caches plus q and o."""
    import torch

    from rbf_attention_amd import ops

    c = DECODE_WORKLOAD
    g = torch.Generator().manual_seed(7)
    shape = (c["B"], c["H"], c["L"], c["D"])
    k = torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn((c["B"], c["H"], c["T"], c["D"]), generator=g).to(torch.bfloat16).to(dev)
    gamma = 1.0 / (2 * c["D"] ** 0.5)
    for _ in range(3):
        ops.rbf_decode(q, k, v, sm_scale=gamma)
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(iters):
        ops.rbf_decode(q, k, v, sm_scale=gamma)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "decode HBM GB/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "us_per_call": round(ms * 1e3, 2),
        "iters": iters,
        "dtype": "bf16",
        "config": dict(c, workload="decode_kv16k_bf16", softmax=True, gamma=gamma),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_GBS, 4), "traffic": measured_traffic("decode_kv16k_bf16", "decode")},
    }


def native_harness(workload: str, steps: int, warmup: int, cold_reps: int, ramp_s: float) -> dict:
    """The same step timed by rbf_attn_bench, the C++ harness that calls the
    C ABI directly (built next to librbfattn.so), as a child process."""
    import subprocess

    exe = os.path.join(REPO, "rbf_attention_amd", "rbf_attn_bench")
    if not os.path.exists(exe):
        return {"error": f"{exe} not built (python -m rbf_attention_amd.build)"}
    cmd = [exe, "--workload", workload, "--steps", str(steps), "--warmup", str(warmup), "--cold-reps",
           str(cold_reps), "--ramp-seconds", str(ramp_s)]
    try:
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    except subprocess.TimeoutExpired:
        return {"error": "timed out after 120 s"}
    if p.returncode != 0:
        return {"error": f"rc={p.returncode}: {p.stderr.strip()[-500:]}"}
    return json.loads(p.stdout.strip().splitlines()[-1])


# Length sweep (--length-sweep): bf16 causal softmax, the same 2^19 tokens per
# step at every N (B x H x N = 524288, H = 8 or 16), so that the step's kernels
# move from the head-resident range to long sequences at a fixed token count.
SWEEP_N = (516, 1028, 2052, 4100, 8196, 16388)


def length_sweep(dev, timer) -> dict:
    """C-ABI fwd+bwd TFLOP/s (14 D P flops per step, the headline formula)
    over SWEEP_N for D = 64 and D = 128."""
    import torch

    from rbf_attention_amd import _lib
    from rbf_attention_amd import workloads as wl

    rows = []
    for D, H in ((64, 8), (128, 16)):
        for N in SWEEP_N:
            B = max(1, (1 << 19) // (H * N))
            w = wl.Workload(f"sweep_d{D}_n{N}", B=B, H=H, content=N - 4, D=D, dtype="bf16", key_lognormal=0.5)
            bufs, a = setup_workload(w, dev)
            sp = timer.stream.cuda_stream

            def step():
                _lib.call("rbf_attn_fwd", a, sp)
                _lib.call("rbf_attn_bwd", a, sp)

            timer.ramp(step, 0.1)
            n = max(3, min(50, int(0.05 / max(w.flops_fwd_bwd() / 700e12, 1e-6))))
            ms = timer.loop(step, n)
            tf = w.flops_fwd_bwd() / (ms * 1e-3) / 1e12
            rows.append({"D": D, "N": N, "B": B, "H": H, "step_us": round(ms * 1e3, 2), "tflops": round(tf, 1),
                         "pct_of_bf16_peak": round(100 * tf / PEAK_TFLOPS["bf16"], 2),
                         "bwd_kernels": _lib.bwd_kernels(a)})
            log(f"  D={D} N={N} B={B} H={H}: {ms * 1e3:.1f} us, {tf:.0f} TFLOP/s")
            del bufs
            torch.cuda.empty_cache()
    return {"config": {"dtype": "bf16", "causal": True, "softmax": True, "tokens_per_step": 1 << 19,
                       "gamma": "1/(2 sqrt(D))"}, "rows": rows}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--ramp-seconds", type=float, default=0.4,
                    help="untimed steps run for this long before the warmup steps (GPU clock ramp)")
    ap.add_argument("--cold-reps", type=int, default=25)
    ap.add_argument("--kernel-seconds", type=float, default=0.2,
                    help="each kernel's own timing loop runs at least this long ...")
    ap.add_argument("--kernel-launches", type=int, default=200, help="... and at least this many launches")
    ap.add_argument("--workload", default="c2_model_bf16")
    ap.add_argument("--quick", action="store_true",
                    help="only the headline workload: no C3/C4 objects, reference sweep, train step or decode")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train-step", action="store_true", help="skip the config-5 train-step measurement")
    ap.add_argument("--train-steps", type=int, default=20)
    ap.add_argument("--no-decode", action="store_true", help="skip the KV-cache decode measurement")
    ap.add_argument("--no-extra-configs", action="store_true", help="skip the C3/C4 objects")
    ap.add_argument("--no-ref-sweep", action="store_true", help="skip the reference's own fp16 length sweep")
    ap.add_argument("--no-native", action="store_true", help="skip the C++ harness (rbf_attn_bench) timings")
    ap.add_argument("--length-sweep", action="store_true",
                    help="add a bf16 fwd+bwd TFLOP/s sweep over N (D = 64 and 128, fixed tokens per step)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="run one device copy of this many MiB before timing (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU; every (b, h) slice is "
            "independent, so data/head-parallel sharding needs no communication inside the op.",
            file=sys.stderr,
        )
        return 2
    if args.quick:
        args.no_extra_configs = args.no_ref_sweep = args.no_train_step = args.no_decode = True

    import torch

    from rbf_attention_amd import workloads as wl

    w = wl.CONFIGS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    timer = Timer(torch, dev, stream)

    if args.copy_probe_mb:
        src = torch.empty(args.copy_probe_mb << 18, device=dev, dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"workload {w.name}: B={w.B} H={w.H} N={w.N} D={w.D} {w.dtype} causal={w.causal} gamma={w.sm_scale:.6f}")
    # the peak-memory probe runs first, so that every kernel's last launches
    # are its own timing loop's (what a profile of this run averages)
    peak_mb = peak_fwd_mb(dev, w)
    head, ms_step = measure_workload(w, dev, timer, args.steps, args.warmup, args.ramp_seconds, args.cold_reps,
                                     graph=True, kernel_s=args.kernel_seconds, kernel_n=args.kernel_launches)
    result = {
        "metric": METRIC,
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic (seeded N(0,1) q/v/dO, lognormal-scaled keys, 4 zero register rows)",
        "config": head["config"],
        "pct_of_bf16_peak": head["pct_of_bf16_peak"],
        "clock_ramp_s": args.ramp_seconds,
        "cold": head["cold"],
        "graph_step_us": head["graph_step_us"],
        "op_step_us": head["op_step_us"],
        "op_graph_step_us": head["op_graph_step_us"],
        "kernel_us": head["kernel_us"],
        "kernel_sum_us": head["kernel_sum_us"],
        "step_kernels": head["step_kernels"],
        "roofline": head["roofline"],
        "peak_fwd_activation_mb": peak_mb,
    }
    if not args.no_native:
        log("native harness (C++, C ABI) ...")
        result["native_harness"] = native_harness(w.name, args.steps, args.warmup, args.cold_reps, args.ramp_seconds)
        log(f"  {result['native_harness']}")
    if not args.no_extra_configs:
        for name in ("c3_long_bf16", "c4_nonsoftmax_bf16"):
            if name == w.name:
                continue
            r, _ = measure_workload(wl.CONFIGS[name], dev, timer, 20, 5, 0.2, 20, graph=False,
                                    kernel_s=args.kernel_seconds, kernel_n=args.kernel_launches)
            if not args.no_native:
                r["native_harness"] = native_harness(name, 20, 5, 20, 0.2)
            result[name.split("_")[0]] = r
            torch.cuda.empty_cache()
    if not args.no_ref_sweep:
        log("reference sweep (fp16 B4 H8 D64, rbf_attention.py:1819-1911) ...")
        result["reference_sweep"] = reference_sweep(dev, timer, 20)
        torch.cuda.empty_cache()
    if not args.no_train_step:
        log("train step (config 5) ...")
        result["train_step"] = train_step_bench(dev, args.train_steps, 3)
        log(f"  {result['train_step']['value']} tokens/s, {result['train_step']['ms_per_step']} ms/step")
    if not args.no_decode:
        log("decode (KV cache) ...")
        result["decode"] = decode_bench(dev, 50)
        log(f"  {result['decode']['value']} GB/s, {result['decode']['us_per_call']} us/call")
    if args.length_sweep:
        log("length sweep ...")
        result["length_sweep"] = length_sweep(dev, timer)
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
        log(f"  {result['cpu_baseline']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
