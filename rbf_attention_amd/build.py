"""Build librbfattn.so (HIP kernels for gfx950 + the C ABI) in-tree.

Usage:  python -m rbf_attention_amd.build      (or build() from Python)

The library lands next to this file, so it travels with the source tree.
Each element type's kernels are a separate translation unit (bf16's two: the
dQ launcher and the rest, for their scheduler strategies), compiled in
parallel, then linked with the C ABI into one shared object.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "librbfattn.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# Native timing harness of the C ABI (csrc/rbf_attn_bench.cpp), linked
# against the library next to it.
BENCH_NAME = "rbf_attn_bench"
BENCH_PATH = os.path.join(PKG_DIR, BENCH_NAME)
ARCH = os.environ.get("RBF_ATTN_ARCH", "gfx950")

# Packed-FP32 VALU ops are disabled for all device code.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # NaN never reaches a max/compare on a path whose result is used (masked
    # logits are -inf, never NaN), so fmaxf needs no NaN canonicalisation.
    "-fno-honor-nans",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    "-Wno-unused-command-line-argument",
]


# Machine-scheduler strategy per unit, chosen by measurement on MI355X: the
# head-resident kernels (short heads held in LDS, one work-group per head)
# run 3-5 % faster with the ILP-maximising scheduler, which slows the
# long-sequence streaming dQ by 15 %; the streaming kernels run 1-2.5 %
# faster with the iterative ILP scheduler (C3 5.74 -> 5.65 ms, C4 495 ->
# 487 us per step).
HR_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
STREAM_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
# The bf16 dQ kernels (their own unit, RBF_PART=2) run faster with the
# occupancy-targeting iterative scheduler: C3 dQ 1571 -> 1543 us, C4 dQ
# 136.0 -> 135.3 us, where the forward and dK/dV kernels lose 1-2 % with it.
DQ_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=iterative-maxocc"]
# MFMA accumulators are kept in ordinary VGPRs (the VGPR form of the MFMA
# instructions), so the softmax VALU work reads them without AGPR<->VGPR
# copies.  Every unit but the fp32 one with 256 features (RBF_WIDE), whose
# fragments and accumulators exceed 512 registers per lane and on which the
# compiler fails with this form forced.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build(verbose: bool = True) -> str:
    """Compile every HIP translation unit for gfx950 and link librbfattn.so."""
    hipcc = _hipcc()
    units = [
        ("rbf_attn_capi.hip", VGPR_FORM),
        ("rbf_attn_launch.hip", ["-DRBF_ELEM_ID=0", "-DRBF_PART=1", *STREAM_FLAGS, *VGPR_FORM]),
        ("rbf_attn_launch.hip", ["-DRBF_ELEM_ID=0", "-DRBF_PART=2", *DQ_FLAGS, *VGPR_FORM]),
        ("rbf_attn_launch.hip", ["-DRBF_ELEM_ID=1", *STREAM_FLAGS, *VGPR_FORM]),
        ("rbf_attn_launch.hip", ["-DRBF_ELEM_ID=2", *STREAM_FLAGS, *VGPR_FORM]),
        ("rbf_attn_launch.hip", ["-DRBF_ELEM_ID=2", "-DRBF_WIDE", *STREAM_FLAGS]),
        ("rbf_attn_launch_hr.hip", ["-DRBF_ELEM_ID=0", *HR_FLAGS, *VGPR_FORM]),
        ("rbf_attn_launch_hr.hip", ["-DRBF_ELEM_ID=1", *HR_FLAGS, *VGPR_FORM]),
    ]
    with tempfile.TemporaryDirectory(prefix="rbfattn_build_") as tmp:
        jobs = []
        for idx, (src, extra) in enumerate(units):
            obj = os.path.join(tmp, f"u{idx}.o")
            cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
            jobs.append((cmd, obj))
        workers = min(len(jobs), max(1, min(16, os.cpu_count() or 1)))
        with cf.ThreadPoolExecutor(workers) as ex:
            list(ex.map(lambda j: _run(j[0]), jobs))
        tmp_lib = os.path.join(tmp, LIB_NAME)
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib, *[o for _, o in jobs]])
        shutil.copyfile(tmp_lib, LIB_PATH + ".tmp")
        os.replace(LIB_PATH + ".tmp", LIB_PATH)
        tmp_bench = os.path.join(tmp, BENCH_NAME)
        _run([hipcc, f"--offload-arch={ARCH}", "-O2", "-std=c++17", f"-I{INCLUDE}",
              os.path.join(CSRC, "rbf_attn_bench.cpp"), f"-L{PKG_DIR}", "-lrbfattn", "-Wl,-rpath,$ORIGIN",
              "-o", tmp_bench])
        shutil.copyfile(tmp_bench, BENCH_PATH + ".tmp")
        os.chmod(BENCH_PATH + ".tmp", 0o755)
        os.replace(BENCH_PATH + ".tmp", BENCH_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {BENCH_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
