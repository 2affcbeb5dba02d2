"""Seeded synthetic workloads of the benchmark configurations.

Inputs are drawn on the CPU from torch.Generator(seed) in float32, in the
order q, k, v, dO, then the key scales; they are rounded to the config dtype
and only then moved to the device, so a CPU checker can upcast the very same
values.  Register tokens (the first ``registers`` rows) of q, k and v are zero,
as the reference's zero-initialised registers are (train_rbf_transformer.py:228-230);
dO is random on every row.
"""
from __future__ import annotations

import dataclasses
import math

import torch

FLOAT_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    B: int
    H: int
    content: int        # content tokens
    D: int
    dtype: str          # "bf16" | "fp16" | "fp32"
    softmax: bool = True
    registers: int = 4  # zero register tokens prepended
    causal: bool = True
    std: float = 1.0    # std of q, k, v, dO
    key_lognormal: float = 0.0  # sigma of the per-key-row lognormal scale (0 = none)
    gamma: float | None = None  # None -> 1/(2 sqrt(D))
    seed: int = 42

    @property
    def N(self) -> int:
        return self.content + self.registers

    @property
    def sm_scale(self) -> float:
        return self.gamma if self.gamma is not None else 1.0 / (2.0 * math.sqrt(self.D))

    @property
    def torch_dtype(self) -> torch.dtype:
        return FLOAT_DTYPES[self.dtype]

    def visible_pairs(self) -> int:
        n = self.N
        return n * (n + 1) // 2 if self.causal else n * n

    def flops_fwd(self) -> float:
        return 4.0 * self.D * self.B * self.H * self.visible_pairs()

    def flops_bwd(self) -> float:
        return 10.0 * self.D * self.B * self.H * self.visible_pairs()

    def flops_fwd_bwd(self) -> float:
        return 14.0 * self.D * self.B * self.H * self.visible_pairs()

    def with_(self, **kw) -> "Workload":
        return dataclasses.replace(self, **kw)


# The benchmark configurations (C1..C4); C5 is the model train step.
C1_TINY = Workload("c1_tiny_fp32", B=2, H=4, content=128, D=64, dtype="fp32")
C2_MODEL = Workload("c2_model_bf16", B=32, H=8, content=512, D=64, dtype="bf16", key_lognormal=0.5)
C3_LONG = Workload("c3_long_bf16", B=4, H=16, content=8192, D=128, dtype="bf16", key_lognormal=0.5)
C4_NONSOFTMAX = Workload("c4_nonsoftmax_bf16", B=16, H=8, content=2048, D=64, dtype="bf16", softmax=False, std=0.5)

CONFIGS = {w.name: w for w in (C1_TINY, C2_MODEL, C3_LONG, C4_NONSOFTMAX)}


def make_inputs(w: Workload):
    """(q, k, v, dO) as CPU tensors of w's dtype, shape (B, H, N, D)."""
    g = torch.Generator().manual_seed(w.seed)
    shape = (w.B, w.H, w.N, w.D)
    q = torch.randn(shape, generator=g) * w.std
    k = torch.randn(shape, generator=g) * w.std
    v = torch.randn(shape, generator=g) * w.std
    do = torch.randn(shape, generator=g) * w.std
    if w.key_lognormal > 0:
        z = torch.randn((w.B, w.H, w.N, 1), generator=g)
        k = k * torch.exp(w.key_lognormal * z)
    r = w.registers
    if r:
        q[:, :, :r] = 0
        k[:, :, :r] = 0
        v[:, :, :r] = 0
    dt = w.torch_dtype
    return q.to(dt), k.to(dt), v.to(dt), do.to(dt)
