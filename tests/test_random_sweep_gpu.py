"""Seeded random shapes against the float64 oracle, to the bounds of
test_parity_gpu (rel-L2, elementwise O/dV, tensor-wide dQ/dK, rounding-model
ratio).

The fixed parity tests pick one dimension at a time (head dims at N = 77,
ragged N at D = 64, masks at one shape, ...).  These cases draw every
dimension at once from one fixed generator, so that combinations the fixed
tests leave out (a padded head dim with a long prefix, fp16 with a
non-causal mask at a ragged length, strided inputs with D = 24, ...) run
through whichever kernels the launchers pick for them.  Sizes stay where the
oracle finishes in about a second (N <= 2000, B * H <= 9).  A second draw
takes the head-resident kernels (B * H >= 256 heads of N <= 576 tokens,
32 < D <= 64), compared on sampled (b, h) slices.

Inputs are contiguous (B, H, N, D) tensors or (B, H, N, D) views of
token-major (B, N, H, D) storage, the layout a model's QKV projection
produces."""
import math

import numpy as np
import pytest
import torch

from test_parity_gpu import compare_case, rand_inputs

pytestmark = pytest.mark.gpu

DTYPES = (torch.bfloat16, torch.float16, torch.float32)
DT_NAMES = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def draw_cases(n, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = 8 * int(rng.integers(1, 17))
        # log-uniform over 1..2000 (ragged short heads), or uniform over 500..2000
        N = int(np.exp(rng.uniform(0.0, math.log(2000.0)))) if rng.random() < 0.6 else int(rng.integers(500, 2001))
        B = int(rng.integers(1, 4))
        H = int(rng.integers(1, 4))
        dtype = DTYPES[int(rng.choice(3, p=[0.55, 0.3, 0.15]))]
        softmax = bool(rng.random() < 0.6)
        causal = bool(rng.random() < 0.75)
        num_prefix = 0 if rng.random() < 0.6 else int(rng.integers(1, min(N, 64) + 1))
        gamma = float(rng.choice([1.0 / math.sqrt(D), 0.5 / math.sqrt(D), rng.uniform(0.02, 0.3)]))
        token_major = bool(rng.random() < 0.35)
        cases.append((i, B, H, N, D, dtype, softmax, causal, num_prefix, gamma, token_major))
    return cases


CASES = draw_cases(64)


def draw_hr_cases(n, seed=5760):
    """Cases for the head-resident kernels: 16-bit, 32 < D <= 64, N <= 576 and
    at least as many heads as the 256 CUs."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = 8 * int(rng.integers(5, 9))
        N = int(rng.integers(1, 577))
        B = int(rng.integers(16, 41))
        H = 16
        dtype = (torch.bfloat16, torch.float16)[int(rng.random() < 0.35)]
        softmax = bool(rng.random() < 0.6)
        causal = bool(rng.random() < 0.8)
        num_prefix = 0 if rng.random() < 0.5 else int(rng.integers(1, min(N, 64) + 1))
        gamma = float(rng.choice([1.0 / math.sqrt(D), 0.5 / math.sqrt(D), rng.uniform(0.02, 0.2)]))
        token_major = bool(rng.random() < 0.35)
        cases.append((100 + i, B, H, N, D, dtype, softmax, causal, num_prefix, gamma, token_major))
    return cases


HR_CASES = draw_hr_cases(12)


def case_id(c):
    i, B, H, N, D, dtype, softmax, causal, npre, gamma, tm = c
    return (f"r{i}_B{B}H{H}N{N}D{D}_{DT_NAMES[dtype]}_{'sm' if softmax else 'ns'}_"
            f"{'causal' if causal else 'full'}_p{npre}{'_tm' if tm else ''}")


def test_draw_covers_the_dispatch_space():
    """The fixed draw reaches every dtype, both variants, both masks, prefixes,
    strided inputs, each head-dim padding class (<= 32, <= 64, <= 128), and
    lengths from below one 64-token tile to past 1200 tokens (where the D = 128
    dQ switches kernels)."""
    assert {c[5] for c in CASES} == set(DTYPES)
    assert {c[6] for c in CASES} == {True, False}
    assert {c[7] for c in CASES} == {True, False}
    assert any(c[8] > 0 for c in CASES) and any(c[10] for c in CASES)
    assert {(c[4] > 32) + (c[4] > 64) for c in CASES} == {0, 1, 2}
    assert min(c[3] for c in CASES) < 64 and max(c[3] for c in CASES) > 1200


def test_hr_draw_takes_the_head_resident_path():
    """Every drawn head-resident case satisfies the launchers' conditions for
    those kernels (16-bit, 32 < D <= 64, N <= 576, B * H >= 256), and the draw
    spans short and long heads, both variants and strided inputs."""
    for c in HR_CASES:
        assert c[5] != torch.float32 and 32 < c[4] <= 64 and c[3] <= 576 and c[1] * c[2] >= 256
    assert min(c[3] for c in HR_CASES) < 64 and max(c[3] for c in HR_CASES) > 448
    assert {c[6] for c in HR_CASES} == {True, False} and any(c[10] for c in HR_CASES)


def make_inputs(case, dev):
    i, B, H, N, D, dtype, softmax, causal, npre, gamma, token_major = case
    q, k, v, do = rand_inputs(B, H, N, D, dtype, dev, std=1.0 if softmax else 0.5, seed=1000 + i,
                              key_scale=0.5 if softmax else 0.0)
    if token_major:
        # same values, (B, H, N, D) views of (B, N, H, D) storage
        q, k, v, do = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, do))
        assert q.stride(2) == H * D
    return q, k, v, do


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_random_shape(cuda_device, case):
    i, B, H, N, D, dtype, softmax, causal, npre, gamma, token_major = case
    q, k, v, do = make_inputs(case, cuda_device)
    compare_case(q, k, v, do, softmax=softmax, causal=causal, gamma=gamma, num_prefix=npre, tag=case_id(case))


@pytest.mark.parametrize("case", HR_CASES, ids=case_id)
def test_random_head_resident(cuda_device, case):
    """One run over every head; the oracle on the first, the last and one
    drawn (b, h) slice (every slice is an independent problem)."""
    i, B, H, N, D, dtype, softmax, causal, npre, gamma, token_major = case
    q, k, v, do = make_inputs(case, cuda_device)
    rng = np.random.default_rng(i)
    picks = [(0, 0), (B - 1, H - 1), (int(rng.integers(0, B)), int(rng.integers(0, H)))]
    outs = None
    for b, h in picks:
        outs = compare_case(q, k, v, do, softmax=softmax, causal=causal, gamma=gamma, num_prefix=npre,
                            sl=(slice(b, b + 1), slice(h, h + 1)), tag=f"{case_id(case)} b{b}h{h}", outs=outs)
