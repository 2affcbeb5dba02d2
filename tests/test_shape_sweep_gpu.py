"""Parity against the float64 oracle on shapes that straddle the launchers'
dispatch boundaries, each checked to the bounds of test_parity_gpu:

  * head-resident kernels up to N = 576 at 32 < D <= 64, streaming above;
  * paired dK/dV kernel at D = 128, with LDS-DMA tile staging from
    N = 2048 and register staging below (D = 128 exactly; padded head dims
    such as 96 or 120 always stage through registers);
  * D = 64 forward and dQ with LDS-DMA at every length, dK/dV from N = 4096;
  * head dims padded to 32 / 64 / 128 (24, 40, 96, 120);
  * B*H not a multiple of 8 (no per-XCD head chunks), B*H = 1;
  * num_prefix register tokens, non-causal masks, fp16 and fp32.

Large heads are compared on their first and last (b, h) slices (every slice
is an independent problem)."""
import math

import pytest
import torch

from test_parity_gpu import compare_case, rand_inputs

pytestmark = pytest.mark.gpu

BF, FP, F32 = torch.bfloat16, torch.float16, torch.float32

# B, H, N, D, dtype, softmax, causal, num_prefix, gamma ("ref" = 1/sqrt(D), "bench" = 1/(2 sqrt(D)))
CASES = [
    (1, 3, 577, 64, BF, True, True, 0, "bench"),  # one block past the head-resident limit
    (2, 8, 576, 64, BF, True, True, 4, "ref"),  # at the limit, fewer heads than CUs
    (1, 2, 2047, 128, BF, True, True, 0, "bench"),  # paired dK/dV, register staging
    (1, 2, 2048, 128, BF, False, True, 0, "bench"),  # paired dK/dV, LDS-DMA from here on
    (3, 3, 4095, 64, FP, True, False, 0, "ref"),  # D = 64 forward with DMA, dK/dV without
    (1, 3, 4096, 64, BF, False, True, 40, "bench"),  # D = 64 dK/dV with DMA, long prefix
    (5, 3, 1000, 96, BF, True, True, 0, "ref"),  # D = 96 padded to 128
    (2, 5, 2500, 120, FP, True, True, 0, "bench"),  # D = 120 padded to 128, long
    (1, 1, 3000, 40, BF, False, False, 0, "bench"),  # D = 40 padded to 64, one head
    (4, 4, 300, 24, BF, True, True, 7, "ref"),  # D = 24 padded to 32
    (1, 2, 1500, 128, F32, True, True, 0, "ref"),  # fp32, D = 128
    (9, 1, 2100, 128, BF, True, True, 0, "bench"),  # B*H = 9, D = 128 DMA
    (16, 1, 700, 64, BF, True, True, 0, "bench"),  # 16 heads, streaming D = 64
    (1, 2, 6000, 64, BF, False, True, 0, "bench"),  # long non-softmax, every DMA path
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}N{}D{}_{}_{}_{}_p{}".format(
    c[0], c[1], c[2], c[3], {BF: "bf16", FP: "fp16", F32: "fp32"}[c[4]], "sm" if c[5] else "ns",
    "causal" if c[6] else "full", c[7]))
def test_shape_sweep(cuda_device, case):
    B, H, N, D, dtype, softmax, causal, npre, gname = case
    gamma = 1.0 / math.sqrt(D) if gname == "ref" else 1.0 / (2.0 * math.sqrt(D))
    seed = (N * 131 + D * 7 + B * 3 + H) % 10007
    q, k, v, do = rand_inputs(B, H, N, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=seed,
                              key_scale=0.5 if softmax else 0.0)
    big = N >= 2000 or B * H > 12
    sl = None
    if big:
        sl = (slice(0, 1), slice(0, 1)) if B * H == 1 else None
    tag = f"sweep B{B} H{H} N{N} D{D}"
    if not big or sl is not None:
        compare_case(q, k, v, do, softmax=softmax, causal=causal, gamma=gamma, num_prefix=npre, sl=sl, tag=tag)
        return
    # first and last (b, h) slices of one run
    outs = None
    for b, h in ((0, 0), (B - 1, H - 1)):
        outs = compare_case(q, k, v, do, softmax=softmax, causal=causal, gamma=gamma, num_prefix=npre,
                            sl=(slice(b, b + 1), slice(h, h + 1)), tag=f"{tag} b{b}h{h}", outs=outs)
