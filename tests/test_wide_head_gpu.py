"""GPU parity for head dims above 128 (128 < D <= 256) against the float64
oracle: the reference pads any D to BLOCK_DMODEL = max(16, next_pow2(D))
(rbf_attention.py:661 forward, 715 backward, 1363 non-softmax) and runs it,
so these shapes must give the reference's results here too.  They run on the
streaming kernels at a padded width of 256 features (features D..255 zero).
Tolerances as tests/test_parity_gpu.py (fp32 max-abs <= 1e-4; 16-bit rel-L2
<= 1e-2, elementwise O/dV and tensor-wide dQ/dK bounds, kernel error at most
1.2x the rounding model's).
"""
import math

import pytest
import torch

from rbf_attention_amd import _lib
from test_decode_gpu import make as make_decode
from test_decode_gpu import run_case as run_decode_case
from test_parity_gpu import compare_case, rand_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [136, 192, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("softmax", [True, False])
def test_wide_head_dims(cuda_device, D, dtype, softmax):
    """Both variants, forward and backward, at D = 136 (padded from 136 to
    256), 192 and 256, bf16 and fp32, on a ragged length."""
    q, k, v, do = rand_inputs(1, 2, 77, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=D + 1)
    compare_case(q, k, v, do, softmax=softmax, gamma=1.0 / math.sqrt(D), tag=f"wide D{D} {dtype} sm{softmax}")


@pytest.mark.parametrize(
    "N,D,dtype,softmax",
    [
        (700, 256, torch.bfloat16, True),  # past the 576 tokens of the head-resident kernels
        (700, 256, torch.bfloat16, False),
        (1100, 192, torch.bfloat16, True),
        (650, 136, torch.float16, True),
        (650, 256, torch.float16, False),
        (600, 256, torch.float32, True),
        (601, 200, torch.float32, False),
    ],
)
def test_wide_head_ragged_long(cuda_device, N, D, dtype, softmax):
    """Lengths past one LDS tile and past the head-resident range, ragged in
    32 and in the 64-token tiles, on two heads of two batch entries."""
    q, k, v, do = rand_inputs(2, 2, N, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=N + D)
    compare_case(q, k, v, do, softmax=softmax, gamma=1.0 / (2 * math.sqrt(D)),
                 tag=f"wide N{N} D{D} {dtype} sm{softmax}")


@pytest.mark.parametrize("causal,num_prefix", [(False, 0), (True, 40)])
@pytest.mark.parametrize("softmax", [True, False])
def test_wide_head_masks(cuda_device, causal, num_prefix, softmax):
    q, k, v, do = rand_inputs(1, 2, 300, 256, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=9)
    compare_case(q, k, v, do, softmax=softmax, causal=causal, num_prefix=num_prefix, gamma=0.04,
                 tag=f"wide mask c{causal} p{num_prefix} sm{softmax}")


def test_wide_head_strided_views(cuda_device):
    """q/k/v as views of one packed projection (token stride 3 H D) and a
    permuted dout, at D = 256."""
    B, N, H, D = 2, 200, 2, 256
    g = torch.Generator().manual_seed(8)
    qkv = torch.randn(B, N, 3 * H * D, generator=g).to(torch.bfloat16).to(cuda_device)
    q, k, v = qkv.view(B, N, 3, H, D).permute(2, 0, 3, 1, 4)
    do = torch.randn(B, N, H, D, generator=g).to(torch.bfloat16).to(cuda_device).permute(0, 2, 1, 3)
    compare_case(q, k, v, do, gamma=0.05, tag="wide strided")


def test_wide_head_c_abi_backward_kernels(cuda_device):
    """At D = 256 the backward is the two-kernel form (dQ, then dK/dV)."""
    q = torch.zeros(1, 1, 64, 256, device=cuda_device, dtype=torch.bfloat16)
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0, _lib.DTYPE_CODES[torch.bfloat16]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = 1, 1, 64, 256, 1, 0.1
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(q))
    assert _lib.bwd_kernels(a) == 2


@pytest.mark.parametrize(
    "D,dtype,softmax,T,L",
    [(256, torch.bfloat16, True, 1, 3000), (256, torch.bfloat16, False, 4, 700), (192, torch.float16, True, 32, 900),
     (136, torch.bfloat16, True, 2, 1500), (256, torch.float32, True, 3, 800), (256, torch.float32, False, 1, 300)],
)
def test_wide_head_decode(cuda_device, D, dtype, softmax, T, L):
    q, k, v = make_decode(2, 3, T, L, D, dtype, cuda_device, seed=D + T + L, std=1.0 if softmax else 0.5)
    run_decode_case(q, k, v, softmax, 1.0 / (2 * D ** 0.5), tag=f"wide decode D{D} {dtype} T{T} L{L}")
