"""GPU parity of the KV-cache decode kernels (rbf_attn_decode) against the
oracle's decode restatement (oracle/rbf_oracle.py decode_forward, pinned to the
full causal forward in tests/test_oracle.py), on identical seeded inputs.
Tolerances as tests/test_parity_gpu.py; the base-2 LSE within 1e-4 (fp32
inputs) or 2e-2 (16-bit inputs, whose P enters the MFMA sums rounded).
"""
import numpy as np
import pytest
import torch

import rbf_attention_amd as ra
from oracle import rbf_oracle as ro
from test_parity_gpu import check, np64

pytestmark = pytest.mark.gpu


def make(B, H, T, L, D, dtype, dev, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, T, D, generator=g) * std).to(dtype)
    k = (torch.randn(B, H, L, D, generator=g) * std).to(dtype)
    v = torch.randn(B, H, L, D, generator=g).to(dtype)
    return q.to(dev), k.to(dev), v.to(dev)


def run_case(q, k, v, softmax, gamma, lens=None, tag=""):
    print(f"case {tag} q={tuple(q.shape)} cache={tuple(k.shape)} {q.dtype} softmax={softmax} lens={lens}", flush=True)
    lt = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=q.device)
    out, lse = ra.rbf_decode(q, k, v, lt, softmax=softmax, sm_scale=gamma)
    torch.cuda.synchronize()
    O, L = ro.decode_forward(np64(q), np64(k), np64(v), gamma, softmax, lens)
    model = None
    if q.dtype != torch.float32:
        r = ro.rounder("bf16" if q.dtype == torch.bfloat16 else "fp16")
        model, _ = ro.decode_forward(np64(q), np64(k), np64(v), gamma, softmax, lens, rnd=r, out_rnd=r)
    check(f"{tag} O", out, O, q.dtype, kind="O", model=model)
    if softmax:
        err = float(np.abs(np64(lse) - L).max())
        print(f"{tag} L max_abs={err:.3e}", flush=True)
        assert err <= (1e-4 if q.dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("T", [1, 3, 32])
@pytest.mark.parametrize("L", [32, 100, 1000, 4100])
def test_decode_bf16_d128(cuda_device, T, L):
    if L < T:
        pytest.skip("cache shorter than the query block")
    q, k, v = make(2, 3, T, L, 128, torch.bfloat16, cuda_device, seed=L + T)
    run_case(q, k, v, True, 1.0 / (2 * 128 ** 0.5), tag=f"T{T} L{L}")


@pytest.mark.parametrize("D", [8, 40, 64, 128])
@pytest.mark.parametrize("softmax", [True, False])
def test_decode_head_dims(cuda_device, D, softmax):
    q, k, v = make(2, 2, 4, 300, D, torch.bfloat16, cuda_device, seed=D, std=1.0 if softmax else 0.5)
    run_case(q, k, v, softmax, 1.0 / (2 * D ** 0.5), tag=f"D{D}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("softmax", [True, False])
def test_decode_dtypes(cuda_device, dtype, softmax):
    q, k, v = make(2, 2, 2, 700, 64, dtype, cuda_device, seed=9, std=1.0 if softmax else 0.5)
    run_case(q, k, v, softmax, 0.0625, tag=f"{dtype}")


@pytest.mark.parametrize("softmax", [True, False])
def test_decode_ragged_lengths(cuda_device, softmax):
    """Per-batch cache lengths inside one padded cache; the tail of the
    shorter entries is never read."""
    B, L = 4, 1500
    q, k, v = make(B, 2, 5, L, 64, torch.bfloat16, cuda_device, seed=77, std=1.0 if softmax else 0.5)
    lens = [1500, 5, 700, 1029]
    k[1, :, lens[1]:] = float("nan")  # padding past the length must not be read
    v[1, :, lens[1]:] = float("nan")
    run_case(q, k, v, softmax, 0.0625, lens=lens, tag="ragged")


def test_decode_equals_last_rows_of_forward(cuda_device):
    """T = L: decode is the full causal forward of the cache."""
    q, k, v = make(2, 2, 32, 32, 64, torch.bfloat16, cuda_device, seed=3)
    out, lse = ra.rbf_decode(q, k, v, sm_scale=0.1)
    ref, L = ra.ops.rbf_scaled_fwd_ex(q, k, v, True, 0.1, 0)
    torch.cuda.synchronize()
    err = (out.float() - ref.float()).abs().max().item()
    print(f"decode vs forward max_abs={err:.3e}")
    assert err <= 2e-2
    assert (lse - L).abs().max().item() <= 2e-2


def test_decode_strided_cache_views(cuda_device):
    """Caches as head-interleaved views of one (B, L, H, D) buffer."""
    B, H, L, D, T = 2, 4, 600, 64, 2
    g = torch.Generator().manual_seed(12)
    kb = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16).to(cuda_device)
    vb = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16).to(cuda_device)
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)
    run_case(q, kb.transpose(1, 2), vb.transpose(1, 2), True, 0.0625, tag="strided")
