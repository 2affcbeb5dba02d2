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


@pytest.mark.parametrize("softmax", [True, False])
def test_decode_wrapper_equals_registered_op(cuda_device, softmax):
    """Eager rbf_decode on plain GPU tensors calls the op's implementation
    directly; the registered op (rbf_attn_amd::decode) gives the same bits."""
    q, k, v = make(2, 3, 4, 500, 64, torch.bfloat16, cuda_device, seed=21, std=1.0 if softmax else 0.5)
    lens = torch.tensor([500, 77], dtype=torch.int32)
    for lt in (None, lens, lens.to(cuda_device)):
        out, lse = ra.rbf_decode(q, k, v, lt, softmax=softmax, sm_scale=0.0625)
        ref, rl = torch.ops.rbf_attn_amd.decode(q, k, v, lt, softmax, 0.0625)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        if softmax:
            assert torch.equal(lse, rl)


def test_decode_strided_cache_views(cuda_device):
    """Caches as head-interleaved views of one (B, L, H, D) buffer."""
    B, H, L, D, T = 2, 4, 600, 64, 2
    g = torch.Generator().manual_seed(12)
    kb = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16).to(cuda_device)
    vb = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16).to(cuda_device)
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)
    run_case(q, kb.transpose(1, 2), vb.transpose(1, 2), True, 0.0625, tag="strided")


def draw_decode_cases(n, seed=16384):
    """Every dimension of a decode call drawn at once from one fixed generator
    (B, H, the query block T, cache length L, D, dtype, variant, gamma,
    per-batch lengths, head-interleaved cache views)."""
    rng = np.random.default_rng(seed)
    dtypes = (torch.bfloat16, torch.float16, torch.float32)
    cases = []
    for i in range(n):
        B = int(rng.integers(1, 5))
        H = int(rng.integers(1, 5))
        T = int(rng.choice([1, 1, 2, int(rng.integers(1, 33))]))
        L = int(np.exp(rng.uniform(np.log(max(T, 2)), np.log(6000.0))))
        L = max(L, T)
        D = 8 * int(rng.integers(1, 17))
        dtype = dtypes[int(rng.choice(3, p=[0.55, 0.3, 0.15]))]
        softmax = bool(rng.random() < 0.65)
        gamma = float(rng.choice([1.0 / D ** 0.5, 0.5 / D ** 0.5, rng.uniform(0.02, 0.3)]))
        lens = [int(rng.integers(T, L + 1)) for _ in range(B)] if rng.random() < 0.4 else None
        strided = bool(rng.random() < 0.35)
        cases.append((i, B, H, T, L, D, dtype, softmax, gamma, lens, strided))
    return cases


DECODE_CASES = draw_decode_cases(24)


def decode_id(c):
    i, B, H, T, L, D, dtype, softmax, gamma, lens, strided = c
    return (f"d{i}_B{B}H{H}T{T}L{L}D{D}_{str(dtype).split('.')[-1]}_{'sm' if softmax else 'ns'}"
            f"{'_ragged' if lens else ''}{'_strided' if strided else ''}")


def test_decode_draw_coverage():
    """The draw reaches every dtype, both variants, single-token and block
    queries, ragged lengths, strided caches and caches past 4096 tokens."""
    assert {c[6] for c in DECODE_CASES} == {torch.bfloat16, torch.float16, torch.float32}
    assert {c[7] for c in DECODE_CASES} == {True, False}
    assert any(c[3] == 1 for c in DECODE_CASES) and any(c[3] > 4 for c in DECODE_CASES)
    assert any(c[9] for c in DECODE_CASES) and any(c[10] for c in DECODE_CASES)
    assert max(c[4] for c in DECODE_CASES) > 4096


@pytest.mark.parametrize("case", DECODE_CASES, ids=decode_id)
def test_decode_random(cuda_device, case):
    i, B, H, T, L, D, dtype, softmax, gamma, lens, strided = case
    std = 1.0 if softmax else 0.5
    if strided:
        g = torch.Generator().manual_seed(500 + i)
        q = (torch.randn(B, H, T, D, generator=g) * std).to(dtype).to(cuda_device)
        k = (torch.randn(B, L, H, D, generator=g) * std).to(dtype).to(cuda_device).transpose(1, 2)
        v = torch.randn(B, L, H, D, generator=g).to(dtype).to(cuda_device).transpose(1, 2)
    else:
        q, k, v = make(B, H, T, L, D, dtype, cuda_device, seed=500 + i, std=std)
    run_case(q, k, v, softmax, gamma, lens=lens, tag=decode_id(case))
