"""Pin of oracle/math_path.py (the reference's fp32 torch math path, used as
bench.py's CPU baseline and as the model test's attention stand-in) against
the float64 oracle (oracle/rbf_oracle.py), forward and autograd gradients,
for both variants; and a copy of the math path with a planted mistake must
fail the same check."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import math_path
from oracle import rbf_oracle as ro

TOL = 1e-5  # fp32 math path vs float64, relative to the tensor's largest magnitude


def inputs(softmax, seed=3, B=2, H=2, N=37, D=16):
    g = torch.Generator().manual_seed(seed)
    std = 1.0 if softmax else 0.5
    return [torch.randn(B, H, N, D, generator=g, dtype=torch.float64) * std for _ in range(4)]


def oracle(q, k, v, do, gamma, softmax, causal):
    a = [t.numpy() for t in (q, k, v, do)]
    if softmax:
        O, _ = ro.softmax_forward(a[0], a[1], a[2], gamma, causal)
        return (O,) + ro.softmax_backward(*a, gamma, causal)
    O = ro.non_softmax_forward(a[0], a[1], a[2], gamma, causal)
    return (O,) + ro.non_softmax_backward(*a, gamma, causal)


def worst(got, ref):
    """Largest error of (O, dQ, dK, dV), each relative to its tensor's max."""
    return max(float(np.abs(g.double().numpy() - r).max() / np.abs(r).max()) for g, r in zip(got, ref))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("softmax", [True, False])
def test_math_path_matches_oracle(softmax, causal):
    q, k, v, do = inputs(softmax)
    gamma = 1.0 / (2.0 * 16 ** 0.5)
    got = math_path.fwd_bwd(q, k, v, do, gamma, softmax=softmax, is_causal=causal)
    err = worst(got, oracle(q, k, v, do, gamma, softmax, causal))
    print(f"softmax={softmax} causal={causal}: worst relative error {err:.2e}")
    assert err <= TOL


def test_math_path_reference_gamma_and_registers():
    """gamma = 1/sqrt(D) (the reference's default) with zero register rows in
    front, as the benchmark configurations prepend them."""
    q, k, v, do = inputs(True, seed=9, N=40, D=24)
    for t in (q, k, v):
        t[:, :, :4] = 0
    gamma = 1.0 / 24 ** 0.5
    got = math_path.fwd_bwd(q, k, v, do, gamma, softmax=True, is_causal=True)
    assert worst(got, oracle(q, k, v, do, gamma, True, True)) <= TOL


def _softmax_without_half(q, k, v, gamma, is_causal=True):
    """Planted mistake: the augmented key column carries -||k||^2 instead of
    -||k||^2 / 2 (the augmented logits then carry the key norm twice)."""
    k_sq = k.float().pow(2).sum(dim=-1, keepdim=True)
    qf, kf = q.float(), k.float()
    qp = torch.cat([qf, torch.ones_like(qf[..., :1])], dim=-1)
    kp = torch.cat([kf, -k_sq], dim=-1)
    pad = (8 - qp.shape[-1] % 8) % 8
    qp, kp = F.pad(qp, (0, pad)), F.pad(kp, (0, pad))
    return F.scaled_dot_product_attention(qp, kp, v.float(), is_causal=is_causal, scale=2.0 * gamma)


_NON_SOFTMAX = math_path.non_softmax_math_forward


def _non_softmax_anticausal(q, k, v, gamma, is_causal=True, chunk=8):
    """Planted mistake: the causal mask transposed (keys after the query)."""
    return _NON_SOFTMAX(q.flip(2), k.flip(2), v.flip(2), gamma, is_causal, chunk).flip(2)


@pytest.mark.parametrize(
    "softmax,attr,mutant",
    [(True, "softmax_math_forward", _softmax_without_half), (False, "non_softmax_math_forward", _non_softmax_anticausal)],
)
def test_planted_mistakes_fail_the_pin(monkeypatch, softmax, attr, mutant):
    q, k, v, do = inputs(softmax, seed=5)
    if softmax:
        k = k * torch.exp(0.5 * torch.randn(k.shape[:-1] + (1,), generator=torch.Generator().manual_seed(1),
                                            dtype=torch.float64))
    gamma = 0.125
    monkeypatch.setattr(math_path, attr, mutant)
    got = math_path.fwd_bwd(q, k, v, do, gamma, softmax=softmax, is_causal=True)
    err = worst(got, oracle(q, k, v, do, gamma, softmax, True))
    print(f"mutant {mutant.__name__}: worst relative error {err:.2e}")
    assert err > 100 * TOL
