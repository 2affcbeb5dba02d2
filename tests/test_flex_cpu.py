"""The flex-attention cross-check path (rbf_attention_amd.flex, the
reference's rbf_flex_attention, rbf_attention.py:1590-1605) against the
float64 oracle on the CPU: forward and autograd gradients, causal and not."""
import math
import warnings

import numpy as np
import pytest
import torch

from oracle import rbf_oracle as ro
from rbf_attention_amd.flex import rbf_flex_attention


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("gamma", [None, 0.0625])
def test_flex_path_matches_oracle(causal, gamma):
    g = torch.Generator().manual_seed(5)
    B, H, N, D = 1, 2, 70, 32
    q, k, v, do = (torch.randn(B, H, N, D, generator=g) for _ in range(4))
    k = k * 1.5
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        o = rbf_flex_attention(qq, kk, vv, is_causal=causal, sm_scale=gamma)
    o.backward(do)
    gam = 1.0 / math.sqrt(D) if gamma is None else gamma
    arrs = [t.double().numpy() for t in (q, k, v, do)]
    O, _ = ro.softmax_forward(*arrs[:3], gam, causal, 0)
    grads = ro.softmax_backward(*arrs, gam, causal, 0)
    for got, ref in zip((o, qq.grad, kk.grad, vv.grad), (O,) + tuple(grads)):
        err = np.abs(got.detach().double().numpy() - ref).max()
        assert err <= 2e-5 * max(1.0, np.abs(ref).max()), err
