"""RBF attention through torch's flex_attention: the reference's comparator
path (rbf_attention.py:1590-1605, `rbf_flex_attention`), kept as an
independent cross-check of the HIP kernels on the GPU.

It is not the product path (`run_triton_rbf` and the ops never call it): the
scores come from torch's own flex_attention -- a generated kernel under
torch.compile, or the unfused implementation that materialises the score
matrix when called eagerly -- with the RBF logit built by a score_mod:

    score_mod(s) = 2 s - gamma ||k||^2,   s = gamma q.k  (flex's scale)

which is 2 gamma q.k - gamma ||k||^2, the reference's logit
(rbf_attention.py:1594-1600).  The causal mask is a flex block mask
(q_idx >= k_idx, rbf_attention.py:1570-1587).
"""
from __future__ import annotations

import math

import torch
from torch.nn.attention.flex_attention import create_block_mask, flex_attention

_MASKS: dict = {}


def _causal(b, h, q_idx, k_idx):
    return q_idx >= k_idx


def causal_block_mask(n: int, device) -> object:
    key = (n, str(torch.device(device)))
    if key not in _MASKS:
        _MASKS[key] = create_block_mask(_causal, B=None, H=None, Q_LEN=n, KV_LEN=n, device=str(torch.device(device)))
    return _MASKS[key]


def rbf_flex_attention(q, k, v, is_causal: bool = True, sm_scale: float | None = None):
    """Softmax RBF attention of (B, H, N, D) tensors with torch's
    flex_attention; gamma = sm_scale (default 1/sqrt(D), as the reference)."""
    d = q.shape[-1]
    gamma = 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)
    kn = torch.sum(k.float() * k.float(), dim=-1) * gamma  # (B, H, N) fp32

    def score_mod(score, b, h, q_idx, k_idx):
        return 2.0 * score - kn[b, h, k_idx]

    mask = causal_block_mask(q.shape[2], q.device) if is_causal else None
    return flex_attention(q, k, v, score_mod=score_mod, block_mask=mask, scale=gamma)
