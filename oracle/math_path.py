"""The reference's PyTorch math path, restated for the CPU -- TEST AND CPU-BASELINE
INFRASTRUCTURE ONLY (used by tests/ and by bench.py's cpu_baseline leg).

softmax:      augmented-dimension SDPA in float32 with autograd backward,
              following test_equivalence.py:9-33 (q' = [q, 1], k' = [k, -||k||^2/2],
              zero-padded to a multiple of 8, scale = 2*gamma, fp32 upcast).
non-softmax:  exp(-gamma||q-k||^2) @ V with the causal mask, following
              rbf_attention.py:1747-1753 (compute_rbf_logits 1547-1553), in
              float32, chunked over (b, h) to bound memory.

num_prefix = 0 only (the reference path has no register-visibility mask).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def softmax_math_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: float, is_causal: bool = True):
    k_sq = k.float().pow(2).sum(dim=-1, keepdim=True)
    qf, kf = q.float(), k.float()
    qp = torch.cat([qf, torch.ones_like(qf[..., :1])], dim=-1)
    kp = torch.cat([kf, -0.5 * k_sq], dim=-1)
    pad = (8 - qp.shape[-1] % 8) % 8
    if pad:
        qp = F.pad(qp, (0, pad))
        kp = F.pad(kp, (0, pad))
    return F.scaled_dot_product_attention(qp, kp, v.float(), is_causal=is_causal, scale=2.0 * gamma)


def non_softmax_math_forward(q, k, v, gamma: float, is_causal: bool = True, chunk: int = 8):
    B, H, N, D = q.shape
    qf = q.float().reshape(B * H, N, D)
    kf = k.float().reshape(B * H, N, D)
    vf = v.float().reshape(B * H, N, D)
    mask = torch.ones(N, N, dtype=torch.bool, device=q.device).triu_(1) if is_causal else None
    outs = []
    for s in range(0, B * H, chunk):
        qs, ks, vs = qf[s : s + chunk], kf[s : s + chunk], vf[s : s + chunk]
        qq = qs.pow(2).sum(-1, keepdim=True)
        kk = ks.pow(2).sum(-1).unsqueeze(-2)
        logits = -gamma * (qq + kk - 2.0 * qs @ ks.transpose(-2, -1))
        if mask is not None:
            logits = logits.masked_fill(mask, float("-inf"))
        outs.append(torch.exp(logits) @ vs)
    return torch.cat(outs).reshape(B, H, N, D)


def fwd_bwd(q, k, v, dout, gamma: float, softmax: bool = True, is_causal: bool = True):
    """One forward + backward of the math path on CPU float32 copies.
    Returns (O, dQ, dK, dV)."""
    q = q.detach().float().clone().requires_grad_(True)
    k = k.detach().float().clone().requires_grad_(True)
    v = v.detach().float().clone().requires_grad_(True)
    fn = softmax_math_forward if softmax else non_softmax_math_forward
    out = fn(q, k, v, gamma, is_causal)
    out.backward(dout.float())
    return out.detach(), q.grad, k.grad, v.grad
