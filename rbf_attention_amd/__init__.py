"""MI355X-native fused RBF attention (softmax and non-softmax), forward and
backward, as hand-written HIP kernels for gfx950 behind a C ABI
(include/rbf_attn.h) and the reference's torch.library operator surface.
"""
from .ops import (  # noqa: F401
    TritonNonSoftmaxRBFAttention,
    TritonRBFAttention,
    rbf_decode,
    rbf_non_softmax_bwd,
    rbf_non_softmax_fwd,
    rbf_scaled_bwd,
    rbf_scaled_fwd,
    run_triton_non_softmax_rbf,
    run_triton_rbf,
)

__all__ = [
    "run_triton_rbf",
    "run_triton_non_softmax_rbf",
    "TritonRBFAttention",
    "TritonNonSoftmaxRBFAttention",
    "rbf_scaled_fwd",
    "rbf_scaled_bwd",
    "rbf_non_softmax_fwd",
    "rbf_non_softmax_bwd",
    "rbf_decode",
]
