"""torch.compile tracing of the drop-in on the CPU, with meta tensors: the
ops dispatch to their fake implementations, so dynamo + AOTAutograd trace
the forward and the registered autograd (fullgraph=True, no graph break)
without a GPU, and the compiled graph's output and gradient shapes and
strides equal eager's (the token-major output included).  The GPU run of the
same graphs is tests/test_compile_gpu.py."""
import pytest
import torch

import rbf_attention_amd as ra

META = torch.device("meta")

CASES = {
    "v5_softmax": lambda q, k, v, p: ra.run_triton_rbf(q, k, v, True),
    "v5_non_softmax": lambda q, k, v, p: ra.run_triton_non_softmax_rbf(q, k, v, False),
    "ex_softmax_pos_token_major": lambda q, k, v, p: ra.run_triton_rbf(q, k, v, True, sm_scale=0.0625, num_prefix=4,
                                                                       token_major=True, pos=p),
    "ex_non_softmax_pos_token_major": lambda q, k, v, p: ra.run_triton_non_softmax_rbf(q, k, v, True, sm_scale=0.05,
                                                                                       token_major=True, pos=p),
}


def fwd_bwd(fn, B=2, H=4, N=130, D=64):
    leaves = [torch.empty(B, H, N, D, device=META, dtype=torch.bfloat16).requires_grad_(True) for _ in range(3)]
    leaves.append(torch.empty(1, H, N, D, device=META, dtype=torch.bfloat16).requires_grad_(True))
    out = fn(*leaves)
    out.backward(torch.empty_like(out))
    return [out] + [x.grad for x in leaves]


@pytest.mark.parametrize("name", sorted(CASES))
def test_compiled_trace_matches_eager_meta(name):
    torch._dynamo.reset()
    fn = CASES[name]
    eager = fwd_bwd(fn)
    got = fwd_bwd(torch.compile(fn, backend="aot_eager", fullgraph=True))
    for i, (a, b) in enumerate(zip(eager, got)):
        if a is None:
            assert b is None, i
            continue
        assert a.shape == b.shape and a.stride() == b.stride() and a.dtype == b.dtype, (i, a.stride(), b.stride())
    if "token_major" in name:
        out = got[0]
        assert out.stride() == (130 * 4 * 64, 64, 4 * 64, 1)  # a (B, N, H, D) buffer seen as (B, H, N, D)
    if "pos" in name:
        assert got[4] is not None and got[4].shape == (1, 4, 130, 64)
    else:
        assert got[4] is None
