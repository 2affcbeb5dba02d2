"""CPU tests of the operator layer: the reference op names and schemas are
registered, the fake (meta) implementations give the reference's output
shapes, and non-GPU tensors are refused (there is no CPU fallback)."""
import pytest
import torch

import rbf_attention_amd as ra  # noqa: F401  (registers the ops)

EXPECTED_SCHEMAS = {
    # rbf_attention.py:651-654, 702-712, 1355-1358, 1399-1407
    "scaled_fwd": "rbf_attn_v5::scaled_fwd(Tensor q, Tensor k, Tensor v, bool is_causal) -> (Tensor, Tensor)",
    "scaled_bwd": "rbf_attn_v5::scaled_bwd(Tensor q, Tensor k, Tensor v, Tensor out, Tensor L, Tensor dout, "
    "bool is_causal, float sm_scale) -> (Tensor, Tensor, Tensor)",
    "non_softmax_fwd": "rbf_attn_v5::non_softmax_fwd(Tensor q, Tensor k, Tensor v, bool is_causal) -> Tensor",
    "non_softmax_bwd": "rbf_attn_v5::non_softmax_bwd(Tensor q, Tensor k, Tensor v, Tensor dout, bool is_causal, "
    "float sm_scale) -> (Tensor, Tensor, Tensor)",
}


@pytest.mark.parametrize("name", sorted(EXPECTED_SCHEMAS))
def test_reference_schema(name):
    op = getattr(torch.ops.rbf_attn_v5, name).default
    assert str(op._schema) == EXPECTED_SCHEMAS[name]


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(shape, device="meta", dtype=dtype)


def test_fake_shapes():
    q = meta(2, 3, 37, 64)
    out, L = torch.ops.rbf_attn_v5.scaled_fwd(q, q, q, True)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert L.shape == (2, 3, 37) and L.dtype == torch.float32
    dq, dk, dv = torch.ops.rbf_attn_v5.scaled_bwd(q, q, q, out, L, q, True, 0.125)
    assert dq.shape == dk.shape == dv.shape == q.shape
    o2 = torch.ops.rbf_attn_v5.non_softmax_fwd(q, q, q, True)
    assert o2.shape == q.shape
    g = torch.ops.rbf_attn_v5.non_softmax_bwd(q, q, q, q, True, 0.125)
    assert all(t.shape == q.shape for t in g)
    o3, L3 = torch.ops.rbf_attn_amd.scaled_fwd_ex(q, q, q, True, 0.0625, 4)
    assert o3.shape == q.shape and L3.shape == (2, 3, 37)


def test_cpu_tensors_refused():
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ra.run_triton_rbf(q, q, q)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ra.run_triton_non_softmax_rbf(q, q, q)


def test_shape_and_dtype_checks():
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(ValueError):
        ra.run_triton_rbf(q, q[:, :, :4], q)
    with pytest.raises(TypeError):
        ra.run_triton_rbf(q, q.double(), q)
    with pytest.raises(ValueError):
        ra.run_triton_rbf(q[0], q[0], q[0])
    big = torch.randn(1, 1, 4, 264)
    with pytest.raises(ValueError):
        ra.run_triton_rbf(big, big, big)


def test_public_surface():
    for name in ("run_triton_rbf", "run_triton_non_softmax_rbf", "TritonRBFAttention", "TritonNonSoftmaxRBFAttention"):
        assert hasattr(ra, name)


def test_eager_path_predicate():
    """The wrappers take their eager autograd.Function path only for plain GPU
    tensors outside tracing, dispatch modes and functorch transforms; CPU and
    meta tensors, tensor subclasses and active dispatch modes go through the
    registered ops (which refuse CPU tensors and trace meta ones)."""
    from torch.utils._python_dispatch import TorchDispatchMode
    from rbf_attention_amd import ops

    cpu = torch.randn(1, 1, 8, 64)
    assert not ops._eager_plain(cpu, cpu, cpu, None)
    m = meta(1, 1, 8, 64)
    assert not ops._eager_plain(m, m, m, None)

    class Sub(torch.Tensor):
        pass

    assert not ops._eager_plain(cpu.as_subclass(Sub), cpu, cpu, None)

    class Mode(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with Mode():
        assert not ops._eager_plain(cpu, cpu, cpu, None)
    # the meta tensors go through the ops' fake implementations
    assert ra.run_triton_rbf(m, m, m).shape == m.shape
    assert ra.run_triton_non_softmax_rbf(m, m, m, sm_scale=0.1, num_prefix=2).shape == m.shape
