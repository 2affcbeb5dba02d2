"""The drop-in under torch.compile, as the reference's callers use it
(train_rbf_transformer.py:280 compiles the model, rbf_attention.py:1832 the
op wrapper): the ops, their autograd and fake implementations traced by
dynamo + AOTAutograd with fullgraph=True (no graph break around the ops),
including the Optional[Tensor] pos argument and the token-major output's
fake strides; every output and gradient must equal eager bit for bit."""
import pytest
import torch

import rbf_attention_amd as ra
from rbf_attention_amd import model as M

pytestmark = pytest.mark.gpu


def inputs(dev, B=2, H=4, N=130, D=64, seed=0, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = ((torch.randn(B, H, N, D, generator=g) * std).to(torch.bfloat16).to(dev) for _ in range(4))
    P = (torch.randn(1, H, N, D, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    return q, k, v, do, P


def fwd_bwd(fn, q, k, v, do, P=None):
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)] + ([P.clone().requires_grad_(True)] if P is not None
                                                                    else [])
    out = fn(*leaves)
    out.backward(do)
    torch.cuda.synchronize()
    return [out.detach()] + [x.grad for x in leaves]


def assert_same(a, b):
    assert len(a) == len(b)
    for i, (x, y) in enumerate(zip(a, b)):
        assert x.shape == y.shape and x.stride() == y.stride(), (i, x.shape, y.shape, x.stride(), y.stride())
        assert torch.equal(x, y), f"output {i}: max diff {(x.float() - y.float()).abs().max().item():.3e}"


CASES = {
    # the reference's own call: rbf_attn_v5 ops, gamma = 1/sqrt(D)
    "v5_softmax": (lambda q, k, v: ra.run_triton_rbf(q, k, v, True), False),
    "v5_non_softmax": (lambda q, k, v: ra.run_triton_non_softmax_rbf(q, k, v, True), False),
    # the extensions: explicit gamma, register prefix, token-major output, fused position term
    "ex_softmax_pos_token_major": (
        lambda q, k, v, p: ra.run_triton_rbf(q, k, v, True, sm_scale=0.0625, num_prefix=4, token_major=True, pos=p),
        True),
    "ex_non_softmax_pos": (lambda q, k, v, p: ra.run_triton_non_softmax_rbf(q, k, v, True, sm_scale=0.0625, pos=p),
                           True),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_compiled_op_equals_eager(cuda_device, name):
    torch._dynamo.reset()
    fn, with_pos = CASES[name]
    q, k, v, do, P = inputs(cuda_device, std=1.0 if "non" not in name else 0.5)
    args = (q, k, v, do, P) if with_pos else (q, k, v, do)
    eager = fwd_bwd(fn, *args)
    compiled = torch.compile(fn, backend="aot_eager", fullgraph=True)
    got = fwd_bwd(compiled, *args)
    assert_same(eager, got)
    if "token_major" in name:
        assert got[0].transpose(1, 2).is_contiguous()


def test_compiled_train_step_equals_eager(cuda_device):
    """One bf16-autocast training step of a small CausalLM (fused position
    term, registers, token-major attention output), compiled whole with
    fullgraph=True: loss and every parameter gradient equal eager's."""
    torch._dynamo.reset()
    torch.manual_seed(0)
    cfg = M.ModelConfig(vocab_size=256, d_model=128, num_layers=2, num_heads=2, max_seq_len=64, num_registers=4)
    model = M.CausalLM(cfg).to(cuda_device)
    tokens = M.synthetic_tokens(4, 60, cfg.vocab_size, device=cuda_device)

    def loss_fn(m, x, y):
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            logits = m(x)
        return torch.nn.functional.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), y.reshape(-1))

    def step(fn):
        model.zero_grad(set_to_none=True)
        loss = fn(model, tokens[:, :-1], tokens[:, 1:])
        loss.backward()
        torch.cuda.synchronize()
        return loss.detach(), {n: p.grad.clone() for n, p in model.named_parameters()}

    l_eager, g_eager = step(loss_fn)
    l_comp, g_comp = step(torch.compile(loss_fn, backend="aot_eager", fullgraph=True))
    assert torch.equal(l_eager, l_comp), (l_eager.item(), l_comp.item())
    for n in g_eager:
        assert torch.equal(g_eager[n], g_comp[n]), n
