"""GPU tests of the model layer: the CausalLM with the HIP attention matches
the same model with the attention replaced by the reference math path
(oracle/math_path.py, fp32 torch on the GPU), loss and every parameter
gradient; and the training step drives the loss down on a repeated batch."""
import pytest
import torch

from oracle import math_path
from rbf_attention_amd import model as M
from rbf_attention_amd import ops

pytestmark = pytest.mark.gpu


def small_cfg(**kw):
    base = dict(vocab_size=128, d_model=64, num_layers=2, num_heads=2, max_seq_len=64, num_registers=4)
    base.update(kw)
    return M.ModelConfig(**base)


def math_rbf(q, k, v, is_causal=True, *, sm_scale=None, num_prefix=0, token_major=False, pos=None):
    assert num_prefix == 0
    if pos is not None:
        q, k = q + pos, k + pos
    g = sm_scale if sm_scale is not None else q.shape[-1] ** -0.5
    return math_path.softmax_math_forward(q.contiguous(), k.contiguous(), v.contiguous(), g, is_causal).to(q.dtype)


def math_rbf_ns(q, k, v, is_causal=True, *, sm_scale=None, num_prefix=0, token_major=False, pos=None):
    assert num_prefix == 0
    if pos is not None:
        q, k = q + pos, k + pos
    g = sm_scale if sm_scale is not None else q.shape[-1] ** -0.5
    return math_path.non_softmax_math_forward(q, k, v, g, is_causal).to(q.dtype)


def loss_and_grads(model, tokens):
    model.zero_grad(set_to_none=True)
    logits = model(tokens[:, :-1])
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
    loss.backward()
    return loss.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}


@pytest.mark.parametrize("attention_type", ["rbf", "rbf_non_softmax"])
def test_model_matches_math_path_fp32(cuda_device, monkeypatch, attention_type):
    torch.manual_seed(0)
    cfg = small_cfg(attention_type=attention_type)
    model = M.CausalLM(cfg).to(cuda_device)
    # non-zero registers so the register path carries gradient signal
    with torch.no_grad():
        model.register_tokens.normal_(0, 0.5)
    tokens = M.synthetic_tokens(2, 60, cfg.vocab_size, device=cuda_device)
    loss_hip, g_hip = loss_and_grads(model, tokens)
    if attention_type == "rbf":
        monkeypatch.setattr(ops, "run_triton_rbf", math_rbf)
    else:
        monkeypatch.setattr(ops, "run_triton_non_softmax_rbf", math_rbf_ns)
    loss_ref, g_ref = loss_and_grads(model, tokens)
    print(f"loss hip={loss_hip.item():.6f} ref={loss_ref.item():.6f}")
    assert abs(loss_hip.item() - loss_ref.item()) <= 1e-4 * abs(loss_ref.item())
    for n in g_ref:
        ref, got = g_ref[n].double(), g_hip[n].double()
        rel = (got - ref).norm() / max(ref.norm().item(), 1e-30)
        assert rel <= 1e-3, f"{n}: rel_l2 {rel:.3e}"


def test_train_step_reduces_loss(cuda_device):
    torch.manual_seed(0)
    cfg = small_cfg()
    model = M.CausalLM(cfg).to(cuda_device)
    tr = M.Trainer(model, lr=3e-3)
    tokens = M.synthetic_tokens(4, 48, cfg.vocab_size, device=cuda_device)
    losses = [tr.step(tokens).item() for _ in range(30)]
    print("losses", losses[0], losses[-1])
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < 0.7 * losses[0]
