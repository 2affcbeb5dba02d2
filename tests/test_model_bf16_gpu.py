"""The config-5 attention path inside the model: a bf16-autocast CausalLM
with 64-feature heads, whose attention takes the fused position-term,
head-resident kernels with token-major output, against the same model with
the attention replaced by the reference's fp32 math path (oracle/math_path.py:
the augmented-dimension SDPA of test_equivalence.py:9-33, on q + pos and
k + pos rounded to bf16 as the model's adds store them) -- loss and every
parameter gradient, including pos_weight and reg_pos_emb."""
import pytest
import torch

from oracle import math_path
from rbf_attention_amd import _lib
from rbf_attention_amd import model as M
from rbf_attention_amd import ops

pytestmark = pytest.mark.gpu


def math_rbf(q, k, v, is_causal=True, *, sm_scale=None, num_prefix=0, token_major=False, pos=None):
    assert num_prefix == 0
    if pos is not None:
        q, k = q + pos, k + pos
    g = sm_scale if sm_scale is not None else q.shape[-1] ** -0.5
    return math_path.softmax_math_forward(q, k, v, g, is_causal).to(q.dtype)


def loss_and_grads(model, tokens):
    model.zero_grad(set_to_none=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = model(tokens[:, :-1])
    loss = torch.nn.functional.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
    loss.backward()
    return loss.detach(), {n: p.grad.detach().float().clone() for n, p in model.named_parameters()}


def test_bf16_model_fused_pos_path_matches_math_path(cuda_device, monkeypatch):
    torch.manual_seed(0)
    cfg = M.ModelConfig(vocab_size=512, d_model=256, num_layers=2, num_heads=4, max_seq_len=128, num_registers=4)
    model = M.CausalLM(cfg).to(cuda_device)
    with torch.no_grad():
        model.register_tokens.normal_(0, 0.5)
    tokens = M.synthetic_tokens(8, 124, cfg.vocab_size, device=cuda_device)  # N = 124 + 4 registers = 128

    launched = []
    real_launch_pos = ops._launch_pos

    def spy(fn, a, pos, device):
        launched.append((fn, a.D, a.N, a.dtype))
        return real_launch_pos(fn, a, pos, device)

    monkeypatch.setattr(ops, "_launch_pos", spy)
    loss_hip, g_hip = loss_and_grads(model, tokens)
    # every layer's forward and backward went through the fused bf16 entry points
    assert [x[0] for x in launched] == ["rbf_attn_fwd_pos"] * 2 + ["rbf_attn_bwd_pos"] * 2, launched
    assert all(x[1:] == (64, 128, _lib.DTYPE_CODES[torch.bfloat16]) for x in launched)

    monkeypatch.setattr(ops, "run_triton_rbf", math_rbf)
    loss_ref, g_ref = loss_and_grads(model, tokens)
    print(f"loss hip={loss_hip.item():.6f} ref={loss_ref.item():.6f}")
    assert abs(loss_hip.item() - loss_ref.item()) <= 2e-3 * abs(loss_ref.item())
    worst = 0.0
    for n in g_ref:
        ref, got = g_ref[n].double(), g_hip[n].double()
        rel = ((got - ref).norm() / max(ref.norm().item(), 1e-30)).item()
        worst = max(worst, rel)
        print(f"{n}: rel_l2 {rel:.3e}")
        assert rel <= 3e-2, f"{n}: rel_l2 {rel:.3e}"
    for n in ("blocks.0.attn.pos_weight", "blocks.1.attn.reg_pos_emb"):
        assert g_hip[n].abs().sum() > 0, n
    print(f"worst gradient rel_l2 {worst:.3e}")
