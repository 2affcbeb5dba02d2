"""CPU tests of the model layer (rbf_attention_amd/model.py): structure,
parameter count, SuSiE position embedding, and that the forward refuses CPU
tensors (the attention has no fallback)."""
import pytest
import torch

from rbf_attention_amd import model as M


def small_cfg(**kw):
    base = dict(vocab_size=64, d_model=32, num_layers=2, num_heads=2, max_seq_len=40, num_registers=3)
    base.update(kw)
    return M.ModelConfig(**base)


def test_param_count_tied_and_untied():
    cfg = small_cfg()
    m = M.CausalLM(cfg)
    d, V, L, H, R, hd = cfg.d_model, cfg.vocab_size, cfg.num_layers, cfg.num_heads, cfg.num_registers, 16
    per_block = (d * 3 * d + 3 * d) + (d * d + d) + H * hd // 2 + H * R * hd + 2 * 2 * d + (d * 4 * d + 4 * d) + (4 * d * d + d)
    expect = R * d + V * d + L * per_block + 2 * d
    assert M.gpt_param_count(m) == expect
    m2 = M.CausalLM(small_cfg(tie_embeddings=False))
    assert M.gpt_param_count(m2) == expect + d * V + V


def test_register_tokens_start_at_zero():
    m = M.CausalLM(small_cfg())
    assert torch.count_nonzero(m.register_tokens) == 0


def test_susie_position_embedding():
    att = M.RBFAttention(num_heads=2, emb_dims=32, max_seq_len=40, num_registers=3, pos_weight_init=1.0)
    s = 10
    pos = att.position_embedding(s, torch.float32)
    assert pos.shape == (1, 2, s, 16)
    table = M.unrotated_sinusoids(40, 16)
    # content token t (after the 3 registers) gets table[t] * weight (weight = 1)
    torch.testing.assert_close(pos[0, 1, 3:], table[: s - 3])
    torch.testing.assert_close(pos[0, :, :3], att.reg_pos_emb[0])
    # sin/cos halves: row 0 is [0..0, 1..1]
    assert torch.all(table[0, :8] == 0) and torch.all(table[0, 8:] == 1)


def test_bad_attention_type():
    with pytest.raises(ValueError):
        M.RBFAttention(2, 32, attention_type="standard")


def test_cpu_forward_refused():
    m = M.CausalLM(small_cfg())
    idx = torch.randint(0, 64, (1, 8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m(idx)


def test_attention_flops_formula():
    cfg = M.ModelConfig()
    f = M.attention_flops_per_step(cfg, 32, 512)
    n = 516
    assert f == 14 * 64 * n * (n + 1) / 2 * 32 * 8 * 8
