"""Shared test fixtures: tiny random-init Qwen2 models, a stub tokenizer, seeded chunk data."""

from __future__ import annotations

import numpy as np
import torch


class StubTokenizer:
    """Offline stand-in: the engines only read eos_token_id (and decode for display)."""

    eos_token_id = 0

    def encode(self, text, add_special_tokens=False):
        return [1 + (ord(c) % 200) for c in text]

    def decode(self, ids):
        return " ".join(str(i) for i in ids)


def tiny_qwen2(layers=3, hidden=256, heads=4, kv=2, inter=512, vocab=512, theta=1e6, seed=0, dtype=torch.float32):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(
        vocab_size=vocab, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
        num_attention_heads=heads, num_key_value_heads=kv, max_position_embeddings=1 << 16,
        rope_theta=theta, tie_word_embeddings=True,
    )
    torch.manual_seed(seed)
    model = Qwen2ForCausalLM(cfg).to(dtype).eval()
    # Larger weights than the default 0.02 init so layers mix tokens visibly.
    with torch.no_grad():
        g = torch.Generator().manual_seed(seed + 1)
        for p in model.parameters():
            if p.dim() == 2:
                p.copy_((torch.randn(p.shape, generator=g) * (1.0 / p.shape[1] ** 0.5)).to(dtype))
    return model


def rope_reference_f64(x: np.ndarray, positions: np.ndarray, theta: float) -> np.ndarray:
    """Textbook half-split RoPE in fp64 (what nn.RoPE(traditional=False) computes)."""
    D = x.shape[-1]
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = positions.astype(np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x = x.astype(np.float64)
    a, b = x[..., : D // 2], x[..., D // 2 :]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


def bf16_ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two arrays of bf16 bit patterns (sign-magnitude aware)."""
    def ordered(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + (u & 0x7FFF))

    return np.abs(ordered(a_bits) - ordered(b_bits))


def random_qwen25_7b(device, layers: int = 28):
    """Random-init Qwen2.5-7B architecture in bf16 on `device` (28 layers, hidden 3584, 28 query
    / 4 KV heads, head_dim 128, intermediate 18944, vocab 152064, theta 1e6)."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=layers,
                      num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=32768,
                      rope_theta=1e6, tie_word_embeddings=False, rms_norm_eps=1e-6)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()
