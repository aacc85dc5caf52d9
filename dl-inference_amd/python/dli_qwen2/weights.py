"""Seeded synthetic Qwen2 weights, named as the reference exporter names them
(python/dli_export/export.py:263-440)."""
from __future__ import annotations

import torch

from .config import Qwen2Config


def rope_tables(cfg: Qwen2Config, max_pos: int | None = None):
    """cos/sin [max_pos, head_dim/2] fp32 (closed form of export.py:242-247)."""
    max_pos = max_pos or cfg.max_pos
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float32) / cfg.head_dim))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv_freq)
    return torch.cos(freqs), torch.sin(freqs)


def random_weights(cfg: Qwen2Config, seed: int = 0, device: str = "cpu",
                   dtype: torch.dtype = torch.bfloat16, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Linear weights and biases ~N(0, std); norm weights 1 + N(0, std); embeddings ~N(0, std).
    Generated with a seeded generator on `device`."""
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(*shape, mean=0.0):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std + mean).to(dtype)

    w: dict[str, torch.Tensor] = {}
    w["model.embed_tokens.weight"] = normal(cfg.vocab, cfg.hidden)
    cos, sin = rope_tables(cfg)
    w["rotary_cos"] = cos.to(device)
    w["rotary_sin"] = sin.to(device)
    q_out, kv_out = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        w[f"{p}.input_layernorm.weight"] = normal(cfg.hidden, mean=1.0)
        w[f"{p}.self_attn.q_proj.weight"] = normal(q_out, cfg.hidden)
        w[f"{p}.self_attn.q_proj.bias"] = normal(q_out)
        w[f"{p}.self_attn.k_proj.weight"] = normal(kv_out, cfg.hidden)
        w[f"{p}.self_attn.k_proj.bias"] = normal(kv_out)
        w[f"{p}.self_attn.v_proj.weight"] = normal(kv_out, cfg.hidden)
        w[f"{p}.self_attn.v_proj.bias"] = normal(kv_out)
        w[f"{p}.self_attn.o_proj.weight"] = normal(cfg.hidden, q_out)
        w[f"{p}.post_attention_layernorm.weight"] = normal(cfg.hidden, mean=1.0)
        w[f"{p}.mlp.gate_proj.weight"] = normal(cfg.ffn, cfg.hidden)
        w[f"{p}.mlp.up_proj.weight"] = normal(cfg.ffn, cfg.hidden)
        w[f"{p}.mlp.down_proj.weight"] = normal(cfg.hidden, cfg.ffn)
    w["model.norm.weight"] = normal(cfg.hidden, mean=1.0)
    w["lm_head.weight"] = (w["model.embed_tokens.weight"] if cfg.tied_embeddings
                           else normal(cfg.vocab, cfg.hidden))
    return w
