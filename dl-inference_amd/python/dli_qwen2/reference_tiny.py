"""The reference's deterministic Qwen2-tiny model (its end-to-end test case), restated.

Configuration: examples/qwen2/qwen2.py:22-35 (vocab 8, hidden 4, intermediate 8, one layer,
2 attention heads, 2 KV heads, so head_dim 2; max positions 16; eps 1e-6; theta 10000; untied
lm_head; q/k/v projections with bias, as Qwen2 always has). Weights: parameter number i in the
model's parameter order gets ((arange(numel) + i) % 13 - 6) / 13 laid out in the parameter's shape
(qwen2.py:38-43). The names are the reference exporter's (export.py:263-440), which are the
module paths of the parameters.
"""
from __future__ import annotations

import torch

from .config import Qwen2Config
from .weights import rope_tables

REFERENCE_TINY = Qwen2Config(hidden=4, layers=1, heads=2, kv_heads=2, head_dim=2, ffn=8, vocab=8,
                             eps=1e-6, theta=10000.0, max_pos=16, tied_embeddings=False)

# (name, shape) in the order the model's parameters are enumerated (the formula's index)
_P = "model.layers.0"
PARAMETER_ORDER = (
    "model.embed_tokens.weight",
    f"{_P}.self_attn.q_proj.weight", f"{_P}.self_attn.q_proj.bias",
    f"{_P}.self_attn.k_proj.weight", f"{_P}.self_attn.k_proj.bias",
    f"{_P}.self_attn.v_proj.weight", f"{_P}.self_attn.v_proj.bias",
    f"{_P}.self_attn.o_proj.weight",
    f"{_P}.mlp.gate_proj.weight", f"{_P}.mlp.up_proj.weight", f"{_P}.mlp.down_proj.weight",
    f"{_P}.input_layernorm.weight", f"{_P}.post_attention_layernorm.weight",
    "model.norm.weight",
    "lm_head.weight",
)


def _shape(name: str, cfg: Qwen2Config) -> tuple[int, ...]:
    q, kv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    table = {
        "embed_tokens.weight": (cfg.vocab, cfg.hidden),
        "q_proj.weight": (q, cfg.hidden), "q_proj.bias": (q,),
        "k_proj.weight": (kv, cfg.hidden), "k_proj.bias": (kv,),
        "v_proj.weight": (kv, cfg.hidden), "v_proj.bias": (kv,),
        "o_proj.weight": (cfg.hidden, q),
        "gate_proj.weight": (cfg.ffn, cfg.hidden), "up_proj.weight": (cfg.ffn, cfg.hidden),
        "down_proj.weight": (cfg.hidden, cfg.ffn),
        "layernorm.weight": (cfg.hidden,), "norm.weight": (cfg.hidden,),
        "lm_head.weight": (cfg.vocab, cfg.hidden),
    }
    for suffix, shape in table.items():
        if name.endswith(suffix):
            return shape
    raise KeyError(name)


def reference_tiny_weights(device: str = "cpu", dtype: torch.dtype = torch.float32) -> dict:
    """Every parameter of the reference's tiny Qwen2 by the formula, plus rotary_cos/sin
    [max_pos, head_dim / 2] (the exporter's closed form)."""
    cfg = REFERENCE_TINY
    w = {}
    for index, name in enumerate(PARAMETER_ORDER):
        shape = _shape(name, cfg)
        n = 1
        for s in shape:
            n *= s
        values = torch.arange(n, dtype=torch.float32).reshape(shape)
        w[name] = (((values + index) % 13 - 6) / 13.0).to(device=device, dtype=dtype)
    cos, sin = rope_tables(cfg)
    w["rotary_cos"] = cos.to(device)
    w["rotary_sin"] = sin.to(device)
    return w
