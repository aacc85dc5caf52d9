"""Qwen2 shapes (hidden, layers, heads, ...) used by the graph builders."""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class Qwen2Config:
    hidden: int = 896
    layers: int = 24
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 4864
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1_000_000.0
    max_pos: int = 32768
    tied_embeddings: bool = True

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes(self, dtype_bytes: int = 2) -> int:
        """Bytes of every parameter a decode step reads (tied lm_head counted once)."""
        per_layer = (self.qkv_rows * self.hidden + self.qkv_rows  # qkv + bias
                     + self.heads * self.head_dim * self.hidden  # o_proj
                     + 3 * self.ffn * self.hidden  # gate, up, down
                     + 2 * self.hidden)  # two norms
        total = self.layers * per_layer + self.vocab * self.hidden + self.hidden
        if not self.tied_embeddings:
            total += self.vocab * self.hidden
        return total * dtype_bytes

    def kv_bytes_per_token(self, dtype_bytes: int = 2) -> int:
        return self.layers * 2 * self.kv_heads * self.head_dim * dtype_bytes


QWEN2_0_5B = Qwen2Config()
QWEN2_7B = Qwen2Config(hidden=3584, layers=28, heads=28, kv_heads=4, head_dim=128, ffn=18944,
                       vocab=152064, tied_embeddings=False)


def tiny_config(**overrides) -> Qwen2Config:
    """A few-layer Qwen2 with the real per-head geometry (fast for tests)."""
    base = replace(QWEN2_0_5B, layers=2, vocab=1024, max_pos=1024)
    return replace(base, **overrides)
