"""Qwen2-shape decoder on the dli graph engine: configs, seeded synthetic weights,
dli.graph.v1 builders (reference-style and fused) and a greedy decode session."""
from .config import QWEN2_0_5B, QWEN2_7B, Qwen2Config, tiny_config
from .graph import build_decode_graph, build_prefill_graph, pack_fused_weights
from .session import DecodeSession
from .weights import random_weights, rope_tables

__all__ = ["Qwen2Config", "QWEN2_0_5B", "QWEN2_7B", "tiny_config", "build_decode_graph",
           "build_prefill_graph", "pack_fused_weights", "DecodeSession", "random_weights", "rope_tables"]
