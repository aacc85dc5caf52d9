"""Writes tests/golden/qwen2_tiny_e2e.json: the reference's Qwen2-tiny end-to-end case.

The reference builds a one-layer Qwen2ForCausalLM (examples/qwen2/qwen2.py:22-35: vocab 8,
hidden 4, intermediate 8, 2 heads, 2 KV heads, max positions 16, eps 1e-6, theta 10000, untied
lm_head) and sets parameter number i (in model.parameters() order) to
((arange(numel) + i) % 13 - 6) / 13 (qwen2.py:38-43). Its e2e test runs input_ids [2] through the
exported graph and compares the logits with the model's at rtol = atol = 1e-3
(tests/e2e/test_models.py:61-71).

This script restates the configuration and the weight formula, builds the same model with
transformers' Qwen2ForCausalLM (third-party, installed in the build container; not the
reference's code), and records its fp32 logits for the reference's prompt [2] and, as an
extension, for every position of the prompt [2, 5, 1, 7] (positions 0..3; with head_dim 2 the
rotate-half and interleaved-pair RoPE conventions coincide, so no weight permutation is needed).
The weights are not stored: tests regenerate them from the formula (dli_qwen2.reference_tiny).
Run: python tests/golden/make_qwen2_tiny.py
"""
from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "dl-inference_amd" / "python"))

from dli_qwen2.reference_tiny import REFERENCE_TINY, PARAMETER_ORDER, reference_tiny_weights  # noqa: E402

PROMPTS = {"reference": [2], "extended": [2, 5, 1, 7]}


def hf_model():
    import transformers

    cfg = REFERENCE_TINY
    hf_cfg = transformers.Qwen2Config(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.ffn,
        num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads,
        num_key_value_heads=cfg.kv_heads, max_position_embeddings=cfg.max_pos,
        rms_norm_eps=cfg.eps, rope_theta=cfg.theta, attention_bias=False,
        tie_word_embeddings=False)
    model = transformers.Qwen2ForCausalLM(hf_cfg).eval()
    names = [n for n, _ in model.named_parameters()]
    assert names == list(PARAMETER_ORDER), names  # the formula's index i is this order
    ours = reference_tiny_weights()
    state = {n: ours[n] for n in names}
    model.load_state_dict(state, strict=True)
    return model


def build():
    model = hf_model()
    cases = {}
    with torch.no_grad():
        for name, ids in PROMPTS.items():
            logits = model(torch.tensor([ids], dtype=torch.int64)).logits[0]  # [S, V]
            cases[name] = {"input_ids": ids, "logits": logits.double().tolist()}
    return {
        "source": "examples/qwen2/qwen2.py:22-44 (config, weight formula); "
                  "tests/e2e/test_models.py:61-71 (prompt [2], rtol = atol = 1e-3)",
        "expected_by": "transformers.Qwen2ForCausalLM fp32 on the CPU",
        "rtol": 1e-3,
        "atol": 1e-3,
        "cases": cases,
    }


if __name__ == "__main__":
    out = HERE / "qwen2_tiny_e2e.json"
    out.write_text(json.dumps(build(), indent=1) + "\n", encoding="utf-8")
    print(f"wrote {os.path.relpath(out)}")
