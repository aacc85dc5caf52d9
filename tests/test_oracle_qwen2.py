"""Pins the Qwen2 decoder oracle (oracle/qwen2.py) on the CPU.

1. Against an independent implementation: transformers' Qwen2ForCausalLM (third-party,
   installed here) in fp32, with the q/k projection rows permuted so that its rotate-half RoPE
   equals the reference's interleaved-pair rotary op (rotary/kernel.py:22-35). The oracle's
   unrounded mode must give the same logits.
2. Causal consistency: feeding a prompt token by token gives the logits of one batched pass.
3. The bf16 mode really rounds: every node output it produces is bf16-representable, and it
   stays close to the fp32 model.
"""
from __future__ import annotations

import pytest
import torch

from dli_qwen2 import random_weights
from dli_qwen2.config import Qwen2Config
from oracle.qwen2 import Qwen2Oracle

CFG = Qwen2Config(hidden=64, layers=2, heads=4, kv_heads=2, head_dim=16, ffn=128, vocab=100,
                  max_pos=64, theta=1_000_000.0)


def _weights():
    w = random_weights(CFG, seed=3, dtype=torch.float32, std=0.2)
    return w


def _hf_model(w):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=CFG.vocab, hidden_size=CFG.hidden, intermediate_size=CFG.ffn,
        num_hidden_layers=CFG.layers, num_attention_heads=CFG.heads,
        num_key_value_heads=CFG.kv_heads, max_position_embeddings=CFG.max_pos,
        rms_norm_eps=CFG.eps, rope_theta=CFG.theta, tie_word_embeddings=True)
    model = transformers.Qwen2ForCausalLM(cfg).eval()
    hd = CFG.head_dim
    # interleaved row 2p <- rotate-half row p, 2p+1 <- p + hd/2; HF rows = ours[inverse]
    perm = torch.stack([torch.arange(hd // 2), torch.arange(hd // 2) + hd // 2], 1).reshape(-1)
    inv = torch.argsort(perm)

    def hf_rows(t, heads):
        shape = t.shape
        return t.reshape(heads, hd, *shape[1:])[:, inv].reshape(shape)

    state = {}
    for name, t in w.items():
        if name in ("rotary_cos", "rotary_sin", "lm_head.weight"):
            continue
        if ".q_proj." in name:
            t = hf_rows(t, CFG.heads)
        elif ".k_proj." in name:
            t = hf_rows(t, CFG.kv_heads)
        state[name] = t
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all("lm_head" in m or "rotary" in m for m in missing), (missing, unexpected)
    return model


def test_oracle_matches_transformers_qwen2_fp32():
    w = _weights()
    model = _hf_model(w)
    ids = torch.tensor([[5, 17, 3, 99, 42, 0, 61], [8, 8, 1, 70, 2, 33, 5]])
    with torch.no_grad():
        ref = model(ids).logits
    oracle = Qwen2Oracle(CFG, w, round_bf16=False)
    oracle.reset(2)
    got = oracle.forward(ids)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    # a wrong RoPE pairing must be caught: use the unpermuted HF rows
    oracle_bad = Qwen2Oracle(CFG, {**w, **{k: model.state_dict()[k] for k in w if ".q_proj." in k}},
                             round_bf16=False)
    oracle_bad.reset(2)
    assert not torch.allclose(oracle_bad.forward(ids), ref, rtol=1e-3, atol=1e-3)


def test_stepwise_equals_batched_prompt():
    w = _weights()
    ids = torch.tensor([[5, 17, 3, 99, 42, 0], [8, 8, 1, 70, 2, 33]])
    # fp32 mode: in bf16 mode the two orders of summation may round a few values differently
    a = Qwen2Oracle(CFG, w, round_bf16=False)
    a.reset(2)
    full = a.forward(ids)
    b = Qwen2Oracle(CFG, w, round_bf16=False)
    b.reset(2)
    steps = torch.cat([b.forward(ids[:, t:t + 1]) for t in range(ids.shape[1])], 1)
    torch.testing.assert_close(steps, full, rtol=1e-5, atol=1e-5)


def test_bf16_mode_rounds_and_stays_close():
    w = {k: v.to(torch.bfloat16).float() for k, v in _weights().items()}
    ids = torch.tensor([[5, 17, 3, 99]])
    exact = Qwen2Oracle(CFG, w, round_bf16=False)
    exact.reset(1)
    rounded = Qwen2Oracle(CFG, w)
    rounded.reset(1)
    lo, hi = rounded.forward(ids), exact.forward(ids)
    assert not torch.equal(lo, hi)
    assert float((lo - hi).norm() / hi.norm()) < 0.05
    k = rounded.k_cache[0]
    assert torch.equal(k, k.to(torch.bfloat16).float())
    tokens, margins = rounded.generate(ids, 3)
    assert tokens.shape == (1, 3) and bool((margins >= 0).all())


def test_teacher_forced_reproduces_free_running_greedy():
    # fp32 mode, so batched and stepwise passes agree to 1e-5 and the argmax is the same
    w = _weights()
    prompt = torch.tensor([[5, 17, 3, 99], [8, 8, 1, 70]])
    o = Qwen2Oracle(CFG, w, round_bf16=False)
    tokens, margins = o.generate(prompt, 5)
    ids, tf_margins, logits = o.teacher_forced(prompt, tokens)
    assert torch.equal(ids, tokens)
    torch.testing.assert_close(tf_margins, margins, rtol=1e-4, atol=1e-4)
    assert logits.shape == (2, 5, CFG.vocab)


def test_static_cache_step_equals_forward():
    # the preallocated-cache step used for CPU timing computes the same logits as forward()
    w = _weights()
    prompt = torch.tensor([[5, 17, 3], [8, 8, 1]])
    a = Qwen2Oracle(CFG, w, round_bf16=False)
    a.reset(2)
    full = a.forward(prompt)
    b = Qwen2Oracle(CFG, w, round_bf16=False)
    b.reset_static(2, 8)
    steps = torch.stack([b.step_static(prompt[:, t], t) for t in range(3)], 1)
    torch.testing.assert_close(steps, full, rtol=1e-5, atol=1e-5)


def test_oracle_reproduces_reference_tiny_fixture():
    """The reference's Qwen2-tiny case (examples/qwen2/qwen2.py:22-44, weights by its formula):
    the fp32 oracle gives transformers' logits recorded in tests/golden/qwen2_tiny_e2e.json, for
    the reference's prompt [2] and at every position of [2, 5, 1, 7]."""
    import json
    import os

    from dli_qwen2.reference_tiny import REFERENCE_TINY, reference_tiny_weights

    path = os.path.join(os.path.dirname(__file__), "golden", "qwen2_tiny_e2e.json")
    fixture = json.load(open(path, encoding="utf-8"))
    oracle = Qwen2Oracle(REFERENCE_TINY, reference_tiny_weights(), round_bf16=False)
    for name, case in fixture["cases"].items():
        ids = torch.tensor([case["input_ids"]], dtype=torch.int64)
        oracle.reset(1)
        logits = oracle.forward(ids)[0].double()
        expect = torch.tensor(case["logits"], dtype=torch.float64)
        torch.testing.assert_close(logits, expect, rtol=1e-5, atol=1e-6, msg=name)
