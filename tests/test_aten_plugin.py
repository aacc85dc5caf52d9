"""The ATen CPU reference plugin (lib/libdli_aten_ops.so) on the CPU: the reference's operator
known answers, the reference-style Qwen2 decode graph against the oracle, the reference's
Qwen2-tiny fixture, and the config-1 single linear layer through the reference's "aten" node
(aten::linear through c10's dispatcher, src/aten_operator.cc:65-106) bit for bit against
torch.nn.functional.linear."""
from __future__ import annotations

import json
import os

import pytest
import torch
import torch.nn.functional as F

import dli
from dli_qwen2 import DecodeSession, random_weights, tiny_config
from dli_qwen2.reference_tiny import REFERENCE_TINY, reference_tiny_weights
from oracle.qwen2 import Qwen2Oracle
from support import assert_close, kat_inputs, kat_outputs, load_kat, one_node_graph

KAT = load_kat()


def _engine():
    return dli.Engine().load_aten_plugin()


def test_registers_the_reference_operator_names():
    from test_core import REF_OPS

    names = set(_engine().operator_names())
    assert set(REF_OPS) <= names and "argmax" in names


@pytest.mark.parametrize("case", KAT, ids=[c["op"] for c in KAT])
def test_reference_known_answers(case):
    inputs = kat_inputs(case)
    engine = _engine()
    outs = engine.run(one_node_graph(case["op"], inputs, list(case["outputs"]), case["attrs"]),
                      inputs)
    for name, expected in kat_outputs(case).items():
        assert_close(outs[name], expected, "float32")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tiny_decode_graph_matches_oracle(dtype):
    """The reference-style decode graph (19 nodes per layer, batch 3) stepped on host tensors
    through the Engine: greedy tokens equal the oracle's (fp32: the plain model; bf16: the oracle
    with the graph's bf16 rounding points), logits within the dtype's bar."""
    cfg = tiny_config()
    w = random_weights(cfg, seed=5, dtype=dtype)
    prompt = torch.randint(0, cfg.vocab, (3, 6), generator=torch.Generator().manual_seed(6))
    session = DecodeSession(cfg, w, 3, max_seq_len=32, fused=False, engine=_engine(), device="cpu")
    pos = torch.zeros(3, dtype=torch.int64)
    logits = []
    for t in range(6):
        lg, _ = session.step(prompt[:, t], pos)
        logits.append(lg.float())
        pos += 1
    oracle = Qwen2Oracle(cfg, w, round_bf16=dtype == torch.bfloat16)
    oracle.reset(3)
    ref = oracle.forward(prompt)  # [B, S, V]
    got = torch.stack(logits, 1)
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(got, ref, **tol)
    assert torch.equal(got.argmax(-1), ref.argmax(-1))


def test_reference_qwen2_tiny_fixture():
    fixture = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                          "qwen2_tiny_e2e.json"), encoding="utf-8"))
    spec = fixture["cases"]["extended"]
    session = DecodeSession(REFERENCE_TINY, reference_tiny_weights(), 1, max_seq_len=16,
                            fused=False, engine=_engine(), device="cpu")
    for t, token in enumerate(spec["input_ids"]):
        lg, _ = session.step(torch.tensor([token]), torch.tensor([t]))
        torch.testing.assert_close(lg[0].double(), torch.tensor(spec["logits"][t], dtype=torch.float64),
                                   rtol=1e-5, atol=1e-6)


def linear_config1_inputs(seed: int = 0):
    """Config 1's single linear layer: x ~ N(0, 1) [64, 1024]; W [4096, 1024] and b [4096]
    ~ U(-1/32, 1/32) (Kaiming-uniform bound 1/sqrt(1024)), seeded on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(64, 1024, generator=g)
    w = torch.rand(4096, 1024, generator=g) * (2 / 32) - 1 / 32
    b = torch.rand(4096, generator=g) * (2 / 32) - 1 / 32
    return x, w, b


def aten_linear_graph():
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "single_linear", "inputs": ["x", "w", "b"],
        "outputs": ["y"],
        "nodes": [{"name": "fc", "op": "aten", "inputs": ["x", "w", "b"], "outputs": ["y"],
                   "attrs": {"name": "aten::linear"}}]}))


def test_config1_aten_linear_is_bit_identical_to_torch():
    """The reference's CPU path for config 1: one "aten" node (aten::linear through the c10
    dispatcher) on the Engine, bit for bit equal to torch.nn.functional.linear on the same seeded
    inputs; the ATen plugin's own linear node gives the same bits."""
    x, w, b = linear_config1_inputs()
    expect = F.linear(x, w, b)
    engine = dli.Engine()
    y = engine.run(aten_linear_graph(), {"x": x, "w": w, "b": b})["y"]
    assert y.dtype == torch.float32 and y.shape == (64, 4096)
    assert torch.equal(y, expect)
    y2 = _engine().run(one_node_graph("linear", {"x": x, "w": w, "b": b}),
                       {"x": x, "w": w, "b": b})["output"]
    assert torch.equal(y2, expect)


def test_prefill_graph_then_decode_matches_oracle_greedy():
    """The prefill graph (all layers over the [B, S] prompt at once, build_prefill_graph) then
    decode steps, on host tensors in fp32: the same greedy tokens as the oracle's free-running
    greedy (batched prefill, then one token per step)."""
    cfg = tiny_config()
    w = random_weights(cfg, seed=7, dtype=torch.float32)
    prompt = torch.randint(0, cfg.vocab, (3, 9), generator=torch.Generator().manual_seed(8))
    session = DecodeSession(cfg, w, 3, max_seq_len=32, fused=False, engine=_engine(),
                            device="cpu", prefill=True)
    got = session.generate(prompt, 6)
    expect, _ = Qwen2Oracle(cfg, w, round_bf16=False).generate(prompt, 6)
    assert torch.equal(got, expect)


def test_prefill_layer_graph_matches_oracle_layer():
    """One decoder layer of prefill (config 3's computation at a small size) on host tensors in
    bf16: the oracle's layer with the graph's bf16 rounding points, within the bf16 bar."""
    from dli_qwen2 import build_prefill_graph

    cfg = tiny_config()
    w = random_weights(cfg, seed=9)
    h = torch.randn(2, 40, cfg.hidden, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    engine = _engine()
    engine.configure_kv_cache(block_size=64, max_seq_len=64)
    out = engine.run(build_prefill_graph(cfg, 2, 40, layers=1, from_hidden=True),
                     {**w, "hidden_states": h})["output"]
    oracle = Qwen2Oracle(cfg, w)
    oracle.reset(2)
    ref = oracle.forward_hidden(h.float(), [0])
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2)


def test_large_hidden_decode_graph_matches_oracle():
    """The large-hidden decode graph (hidden above what the fused kernels hold, head_dim 128 as
    in the Qwen2-7B geometry) on host tensors in fp32: greedy tokens and logits of the oracle."""
    from dli_qwen2 import Qwen2Config
    from dli_qwen2.graph import uses_large_graph

    cfg = Qwen2Config(hidden=1152, layers=2, heads=9, kv_heads=3, head_dim=128, ffn=512,
                      vocab=300, max_pos=64, tied_embeddings=False)
    assert uses_large_graph(cfg, True)
    w = random_weights(cfg, seed=11, dtype=torch.float32)
    prompt = torch.randint(0, cfg.vocab, (2, 5), generator=torch.Generator().manual_seed(12))
    session = DecodeSession(cfg, w, 2, max_seq_len=32, engine=_engine(), device="cpu")
    got = session.generate(prompt, 4)
    expect, _ = Qwen2Oracle(cfg, w, round_bf16=False).generate(prompt, 4)
    assert torch.equal(got, expect)
