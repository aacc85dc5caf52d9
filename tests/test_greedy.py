"""C++ greedy decode driver (dli.GreedyDecoder) argument checks and the dli.weights.v1 writer
(dli.weights.save_weights) round trip through the C++ loader. Decoding itself needs the gfx950
plugin: tests/test_greedy_gpu.py."""
from __future__ import annotations

import json

import pytest
import torch

import dli
from dli.weights import save_weights


def _graph(outputs=("next_ids",)):
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "greedy_test",
        "inputs": ["input_ids", "positions", "table"], "outputs": list(outputs),
        "nodes": [{"name": "emb", "op": "aten", "inputs": ["table", "input_ids"],
                   "outputs": ["next_ids"], "attrs": {"name": "aten::embedding"}}]}))


def test_weights_round_trip_all_dtypes(tmp_path):
    g = torch.Generator().manual_seed(0)
    tensors = {
        "f32": torch.randn(3, 5, generator=g),
        "bf16": torch.randn(7, 9, generator=g).to(torch.bfloat16),
        "f16": torch.randn(4, generator=g).to(torch.float16),
        "i64": torch.randint(-2**40, 2**40, (6,), generator=g),
        "i32": torch.randint(-2**30, 2**30, (2, 3), generator=g, dtype=torch.int32),
        "empty": torch.zeros(0, 4),
    }
    path = save_weights(tmp_path, "m", tensors)
    assert path.name == "m.dli.weights.json"
    manifest = json.loads(path.read_text())
    assert manifest["format"] == "dli.weights.v1" and manifest["data"] == "m.dli.weights.bin"
    assert all(m["offset"] % 64 == 0 for m in manifest["tensors"].values())
    assert manifest["tensors"]["bf16"]["dtype"] == "bfloat16"
    assert manifest["tensors"]["bf16"]["nbytes"] == 7 * 9 * 2
    back = dli.load_weights(str(path))
    assert set(back) == set(tensors)
    for name, t in tensors.items():
        assert back[name].dtype == t.dtype and back[name].shape == t.shape
        assert torch.equal(back[name], t), name  # bit-exact, bf16 included


def test_weights_writer_rejects_unsupported_dtype(tmp_path):
    with pytest.raises(TypeError):
        save_weights(tmp_path, "bad", {"b": torch.zeros(2, dtype=torch.bool)})


def test_decoder_rejects_bad_graphs_and_arguments():
    e = dli.Engine()
    table = {"table": torch.randn(10, 4)}
    with pytest.raises(ValueError, match="next_ids"):
        dli.GreedyDecoder(e, _graph(outputs=("y",)), table, 2)
    with pytest.raises(ValueError, match="step input"):
        dli.GreedyDecoder(e, _graph(), {**table, "input_ids": torch.zeros(2, dtype=torch.int64)}, 2)
    with pytest.raises(ValueError, match="batch"):
        dli.GreedyDecoder(e, _graph(), table, 0)
    d = dli.GreedyDecoder(e, _graph(), table, 2, max_seq_len=8)
    assert d.batch == 2 and not d.captured  # host weights: eager steps
    pos = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="ids"):
        d.step(torch.zeros(3, dtype=torch.int64), pos)
    with pytest.raises(ValueError, match="ids"):
        d.step(torch.zeros(2, dtype=torch.int32), pos)
    with pytest.raises(IndexError):
        d.step(torch.zeros(2, dtype=torch.int64), torch.tensor([0, 8]))
    with pytest.raises(ValueError, match="prompt"):
        d.generate(torch.zeros(2, 0, dtype=torch.int64), 3)
    with pytest.raises(ValueError, match="prompt"):
        d.generate(torch.zeros(3, 2, dtype=torch.int64), 3)
    with pytest.raises(IndexError):  # 6 prompt positions + 3 tokens need positions up to 7 + 1
        d.generate(torch.zeros(2, 6, dtype=torch.int64), 4)


def _status_graph():
    """A decode-step graph with a `status` output, as the decoder_stack graph has: here
    status = clone(flag) on the host, so the test controls what a step reports."""
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "greedy_status_test",
        "inputs": ["input_ids", "positions", "table", "flag"],
        "outputs": ["next_ids", "status"],
        "nodes": [
            {"name": "emb", "op": "aten", "inputs": ["table", "input_ids"],
             "outputs": ["ids2"], "attrs": {
                 "name": "aten::embedding", "padding_idx": -1, "scale_grad_by_freq": False,
                 "sparse": False, "attr_order": ["padding_idx", "scale_grad_by_freq", "sparse"]}},
            {"name": "pick", "op": "aten", "inputs": ["ids2"], "outputs": ["next_ids"],
             "attrs": {"name": "aten::select", "overload": "int", "dim": 1, "index": 0,
                       "attr_order": ["dim", "index"]}},
            {"name": "status", "op": "aten", "inputs": ["flag"], "outputs": ["status"],
             "attrs": {"name": "aten::abs"}}]}))


def test_decoder_raises_on_a_reported_launch_failure():
    """A step whose `status` output is non-zero (a decoder_stack wait gave up) makes the next
    synchronizing call raise; generate() checks once at its end, after its own sync."""
    e = dli.Engine()
    table = torch.arange(40, dtype=torch.int64).reshape(10, 4)
    ok = dli.GreedyDecoder(e, _status_graph(), {"table": table,
                                                "flag": torch.zeros(1, dtype=torch.int32)}, 2)
    pos = torch.zeros(2, dtype=torch.int64)
    ok.step(torch.zeros(2, dtype=torch.int64), pos)
    ok.step(torch.zeros(2, dtype=torch.int64), pos + 1)
    ok.check_status()

    bad = dli.GreedyDecoder(e, _status_graph(), {"table": table,
                                                 "flag": torch.ones(1, dtype=torch.int32)}, 2)
    bad.step(torch.zeros(2, dtype=torch.int64), pos)  # reports, nothing checked yet
    with pytest.raises(RuntimeError, match="gave up waiting"):
        bad.step(torch.zeros(2, dtype=torch.int64), pos + 1)
    bad.check_status()  # the word was cleared when it was reported
    with pytest.raises(RuntimeError, match="gave up waiting"):
        bad.generate(torch.zeros(2, 1, dtype=torch.int64), 2)


def test_stack_graph_folds_the_embedding_into_the_decoder_stack_node():
    """The stack graph has no embedding node: its decoder_stack node reads the token ids and,
    after the layer weights, the embedding table (the launch gathers the rows itself). The
    fused graph keeps the embedding node."""
    from dli_qwen2 import tiny_config
    from dli_qwen2.graph import build_decode_graph

    cfg = tiny_config(layers=2)
    stack = json.loads(build_decode_graph(cfg, 4, fused=True, stack=True,
                                          stack_trace=True).to_json())
    ops = [n["op"] for n in stack["nodes"]]
    assert ops == ["decoder_stack", "lm_head_argmax"]
    node = stack["nodes"][0]
    assert node["inputs"][:4] == ["input_ids", "positions", "rotary_cos", "rotary_sin"]
    assert node["inputs"][-2:] == ["model.embed_tokens.weight", "stack_trace"]
    assert len(node["inputs"]) == 4 + 7 * cfg.layers + 2
    fused = json.loads(build_decode_graph(cfg, 4, fused=True).to_json())
    assert fused["nodes"][0]["op"] == "embedding"
