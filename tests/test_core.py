"""Host runtime behaviour on the CPU, through the Python bindings.

Re-expresses the reference's C++ unit tests (tests/cpp/test_{graph,attributes,engine,
operator_registry,weights,aten_operator,kv_cache,tensor}.cc) and its binding test
(tests/python/test_dli_module.py) against this runtime, plus the libpython linkage guard
(cmake/check_no_libpython.cmake).
"""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest
import torch

import dli
from support import one_node_graph

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

REF_OPS = ["add", "attention", "batch_norm2d", "conv2d", "embedding", "linear", "matmul",
           "max_pool2d", "mul", "relu", "reshape", "rms_norm", "rotary_embedding", "silu",
           "softmax", "transpose"]


def test_graph_json_types_and_round_trip():
    # tests/cpp/test_graph.cc:10-51
    g = dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "graph_test", "weights": "weights.json",
        "inputs": ["x"], "outputs": ["y"],
        "nodes": [{"name": "node", "op_type": "aten", "inputs": ["x"], "outputs": ["y"],
                   "attrs": {"name": "aten::relu", "flag": True, "int": 2, "number": 1.5,
                             "ints": [1, 2], "numbers": [1, 2.5], "strings": ["a", "b"],
                             "empty": [], "whole": 2.0}}]}))
    assert g.model_type == "graph_test" and g.weights == "weights.json"
    assert len(g.nodes) == 1 and g.nodes[0].op_type == "aten"
    again = json.loads(g.to_json())
    attrs = again["nodes"][0]["attrs"]
    assert attrs["flag"] is True and attrs["int"] == 2 and attrs["number"] == 1.5
    assert attrs["ints"] == [1, 2] and attrs["numbers"] == [1.0, 2.5]
    assert attrs["strings"] == ["a", "b"] and attrs["empty"] == []
    # a double stays a double through to_json/from_json (written with a decimal point)
    assert isinstance(attrs["whole"], float)
    assert dli.Graph.from_json(g.to_json()).to_json() == g.to_json()
    with pytest.raises(ValueError):
        dli.Graph.from_json('{"format":"bad","nodes":[]}')
    with pytest.raises(ValueError):
        dli.Graph.from_json('{"format":"dli.graph.v1"}')
    with pytest.raises(ValueError):
        dli.Graph.from_json('{"format":"dli.graph.v1","nodes":[{"name":"n","op":"x","inputs":[],'
                            '"outputs":[],"attrs":{"bad":[1,"a"]}}]}')
    with pytest.raises(RuntimeError):
        dli.Graph.from_json_file("/nonexistent/graph.json")


def test_graph_op_wins_over_op_type_and_escapes_round_trip():
    g = dli.Graph.from_json(json.dumps({"format": "dli.graph.v1", "nodes": [
        {"name": "q\"\n\\", "op": "linear", "op_type": "ignored", "inputs": ["a"], "outputs": ["b"]}]}))
    assert g.nodes[0].op_type == "linear"
    assert dli.Graph.from_json(g.to_json()).nodes[0].name == "q\"\n\\"


def test_engine_builtins_and_errors():
    # tests/cpp/test_engine.cc:27-48
    e = dli.Engine()
    assert e.has_operator("aten")
    for name in ("conv2d", "attention", "linear", "rms_norm"):
        assert not e.has_operator(name)
    g = one_node_graph("aten", ["x"], ["y"], {"name": "aten::relu"})
    with pytest.raises(ValueError, match="missing input tensor"):
        e.run(g, {})
    g2 = dli.Graph.from_json(json.dumps({"format": "dli.graph.v1", "outputs": ["missing"],
                                         "nodes": [{"name": "relu", "op": "aten", "inputs": ["x"],
                                                    "outputs": ["y"], "attrs": {"name": "aten::relu"}}]}))
    with pytest.raises(ValueError, match="not produced"):
        e.run(g2, {"x": torch.ones(1)})
    with pytest.raises(ValueError, match="not registered"):
        e.run(one_node_graph("nope", ["x"]), {"x": torch.ones(1)})


def test_engine_returns_all_tensors_when_outputs_empty():
    g = dli.Graph.from_json(json.dumps({"format": "dli.graph.v1", "nodes": [
        {"name": "r", "op": "aten", "inputs": ["x"], "outputs": ["y"], "attrs": {"name": "aten::relu"}}]}))
    out = dli.Engine().run(g, {"x": torch.tensor([-1.0, 2.0])})
    assert set(out) == {"x", "y"}
    assert out["y"].tolist() == [0.0, 2.0]


def test_aten_operator():
    # tests/cpp/test_aten_operator.cc:14-68 and tests/python/test_dli_module.py:10-41
    e = dli.Engine()
    x = torch.tensor([-1.0, 0.5, 2.0, -3.0])
    y = e.run(one_node_graph("aten", ["x"], ["y"], {"name": "aten::relu"}), {"x": x})["y"]
    torch.testing.assert_close(y, torch.relu(x), atol=1e-6, rtol=0)
    lhs, rhs = torch.tensor([[1.0, 2.0], [3.0, 4.0]]), torch.tensor([10.0, 20.0])
    out = e.run(one_node_graph("aten", ["x", "bias"], ["y"],
                               {"name": "aten::add", "overload": "Tensor", "attr_order": ["alpha"],
                                "alpha": 1.5}), {"x": lhs, "bias": rhs})
    torch.testing.assert_close(out["y"], lhs + rhs * 1.5)
    with pytest.raises(ValueError):
        e.run(one_node_graph("aten", ["x"], ["y"], {}), {"x": x})
    with pytest.raises(ValueError, match="reserved"):
        e.run(one_node_graph("aten", ["x"], ["y"], {"name": "aten::relu", "attr_order": ["name"]}),
              {"x": x})
    # bfloat16 tensors flow through the engine (dtype extension)
    xb = torch.tensor([-1.0, 2.0], dtype=torch.bfloat16)
    yb = e.run(one_node_graph("aten", ["x"], ["y"], {"name": "aten::relu"}), {"x": xb})["y"]
    assert yb.dtype == torch.bfloat16 and yb.tolist() == [0.0, 2.0]


def test_plugin_registry_contract(tmp_path):
    # tests/cpp/test_operator_registry.cc:36-63
    e = dli.Engine()
    for name in REF_OPS:
        assert not e.has_operator(name)
    with pytest.raises(RuntimeError, match="failed to load operator library"):
        e.load_library(str(tmp_path / "missing_plugin.so"))
    with pytest.raises(RuntimeError, match="missing dli_register_operators"):
        e.load_library(dli.hip_library_path())
    e.load_plugin()
    for name in REF_OPS:
        assert e.has_operator(name), name


def test_plugin_ops_reject_host_tensors():
    e = dli.Engine().load_plugin()
    x = torch.ones(2, 3)
    with pytest.raises(ValueError, match="CUDA"):
        e.run(one_node_graph("add", ["x", "b"]), {"x": x, "b": x})
    with pytest.raises(ValueError, match="CUDA"):
        e.run(one_node_graph("attention", ["q", "k", "v"], attrs={"kv_cache": "layer"}),
              {"q": torch.ones(1, 1, 1, 2), "k": torch.ones(1, 1, 1, 2), "v": torch.ones(1, 1, 1, 2)})


def _write_weights(path, tensors):
    data, meta, offset = bytearray(), {}, 0
    for name, t in tensors.items():
        raw = t.contiguous().view(torch.uint8).numpy().tobytes() if t.dtype == torch.bfloat16 else \
            t.contiguous().numpy().tobytes()
        meta[name] = {"dtype": {torch.float32: "float32", torch.int64: "int64",
                                torch.bfloat16: "bfloat16", torch.int32: "int32",
                                torch.float16: "float16"}[t.dtype],
                      "shape": list(t.shape), "offset": offset, "nbytes": len(raw)}
        data += raw
        offset += len(raw)
    (path / "w.bin").write_bytes(bytes(data))
    (path / "w.json").write_text(json.dumps({"format": "dli.weights.v1", "data": "w.bin",
                                             "tensors": meta}))
    return str(path / "w.json")


def test_weights_loader(tmp_path):
    # tests/cpp/test_weights.cc:9-58, plus bfloat16/float16/int32 dtypes
    tensors = {"linear.weight": torch.tensor([[1.0, 2.0], [3.0, 4.0]]),
               "ids": torch.tensor([7, 8], dtype=torch.int64),
               "bf": torch.tensor([1.5, -2.25, 3.0], dtype=torch.bfloat16),
               "hf": torch.tensor([0.5], dtype=torch.float16),
               "i32": torch.tensor([[1, -2]], dtype=torch.int32)}
    loaded = dli.load_weights(_write_weights(tmp_path, tensors))
    for name, t in tensors.items():
        assert loaded[name].dtype == t.dtype and torch.equal(loaded[name], t), name
    bad = tmp_path / "bad.json"
    bad.write_text('{"format":"bad","data":"missing.bin","tensors":{}}')
    with pytest.raises(ValueError):
        dli.load_weights(str(bad))
    over = tmp_path / "over.json"
    over.write_text(json.dumps({"format": "dli.weights.v1", "data": "w.bin", "tensors": {
        "x": {"dtype": "float32", "shape": [1000], "offset": 0, "nbytes": 4000}}}))
    with pytest.raises(ValueError, match="exceeds"):
        dli.load_weights(str(over))


def test_kv_cache_controls():
    e = dli.Engine()
    assert e.kv_cache_size() == 0 and e.kv_cache_entry("missing") is None
    e.configure_kv_cache(block_size=16, max_seq_len=100)
    with pytest.raises(ValueError):
        e.configure_kv_cache(block_size=0, max_seq_len=10)
    e.clear_kv_cache()
    assert e.kv_cache_size() == 0


@pytest.mark.parametrize("lib", ["libdli_core.so", "libdli_hip_ops.so", "libdli_hip.so"])
def test_native_libraries_do_not_link_libpython(lib):
    # cmake/check_no_libpython.cmake:25-32
    out = subprocess.run(["ldd", os.path.join(dli.LIB_DIR, lib)], capture_output=True, text=True,
                         check=True).stdout
    assert "libpython" not in out


def test_device_library_has_no_torch_dependency():
    out = subprocess.run(["ldd", dli.hip_library_path()], capture_output=True, text=True,
                         check=True).stdout
    assert "torch" not in out and "c10" not in out


def _compile_snippet(tmp_path, body):
    torch_dir = os.path.dirname(torch.__file__)
    src = tmp_path / "snippet.cc"
    src.write_text('#include "dli/kv_cache.h"\nint probe(dli::KVCacheEntry& e) {\n' + body +
                   "\n  return 0;\n}\n")
    return subprocess.run(
        ["g++", "-std=c++20", "-fsyntax-only", f"-I{ROOT}/include",
         "-isystem", f"{torch_dir}/include", "-isystem",
         f"{torch_dir}/include/torch/csrc/api/include", str(src)],
        capture_output=True, text=True)


def test_reference_kv_entry_fields_do_not_compile(tmp_path):
    """Plugin source written against the reference's KV entry (contiguous [B,H,S,D] tensors
    `key` / `value`, which its attention template binds straight as K and V) must not compile
    against the paged entry here, whose pools are `key_pool` / `value_pool`."""
    assert _compile_snippet(tmp_path, "(void)e.key_pool; (void)e.value_pool;").returncode == 0
    bad = _compile_snippet(tmp_path, "(void)e.key; (void)e.value;")
    assert bad.returncode != 0 and "key" in bad.stderr
