"""Helpers shared by the tests: one-node dli.graph.v1 runs (the in-process counterpart of the
reference's tests/operators/operator_test_support.py:108-137) and golden fixtures."""
from __future__ import annotations

import json
import os

import numpy as np
import torch

import dli

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TORCH_DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16,
                "int64": torch.int64, "int32": torch.int32}

# Tolerances stated by the parity contract: fp32 1e-4 relative, bf16 2e-2 (fp16 uses 2e-3).
TOL = {"float32": dict(rtol=1e-4, atol=1e-5), "bfloat16": dict(rtol=2e-2, atol=2e-2),
       "float16": dict(rtol=2e-3, atol=2e-3)}


def one_node_graph(op, inputs, outputs=("output",), attrs=None):
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1",
        "model_type": "operator_numeric_test",
        "inputs": list(inputs),
        "outputs": list(outputs),
        "nodes": [{"name": op, "op": op, "inputs": list(inputs), "outputs": list(outputs),
                   "attrs": attrs or {}}],
    }))


_ENGINE = None


def plugin_engine() -> dli.Engine:
    global _ENGINE
    if _ENGINE is None:
        _ENGINE = dli.Engine().load_plugin()
    return _ENGINE


def run_op(op, inputs: dict, outputs=("output",), attrs=None, engine=None):
    engine = engine or plugin_engine()
    result = engine.run(one_node_graph(op, inputs, outputs, attrs), inputs)
    torch.cuda.synchronize()
    return result


def load_kat():
    with open(os.path.join(GOLDEN, "kat_ops.json"), encoding="utf-8") as f:
        return json.load(f)["cases"]


def kat_inputs(case, device="cpu", float_dtype=torch.float32):
    out = {}
    for name, spec in case["inputs"].items():
        dtype = torch.int64 if spec["dtype"] == "int64" else float_dtype
        out[name] = torch.tensor(spec["data"], dtype=torch.float64).reshape(spec["shape"]).to(
            dtype).to(device)
    return out


def kat_outputs(case):
    return {name: np.asarray(spec["data"], dtype=np.float64).reshape(spec["shape"])
            for name, spec in case["outputs"].items()}


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy() if t.is_floating_point() else t.cpu().numpy()


def assert_close(actual, expected, dtype="float32", **override):
    tol = dict(TOL[dtype])
    tol.update(override)
    a = to_np(actual) if isinstance(actual, torch.Tensor) else np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"shape {a.shape} != {e.shape}"
    np.testing.assert_allclose(a, e, **tol)
