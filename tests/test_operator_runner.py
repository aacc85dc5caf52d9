"""The C++ operator runner (bin/dli_operator_engine_runner): a dli.graph.v1 graph, a
dli.weights.v1 inputs manifest and a plugin path in, dli.outputs.v1 out, with no Python in the
process. It is the counterpart of the reference's tests/operator_engine_runner.cc:114-137, which
drives every per-operator test of the reference (tests/operators/operator_test_support.py:108-137).
On the CPU the runner drives the ATen reference plugin; on the GPU the gfx950 plugin, for the
reference operators' known answers and a fused decode operator, against the oracle."""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest
import torch

import dli
from dli.weights import save_weights
from oracle import ops
from support import assert_close, kat_inputs, kat_outputs, load_kat

RUNNER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "dl-inference_amd", "bin", "dli_operator_engine_runner")
KAT = load_kat()
_NP = {"float32": np.float32, "int64": np.int64, "int32": np.int32, "float16": np.float16}


def run_runner(tmp, nodes, inputs, outputs, plugin, device):
    """Writes the graph and the inputs manifest under tmp, runs the runner and returns
    (returncode, stderr, {output name: float64/int array})."""
    graph = {"format": "dli.graph.v1", "model_type": "operator_runner_test",
             "inputs": list(inputs), "outputs": list(outputs), "nodes": nodes}
    (tmp / "g.json").write_text(json.dumps(graph))
    manifest = save_weights(tmp, "inputs", inputs)
    out_dir = tmp / "out"
    proc = subprocess.run([RUNNER, "--graph", str(tmp / "g.json"), "--inputs", str(manifest),
                           "--plugin", plugin, "--output-dir", str(out_dir), "--device", device],
                          capture_output=True, text=True, timeout=120)
    if proc.returncode != 0:
        return proc.returncode, proc.stderr, {}
    meta = json.loads((out_dir / "outputs.json").read_text())
    assert meta["format"] == "dli.outputs.v1"
    assert list(meta["tensors"]) == list(outputs)
    result = {}
    for name, spec in meta["tensors"].items():
        raw = (out_dir / spec["file"]).read_bytes()
        if spec["dtype"] == "bfloat16":  # bf16 bits are the upper half of an fp32
            bits = np.frombuffer(raw, np.uint16).astype(np.uint32) << 16
            arr = bits.view(np.float32).astype(np.float64)
        else:
            arr = np.frombuffer(raw, _NP[spec["dtype"]])
        result[name] = arr.reshape(spec["shape"])
    return 0, proc.stderr, result


def one_node(case):
    return [{"name": case["op"], "op": case["op"], "inputs": list(case["inputs"]),
             "outputs": list(case["outputs"]), "attrs": case["attrs"]}]


@pytest.mark.parametrize("case", KAT, ids=[c["op"] for c in KAT])
def test_runner_reference_known_answers_on_the_aten_cpu_plugin(case, tmp_path):
    rc, err, out = run_runner(tmp_path, one_node(case), kat_inputs(case), case["outputs"],
                              dli.aten_plugin_path(), "cpu")
    assert rc == 0, err
    for name, expected in kat_outputs(case).items():
        assert_close(out[name], expected, "float32")


def test_runner_reports_errors_with_status_1(tmp_path):
    case = KAT[0]
    rc, err, _ = run_runner(tmp_path, one_node(case), kat_inputs(case), case["outputs"],
                            str(tmp_path / "missing_plugin.so"), "cpu")
    assert rc == 1 and "operator engine runner failed" in err
    bad = dict(one_node(case)[0], op="no_such_operator")
    rc, err, _ = run_runner(tmp_path, [bad], kat_inputs(case), case["outputs"],
                            dli.aten_plugin_path(), "cpu")
    assert rc == 1 and "no_such_operator" in err
    proc = subprocess.run([RUNNER, "--graph"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 1 and "usage" in proc.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["linear", "attention", "rms_norm", "rotary_embedding", "conv2d"])
def test_runner_reference_known_answers_on_the_gfx950_plugin(op, tmp_path):
    case = next(c for c in KAT if c["op"] == op)
    rc, err, out = run_runner(tmp_path, one_node(case), kat_inputs(case), case["outputs"],
                              dli.plugin_path(), "cuda")
    assert rc == 0, err
    for name, expected in kat_outputs(case).items():
        assert_close(out[name], expected, "float32")


@pytest.mark.gpu
def test_runner_fused_gate_up_silu_decode_op(tmp_path):
    """The decode MLP's fused gate_up_silu (post-attention RMSNorm, gate and up projections over
    the 16-row interleaved weight, SwiGLU) at the Qwen2-0.5B shape, batch 32, from the runner
    against the oracle's composition of the reference nodes it replaces, at the bf16 bar."""
    from dli_qwen2.graph import interleave_gate_up

    g = torch.Generator().manual_seed(7)
    b, h, f = 32, 896, 4864
    x = torch.randn(b, h, generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    wg = (0.05 * torch.randn(f, h, generator=g)).to(torch.bfloat16)
    wu = (0.05 * torch.randn(f, h, generator=g)).to(torch.bfloat16)
    inputs = {"x": x, "nw": nw, "w": interleave_gate_up(wg, wu)}
    nodes = [{"name": "mlp.gate_up", "op": "gate_up_silu", "inputs": ["x", "nw", "w"],
              "outputs": ["act"], "attrs": {"eps": 1e-6}}]
    rc, err, out = run_runner(tmp_path, nodes, inputs, ["act"], dli.plugin_path(), "cuda")
    assert rc == 0, err
    R = ops.round_bf16
    xn = R(ops.rms_norm(x.float().numpy(), nw.float().numpy(), 1e-6))
    gate = R(ops.linear(xn, wg.float().numpy()))
    up = R(ops.linear(xn, wu.float().numpy()))
    assert_close(out["act"], R(R(ops.silu(gate)) * up), "bfloat16")
