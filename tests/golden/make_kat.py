"""Writes tests/golden/kat_ops.json: the reference's per-operator known-answer cases.

Inputs are the literal tensors of the reference's tests/operators/test_<op>.py (transcribed
as data; file:line cited per case). Expected outputs are computed here with the same torch
closed forms those tests compare against (F.linear, F.conv2d, torch.softmax, ...), in float64.
Run: python tests/golden/make_kat.py
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import torch
import torch.nn.functional as F

D = torch.float64


def t(data):
    return torch.tensor(data, dtype=D)


def case(op, source, inputs, expected, attrs=None, outputs=None):
    return {
        "op": op,
        "source": source,
        "attrs": attrs or {},
        "inputs": {k: {"dtype": "int64" if v.dtype == torch.int64 else "float32",
                       "shape": list(v.shape), "data": v.reshape(-1).tolist()}
                   for k, v in inputs.items()},
        "outputs": {k: {"shape": list(v.shape), "data": v.reshape(-1).tolist()}
                    for k, v in zip(outputs or ["output"], expected)},
    }


def build():
    cases = []
    x = t([[1.0, -2.0, 3.0], [4.0, 5.0, -6.0]])
    b = t([0.5, -1.0, 2.0])
    cases.append(case("add", "tests/operators/test_add.py:13-15", {"x": x, "b": b}, [x + b]))
    cases.append(case("mul", "tests/operators/test_mul.py:13-15", {"x": x, "b": b}, [x * b]))

    q = t([[[[0.2, -0.4], [1.0, 0.5]], [[-0.3, 0.7], [0.8, -0.6]]]])
    k = t([[[[0.1, 0.9], [-0.5, 0.2]], [[0.6, -0.1], [0.3, 0.4]]]])
    v = t([[[[1.0, -1.0], [0.5, 0.25]], [[-0.2, 0.8], [1.2, -0.7]]]])
    scores = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    mask = torch.tril(torch.ones(2, 2, dtype=torch.bool))
    att = torch.softmax(scores.masked_fill(~mask, float("-inf")), dim=-1) @ v
    cases.append(case("attention", "tests/operators/test_attention.py:14-23",
                      {"q": q, "k": k, "v": v}, [att], attrs={"causal": True}))

    xb = torch.arange(48, dtype=D).reshape(2, 3, 2, 4) / 8.0
    w = t([1.25, -0.5, 2.0])
    bb = t([0.25, 1.0, -0.75])
    rm = t([0.5, 1.5, 2.5])
    rv = t([0.25, 1.0, 4.0])
    bn = F.batch_norm(xb, rm, rv, w, bb, training=False, eps=1e-4)
    cases.append(case("batch_norm2d", "tests/operators/test_batch_norm2d.py:13-33",
                      {"x": xb, "weight": w, "bias": bb, "running_mean": rm, "running_var": rv},
                      [bn], attrs={"eps": 1e-4}))

    xc = torch.arange(16, dtype=D).reshape(1, 1, 4, 4) / 8.0
    wc = t([[[[1.0, 0.0], [0.0, -1.0]]], [[[0.5, -0.25], [0.75, 0.125]]]])
    bc = t([0.25, -0.5])
    cases.append(case("conv2d", "tests/operators/test_conv2d.py:13-21",
                      {"x": xc, "weight": wc, "bias": bc}, [F.conv2d(xc, wc, bias=bc)],
                      attrs={"stride": [1, 1], "padding": [0, 0]}))

    ids = torch.tensor([[2, 1], [0, 3]], dtype=torch.int64)
    table = torch.arange(20, dtype=D).reshape(5, 4) / 10.0
    cases.append(case("embedding", "tests/operators/test_embedding.py:13-17",
                      {"ids": ids, "table": table}, [table[ids]]))

    xl = t([[1.0, 2.0, -1.0, 0.5], [-0.5, 3.0, 1.5, 2.0]])
    wl = t([[0.5, -1.0, 0.25, 2.0], [1.5, 0.0, -0.5, 0.75], [-1.0, 1.0, 0.5, 0.0]])
    bl = t([0.1, -0.2, 0.3])
    cases.append(case("linear", "tests/operators/test_linear.py:13-19",
                      {"x": xl, "weight": wl, "bias": bl}, [F.linear(xl, wl, bl)]))

    a = t([[1.0, -2.0, 0.5, 3.0], [0.25, 1.5, -1.0, 2.0]])
    bm = t([[0.5, 1.0, -0.75], [1.5, -0.5, 0.25], [-1.0, 0.0, 2.0], [0.25, 0.75, -1.5]])
    cases.append(case("matmul", "tests/operators/test_matmul.py:13-17", {"a": a, "b": bm},
                      [a @ bm]))

    xp = t([[[[1.0, -1.0, 3.0, 2.0], [0.5, 4.0, -2.0, 1.5], [2.5, 0.0, 5.0, -0.5],
               [1.0, 3.5, 2.0, 4.5]]]])
    cases.append(case("max_pool2d", "tests/operators/test_max_pool2d.py:13-33", {"x": xp},
                      [F.max_pool2d(xp, kernel_size=2, stride=2)],
                      attrs={"kernel_size": [2, 2], "stride": [2, 2], "padding": [0, 0]}))

    xr = t([[-1.0, 0.0, 2.0], [3.5, -4.0, 5.0]])
    cases.append(case("relu", "tests/operators/test_relu.py:13-14", {"x": xr}, [torch.relu(xr)]))
    cases.append(case("silu", "tests/operators/test_silu.py:13-14", {"x": xr}, [F.silu(xr)]))

    xs = torch.arange(6, dtype=D).reshape(2, 3)
    cases.append(case("reshape", "tests/operators/test_reshape.py:13-15", {"x": xs},
                      [xs.reshape(3, 2)], attrs={"shape": [3, 2]}))

    xn = t([[1.0, 2.0, -1.0, 0.5], [-0.5, 3.0, 1.5, 2.0]])
    wn = t([0.5, 1.0, -1.5, 2.0])
    rms = xn * torch.rsqrt((xn * xn).mean(dim=-1, keepdim=True) + 1e-6) * wn
    cases.append(case("rms_norm", "tests/operators/test_rms_norm.py:13-19",
                      {"x": xn, "weight": wn}, [rms], attrs={"eps": 1e-6}))

    qr = t([[[[1.0, 2.0], [-1.0, 0.5]]]])
    kr = t([[[[0.25, -0.75], [1.5, -2.0]]]])
    cos = t([[1.0], [0.5], [-0.25], [0.75]])
    sin = t([[0.0], [0.25], [0.5], [-0.5]])

    def rotate(z):
        out = z.clone()
        c = cos[1:3, 0].reshape(1, 1, 2)
        s = sin[1:3, 0].reshape(1, 1, 2)
        out[..., 0] = z[..., 0] * c - z[..., 1] * s
        out[..., 1] = z[..., 0] * s + z[..., 1] * c
        return out

    cases.append(case("rotary_embedding", "tests/operators/test_rotary_embedding.py:13-38",
                      {"q": qr, "k": kr, "cos": cos, "sin": sin}, [rotate(qr), rotate(kr)],
                      attrs={"start_pos": 1}, outputs=["out_q", "out_k"]))

    xsm = t([[1.0, 0.0, -1.0, 2.0, 0.5], [-0.5, 1.5, 2.5, -1.0, 0.0]])
    cases.append(case("softmax", "tests/operators/test_softmax.py:13-14", {"x": xsm},
                      [torch.softmax(xsm, dim=-1)]))

    xt = t([[1.0, -2.0, 3.0], [4.0, 5.0, -6.0]])
    cases.append(case("transpose", "tests/operators/test_transpose.py:13-15", {"x": xt},
                      [xt.t()], attrs={"perm": [1, 0]}))
    return cases


def main():
    out = Path(__file__).with_name("kat_ops.json")
    out.write_text(json.dumps({"format": "dli.kat.v1", "cases": build()}, indent=1) + "\n",
                   encoding="utf-8")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
