"""AlexNet-style CNN as a dli.graph.v1 graph (the shape of the reference's examples/alexnet,
widened to the CIFAR-size AlexNet of the fp32 CNN benchmark): NCHW fp32 input [B, 3, 32, 32];
conv 64@3x3 s1p1, ReLU, max_pool 2; conv 192@3x3, ReLU, max_pool 2; conv 384/256/256@3x3, ReLU;
flatten; fully connected 4096, ReLU, 4096, ReLU, 10.

With fused=True each conv2d / linear node carries activation = "relu" (the ReLU runs in the MFMA
GEMM epilogue); with fused=False the graph has separate relu nodes as the reference exporter
emits them. Weights are random (Kaiming-uniform, seeded) and live only in memory."""
from __future__ import annotations

import json
import math

import torch

import dli

CONVS = [(3, 64), (64, 192), (192, 384), (384, 256), (256, 256)]  # (in, out) channels, 3x3 s1p1
POOL_AFTER = {0, 1}  # max_pool2d 2x2 after these convs
FCS = [(256 * 8 * 8, 4096), (4096, 4096), (4096, 10)]
IMAGE = (3, 32, 32)


def build_graph(batch: int, fused: bool = True) -> "dli.Graph":
    nodes = []

    def node(name, op, inputs, outputs, attrs=None):
        nodes.append({"name": name, "op": op, "inputs": inputs, "outputs": outputs,
                      **({"attrs": attrs} if attrs else {})})

    h = "x"
    for i, _ in enumerate(CONVS):
        attrs = {"stride": [1, 1], "padding": [1, 1]}
        if fused:
            attrs["activation"] = "relu"
        node(f"features.conv{i}", "conv2d", [h, f"conv{i}.weight", f"conv{i}.bias"], [f"c{i}"],
             attrs)
        h = f"c{i}"
        if not fused:
            node(f"features.relu{i}", "relu", [h], [f"r{i}"])
            h = f"r{i}"
        if i in POOL_AFTER:
            node(f"features.pool{i}", "max_pool2d", [h], [f"p{i}"],
                 {"kernel_size": [2, 2], "stride": [2, 2]})
            h = f"p{i}"
    node("flatten", "reshape", [h], ["flat"], {"shape": [batch, FCS[0][0]]})
    h = "flat"
    for i, _ in enumerate(FCS):
        last = i == len(FCS) - 1
        attrs = {"activation": "relu"} if fused and not last else None
        out = "logits" if last else f"f{i}"
        node(f"classifier.fc{i}", "linear", [h, f"fc{i}.weight", f"fc{i}.bias"], [out], attrs)
        h = out
        if not fused and not last:
            node(f"classifier.relu{i}", "relu", [h], [f"fr{i}"])
            h = f"fr{i}"
    inputs = ["x"] + [f"{k}{i}.{p}" for k, n in (("conv", CONVS), ("fc", FCS))
                      for i in range(len(n)) for p in ("weight", "bias")]
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "alexnet_cifar", "inputs": inputs,
        "outputs": ["logits"], "nodes": nodes}))


def random_weights(seed: int = 0, device: str = "cpu") -> dict:
    """Kaiming-uniform weights and biases, U(-1/sqrt(fan_in), 1/sqrt(fan_in)) (torch's default
    Conv2d / Linear initialisation)."""
    g = torch.Generator().manual_seed(seed)
    out = {}

    def uni(shape, fan_in):
        bound = 1.0 / math.sqrt(fan_in)
        return (torch.rand(shape, generator=g) * 2 - 1) * bound

    for i, (cin, cout) in enumerate(CONVS):
        out[f"conv{i}.weight"] = uni((cout, cin, 3, 3), cin * 9)
        out[f"conv{i}.bias"] = uni((cout,), cin * 9)
    for i, (fin, fout) in enumerate(FCS):
        out[f"fc{i}.weight"] = uni((fout, fin), fin)
        out[f"fc{i}.bias"] = uni((fout,), fin)
    return {k: v.to(device) for k, v in out.items()}


def flops_per_image() -> int:
    """Multiply-adds x 2 of the convs and fully connected layers (ReLU and pooling excluded)."""
    total, hw = 0, IMAGE[1] * IMAGE[2]
    for i, (cin, cout) in enumerate(CONVS):
        total += 2 * hw * cout * cin * 9
        if i in POOL_AFTER:
            hw //= 4
    return total + sum(2 * fin * fout for fin, fout in FCS)


def torch_forward(x: torch.Tensor, w: dict) -> torch.Tensor:
    """The same network with ATen functional ops (the CPU ATen path timed beside the GPU)."""
    import torch.nn.functional as F

    h = x
    for i, _ in enumerate(CONVS):
        h = F.relu(F.conv2d(h, w[f"conv{i}.weight"], w[f"conv{i}.bias"], padding=1))
        if i in POOL_AFTER:
            h = F.max_pool2d(h, 2, 2)
    h = h.reshape(h.shape[0], -1)
    for i, _ in enumerate(FCS):
        h = F.linear(h, w[f"fc{i}.weight"], w[f"fc{i}.bias"])
        if i < len(FCS) - 1:
            h = F.relu(h)
    return h
