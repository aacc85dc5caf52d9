"""MFMA GEMMs of the generic operators (csrc/kernels/mfma_gemm.hip) through the plugin: fp32
linear / matmul / conv2d (implicit GEMM; a conv whose patch has 9 or 27 elements takes the
direct kernels conv2d_small_f32_p9 / _p27 in csrc/kernels/conv.hip), tiled bf16 linear, and the fused ReLU epilogue
(attribute activation = "relu"), against the CPU oracle at the parity contract's tolerances
(fp32 1e-4 relative, bf16 2e-2). Ragged shapes cover every tile edge; the larger cases take the
128 x 128 tile path. Last, the reference's TinyAlexNet end-to-end case
(tests/e2e/test_models.py:42-58, examples/alexnet/alexnet.py) as a dli.graph.v1 graph."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import dli
from oracle import ops
from support import assert_close, plugin_engine, run_op, to_np

pytestmark = pytest.mark.gpu


def close_f32(actual, expected):
    """fp32 parity: 1e-4 relative per element, plus an absolute term of 1e-5 x the output's RMS.
    The rounding error of a K-term fp32 sum grows with its partial sums, not with the result,
    so an output that cancels to near zero keeps an absolute error of about sqrt(K) ulps of the
    partial sums (5e-5 at K = 1024 and outputs of size 30); a wrong index, sign or operand moves
    outputs by the size of the RMS itself."""
    e = np.asarray(expected, np.float64)
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    assert_close(actual, e, atol=max(1e-5, 1e-5 * rms))


def rand(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).cuda()


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 17, 3), (64, 4096, 1024), (130, 257, 33),
                                   (300, 70, 1000), (2048, 2048, 72)])
def test_linear_f32(m, n, k):
    x, w, b = rand((m, k), 1), rand((n, k), 2), rand((n,), 3)
    out = run_op("linear", {"x": x, "weight": w, "bias": b})["output"]
    close_f32(out, ops.linear(to_np(x), to_np(w), to_np(b)))
    relu = run_op("linear", {"x": x, "weight": w, "bias": b}, attrs={"activation": "relu"})["output"]
    close_f32(relu, ops.relu(ops.linear(to_np(x), to_np(w), to_np(b))))


@pytest.mark.parametrize("m,n,k", [(32, 1024, 8192), (64, 300, 5000)])
def test_linear_f32_split_k(m, n, k):
    """Few output tiles, long K: the plugin passes a workspace and K is split (8 and 4 ways
    here); the C ABI without a workspace runs unsplit. Both match the oracle."""
    from dli import hip

    x, w, b = rand((m, k), 14), rand((n, k), 15), rand((n,), 16)
    assert hip.lib().dli_hip_linear_workspace(hip.F32, m, n, k) > 0
    ref = ops.relu(ops.linear(to_np(x), to_np(w), to_np(b)))
    close_f32(run_op("linear", {"x": x, "weight": w, "bias": b},
                     attrs={"activation": "relu"})["output"], ref)
    out = torch.empty(m, n, device="cuda")
    hip.call("dli_hip_linear_act", hip.F32, hip.F32, x.data_ptr(), w.data_ptr(), b.data_ptr(),
             out.data_ptr(), m, n, k, 1, None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    close_f32(out, ref)


@pytest.mark.parametrize("m,n,k", [(5, 9, 2), (96, 200, 130), (2048, 2048, 40)])
def test_matmul_f32(m, n, k):
    a, b = rand((m, k), 4), rand((k, n), 5)
    close_f32(run_op("matmul", {"a": a, "b": b})["output"], ops.matmul(to_np(a), to_np(b)))


@pytest.mark.parametrize("out_dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("m,n,k", [(65, 1152, 896), (300, 4864, 896), (2048, 2048, 256),
                                   (100, 33, 8)])
def test_linear_bf16_tiled(m, n, k, out_dtype):
    x, w = rand((m, k), 6, torch.bfloat16), rand((n, k), 7, torch.bfloat16, 0.05)
    b = rand((n,), 8, torch.bfloat16)
    attrs = {"out_dtype": out_dtype} if out_dtype == "float32" else {}
    out = run_op("linear", {"x": x, "weight": w, "bias": b}, attrs=attrs)["output"]
    assert out.dtype == (torch.float32 if out_dtype == "float32" else torch.bfloat16)
    ref = ops.linear(to_np(x), to_np(w), to_np(b))
    assert_close(out, ref, "bfloat16")
    relu = run_op("linear", {"x": x, "weight": w, "bias": b},
                  attrs={**attrs, "activation": "relu"})["output"]
    assert_close(relu, ops.relu(ref), "bfloat16")


CONVS = [  # (N, C, H, W, OC, KH, KW, stride, pad)
    (2, 3, 32, 32, 64, 3, 3, (1, 1), (1, 1)),     # AlexNet-style conv1
    (2, 64, 16, 16, 192, 3, 3, (1, 1), (1, 1)),   # conv2
    (2, 192, 8, 8, 384, 3, 3, (1, 1), (1, 1)),    # conv3
    (3, 5, 11, 13, 10, 3, 2, (2, 1), (1, 0)),     # ragged, strided, asymmetric
    (2, 8, 9, 9, 7, 5, 5, (1, 1), (2, 2)),
    (4, 16, 7, 7, 33, 1, 1, (1, 1), (0, 0)),      # 1x1
    (16, 16, 32, 32, 256, 3, 3, (1, 1), (1, 1)),  # 128 x 128 tiles
    (2, 256, 8, 8, 256, 3, 3, (1, 1), (1, 1)),    # split-K (2 ways)
    (2, 512, 6, 6, 64, 3, 3, (1, 1), (1, 1)),     # split-K (4 ways)
]


@pytest.mark.parametrize("case", CONVS, ids=[str(i) for i in range(len(CONVS))])
def test_conv2d_f32_implicit_gemm(case):
    n, c, h, w_, oc, kh, kw, stride, pad = case
    x, w, b = rand((n, c, h, w_), 9), rand((oc, c, kh, kw), 10, scale=0.2), rand((oc,), 11)
    attrs = {"stride": list(stride), "padding": list(pad)}
    ref = ops.conv2d(to_np(x), to_np(w), to_np(b), stride, pad)
    out = run_op("conv2d", {"x": x, "weight": w, "bias": b}, attrs=attrs)["output"]
    close_f32(out, ref)
    fused = run_op("conv2d", {"x": x, "weight": w, "bias": b},
                   attrs={**attrs, "activation": "relu"})["output"]
    close_f32(fused, ops.relu(ref))
    from dli import hip

    oh, ow = (h + 2 * pad[0] - kh) // stride[0] + 1, (w_ + 2 * pad[1] - kw) // stride[1] + 1
    if c >= 256:  # the plugin passes a workspace, so these split K
        assert hip.lib().dli_hip_conv2d_workspace(hip.F32, n, c, oc, kh, kw, oh, ow) > 0
    nob = run_op("conv2d", {"x": x, "weight": w}, attrs=attrs)["output"]
    close_f32(nob, ops.conv2d(to_np(x), to_np(w), None, stride, pad))


# patch = C x KH x KW of 9 or 27: the direct kernels conv2d_small_f32_p9 / _p27 instead of MFMA
SMALL_CONVS = [  # (N, C, H, W, OC, KH, KW, stride, pad)
    (64, 3, 32, 32, 64, 3, 3, (1, 1), (1, 1)),    # the AlexNet-style input layer, batch 64
    (2, 3, 9, 10, 20, 3, 3, (1, 2), (0, 1)),      # channels not a multiple of 16, strided
    (3, 1, 17, 15, 5, 3, 3, (2, 2), (2, 2)),      # one channel, padding wider than the kernel
    (1, 3, 3, 3, 33, 3, 3, (1, 1), (1, 1)),       # a 3 x 3 image: every tap but the centre clipped
]


@pytest.mark.parametrize("case", SMALL_CONVS, ids=[str(i) for i in range(len(SMALL_CONVS))])
def test_conv2d_f32_small_patch(case):
    n, c, h, w_, oc, kh, kw, stride, pad = case
    assert c * kh * kw in (9, 27)
    x, w, b = rand((n, c, h, w_), 19), rand((oc, c, kh, kw), 20, scale=0.2), rand((oc,), 21)
    attrs = {"stride": list(stride), "padding": list(pad)}
    ref = ops.conv2d(to_np(x), to_np(w), to_np(b), stride, pad)
    close_f32(run_op("conv2d", {"x": x, "weight": w, "bias": b}, attrs=attrs)["output"], ref)
    fused = run_op("conv2d", {"x": x, "weight": w, "bias": b},
                   attrs={**attrs, "activation": "relu"})["output"]
    close_f32(fused, ops.relu(ref))
    nob = run_op("conv2d", {"x": x, "weight": w}, attrs=attrs)["output"]
    close_f32(nob, ops.conv2d(to_np(x), to_np(w), None, stride, pad))


def test_unknown_activation_is_rejected():
    x, w = rand((4, 8), 12), rand((3, 8), 13)
    with pytest.raises(Exception, match="activation"):
        run_op("linear", {"x": x, "weight": w}, attrs={"activation": "gelu"})


# ---- the reference's TinyAlexNet end-to-end case ------------------------------------------------

def _alexnet_params():
    """examples/alexnet/alexnet.py:31-36: every parameter = (arange(numel) % 17 - 8) / 17."""
    shapes = {"features.0.weight": (8, 3, 3, 3), "features.0.bias": (8,),
              "features.3.weight": (16, 8, 3, 3), "features.3.bias": (16,),
              "classifier.1.weight": (8, 1024), "classifier.1.bias": (8,),
              "classifier.3.weight": (4, 8), "classifier.3.bias": (4,)}
    return {k: ((torch.arange(int(np.prod(s)), dtype=torch.float32) % 17 - 8) / 17).reshape(s)
            for k, s in shapes.items()}


def _alexnet_graph(fused):
    nodes = []

    def node(name, op, inputs, outputs, attrs=None):
        nodes.append({"name": name, "op": op, "inputs": inputs, "outputs": outputs,
                      **({"attrs": attrs} if attrs else {})})

    act = {"activation": "relu"} if fused else {}
    h = "x"
    for i, (conv, tag) in enumerate((("features.0", "c1"), ("features.3", "c2"))):
        node(conv, "conv2d", [h, f"{conv}.weight", f"{conv}.bias"], [tag],
             {"stride": [1, 1], "padding": [1, 1], **act})
        if not fused:
            node(f"{conv}.relu", "relu", [tag], [tag + "r"])
            tag = tag + "r"
        node(f"pool{i}", "max_pool2d", [tag], [f"p{i}"], {"kernel_size": [2, 2], "stride": [2, 2]})
        h = f"p{i}"
    node("flatten", "reshape", [h], ["flat"], {"shape": [1, 1024]})
    node("classifier.1", "linear", ["flat", "classifier.1.weight", "classifier.1.bias"], ["f1"],
         act or None)
    f1 = "f1"
    if not fused:
        node("classifier.relu", "relu", ["f1"], ["f1r"])
        f1 = "f1r"
    node("classifier.3", "linear", [f1, "classifier.3.weight", "classifier.3.bias"], ["logits"])
    params = list(_alexnet_params())
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "alexnet_e2e", "inputs": ["x"] + params,
        "outputs": ["logits"], "nodes": nodes}))


def _alexnet_oracle(x, p):
    h = x
    for conv in ("features.0", "features.3"):
        h = ops.relu(ops.conv2d(h, p[f"{conv}.weight"], p[f"{conv}.bias"], (1, 1), (1, 1)))
        h = ops.max_pool2d(h, (2, 2), (2, 2))
    h = h.reshape(1, 1024)
    h = ops.relu(ops.linear(h, p["classifier.1.weight"], p["classifier.1.bias"]))
    return ops.linear(h, p["classifier.3.weight"], p["classifier.3.bias"])


@pytest.mark.parametrize("fused", [False, True], ids=["relu_nodes", "fused_relu"])
def test_reference_tiny_alexnet_end_to_end(fused):
    x = (torch.arange(3 * 32 * 32, dtype=torch.float32).reshape(1, 3, 32, 32) % 29 - 14) / 29
    params = _alexnet_params()
    expect = _alexnet_oracle(x.numpy(), {k: v.numpy() for k, v in params.items()})
    engine = plugin_engine()
    inputs = {"x": x.cuda(), **{k: v.cuda() for k, v in params.items()}}
    out = engine.run(_alexnet_graph(fused), inputs)["logits"]
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, 4)
    close_f32(out, expect)  # the reference test allows rtol 5e-3, atol 2e-2


@pytest.mark.parametrize("batch", [2, 64])
@pytest.mark.parametrize("fused", [False, True], ids=["relu_nodes", "fused_relu"])
def test_alexnet_cifar_graph(fused, batch):
    """The AlexNet-style fp32 benchmark network (dli_alexnet) against ATen in float64 on the CPU
    (per element at the fp32 tolerance). Batch 64 is the benchmark's batch: the split-K and
    tile choices it makes (conv splits over the patch, FC splits over K) run here."""
    import dli_alexnet as net

    w = net.random_weights(seed=3)
    x = torch.randn((batch,) + net.IMAGE, generator=torch.Generator().manual_seed(4))
    ref = net.torch_forward(x.double(), {k: v.double() for k, v in w.items()}).numpy()
    out = plugin_engine().run(net.build_graph(batch, fused=fused),
                              {"x": x.cuda(), **{k: v.cuda() for k, v in w.items()}})["logits"]
    torch.cuda.synchronize()
    close_f32(out, ref)
