"""Per-operator parity on the GPU: one-node dli.graph.v1 graphs through Engine + the gfx950
plugin (the reference's tests/operators/* pattern, in process), checked against the CPU oracle
(oracle/ops.py) and the reference's known-answer literals.

Tolerances (the parity contract): fp32 1e-4 relative, bf16 2e-2, fp16 2e-3. The oracle is
fed the same rounded inputs the device sees and its float64 result is compared directly.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops
from support import (TORCH_DTYPES, assert_close, kat_inputs, kat_outputs, load_kat,
                     plugin_engine, run_op, to_np)

pytestmark = pytest.mark.gpu

DEV = "cuda"
FLOATS = ["float32", "bfloat16", "float16"]
KAT = load_kat()


def rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(TORCH_DTYPES[dtype]).to(DEV)


@pytest.mark.parametrize("case", KAT, ids=[c["op"] for c in KAT])
def test_reference_known_answers(case):
    inputs = kat_inputs(case, DEV)
    outs = run_op(case["op"], inputs, outputs=list(case["outputs"]), attrs=case["attrs"])
    for name, expected in kat_outputs(case).items():
        assert_close(outs[name], expected, "float32")


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape,bshape", [((7, 33), (33,)), ((4, 5, 6), (5, 6)), ((1000,), (1,)),
                                          ((0, 3), (3,))])
def test_add_mul(dtype, shape, bshape):
    a, b = rand(shape, dtype, 1), rand(bshape, dtype, 2)
    for op, fn in (("add", ops.add), ("mul", ops.mul)):
        out = run_op(op, {"x": a, "b": b})["output"]
        assert out.dtype == a.dtype and list(out.shape) == list(shape)
        assert_close(out, fn(to_np(a), to_np(b)), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
def test_activations(dtype):
    x = rand((3, 517), dtype, 3, 4.0)
    assert_close(run_op("silu", {"x": x})["output"], ops.silu(to_np(x)), dtype)
    assert_close(run_op("relu", {"x": x})["output"], ops.relu(to_np(x)), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("rows,hidden", [(1, 896), (37, 896), (1029, 2048), (8192, 896), (5, 4096),
                                         (3, 3000), (2, 4), (6, 8)])
def test_rms_norm(dtype, rows, hidden):
    x, w = rand((rows, hidden), dtype, 4), rand((hidden,), dtype, 5)
    out = run_op("rms_norm", {"x": x, "weight": w}, attrs={"eps": 1e-6})["output"]
    assert_close(out, ops.rms_norm(to_np(x), to_np(w), 1e-6), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_embedding(dtype, ids_dtype):
    table = rand((50, 96), dtype, 6)
    ids = torch.tensor([[3, 0, 49], [7, 7, 1]], dtype=ids_dtype, device=DEV)
    out = run_op("embedding", {"ids": ids, "table": table})["output"]
    assert torch.equal(out.cpu(), table.cpu()[ids.cpu().long()])


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("m,n,k", [(1, 896, 896), (7, 130, 64), (16, 1152, 896), (32, 4864, 896),
                                   (33, 96, 4864), (64, 200, 128), (100, 70, 40), (3, 5, 7),
                                   # decode-sized bf16 on the tiled GEMM: K split into parts
                                   # (tail parts, k % 64 != 0), wide outputs from 16 rows
                                   (64, 3584, 3584), (48, 9000, 520), (16, 8200, 896),
                                   (40, 1032, 1000)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear(dtype, m, n, k, bias):
    scale = 1.0 / np.sqrt(k)
    x, w = rand((m, k), dtype, 7), rand((n, k), dtype, 8, scale)
    inputs = {"x": x, "weight": w}
    if bias:
        inputs["bias"] = rand((n,), dtype, 9)
    out = run_op("linear", inputs)["output"]
    ref = ops.linear(to_np(x), to_np(w), to_np(inputs["bias"]) if bias else None)
    assert_close(out, ref, dtype)


def test_linear_fp32_logits_from_bf16():
    x, w = rand((4, 896), "bfloat16", 10), rand((1000, 896), "bfloat16", 11, 0.03)
    out = run_op("linear", {"x": x, "weight": w}, attrs={"out_dtype": "float32"})["output"]
    assert out.dtype == torch.float32
    assert_close(out, ops.linear(to_np(x), to_np(w)), "float32", rtol=1e-5, atol=1e-5)


def test_linear_single_layer_config():
    """Single linear layer, fp32: x [64,1024] ~N(0,1); W [4096,1024], b [4096] ~U(-1/32, 1/32)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 1024, generator=g)
    w = (torch.rand(4096, 1024, generator=g) * 2 - 1) / 32
    b = (torch.rand(4096, generator=g) * 2 - 1) / 32
    out = run_op("linear", {"x": x.to(DEV), "weight": w.to(DEV), "bias": b.to(DEV)})["output"]
    assert_close(out, ops.linear(x.numpy(), w.numpy(), b.numpy()), "float32")


@pytest.mark.parametrize("dtype", FLOATS)
def test_matmul(dtype):
    a, b = rand((70, 45), dtype, 12), rand((45, 130), dtype, 13)
    assert_close(run_op("matmul", {"a": a, "b": b})["output"], ops.matmul(to_np(a), to_np(b)), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
def test_softmax_transpose(dtype):
    x = rand((9, 1500), dtype, 14, 3.0)
    assert_close(run_op("softmax", {"x": x})["output"], ops.softmax(to_np(x)), dtype)
    y = rand((67, 45), dtype, 15)
    out = run_op("transpose", {"x": y}, attrs={"perm": [1, 0]})["output"]
    assert torch.equal(out.cpu(), y.cpu().t())


@pytest.mark.parametrize("dtype", FLOATS)
def test_conv_pool_bn(dtype):
    x, w, b = rand((2, 3, 11, 10), dtype, 16), rand((5, 3, 3, 3), dtype, 17, 0.3), rand((5,), dtype, 18)
    out = run_op("conv2d", {"x": x, "weight": w, "bias": b}, attrs={"stride": [2, 1], "padding": [1, 1]})
    assert_close(out["output"], ops.conv2d(to_np(x), to_np(w), to_np(b), (2, 1), (1, 1)), dtype)
    p = run_op("max_pool2d", {"x": x}, attrs={"kernel_size": [3, 3], "stride": [2, 2], "padding": [1, 1]})
    assert_close(p["output"], ops.max_pool2d(to_np(x), (3, 3), (2, 2), (1, 1)), dtype)
    g, bb, mu = rand((3,), dtype, 19), rand((3,), dtype, 20), rand((3,), dtype, 21)
    var = (rand((3,), dtype, 22).abs() + 0.5).to(TORCH_DTYPES[dtype])
    bn = run_op("batch_norm2d", {"x": x, "weight": g, "bias": bb, "running_mean": mu, "running_var": var})
    assert_close(bn["output"], ops.batch_norm2d(*(to_np(t) for t in (x, g, bb, mu, var))), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
def test_rotary_positions_and_gqa(dtype):
    q, k = rand((3, 14, 2, 64), dtype, 23), rand((3, 2, 2, 64), dtype, 24)
    ang = torch.rand(64, 32, generator=torch.Generator().manual_seed(25)) * 6.28
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    positions = torch.tensor([0, 5, 60], dtype=torch.int32, device=DEV)
    out = run_op("rotary_embedding", {"q": q, "k": k, "cos": cos, "sin": sin, "positions": positions},
                 outputs=["oq", "ok"], attrs={"start_pos": 1})
    pos = positions.cpu().numpy()
    assert_close(out["oq"], ops.rotary(to_np(q), cos.cpu().numpy(), sin.cpu().numpy(), 1, pos), dtype)
    assert_close(out["ok"], ops.rotary(to_np(k), cos.cpu().numpy(), sin.cpu().numpy(), 1, pos), dtype)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("hq,hkv,sq,sk,d,causal", [(14, 2, 1, 300, 64, True), (4, 4, 17, 17, 128, True),
                                                   (6, 3, 5, 40, 64, False), (2, 1, 3, 3, 2, True)])
def test_attention_dense(dtype, hq, hkv, sq, sk, d, causal):
    q, k, v = rand((2, hq, sq, d), dtype, 26), rand((2, hkv, sk, d), dtype, 27), rand((2, hkv, sk, d), dtype, 28)
    out = run_op("attention", {"q": q, "k": k, "v": v}, attrs={"causal": causal})["output"]
    assert_close(out, ops.attention(to_np(q), to_np(k), to_np(v), causal=causal), dtype)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_attention_kv_cache_prefill_then_decode(dtype):
    """attention with kv_cache: appends grow the cache (across a block boundary and past the
    initial capacity) and each call attends over everything cached so far."""
    import dli

    e = dli.Engine().load_plugin()
    e.configure_kv_cache(block_size=16, max_seq_len=40)
    B, hq, hkv, d = 2, 6, 2, 64
    ks, vs = [], []
    steps = [(20, True), (1, True), (1, True), (30, True)]  # grows past the 48-token capacity
    for i, (s, causal) in enumerate(steps):
        q, k, v = rand((B, hq, s, d), dtype, 100 + i), rand((B, hkv, s, d), dtype, 200 + i), rand((B, hkv, s, d), dtype, 300 + i)
        ks.append(to_np(k))
        vs.append(to_np(v))
        out = run_op("attention", {"q": q, "k": k, "v": v}, attrs={"causal": causal, "kv_cache": "layer_0"}, engine=e)["output"]
        ref = ops.attention(to_np(q), np.concatenate(ks, 2), np.concatenate(vs, 2), causal=causal)
        assert_close(out, ref, dtype)
    assert e.kv_cache_entry("layer_0")["length"] == sum(s for s, _ in steps)


def test_attention_kv_cache_device_positions():
    """Per-sequence lengths (4th input): sequences at different positions in one batch."""
    import dli

    e = dli.Engine().load_plugin()
    e.configure_kv_cache(block_size=32, max_seq_len=128)
    B, hq, hkv, d = 3, 14, 2, 64
    lens = [5, 40, 77]
    hist_k = [rand((1, hkv, L, d), "bfloat16", 400 + b) for b, L in enumerate(lens)]
    hist_v = [rand((1, hkv, L, d), "bfloat16", 500 + b) for b, L in enumerate(lens)]
    # write every prefix with one batched call at positions 0 (tails past lens[b] are padding
    # that the decode step below never attends to)
    maxL = max(lens)
    k_all = torch.zeros(B, hkv, maxL, d, dtype=torch.bfloat16, device=DEV)
    v_all = torch.zeros_like(k_all)
    for b in range(B):
        k_all[b, :, :lens[b]] = hist_k[b][0]
        v_all[b, :, :lens[b]] = hist_v[b][0]
    zero = torch.zeros(B, dtype=torch.int64, device=DEV)
    q0 = rand((B, hq, maxL, d), "bfloat16", 600)
    run_op("attention", {"q": q0, "k": k_all, "v": v_all, "positions": zero},
           attrs={"causal": True, "kv_cache": "L"}, engine=e)
    # decode one token per sequence at its own position
    pos = torch.tensor(lens, dtype=torch.int64, device=DEV)
    q, k, v = rand((B, hq, 1, d), "bfloat16", 601), rand((B, hkv, 1, d), "bfloat16", 602), rand((B, hkv, 1, d), "bfloat16", 603)
    out = run_op("attention", {"q": q, "k": k, "v": v, "positions": pos},
                 attrs={"causal": True, "kv_cache": "L"}, engine=e)["output"]
    for b in range(B):
        kk = np.concatenate([to_np(hist_k[b]), to_np(k[b:b + 1])], 2)
        vv = np.concatenate([to_np(hist_v[b]), to_np(v[b:b + 1])], 2)
        assert_close(out[b:b + 1], ops.attention(to_np(q[b:b + 1]), kk, vv, causal=True), "bfloat16")


@pytest.mark.parametrize("dtype,rows,width", [("float32", 3, 1000), ("bfloat16", 5, 4100),
                                               ("float32", 64, 152064), ("float32", 7, 4096),
                                               ("float32", 2, 4098)])
def test_argmax_first_index_of_maximum(dtype, rows, width):
    """torch.argmax's rule (first index of the maximum) on integer-valued rows with the maximum
    planted several times per row: inside one 16-byte vector, across threads and at both ends.
    Wide fp32 rows take the 16-byte-load kernel, the others the generic one."""
    g = torch.Generator().manual_seed(rows * 7 + width)
    x = torch.randint(-1000, 1000, (rows, width), generator=g).float()
    for r in range(rows):
        a = (r * 977) % (width - 1)
        for p in (a, a + 1, (r * 4099 + 5) % width, width - 1 - r % 3):  # a, a + 1: one vector
            x[r, p] = 5000.0
    x[0, 0] = x[0, width - 1] = 6000.0
    x = x.to(TORCH_DTYPES[dtype])
    out = run_op("argmax", {"x": x.to(DEV)})["output"]
    assert torch.equal(out.cpu(), torch.argmax(x.float(), dim=-1))


def test_reshape_is_a_view():
    x = rand((4, 6), "float32", 30)
    out = run_op("reshape", {"x": x}, attrs={"shape": [3, -1]})["output"]
    assert out.shape == (3, 8) and out.data_ptr() == x.data_ptr()


def test_plugin_uses_native_library():
    import dli

    assert plugin_engine().has_operator("linear")
    maps = open("/proc/self/maps").read()
    assert "libdli_hip_ops.so" in maps and "libdli_hip.so" in maps
    from dli import hip

    assert hip.lib().dli_hip_available() == 1, hip.lib().dli_hip_load_error()


def test_public_launch_and_allocator_abi_runs_a_kernel():
    """The CudaAotKernel / cuda_runtime replacement from the C ABI alone (the reference's
    tests/cpp/test_cuda_aot_kernel.cc and cuda_driver.cc:107-129): the embedded elementwise code
    object through dli_hip_module_load, its add_f32 kernel through dli_hip_module_get_function,
    buffers through dli_hip_malloc and dli_hip_memcpy, one dli_hip_launch, results against the
    oracle's add (add/kernel.py:6-11: out[i] = a[i] + b[i % width]), then unload and free."""
    import ctypes

    from dli import hip

    lib = hip.load()
    image, size = ctypes.c_void_p(), ctypes.c_size_t()
    assert lib.dli_hip_code_object(b"elementwise", ctypes.byref(image), ctypes.byref(size)) == 0
    module, fn = ctypes.c_void_p(), ctypes.c_void_p()
    hip.call("dli_hip_module_load", image, size.value, ctypes.byref(module))
    hip.call("dli_hip_module_get_function", module, b"add_f32", ctypes.byref(fn))
    total, width = 3000, 7
    rng = np.random.default_rng(5)
    a = rng.standard_normal(total).astype(np.float32)
    b = rng.standard_normal(width).astype(np.float32)
    dev = [ctypes.c_void_p() for _ in range(3)]
    for buf, n in zip(dev, (total, width, total)):
        hip.call("dli_hip_malloc", n * 4, ctypes.byref(buf))
    try:
        hip.call("dli_hip_memcpy", dev[0], a.ctypes.data, total * 4, 1)  # host to device
        hip.call("dli_hip_memcpy", dev[1], b.ctypes.data, width * 4, 1)
        n_total, n_width = ctypes.c_int64(total), ctypes.c_int64(width)
        args = (ctypes.c_void_p * 5)(*[ctypes.addressof(x) for x in
                                       (dev[0], dev[1], dev[2], n_total, n_width)])
        # the kernel is grid-strided with 256 threads per workgroup
        hip.call("dli_hip_launch", fn, 4, 1, 1, 256, 1, 1, 0, None, args)
        hip.call("dli_hip_device_synchronize")
        out = np.empty(total, dtype=np.float32)
        hip.call("dli_hip_memcpy", out.ctypes.data, dev[2], total * 4, 2)  # device to host
    finally:
        for buf in dev:
            hip.call("dli_hip_free", buf)
        hip.call("dli_hip_module_unload", module)
    np.testing.assert_array_equal(out, ops.add(a, b).astype(np.float32))
