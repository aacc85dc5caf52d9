"""Pins the CPU oracle (oracle/ops.py) before it is trusted as the parity checker.

Three kinds of checks, chosen so that a dropped term, a wrong sign or index, or a transposed
operand fails at least one:
  1. the reference's own known-answer literals (tests/golden/kat_ops.json);
  2. independent library routines / textbook formulations on seeded random inputs
     (F.linear, F.conv2d, F.scaled_dot_product_attention, complex rotation for RoPE, ...);
  3. invariants (softmax rows sum to 1, rotation preserves pair norms, ...).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops
from support import kat_outputs, load_kat

KAT = load_kat()


def _np(case, name):
    spec = case["inputs"][name]
    dtype = np.int64 if spec["dtype"] == "int64" else np.float64
    return np.asarray(spec["data"], dtype=dtype).reshape(spec["shape"])


def _oracle_for(case):
    op, a = case["op"], case["attrs"]
    g = lambda n: _np(case, n)  # noqa: E731
    if op == "add":
        return {"output": ops.add(g("x"), g("b"))}
    if op == "mul":
        return {"output": ops.mul(g("x"), g("b"))}
    if op == "attention":
        return {"output": ops.attention(g("q"), g("k"), g("v"), causal=a.get("causal", False))}
    if op == "batch_norm2d":
        return {"output": ops.batch_norm2d(g("x"), g("weight"), g("bias"), g("running_mean"),
                                           g("running_var"), a.get("eps", 1e-5))}
    if op == "conv2d":
        return {"output": ops.conv2d(g("x"), g("weight"), g("bias"), tuple(a["stride"]),
                                     tuple(a["padding"]))}
    if op == "embedding":
        return {"output": ops.embedding(g("ids"), g("table"))}
    if op == "linear":
        return {"output": ops.linear(g("x"), g("weight"), g("bias"))}
    if op == "matmul":
        return {"output": ops.matmul(g("a"), g("b"))}
    if op == "max_pool2d":
        return {"output": ops.max_pool2d(g("x"), tuple(a["kernel_size"]), tuple(a["stride"]),
                                         tuple(a["padding"]))}
    if op == "relu":
        return {"output": ops.relu(g("x"))}
    if op == "silu":
        return {"output": ops.silu(g("x"))}
    if op == "reshape":
        return {"output": g("x").reshape(a["shape"])}
    if op == "rms_norm":
        return {"output": ops.rms_norm(g("x"), g("weight"), a.get("eps", 1e-6))}
    if op == "rotary_embedding":
        sp = a.get("start_pos", 0)
        return {"out_q": ops.rotary(g("q"), g("cos"), g("sin"), sp),
                "out_k": ops.rotary(g("k"), g("cos"), g("sin"), sp)}
    if op == "softmax":
        return {"output": ops.softmax(g("x"))}
    if op == "transpose":
        return {"output": ops.transpose(g("x"))}
    raise AssertionError(op)


@pytest.mark.parametrize("case", KAT, ids=[c["op"] for c in KAT])
def test_oracle_matches_reference_known_answers(case):
    got = _oracle_for(case)
    for name, expected in kat_outputs(case).items():
        np.testing.assert_allclose(got[name], expected, rtol=1e-12, atol=1e-12)


def test_kat_covers_every_reference_operator():
    assert {c["op"] for c in KAT} == {
        "add", "attention", "batch_norm2d", "conv2d", "embedding", "linear", "matmul",
        "max_pool2d", "mul", "relu", "reshape", "rms_norm", "rotary_embedding", "silu",
        "softmax", "transpose"}


def _rng(seed=0):
    return np.random.default_rng(seed)


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def test_linear_and_matmul_against_torch():
    r = _rng(1)
    x, w, b = r.normal(size=(5, 3, 7)), r.normal(size=(4, 7)), r.normal(size=4)
    np.testing.assert_allclose(ops.linear(x, w, b), F.linear(_t(x), _t(w), _t(b)).numpy(), rtol=1e-12)
    a, m = r.normal(size=(6, 9)), r.normal(size=(9, 5))
    np.testing.assert_allclose(ops.matmul(a, m), (_t(a) @ _t(m)).numpy(), rtol=1e-12)
    # linear == matmul with the transposed weight, and the bias lands on the output features
    np.testing.assert_allclose(ops.linear(x, w), ops.matmul(x.reshape(-1, 7), w.T).reshape(5, 3, 4),
                               rtol=1e-12)
    np.testing.assert_allclose(ops.linear(x, w, b) - ops.linear(x, w), np.broadcast_to(b, (5, 3, 4)),
                               rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("stride,padding", [((1, 1), (0, 0)), ((1, 1), (1, 1)), ((2, 1), (1, 2))])
def test_conv2d_against_torch(stride, padding):
    r = _rng(2)
    x, w, b = r.normal(size=(2, 3, 9, 8)), r.normal(size=(4, 3, 3, 2)), r.normal(size=4)
    ref = F.conv2d(_t(x), _t(w), _t(b), stride=stride, padding=padding).numpy()
    np.testing.assert_allclose(ops.conv2d(x, w, b, stride, padding), ref, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("k,s,p", [((2, 2), (2, 2), (0, 0)), ((3, 3), (2, 2), (1, 1)), ((3, 2), (1, 2), (1, 0))])
def test_max_pool2d_against_torch(k, s, p):
    x = _rng(3).normal(size=(2, 3, 7, 6))
    ref = F.max_pool2d(_t(x), kernel_size=k, stride=s, padding=p).numpy()
    np.testing.assert_allclose(ops.max_pool2d(x, k, s, p), ref)


def test_norms_and_activations_against_torch():
    r = _rng(4)
    x, w = r.normal(size=(6, 32)), r.normal(size=32)
    np.testing.assert_allclose(ops.rms_norm(x, w, 1e-6),
                               F.rms_norm(_t(x), (32,), _t(w), eps=1e-6).numpy(), rtol=1e-12)
    np.testing.assert_allclose(ops.silu(x), F.silu(_t(x)).numpy(), rtol=1e-12)
    np.testing.assert_allclose(ops.relu(x), F.relu(_t(x)).numpy())
    np.testing.assert_allclose(ops.softmax(x), torch.softmax(_t(x), -1).numpy(), rtol=1e-12)
    np.testing.assert_allclose(ops.softmax(x).sum(-1), np.ones(6), rtol=1e-12)
    xb = r.normal(size=(2, 3, 4, 5))
    g, bb, mu, var = r.normal(size=3), r.normal(size=3), r.normal(size=3), r.uniform(0.5, 2, 3)
    ref = F.batch_norm(_t(xb), _t(mu), _t(var), _t(g), _t(bb), training=False, eps=1e-5).numpy()
    np.testing.assert_allclose(ops.batch_norm2d(xb, g, bb, mu, var, 1e-5), ref, rtol=1e-12)
    m = r.normal(size=(3, 5))
    np.testing.assert_allclose(ops.transpose(m), m.T)


def test_embedding_and_argmax():
    table = _rng(5).normal(size=(11, 4))
    ids = np.array([[3, 0, 10], [7, 7, 1]])
    np.testing.assert_allclose(ops.embedding(ids, table),
                               F.embedding(torch.from_numpy(ids), _t(table)).numpy())
    x = np.array([[1.0, 3.0, 3.0, -1.0], [0.0, 0.0, 0.0, 0.0], [-5.0, -4.0, -4.5, -4.0]])
    assert ops.argmax(x).tolist() == torch.argmax(_t(x), -1).tolist() == [1, 0, 1]


def test_rotary_matches_complex_rotation_and_preserves_norms():
    r = _rng(6)
    b, h, s, d, max_pos = 2, 3, 5, 8, 40
    x = r.normal(size=(b, h, s, d))
    angles = r.uniform(-np.pi, np.pi, size=(max_pos, d // 2))
    cos, sin = np.cos(angles), np.sin(angles)
    positions = np.array([4, 17])
    got = ops.rotary(x, cos, sin, start_pos=2, positions=positions)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    for bi in range(b):
        pos = 2 + positions[bi] + np.arange(s)
        rot = np.exp(1j * angles[pos])[None]
        ref = z[bi] * rot
        np.testing.assert_allclose(got[bi][..., 0::2], ref.real, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(got[bi][..., 1::2], ref.imag, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np.hypot(got[..., 0::2], got[..., 1::2]),
                               np.hypot(x[..., 0::2], x[..., 1::2]), rtol=1e-12)


def _sdpa_ref(q, k, v, causal, past):
    """torch SDPA (float64) with KV heads repeated and an explicit offset causal mask."""
    group = q.shape[1] // k.shape[1]
    kk = _t(k).repeat_interleave(group, dim=1)
    vv = _t(v).repeat_interleave(group, dim=1)
    sq, sk = q.shape[2], k.shape[2]
    mask = None
    if causal:
        mask = torch.arange(sk)[None, :] <= (past + torch.arange(sq))[:, None]
    return F.scaled_dot_product_attention(_t(q), kk, vv, attn_mask=mask).numpy()


@pytest.mark.parametrize("hq,hkv,sq,sk,causal", [(4, 4, 3, 3, True), (6, 2, 1, 9, True),
                                                  (6, 3, 4, 10, True), (2, 1, 5, 7, False)])
def test_attention_against_sdpa(hq, hkv, sq, sk, causal):
    r = _rng(7)
    q, k, v = r.normal(size=(2, hq, sq, 16)), r.normal(size=(2, hkv, sk, 16)), r.normal(size=(2, hkv, sk, 16))
    got = ops.attention(q, k, v, causal=causal)
    np.testing.assert_allclose(got, _sdpa_ref(q, k, v, causal, sk - sq), rtol=1e-10, atol=1e-12)


def test_attention_special_cases():
    r = _rng(8)
    q, k, v = r.normal(size=(1, 2, 1, 8)), r.normal(size=(1, 2, 1, 8)), r.normal(size=(1, 2, 1, 8))
    np.testing.assert_allclose(ops.attention(q, k, v), v)  # a single key returns its value
    q, k, v = r.normal(size=(1, 1, 4, 8)), r.normal(size=(1, 1, 4, 8)), r.normal(size=(1, 1, 4, 8))
    out = ops.attention(q, k, v, causal=True)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0])  # first causal query sees only key 0


def test_round_bf16_matches_torch_including_ties_and_specials():
    r = _rng(9)
    vals = np.concatenate([
        r.normal(size=4000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 1e-40, -3e-39, 3.4e38], np.float32),
        # exact ties at bf16 precision: mantissa bits ...1000 0000 0000 0000
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    ref = torch.from_numpy(vals).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(ops.round_bf16(vals), ref)
    assert np.isnan(ops.round_bf16(np.array([np.nan], np.float32)))[0]
