"""Per-operator parity of the fused operators (plugin ops qkv_rope_append, qkv_rope_heads,
linear_residual, linear_residual_norm, gate_up_silu, lm_head_argmax) against the CPU oracle.

Each fused op stands for a run of nodes of the reference's decoder graph
(python/dli_export/export.py:272-446) with every node's bf16 rounding point; the oracle applies
oracle/ops.py's restatements of those nodes in float64 and rounds at the same points
(round_bf16). Tolerance: bf16 2e-2. Argmax results are exact: the lm_head test builds integer
logits (exact in fp32 in any summation order) with ties inside one tile and across workgroups.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import dli
from dli_qwen2.graph import interleave_gate_up
from oracle import ops
from support import assert_close, run_op, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"
R = ops.round_bf16


def rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def rope_tables(max_pos, d, theta=10000.0):
    inv = 1.0 / theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
    f = torch.outer(torch.arange(max_pos, dtype=torch.float64), inv)
    return f.cos().float().to(DEV), f.sin().float().to(DEV)


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("B,H,hq,hkv,positions", [
    (1, 128, 2, 1, [0]),
    (5, 256, 4, 2, [0, 63, 64, 130, 5]),
    (32, 896, 14, 2, None),   # Qwen2-0.5B shape, positions spread over 4 cache blocks
    (40, 256, 4, 2, None),    # 33..64 rows
])
def test_qkv_rope_append(B, H, hq, hkv, positions, norm):
    _check_qkv_rope_append(B, H, hq, hkv, 64, positions, norm)


@pytest.mark.parametrize("B,H,hq,hkv,d,positions", [
    (64, 3584, 28, 4, 128, None),  # Qwen2-7B geometry at 64 rows: tiled GEMM parts + reduce
    (8, 3584, 28, 4, 128, None),   # ... at 8 rows: skinny parts
    (40, 1152, 9, 3, 128, None),   # 33..64 rows, 1920 q|k|v columns
    (3, 2048, 4, 2, 64, [0, 191, 64]),
])
def test_qkv_rope_append_large_hidden(B, H, hq, hkv, d, positions):
    """Hidden sizes above 1024 (no RMSNorm prologue: the norm is a node of its own): K-split
    parts in the op's workspace, then the reduce that adds the bias, rotates and writes."""
    _check_qkv_rope_append(B, H, hq, hkv, d, positions, False)


def _check_qkv_rope_append(B, H, hq, hkv, d, positions, norm):
    n = (hq + 2 * hkv) * d
    if positions is None:
        positions = [(7 * b + 3) % 250 for b in range(B)]
    x, w, b = rand((B, H), 1), rand((n, H), 2, 0.05), rand((n,), 3, 0.1)
    nw = (1 + rand((H,), 4, 0.1).float()).to(torch.bfloat16)
    cos, sin = rope_tables(256, d)
    pos = torch.tensor(positions, dtype=torch.int64, device=DEV)
    e = dli.Engine().load_plugin()
    e.configure_kv_cache(block_size=64, max_seq_len=256)
    inputs = {"x": x, "nw": nw} if norm else {"x": x}
    inputs.update({"w": w, "b": b, "cos": cos, "sin": sin, "pos": pos})
    out = run_op("qkv_rope_append", inputs,
                 attrs={"kv_cache": "L", "q_heads": hq, "kv_heads": hkv, "head_dim": d, "eps": 1e-6},
                 engine=e)["output"]
    xn = R(ops.rms_norm(to_np(x), to_np(nw), 1e-6)) if norm else to_np(x)
    y = R(ops.linear(xn, to_np(w), to_np(b)))  # [B, n]
    q = y[:, :hq * d].reshape(B, hq, 1, d)
    k = y[:, hq * d:(hq + hkv) * d].reshape(B, hkv, 1, d)
    v = y[:, (hq + hkv) * d:].reshape(B, hkv, 1, d)
    pnp = np.asarray(positions)
    q = R(ops.rotary(q, to_np(cos), to_np(sin), positions=pnp))
    k = R(ops.rotary(k, to_np(cos), to_np(sin), positions=pnp))
    assert_close(out, q, "bfloat16")
    entry = e.kv_cache_entry("L")
    kp, vp, table = to_np(entry["key_pool"]), to_np(entry["value_pool"]), entry["block_table"].cpu().numpy()
    bs = entry["block_size"]
    for i, p in enumerate(positions):
        blk = table[i, p // bs]
        assert_close(kp[blk, :, p % bs, :], k[i, :, 0, :], "bfloat16")
        assert_close(vp[blk, :, :, p % bs], v[i, :, 0, :], "bfloat16")
    # nothing else was written: every other slot of the zero-initialised pools is still zero
    written = np.zeros(kp.shape[0] * bs, bool)
    for i, p in enumerate(positions):
        written[table[i, p // bs] * bs + p % bs] = True
    k_slots = np.abs(kp).sum(axis=(1, 3)).reshape(-1)
    v_slots = np.abs(vp).sum(axis=(1, 2)).reshape(-1)
    assert not k_slots[~written].any() and not v_slots[~written].any()


def _residual_oracle(x, w, res, bias):
    y = ops.linear(to_np(x), to_np(w), None if bias is None else to_np(bias))
    return R(to_np(res) + R(y))


CASES = [  # B, N, K, splits, bias
    (1, 128, 256, 1, False),
    (5, 896, 896, 2, True),
    (32, 896, 896, 4, False),
    (32, 896, 4864, 8, False),
    (33, 896, 4864, 4, False),
    (64, 256, 512, 8, True),
]


@pytest.mark.parametrize("B,N,K,splits,bias", CASES + [
    # n > 1024 (a large hidden size): GEMM parts, then one workgroup per row adds the residual
    # and normalizes; tiled parts from 33 rows, skinny parts below
    (64, 3584, 3584, 4, False),
    (64, 3584, 4864, 4, True),
    (40, 1032, 1000, 4, True),
    (8, 3584, 3584, 2, True),
    (1, 2048, 512, 1, False),
    (16, 4096, 1024, 3, True),
])
def test_linear_residual_norm(B, N, K, splits, bias):
    x, w, res = rand((B, K), 10), rand((N, K), 11, 0.03), rand((B, N), 12)
    nw = (1 + rand((N,), 13, 0.1).float()).to(torch.bfloat16)
    inputs = {"x": x, "w": w, "res": res, "nw": nw}
    if bias:
        inputs["b"] = rand((N,), 14, 0.1)
    out = run_op("linear_residual_norm", inputs, outputs=("h", "xn"),
                 attrs={"splits": splits, "eps": 1e-6})
    h = _residual_oracle(x, w, res, inputs.get("b"))
    assert_close(out["h"], h, "bfloat16")
    assert_close(out["xn"], R(ops.rms_norm(h, to_np(nw), 1e-6)), "bfloat16")


@pytest.mark.parametrize("B,S,H,Hq,Hkv,D,start,max_pos", [
    (1, 1, 64, 2, 1, 64, 0, 16),
    (3, 37, 256, 4, 2, 64, 5, 30),       # ragged; positions 30.. are past the table (unrotated)
    (2, 100, 896, 14, 2, 64, 0, 128),    # Qwen2-0.5B heads, 64-row tiles
    (1, 300, 128, 2, 1, 128, 7, 512),    # head_dim 128
    (2, 2048, 896, 14, 2, 64, 0, 2048),  # 128-row tiles (288 of them)
])
def test_qkv_rope_heads(B, S, H, Hq, Hkv, D, start, max_pos):
    """Prefill q|k|v: linear (bf16 rounding), [B,S,H,D] -> [B,H,S,D], RoPE on q and k."""
    n = (Hq + 2 * Hkv) * D
    x, w, b = rand((B, S, H), 60), rand((n, H), 61, 0.05), rand((n,), 62, 0.1)
    cos, sin = rope_tables(max_pos, D)
    out = run_op("qkv_rope_heads", {"x": x, "w": w, "b": b, "cos": cos, "sin": sin},
                 outputs=("q", "k", "v"),
                 attrs={"q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "start_pos": start})
    # the linear in float64 through torch on the CPU (the oracle's einsum is slow at 4096 rows)
    lin = R((x.cpu().double() @ w.cpu().double().T + b.cpu().double()).numpy())
    heads = lambda a, h: a.reshape(B, S, h, D).transpose(0, 2, 1, 3)
    qr, kr = lin[..., :Hq * D], lin[..., Hq * D:(Hq + Hkv) * D]
    vr = lin[..., (Hq + Hkv) * D:]
    cn, sn = to_np(cos), to_np(sin)
    assert tuple(out["q"].shape) == (B, Hq, S, D) and tuple(out["v"].shape) == (B, Hkv, S, D)
    assert_close(out["q"], R(ops.rotary(heads(qr, Hq), cn, sn, start_pos=start)), "bfloat16")
    assert_close(out["k"], R(ops.rotary(heads(kr, Hkv), cn, sn, start_pos=start)), "bfloat16")
    assert_close(out["v"], heads(vr, Hkv), "bfloat16")


@pytest.mark.parametrize("B,N,K,splits,bias", CASES + [(16, 4096, 1024, 1, True),
                                                      (16, 4096, 1024, 2, True),
                                                      # n > 1024 at 33-64 rows: the tiled GEMM,
                                                      # K split as far as the workspace holds
                                                      (64, 3584, 3584, 4, True),
                                                      (48, 2048, 4096, 2, False),
                                                      (40, 1032, 1000, 4, True),
                                                      (64, 1536, 6144, 1, False)])
def test_linear_residual(B, N, K, splits, bias):
    """splits > 1: the last split to finish a tile sums the partials; the second call checks that
    the first left every arrival counter at zero."""
    x, w, res = rand((B, K), 20), rand((N, K), 21, 0.03), rand((B, N), 22)
    inputs = {"x": x, "w": w, "res": res}
    if bias:
        inputs["b"] = rand((N,), 23, 0.1)
    e = dli.Engine().load_plugin()
    expect = _residual_oracle(x, w, res, inputs.get("b"))
    for _ in range(2):
        out = run_op("linear_residual", inputs, attrs={"splits": splits}, engine=e)["output"]
        assert_close(out, expect, "bfloat16")


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("B,H,F", [(1, 128, 64), (7, 896, 4864), (32, 896, 4864), (64, 256, 512)])
def test_gate_up_silu(B, H, F, norm):
    x, wg, wu = rand((B, H), 30), rand((F, H), 31, 0.05), rand((F, H), 32, 0.05)
    nw = (1 + rand((H,), 33, 0.1).float()).to(torch.bfloat16)
    inputs = {"x": x, "nw": nw} if norm else {"x": x}
    inputs["w"] = interleave_gate_up(wg, wu)
    out = run_op("gate_up_silu", inputs, attrs={"eps": 1e-6})["output"]
    xn = R(ops.rms_norm(to_np(x), to_np(nw), 1e-6)) if norm else to_np(x)
    g = R(ops.linear(xn, to_np(wg)))
    u = R(ops.linear(xn, to_np(wu)))
    assert_close(out, R(R(ops.silu(g)) * u), "bfloat16")


@pytest.mark.parametrize("B,H,F", [(48, 1536, 1024), (64, 2048, 2064), (9, 1032, 96),
                                   (1, 1152, 512)])
def test_gate_up_silu_large_hidden(B, H, F):
    """hidden > 1024 at decode-sized rows (no RMSNorm prologue; the skinny kernels stop at 1024):
    the tiled GEMM with the SwiGLU epilogue; F = 2064 leaves a half 64-column tile."""
    x, wg, wu = rand((B, H), 34), rand((F, H), 35, 0.05), rand((F, H), 36, 0.05)
    out = run_op("gate_up_silu", {"x": x, "w": interleave_gate_up(wg, wu)})["output"]
    g = R(ops.linear(to_np(x), to_np(wg)))
    u = R(ops.linear(to_np(x), to_np(wu)))
    assert_close(out, R(R(ops.silu(g)) * u), "bfloat16")


@pytest.mark.parametrize("B,H,V", [(1, 128, 1000), (5, 896, 4099), (32, 896, 151936 // 8),
                                   (48, 256, 777), (2, 512, 100), (3, 1024, 900),
                                   (48, 256, 120000), (20, 128, 230000)])
@pytest.mark.parametrize("logits_dtype", ["float32", "bfloat16"])
def test_lm_head_argmax(B, H, V, logits_dtype):
    """The last two vocabularies give every workgroup more tiles than it stages in LDS (12) on
    a 256-CU device, at 64 and at 32 rows per tile, so logits are also written inside the tile
    loop; row 8193 (tile 256) is a third tie for row 0, often in the workgroup of row 3."""
    g = torch.Generator().manual_seed(40 + B)
    # small integers: every partial sum is exact in fp32, so logits are exact and ties are real
    x = torch.randint(-2, 3, (B, H), generator=g).to(torch.bfloat16)
    w = torch.randint(-1, 2, (V, H), generator=g).to(torch.bfloat16)
    best = torch.sign(x.float()).to(torch.bfloat16)  # maximises row's logit: sum |x|
    if V > 700:
        w[3], w[700] = best[0], best[0]        # tie across workgroups (256 rows each)
    if V > 8193:
        w[8193] = best[0]
    if B > 1:
        w[9], w[5] = best[1], best[1]          # tie inside one 32-row tile, lower index second
    x, w = x.to(DEV), w.to(DEV)
    out = run_op("lm_head_argmax", {"x": x, "w": w}, outputs=("logits", "ids"),
                 attrs={"logits_dtype": logits_dtype})
    exact = to_np(x) @ to_np(w).T
    ids = out["ids"].cpu().numpy()
    np.testing.assert_array_equal(ids, np.argmax(exact, axis=-1))
    if V > 700:
        assert ids[0] == 3
    if B > 1:
        assert ids[1] == 5
    expect = exact if logits_dtype == "float32" else R(exact)
    np.testing.assert_array_equal(to_np(out["logits"]), expect)


def test_lm_head_argmax_random_logits_match_oracle():
    B, H, V = 32, 896, 20000
    x, w = rand((B, H), 50), rand((V, H), 51, 0.05)
    out = run_op("lm_head_argmax", {"x": x, "w": w}, outputs=("logits", "ids"))
    ref = ops.linear(to_np(x), to_np(w))
    assert_close(out["logits"], ref, "float32", rtol=1e-4, atol=1e-4)
    ids = out["ids"].cpu().numpy()
    np.testing.assert_array_equal(ids, np.argmax(to_np(out["logits"]), axis=-1))
    top2 = np.sort(ref, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-3  # rows whose winner the fp32 sums cannot flip
    np.testing.assert_array_equal(ids[clear], np.argmax(ref, axis=-1)[clear])


@pytest.mark.parametrize("B", [1, 5, 32, 48])
def test_lm_head_argmax_with_final_norm(B):
    """Third input = model.norm's weight: the final RMSNorm (bf16 output) runs in the kernel's
    registers. Against the oracle (RMSNorm rounded to bf16, then fp32 logits) and against the
    separate rms_norm node followed by the two-input form."""
    H, V = 896, 20000
    x, nw, w = rand((B, H), 52, 4.0), rand((H,), 53), rand((V, H), 54, 0.05)
    out = run_op("lm_head_argmax", {"x": x, "w": w, "nw": nw}, outputs=("logits", "ids"),
                 attrs={"eps": 1e-6})
    xn = R(ops.rms_norm(to_np(x), to_np(nw), 1e-6))
    ref = ops.linear(xn, to_np(w))
    # an element of xn may round to the neighbouring bf16 value (fp32 vs float64 row sums)
    assert_close(out["logits"], ref, "bfloat16")
    ids = out["ids"].cpu().numpy()
    np.testing.assert_array_equal(ids, np.argmax(to_np(out["logits"]), axis=-1))
    h = run_op("rms_norm", {"x": x, "weight": nw}, attrs={"eps": 1e-6})["output"]
    two = run_op("lm_head_argmax", {"x": h, "w": w}, outputs=("logits", "ids"))
    assert_close(out["logits"], to_np(two["logits"]), "bfloat16")
    top2 = np.sort(ref, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 0.05  # winners no rounding of xn can flip
    np.testing.assert_array_equal(ids[clear], np.argmax(ref, axis=-1)[clear])
    np.testing.assert_array_equal(ids[clear], two["ids"].cpu().numpy()[clear])


@pytest.mark.parametrize("B,positions,max_seq,geometry", [
    (8, [0, 1, 63, 64, 65, 1000, 2047, 4095], 4160, (14, 2, 64)),  # ragged, partial last blocks
    (32, None, 4160, (14, 2, 64)),       # the decode workload: every row at 4095
    (3, [5, 130, 517], 600, (14, 2, 64)),  # short cache: one split per sequence
    (2, [-1, 10], 256, (14, 2, 64)),     # an empty sequence yields zeros
    # head_dim 128 (the Qwen2-7B geometry, 28 / 4 heads): ragged lengths over several splits,
    # an empty sequence, and long contexts with one split per (sequence, kv head)
    (8, [-1, 0, 31, 32, 63, 64, 1000, 8191], 8256, (28, 4, 128)),
    (64, [8191] * 64, 8256, (28, 4, 128)),
    (3, [5, 130, 517], 600, (28, 4, 128)),
    # every kv head of a sequence in one workgroup: 4 waves per head (2 kv heads), 1 wave per head
    # (8 kv heads); 3 kv heads do not divide the 8 waves (one kv head per workgroup)
    (4, [100, 4000, 8191, 0], 8256, (16, 2, 128)),
    (2, [3000, 77], 4160, (8, 8, 128)),
    (3, [50, 2000, 4100], 4160, (12, 3, 128)),
])
def test_paged_attention_decode(B, positions, max_seq, geometry):
    """paged_attention (decode, 64-key blocks): every (sequence, kv head) is split over
    workgroups whose partials the last one merges; compared with the oracle's attention over the
    cache contents of each sequence (attention/kernel.py:6-62 with past = position)."""
    hq, hkv, d = geometry
    if positions is None:
        positions = [4095] * B
    e = dli.Engine().load_plugin()
    e.configure_kv_cache(block_size=64, max_seq_len=max_seq)
    e.reserve_kv_cache("L", "bfloat16", B, hkv, d)
    entry = e.kv_cache_entry("L")
    g = torch.Generator(device=DEV).manual_seed(60)
    for pool in (entry["key_pool"], entry["value_pool"]):
        pool.copy_(torch.randn(pool.shape, generator=g, device=DEV).to(pool.dtype))
    q = rand((B, hq, 1, d), 61)
    pos = torch.tensor(positions, dtype=torch.int64, device=DEV)
    for _ in range(2):  # the second call reuses the workspace counters the first left at zero
        out = run_op("paged_attention", {"q": q, "pos": pos}, attrs={"kv_cache": "L"},
                     engine=e)["output"]
    kp, vp = to_np(entry["key_pool"]), to_np(entry["value_pool"])
    table, bs = entry["block_table"].cpu().numpy(), entry["block_size"]
    for i, p in enumerate(positions):
        n = p + 1
        if n <= 0:
            assert not to_np(out[i]).any()
            continue
        blocks = [table[i, j] for j in range((n + bs - 1) // bs)]
        k = np.concatenate([kp[blk] for blk in blocks], axis=1)[:, :n]                      # [Hkv, n, D]
        v = np.concatenate([vp[blk].transpose(0, 2, 1) for blk in blocks], axis=1)[:, :n]  # [Hkv, n, D]
        ref = ops.attention(to_np(q[i:i + 1]), k[None], v[None], causal=True)
        assert_close(out[i:i + 1], ref, "bfloat16")


def test_workspace_first_use_inside_a_capture_is_refused():
    """A node whose scratch buffer would be allocated and zero-filled inside a stream capture is
    refused with a clear error (the allocation and its device synchronization cannot be
    captured); after one eager run the same node captures and replays, equal to eager."""
    from support import one_node_graph

    x, w, res = rand((8, 896), 24), rand((896, 896), 25, 0.03), rand((8, 896), 26)
    inputs = {"x": x, "w": w, "res": res}
    graph = one_node_graph("linear_residual", inputs, attrs={"splits": 3})
    e = dli.Engine().load_plugin()  # its linear_residual node has no buffer yet
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="inside a stream capture"):
        with torch.cuda.graph(g):
            e.run(graph, inputs)
    del g
    torch.cuda.synchronize()
    eager = e.run(graph, inputs)["output"].clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = e.run(graph, inputs)["output"]
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert_close(eager, _residual_oracle(x, w, res, None), "bfloat16")
