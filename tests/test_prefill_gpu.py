"""Config 3 on the GPU: one Qwen2 decoder layer of prefill in bf16 at batch 4 x 2048 tokens
(hidden 896, 14 / 2 heads, head_dim 64, RMSNorm eps 1e-6, RoPE theta 1e6, causal GQA, SwiGLU
4864; activations ~N(0, 1), weights ~N(0, 0.02)), run as the chained dli.graph.v1 prefill graph
(build_prefill_graph: RMSNorm -> q/k/v tiled MFMA linears -> [B,S,H,D] -> [B,H,S,D] -> RoPE ->
KV append + flash attention -> o_proj + residual -> RMSNorm -> gate/up -> SiLU * up -> down +
residual) through the Engine and the gfx950 plugin, against the oracle's layer with the same
bf16 rounding points (oracle/qwen2.py forward_hidden)."""
from __future__ import annotations

from dataclasses import replace

import pytest
import torch

import dli
from dli_qwen2 import QWEN2_0_5B, build_prefill_graph, pack_fused_weights, random_weights
from oracle.qwen2 import Qwen2Oracle

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("batch,seq", [(1, 100), (4, 2048)])
def test_qwen2_decoder_layer_prefill_matches_oracle(batch, seq):
    """Both forms of the layer graph: the reference's node sequence and the fused one
    (linear_residual for o_proj and down_proj, gate_up_silu over the interleaved gate/up
    weight), each against the same oracle layer."""
    cfg = QWEN2_0_5B
    w = random_weights(cfg, seed=81, device="cuda")
    packed = pack_fused_weights(replace(cfg, layers=1),
                                {k: v for k, v in w.items() if not k.startswith("model.layers.")
                                 or k.startswith("model.layers.0.")})
    h = torch.randn(batch, seq, cfg.hidden, generator=torch.Generator().manual_seed(82)).to(
        torch.bfloat16)
    oracle = Qwen2Oracle(cfg, w)
    oracle.reset(batch)
    ref = oracle.forward_hidden(h.float(), [0])
    exact_oracle = Qwen2Oracle(cfg, w, round_bf16=False)
    exact_oracle.reset(batch)
    exact = exact_oracle.forward_hidden(h.float(), [0])
    noise = _rel(ref, exact)
    for fused in (False, True):
        engine = dli.Engine().load_plugin()
        engine.configure_kv_cache(block_size=64, max_seq_len=seq)
        graph = build_prefill_graph(cfg, batch, seq, layers=1, from_hidden=True, fused=fused)
        out = engine.run(graph, {**packed, "hidden_states": h.cuda()})["output"]
        torch.cuda.synchronize()
        got = out.float().cpu()
        err, err32 = _rel(got, ref), _rel(got, exact)
        print(f"\nprefill layer {batch}x{seq} ({'fused' if fused else 'reference nodes'}): "
              f"relative L2 error vs bf16 oracle {err:.3e}, vs fp32 model {err32:.3e}; bf16 "
              f"oracle vs fp32 model {noise:.3e}", flush=True)
        torch.testing.assert_close(got, ref, rtol=2e-2, atol=2e-2)
        assert err32 <= 1.25 * noise + 1e-4
        # the prompt's keys and values went into the cache entry (token-major key pool,
        # identity block table): block 0 of sequence 0 holds positions 0..63 of kv head 0
        e = engine.kv_cache_entry("layer_0")
        k_cached = e["key_pool"][0, 0, :min(64, seq)].float().cpu()
        k_ref = oracle.k_cache[0][0, 0, :min(64, seq)]
        torch.testing.assert_close(k_cached, k_ref, rtol=2e-2, atol=2e-2)
