"""The C++ greedy decode driver (dli.GreedyDecoder) on the GPU: HIP-graph replay and eager steps
give the same tokens as the Python DecodeSession over the same plugin, also with the graph and
the bf16 weights read back from dli.graph.v1 / dli.weights.v1 files."""
from __future__ import annotations

import pytest
import torch

import dli
from dli.weights import save_weights
from dli_qwen2 import DecodeSession, random_weights, tiny_config
from dli_qwen2.graph import build_decode_graph, pack_fused_weights

pytestmark = pytest.mark.gpu

BATCH, PROMPT, STEPS, MAX_SEQ = 4, 7, 9, 64


def _case(seed):
    cfg = tiny_config()
    w = random_weights(cfg, seed=seed, device="cuda")
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, cfg.vocab, (BATCH, PROMPT), generator=g)
    return cfg, w, prompt


def _python_tokens(cfg, w, prompt, stack):
    session = DecodeSession(cfg, w, BATCH, max_seq_len=MAX_SEQ, stack=stack).capture()
    return session.generate(prompt.cuda(), STEPS).cpu()


@pytest.mark.parametrize("stack", [False, True], ids=["fused", "stack"])
@pytest.mark.parametrize("capture", [True, False], ids=["replay", "eager"])
def test_cpp_driver_matches_python_session(stack, capture):
    cfg, w, prompt = _case(51)
    expect = _python_tokens(cfg, w, prompt, stack)
    graph = build_decode_graph(cfg, BATCH, fused=True, stack=stack)
    weights = pack_fused_weights(cfg, w, drop_unfused=True)
    engine = dli.Engine().load_plugin()
    d = dli.GreedyDecoder(engine, graph, weights, BATCH, max_seq_len=MAX_SEQ, capture=capture)
    assert not d.captured  # the first step runs eagerly, then is captured
    got = d.generate(prompt, STEPS)
    assert d.captured == capture
    assert got.dtype == torch.int64 and got.shape == (BATCH, STEPS) and not got.is_cuda
    assert torch.equal(got, expect)
    # a second generation from position 0 rewrites the cache and repeats the tokens
    assert torch.equal(d.generate(prompt.cuda(), STEPS), expect)


@pytest.mark.parametrize("stack", [False, True], ids=["fused", "stack"])
def test_cpp_driver_continues_a_cached_prefix(stack):
    """A decoder built on an engine whose cache already holds a prefix (written by another
    decoder) continues it exactly: its first step, which precedes the capture, writes only its
    own position, so generate(start > 0) gives the tokens of one uninterrupted generation."""
    cfg, w, prompt = _case(53)
    expect = _python_tokens(cfg, w, prompt, stack)
    graph = build_decode_graph(cfg, BATCH, fused=True, stack=stack)
    weights = pack_fused_weights(cfg, w, drop_unfused=True)
    engine = dli.Engine().load_plugin()
    first = dli.GreedyDecoder(engine, graph, weights, BATCH, max_seq_len=MAX_SEQ, capture=False)
    first.generate(prompt[:, :4], 1)  # positions 0..3 hold the prompt's first four tokens
    second = dli.GreedyDecoder(engine, graph, weights, BATCH, max_seq_len=MAX_SEQ, capture=True)
    got = second.generate(prompt[:, 4:], STEPS, start=4)
    assert second.captured
    assert torch.equal(got, expect)


def test_cpp_driver_from_files(tmp_path):
    cfg, w, prompt = _case(61)
    expect = _python_tokens(cfg, w, prompt, stack=True)
    graph_path = tmp_path / "qwen2_tiny.dli.graph.json"
    graph_path.write_text(build_decode_graph(cfg, BATCH, fused=True, stack=True).to_json())
    manifest = save_weights(tmp_path, "qwen2_tiny", pack_fused_weights(cfg, w, drop_unfused=True))
    weights = dli.load_weights(str(manifest), device="cuda")
    assert weights["model.embed_tokens.weight"].dtype == torch.bfloat16
    engine = dli.Engine().load_plugin()
    d = dli.GreedyDecoder(engine, dli.Graph.from_json_file(str(graph_path)), weights, BATCH,
                          max_seq_len=MAX_SEQ)
    assert torch.equal(d.generate(prompt, STEPS), expect)


@pytest.mark.slow
def test_cpp_driver_qwen2_0_5b_shape_matches_python_session():
    """Full Qwen2-0.5B shape through the decoder stack: batch 32, 512 random prompt tokens, 64
    greedy tokens; the C++ driver and the Python session replay the same captured step, so
    their tokens are equal."""
    from dli_qwen2 import QWEN2_0_5B

    cfg, b, prompt_len, steps = QWEN2_0_5B, 32, 512, 64
    w = random_weights(cfg, seed=71, device="cuda")
    prompt = torch.randint(0, cfg.vocab, (b, prompt_len), generator=torch.Generator().manual_seed(72))
    session = DecodeSession(cfg, w, b, max_seq_len=prompt_len + steps + 8, stack=True).capture()
    expect = session.generate(prompt.cuda(), steps).cpu()
    del session
    engine = dli.Engine().load_plugin()
    d = dli.GreedyDecoder(engine, build_decode_graph(cfg, b, fused=True, stack=True),
                          pack_fused_weights(cfg, w, drop_unfused=True), b,
                          max_seq_len=prompt_len + steps + 8)
    assert torch.equal(d.generate(prompt, steps), expect)
