"""The persistent decoder stack (plugin op decoder_stack -> C ABI dli_hip_decoder_stack: every
decoder layer in one launch) against the five-launch fused graph.

Per tile, the stack runs the same code in the same order as the one-stage kernels, so the two
graphs must agree bit for bit: logits, greedy ids and every layer's KV cache, step after step.
Repeated steps also check that each launch leaves its arrival counters at zero, and
check_status makes every launch report whether a workgroup gave up waiting (it must not).
The fused graph itself is checked against the CPU oracle in test_decode_gpu.py."""
from __future__ import annotations

import pytest
import torch

from dli_qwen2 import QWEN2_0_5B, DecodeSession, random_weights, tiny_config

pytestmark = pytest.mark.gpu


def _prompt(cfg, batch, length, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.vocab, (batch, length), generator=g)


def _run_steps(session, prompt, steps, start=0):
    b, s = prompt.shape
    pos = torch.full((b,), start, dtype=torch.int64, device="cuda")
    out = []
    nxt = None
    for t in range(s + steps):
        ids = prompt[:, t].cuda() if t < s else nxt
        logits, nxt = session.step(ids, pos)
        nxt = nxt.clone()
        out.append((logits.float().cpu().clone(), nxt.cpu()))
        pos += 1
    return out


def _assert_same(fused, stack, a, b, layers):
    for step, ((la, ia), (lb, ib)) in enumerate(zip(a, b)):
        assert torch.equal(la, lb), f"logits differ at step {step}"
        assert torch.equal(ia, ib), f"ids differ at step {step}"
    for i in range(layers):
        ea = fused.engine.kv_cache_entry(f"layer_{i}")
        eb = stack.engine.kv_cache_entry(f"layer_{i}")
        assert torch.equal(ea["key_pool"], eb["key_pool"]), f"key cache of layer {i} differs"
        assert torch.equal(ea["value_pool"], eb["value_pool"]), f"value cache of layer {i} differs"


def _pair(cfg, w, batch, max_seq_len, down=1, attn=3, **kw):
    """A fused and a stack session with the same down_proj split-K (1: one workgroup reduces a
    tile over the full K; more: the last split to finish merges the partials) and the same
    attention split count per (sequence, kv head) pair (by default the stack spreads attention
    over the CUs its q|k|v stage leaves free, the stand-alone kernel over all CUs)."""
    splits = {"o": 1, "down": down, "attn": attn}
    fused = DecodeSession(cfg, w, batch, max_seq_len=max_seq_len, fused=True, splits=splits)
    stack = DecodeSession(cfg, w, batch, max_seq_len=max_seq_len, fused=True, stack=True,
                          splits=splits, check_status=True, **kw)
    return fused, stack


@pytest.mark.parametrize("down", [1, 3])
@pytest.mark.parametrize("batch", [1, 5, 16, 32, 40])
def test_stack_matches_fused_graph_bitwise(batch, down):
    cfg = tiny_config(layers=3)
    w = random_weights(cfg, seed=31, device="cuda")
    prompt = _prompt(cfg, batch, 6, 32)
    fused, stack = _pair(cfg, w, batch, 256, down)
    print(f"stack vs fused: batch {batch}", flush=True)
    _assert_same(fused, stack, _run_steps(fused, prompt, 4), _run_steps(stack, prompt, 4),
                 cfg.layers)


def test_stack_ragged_positions_cross_cache_blocks():
    """Sequences at different positions, some crossing 64-token cache blocks during the run."""
    cfg = tiny_config(layers=2)
    w = random_weights(cfg, seed=41, device="cuda")
    batch = 6
    fused, stack = _pair(cfg, w, batch, 512)
    start = torch.tensor([0, 61, 62, 127, 200, 300], device="cuda")
    g = torch.Generator().manual_seed(42)
    outs = []
    for sess in (fused, stack):
        pos = start.clone()
        res = []
        for t in range(5):
            ids = torch.randint(0, cfg.vocab, (batch,), generator=g).cuda() if t == 0 else nxt
            logits, nxt = sess.step(ids, pos)
            nxt = nxt.clone()
            res.append((logits.float().cpu().clone(), nxt.cpu()))
            pos += 1
        outs.append(res)
        g.manual_seed(42)
    _assert_same(fused, stack, outs[0], outs[1], cfg.layers)


def test_stack_graph_replay_equals_fused_eager():
    cfg = tiny_config(layers=2)
    w = random_weights(cfg, seed=51, device="cuda")
    prompt = _prompt(cfg, 8, 4, 52)
    splits = {"o": 1, "down": 1, "attn": 3}
    fused = DecodeSession(cfg, w, 8, max_seq_len=64, splits=splits)
    stack = DecodeSession(cfg, w, 8, max_seq_len=64, stack=True, splits=splits).capture()
    _assert_same(fused, stack, _run_steps(fused, prompt, 5), _run_steps(stack, prompt, 5),
                 cfg.layers)


@pytest.mark.parametrize("stack", [True, False])
def test_multi_step_graph_equals_single_steps(stack):
    """capture(chain_ids=True, steps=3): one graph launch runs three greedy steps, each reading
    the previous step's next_ids and its own row of step_positions. The last step's logits and
    ids, the chained input ids and every layer's KV cache (which holds the keys and values of
    all three new tokens) equal three one-step replays, bit for bit."""
    cfg = tiny_config(layers=2)
    w = random_weights(cfg, seed=53, device="cuda")
    prompt = _prompt(cfg, 4, 4, 54)
    single = DecodeSession(cfg, w, 4, max_seq_len=64, stack=stack).capture()
    multi = DecodeSession(cfg, w, 4, max_seq_len=64, stack=stack)
    ids = _run_steps(single, prompt, 0)[-1][1].cuda()
    assert torch.equal(_run_steps(multi, prompt, 0)[-1][1].cuda(), ids)
    pos = torch.full((4,), prompt.shape[1], dtype=torch.int64, device="cuda")
    expect = []
    for t in range(3):
        logits, nxt = single.step(ids if t == 0 else expect[-1][1].cuda(), pos + t)
        expect.append((logits.float().cpu().clone(), nxt.cpu().clone()))
    multi.capture(chain_ids=True, steps=3)
    with pytest.raises(ValueError):
        multi.step(ids, pos)
    multi.ids.copy_(ids)
    for t in range(3):
        multi.step_positions[t].copy_(pos + t)
    out = multi.replay()
    torch.cuda.synchronize()
    assert torch.equal(out["logits"].float().cpu(), expect[-1][0]), "last step's logits differ"
    assert torch.equal(out["next_ids"].cpu(), expect[-1][1]), "last step's ids differ"
    assert torch.equal(multi.ids.cpu(), expect[-1][1]), "chained input ids differ"
    for i in range(cfg.layers):
        ea = single.engine.kv_cache_entry(f"layer_{i}")
        eb = multi.engine.kv_cache_entry(f"layer_{i}")
        assert torch.equal(ea["key_pool"], eb["key_pool"]), f"key cache of layer {i} differs"
        assert torch.equal(ea["value_pool"], eb["value_pool"]), f"value cache of layer {i} differs"


def test_stack_qwen2_0_5b_shape_batch32_bitwise():
    """All 24 layers of the Qwen2-0.5B shape at batch 32 (one launch)."""
    cfg = QWEN2_0_5B
    w = random_weights(cfg, seed=61, device="cuda")
    prompt = _prompt(cfg, 32, 3, 62)
    fused, stack = _pair(cfg, w, 32, 128)
    _assert_same(fused, stack, _run_steps(fused, prompt, 3, start=60),
                 _run_steps(stack, prompt, 3, start=60), cfg.layers)


def test_bench_step_matches_the_fp32_logit_session():
    """The benchmark's own step: Qwen2-0.5B shape, batch 32, every sequence at position 4095 of
    a seeded 4095-key context, the stack graph with bf16 logits, captured as 5 chained greedy
    steps in one graph. Against a stack session with fp32 logits stepped one replay at a time:
    lm_head_argmax picks the ids from the fp32 logits before it rounds them, so after 5 steps
    the ids are equal and the bf16 logits are the fp32 logits rounded, bit for bit."""
    cfg, b, ctx = QWEN2_0_5B, 32, 4096
    w = random_weights(cfg, seed=81, device="cuda")
    ref = DecodeSession(cfg, w, b, max_seq_len=ctx + 64, stack=True)
    bench = DecodeSession(cfg, w, b, max_seq_len=ctx + 64, stack=True,
                          logits_dtype="bfloat16")
    g = torch.Generator(device="cuda").manual_seed(82)
    ids = torch.randint(0, cfg.vocab, (b,), generator=g, device="cuda")
    pos = torch.full((b,), ctx - 1, dtype=torch.int64, device="cuda")
    for sess in (ref, bench):
        sess.ids.copy_(ids)
        sess.positions.copy_(pos)
        sess.run_eager()  # reserves the caches
    _fill_caches([ref, bench], cfg, 83)
    ref.capture()
    nxt = ids
    for _ in range(5):
        logits, nxt = ref.step(nxt, pos)
        nxt = nxt.clone()
    bench.ids.copy_(ids)
    bench.positions.copy_(pos)
    bench.capture(chain_ids=True, steps=5)
    bench.ids.copy_(ids)
    out = bench.replay()
    torch.cuda.synchronize()
    bench.check_status()
    assert torch.equal(out["next_ids"], nxt), "ids differ after 5 steps"
    assert torch.equal(bench.ids, nxt), "chained input ids differ"
    assert out["logits"].dtype == torch.bfloat16
    assert torch.equal(out["logits"], logits.to(torch.bfloat16)), "bf16 logits != rounded fp32"


def test_stack_more_layers_than_one_launch():
    """40 layers run as two launches (32 + 8) that continue from the same output buffer."""
    cfg = tiny_config(layers=40)
    w = random_weights(cfg, seed=71, device="cuda")
    prompt = _prompt(cfg, 4, 3, 72)
    fused, stack = _pair(cfg, w, 4, 64, down=4)
    _assert_same(fused, stack, _run_steps(fused, prompt, 2), _run_steps(stack, prompt, 2),
                 cfg.layers)


def _fill_caches(sessions, cfg, seed):
    """The same seeded context in every layer's cache of each session."""
    for i in range(cfg.layers):
        g = torch.Generator(device="cuda").manual_seed(seed + i)
        pools = [sess.engine.kv_cache_entry(f"layer_{i}") for sess in sessions]
        for name in ("key_pool", "value_pool"):
            val = torch.randn(pools[0][name].shape, generator=g, device="cuda").to(torch.bfloat16)
            for p in pools:
                p[name].copy_(val)


@pytest.mark.parametrize("batch,splits", [(32, 3), (32, 4), (4, 6), (2, 9)])
def test_stack_long_context_split_merge_bitwise(batch, splits):
    """Context up to 4096 keys: every pair's keys are split over several workgroups and merged
    by the last to finish, in both paths (up to 9 splits, the most a 65-block context uses)."""
    cfg = tiny_config(layers=2)
    w = random_weights(cfg, seed=81, device="cuda")
    fused, stack = _pair(cfg, w, batch, 4096 + 64, attn=splits)
    start = torch.tensor([4000 - 37 * b for b in range(batch)], device="cuda")
    ids0 = torch.randint(0, cfg.vocab, (batch,), generator=torch.Generator().manual_seed(82))
    outs = []
    for sess in (fused, stack):
        sess.step(ids0.cuda(), start)  # reserves the caches
    _fill_caches((fused, stack), cfg, 83)
    for sess in (fused, stack):
        pos = start.clone()
        res, nxt = [], ids0.cuda()
        for _ in range(3):
            logits, nxt = sess.step(nxt, pos)
            nxt = nxt.clone()
            res.append((logits.float().cpu().clone(), nxt.cpu()))
            pos += 1
        outs.append(res)
    _assert_same(fused, stack, outs[0], outs[1], cfg.layers)


def test_stack_trace_timeline():
    """The stage timeline (a trace buffer input of the decoder_stack node, DliStackOptions.trace):
    every workgroup stamps its layer entries in order, each layer's stage stamps after its entry,
    and the stamps do not change the results (the traced run matches the fused graph bit for
    bit). A session without the buffer, running at the same time, leaves it alone."""
    cfg = tiny_config(layers=3)
    w = random_weights(cfg, seed=71, device="cuda")
    prompt = _prompt(cfg, 8, 3, 72)
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    events = 32  # DLI_STACK_TRACE_EVENTS
    trace = torch.zeros(cfg.layers * grid * events, dtype=torch.int64, device="cuda")
    fused, stack = _pair(cfg, w, 8, 128, down=3, stack_trace=trace)
    _, untraced = _pair(cfg, w, 8, 128, down=3)
    traced = _run_steps(stack, prompt, 1)
    torch.cuda.synchronize()
    _assert_same(fused, stack, _run_steps(fused, prompt, 1), traced, cfg.layers)
    t = trace.view(cfg.layers, grid, events).cpu()
    start = t[:, :, 0]  # kTrLayerStart: written by every workgroup in every layer
    assert bool((start > 0).all()), "a workgroup did not stamp a layer entry"
    assert bool((start[1:] >= start[:-1]).all()), "layer entries out of order"
    later = t[:, :, 1:]
    reached = later > 0  # a workgroup without work in a stage leaves its events at 0
    assert bool(reached.any()), "no stage stamps"
    assert bool((later[reached] >= start.unsqueeze(2).expand_as(later)[reached]).all())
    # the stamps of one layer end before the next layer's entries of the same workgroup
    assert bool((later[:-1].amax(dim=2) <= start[1:]).all())
    before = trace.clone()
    _run_steps(untraced, prompt[:, :1], 0, start=3)
    torch.cuda.synchronize()
    assert torch.equal(trace, before), "a session without the trace buffer wrote to it"


def test_stack_trace_buffer_too_small_is_rejected():
    cfg = tiny_config(layers=2)
    w = random_weights(cfg, seed=73, device="cuda")
    buf = torch.zeros(16, dtype=torch.int64, device="cuda")  # less than one layer
    _, stack = _pair(cfg, w, 4, 64, stack_trace=buf)
    with pytest.raises(ValueError, match="trace buffer"):
        stack.step(torch.zeros(4, dtype=torch.int64, device="cuda"),
                   torch.zeros(4, dtype=torch.int64, device="cuda"))
