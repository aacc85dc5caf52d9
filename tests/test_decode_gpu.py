"""Qwen2 decode on the GPU through Engine + the gfx950 plugin. The fused graph and the
reference-style graph, and HIP-graph replay and eager runs, must give identical greedy tokens;
against the CPU oracle (oracle/qwen2.py) the bar is bf16 logit parity, teacher-forced on the
GPU's own tokens."""
from __future__ import annotations

import pytest
import torch

from dli_qwen2 import QWEN2_0_5B, DecodeSession, random_weights, tiny_config
from oracle.qwen2 import Qwen2Oracle

pytestmark = pytest.mark.gpu


def _prompt(cfg, batch, length, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.vocab, (batch, length), generator=g)


def _run_prefill_steps(session, prompt, steps):
    """The prompt through the prefill graph in one run, then `steps` greedy decode steps; the
    same (logits, next_ids) list as _run_steps."""
    b, s = prompt.shape
    logits, nxt = session.run_prefill(prompt.cuda())
    out = [(logits.float().cpu().clone(), nxt.cpu().clone())]
    pos = torch.full((b,), s, dtype=torch.int64, device="cuda")
    for _ in range(steps):
        logits, nxt = session.step(nxt.clone(), pos)
        out.append((logits.float().cpu().clone(), nxt.cpu().clone()))
        pos += 1
    return out


def _run_steps(session, prompt, steps):
    """Feeds the prompt then `steps` greedy tokens; returns per-step (logits, next_ids) after the
    prompt's last token and after each generated token."""
    b, s = prompt.shape
    pos = torch.zeros(b, dtype=torch.int64, device="cuda")
    out = []
    nxt = None
    for t in range(s + steps):
        ids = prompt[:, t].cuda() if t < s else nxt
        logits, nxt = session.step(ids, pos)
        nxt = nxt.clone()
        if t >= s - 1:
            out.append((logits.float().cpu().clone(), nxt.cpu()))
        pos += 1
    return out


@pytest.mark.parametrize("batch", [1, 5, 16])
def test_fused_graph_matches_reference_graph(batch):
    cfg = tiny_config()
    w = random_weights(cfg, seed=11, device="cuda")
    prompt = _prompt(cfg, batch, 6, 12)
    fused = DecodeSession(cfg, w, batch, max_seq_len=64, fused=True)
    ref = DecodeSession(cfg, w, batch, max_seq_len=64, fused=False)
    a = _run_steps(fused, prompt, 5)
    b = _run_steps(ref, prompt, 5)
    for (la, ia), (lb, ib) in zip(a, b):
        torch.testing.assert_close(la, lb, rtol=2e-2, atol=2e-2)
        assert torch.equal(ia, ib)


def test_capture_replay_equals_eager():
    cfg = tiny_config()
    w = random_weights(cfg, seed=21, device="cuda")
    prompt = _prompt(cfg, 8, 5, 22)
    eager = DecodeSession(cfg, w, 8, max_seq_len=64)
    # capture's warm-up step writes position 0, which the first real step overwrites
    graphed = DecodeSession(cfg, w, 8, max_seq_len=64).capture()
    a = _run_steps(eager, prompt, 6)
    b = _run_steps(graphed, prompt, 6)
    for (la, ia), (lb, ib) in zip(a, b):  # deterministic kernels: bitwise equal every replay
        assert torch.equal(la, lb)
        assert torch.equal(ia, ib)


def _flip_report(logits, ref, exact, gpu_ids, expect):
    """Per-token check of the steps where the GPU's greedy token differs from the oracle's argmax
    (same prefix). A flip from the oracle's b to the GPU's a is accepted only as a near-tie:
    the oracle's margin ref[b] - ref[a] is within 4 sqrt(2) sigma, and each of the two logits the
    GPU got wrong is within 6 sigma of the oracle's value, where sigma is that step's RMS of
    (bf16 oracle - fp32 model) over the vocabulary: the rounding noise the graph's bf16 rounding
    points produce at that step. Returns the flips as dicts; raises on one outside the band."""
    sigma = (ref - exact).pow(2).mean(-1).sqrt()  # [R, T]
    flips = []
    for r, t in (~(gpu_ids == expect)).nonzero().tolist():
        a, b = int(gpu_ids[r, t]), int(expect[r, t])
        gap = float(ref[r, t, b] - ref[r, t, a])
        e_a = float((logits[r, t, a] - ref[r, t, a]).abs())
        e_b = float((logits[r, t, b] - ref[r, t, b]).abs())
        sg = float(sigma[r, t])
        flips.append({"row": r, "step": t, "gpu": a, "oracle": b, "gap": gap, "err_gpu_tok": e_a,
                      "err_oracle_tok": e_b, "sigma": sg})
        assert gap <= 4 * 2 ** 0.5 * sg and e_a <= 6 * sg and e_b <= 6 * sg, (
            f"token flip outside the rounding-noise band: {flips[-1]}")
    return flips


def _teacher_forced_parity(cfg, w, batch, prompt_len, steps, seed, agree_min, stack=False,
                           prefill=False):
    """Free-running greedy decode on the GPU, then the oracle teacher-forced on the GPU's own
    tokens (one batched CPU pass over prompt + generated tokens) for every row, so both score
    the same prefixes at every step.

    Two bf16 implementations that sum in different orders cannot promise identical tokens or
    logits: every node output is rounded to bf16, and where the two orders round a value
    differently the difference propagates through the remaining layers. The size of that noise
    is measured here rather than assumed: the oracle is run twice, with its bf16 rounding points
    (the graph's arithmetic) and in plain fp32 (the same model without rounding). Criteria:
      1. next_ids is exactly argmax(logits) (first index of the maximum) at every step;
      2. the GPU's logits are no further from the bf16 oracle, and no further from the fp32
         model, than bf16 rounding itself moves the oracle (relative L2 error per step, ratio
         bounds below); a wrong index, sign or operand gives errors of order 1 and fails;
      3. every token flip passes the per-token near-tie test of _flip_report, and the tokens
         agree on at least `agree_min` of the (row, step) pairs.
    The first step at which a row's tokens differ from the oracle's argmax is also the step at
    which a free-running oracle would first diverge from the GPU (the prefixes agree up to it).
    """
    prompt = _prompt(cfg, batch, prompt_len, seed)
    session = DecodeSession(cfg, w, batch, max_seq_len=prompt_len + steps + 8, stack=stack,
                            prefill=prefill).capture()
    run = _run_prefill_steps if prefill else _run_steps
    got = run(session, prompt, steps - 1)  # logits after the prompt + steps-1 tokens
    logits = torch.stack([lg for lg, _ in got], 1)  # [B, T, V]
    ids = torch.stack([nx for _, nx in got], 1)  # [B, T]
    assert torch.equal(ids, torch.argmax(logits, -1)), "next_ids != argmax(logits)"
    expect, _, ref = Qwen2Oracle(cfg, w).teacher_forced(prompt, ids)
    _, _, exact = Qwen2Oracle(cfg, w, round_bf16=False).teacher_forced(prompt, ids)

    def rel(a, b):  # [R, T]
        return (a - b).norm(dim=-1) / b.norm(dim=-1)

    err_bf16, err_fp32, noise = rel(logits, ref), rel(logits, exact), rel(ref, exact)
    print(f"\nteacher-forced parity, {batch} rows, {logits.shape[1]} steps: relative logit "
          f"error vs bf16 oracle mean {float(err_bf16.mean()):.3e} max {float(err_bf16.max()):.3e}; "
          f"vs fp32 model mean {float(err_fp32.mean()):.3e} max {float(err_fp32.max()):.3e}; "
          f"bf16 oracle vs fp32 model mean {float(noise.mean()):.3e} max {float(noise.max()):.3e}")
    assert float(err_bf16.mean()) <= 1.25 * float(noise.mean())
    assert float(err_fp32.mean()) <= 1.25 * float(noise.mean())
    assert float(err_bf16.max()) <= 1.5 * float(noise.max())
    assert float(err_fp32.max()) <= 1.5 * float(noise.max())
    flips = _flip_report(logits, ref, exact, ids, expect)
    agree = ids == expect
    rate = float(agree.float().mean())
    first = [int((~agree[r]).nonzero()[0]) if not bool(agree[r].all()) else None
             for r in range(batch)]
    worst = max((f["gap"] / f["sigma"] for f in flips), default=0.0)
    print(f"token agreement {rate:.3f} over {agree.numel()} (row, step) pairs; {len(flips)} flips, "
          f"largest oracle margin at a flip {worst:.2f} sigma; first divergence step per row "
          f"{first}", flush=True)
    assert rate >= agree_min, f"token agreement {rate:.3f} < {agree_min}"


@pytest.mark.parametrize("prefill", [False, True], ids=["stepwise", "prefill"])
@pytest.mark.parametrize("stack", [False, True], ids=["fused", "stack"])
def test_tiny_decode_teacher_forced_parity(stack, prefill):
    cfg = tiny_config()
    w = random_weights(cfg, seed=31, device="cuda")
    _teacher_forced_parity(cfg, w, batch=6, prompt_len=12, steps=24, seed=32, agree_min=0.9,
                           stack=stack, prefill=prefill)


@pytest.mark.slow
def test_qwen2_0_5b_shape_prefill_graph_then_decode_teacher_forced_parity():
    """The 512-token prompt through the prefill graph (all layers over [8, 512] tokens: tiled
    bf16 MFMA linears, flash attention), then 64 greedy steps through the decoder stack;
    every row scored by the oracle."""
    cfg = QWEN2_0_5B
    w = random_weights(cfg, seed=41, device="cuda")
    _teacher_forced_parity(cfg, w, batch=8, prompt_len=512, steps=64, seed=42, agree_min=0.92,
                           stack=True, prefill=True)


@pytest.mark.slow
@pytest.mark.parametrize("batch", [1, 8, 32])
def test_qwen2_0_5b_shape_64_steps_teacher_forced_parity(batch):
    """Full Qwen2-0.5B shape through the decoder stack (the product graph), 512 random prompt
    tokens, 64 greedy steps; the oracle scores every row on the CPU."""
    cfg = QWEN2_0_5B
    w = random_weights(cfg, seed=41, device="cuda")
    # measured agreement: 0.969 (batch 1, 64 tokens), 0.947 (batch 8), 0.958 (batch 32)
    _teacher_forced_parity(cfg, w, batch=batch, prompt_len=512, steps=64, seed=42,
                           agree_min={1: 0.9, 8: 0.92, 32: 0.93}[batch], stack=True)


def _fill_paged_cache(engine, oracle, layers, batch, fill):
    """Copies the oracle's synthetic context (positions [0, fill) of its preallocated caches)
    into the paged pools of the engine's cache entries layer_0.. (layouts in
    include/dli/kv_cache.h: key [blocks, Hkv, 64, D], value [blocks, Hkv, D, 64])."""
    for i in range(layers):
        e = engine.kv_cache_entry(f"layer_{i}")
        bs = e["block_size"]
        nblk = (fill + bs - 1) // bs
        table = e["block_table"].long()
        kp, vp = e["key_pool"], e["value_pool"]
        hkv, d = kp.shape[1], kp.shape[3]
        for b in range(batch):
            k = torch.zeros(hkv, nblk * bs, d)
            v = torch.zeros(hkv, nblk * bs, d)
            k[:, :fill] = oracle.k_static[i][b, :, :fill]
            v[:, :fill] = oracle.v_static[i][b, :, :fill]
            blocks = table[b, :nblk]
            kp[blocks] = k.view(hkv, nblk, bs, d).permute(1, 0, 2, 3).to(kp.dtype).cuda()
            vp[blocks] = v.view(hkv, nblk, bs, d).permute(1, 0, 3, 2).to(vp.dtype).cuda()


@pytest.mark.slow
@pytest.mark.parametrize("batch", [1, 8, 32])
def test_qwen2_0_5b_shape_step_at_context_4096_matches_oracle(batch):
    """The bench workload's step: every row at position 4095 over a seeded synthetic context of
    4095 keys per layer, through the decoder stack; the oracle's preallocated-cache step on the
    same context. Logits: within the noise bounds of _teacher_forced_parity (relative L2 error
    against the bf16 oracle and the fp32 model no larger than bf16 rounding moves the oracle);
    tokens: the oracle's argmax except near-ties (_flip_report)."""
    cfg, ctx = QWEN2_0_5B, 4096
    w = random_weights(cfg, seed=43, device="cuda")
    ids = torch.randint(0, cfg.vocab, (batch,), generator=torch.Generator().manual_seed(44))
    oracle = Qwen2Oracle(cfg, w)
    oracle.reset_static(batch, ctx, seed=45, fill=ctx - 1)
    exact_oracle = Qwen2Oracle(cfg, w, round_bf16=False)
    exact_oracle.k_static, exact_oracle.v_static = oracle.k_static, oracle.v_static
    session = DecodeSession(cfg, w, batch, max_seq_len=ctx + 8, stack=True)
    pos = torch.full((batch,), ctx - 1, dtype=torch.int64, device="cuda")
    session.step(ids.cuda(), pos)  # creates the cache entries (the context is written next)
    torch.cuda.synchronize()
    _fill_paged_cache(session.engine, oracle, cfg.layers, batch, ctx - 1)
    torch.cuda.synchronize()
    logits, nxt = session.step(ids.cuda(), pos)
    logits = logits.float().cpu()[:, None]  # [B, 1, V]
    nxt = nxt.cpu()[:, None]
    ref = oracle.step_static(ids, ctx - 1)[:, None]
    exact = exact_oracle.step_static(ids, ctx - 1)[:, None]
    session.check_status()
    assert torch.equal(nxt, torch.argmax(logits, -1))

    def rel(a, b):
        return (a - b).norm(dim=-1) / b.norm(dim=-1)

    err_bf16, err_fp32, noise = rel(logits, ref), rel(logits, exact), rel(ref, exact)
    print(f"\ncontext {ctx}, batch {batch}: relative logit error vs bf16 oracle mean "
          f"{float(err_bf16.mean()):.3e} max {float(err_bf16.max()):.3e}; vs fp32 model mean "
          f"{float(err_fp32.mean()):.3e} max {float(err_fp32.max()):.3e}; bf16 oracle vs fp32 "
          f"model mean {float(noise.mean()):.3e} max {float(noise.max()):.3e}", flush=True)
    # 2e-2 is the per-operator bf16 bar. End to end at this context the bf16 model's own
    # rounding noise is larger (the bf16 oracle sits about 3.4e-2 from the fp32 model), so the
    # logits are held to that measured noise instead, as in _teacher_forced_parity.
    assert float(err_bf16.mean()) <= 1.25 * float(noise.mean())
    assert float(err_fp32.mean()) <= 1.25 * float(noise.mean())
    assert float(err_bf16.max()) <= 1.5 * float(noise.max())
    assert float(err_fp32.max()) <= 1.5 * float(noise.max())
    expect = torch.argmax(ref, -1)
    flips = _flip_report(logits, ref, exact, nxt, expect)
    print(f"tokens: {batch - len(flips)}/{batch} equal to the oracle's argmax; flips {flips}",
          flush=True)


@pytest.mark.slow
@pytest.mark.parametrize("batch", [1, 4, 8, 32])
def test_qwen2_0_5b_shape_fp32_reference_graph_identical_greedy_ids(batch):
    """The reference's own precision: the reference-style graph (the exporter's 19 nodes per
    layer) in fp32 at the Qwen2-0.5B shape, 512 random prompt tokens fed through the decode step,
    then 64 greedy tokens, at the config's batches 1, 8 and 32 (and 4). Every row must equal the
    fp32 oracle's free-running greedy tokens exactly (prefill as one batched pass, then one step
    per token): the bar of the reference's end-to-end test (tests/e2e/test_models.py:61-71)."""
    cfg = QWEN2_0_5B
    w = random_weights(cfg, seed=47, device="cuda", dtype=torch.float32)
    prompt = _prompt(cfg, batch, 512, 48)
    session = DecodeSession(cfg, w, batch, max_seq_len=512 + 64 + 8, fused=False).capture()
    got = session.generate(prompt.cuda(), 64).cpu()
    expect, margins = Qwen2Oracle(cfg, w, round_bf16=False).generate(prompt, 64)
    differ = [r for r in range(batch) if not torch.equal(got[r], expect[r])]
    first = {r: int((got[r] != expect[r]).nonzero()[0]) for r in differ}
    print(f"\nfp32 greedy, batch {batch}, 64 steps: smallest top-1/top-2 oracle margin "
          f"{float(margins.min()):.3e}; rows differing {len(differ)} of {batch}, first differing "
          f"step per such row {first}", flush=True)
    assert torch.equal(got, expect)


@pytest.mark.slow
def test_qwen2_7b_shape_two_layers_teacher_forced_parity():
    """The Qwen2-7B geometry (hidden 3584, 28 / 4 heads, head_dim 128, MLP 18944, vocab 152064,
    untied lm_head) with 2 of its 28 layers, batch 64: the large-hidden decode graph (head_dim-128
    MFMA decode attention, skinny MFMA linears) against the oracle, every row scored."""
    from dataclasses import replace

    from dli_qwen2 import QWEN2_7B

    cfg = replace(QWEN2_7B, layers=2)
    w = random_weights(cfg, seed=91, device="cuda")
    _teacher_forced_parity(cfg, w, batch=64, prompt_len=16, steps=8, seed=92, agree_min=0.9)


@pytest.mark.slow
def test_qwen2_7b_shape_step_at_context_8192_matches_oracle():
    """The config-5 step geometry at context 8192 (position 8191 over a seeded 8191-key context
    per layer) with 2 of the 28 layers, batch 8, against the oracle's preallocated-cache step."""
    from dataclasses import replace

    from dli_qwen2 import QWEN2_7B

    cfg, ctx, batch = replace(QWEN2_7B, layers=2), 8192, 8
    w = random_weights(cfg, seed=93, device="cuda")
    ids = torch.randint(0, cfg.vocab, (batch,), generator=torch.Generator().manual_seed(94))
    oracle = Qwen2Oracle(cfg, w)
    oracle.reset_static(batch, ctx, seed=95, fill=ctx - 1)
    exact_oracle = Qwen2Oracle(cfg, w, round_bf16=False)
    exact_oracle.k_static, exact_oracle.v_static = oracle.k_static, oracle.v_static
    session = DecodeSession(cfg, w, batch, max_seq_len=ctx + 8)
    pos = torch.full((batch,), ctx - 1, dtype=torch.int64, device="cuda")
    session.step(ids.cuda(), pos)
    torch.cuda.synchronize()
    _fill_paged_cache(session.engine, oracle, cfg.layers, batch, ctx - 1)
    torch.cuda.synchronize()
    logits, nxt = session.step(ids.cuda(), pos)
    logits = logits.float().cpu()[:, None]
    nxt = nxt.cpu()[:, None]
    ref = oracle.step_static(ids, ctx - 1)[:, None]
    exact = exact_oracle.step_static(ids, ctx - 1)[:, None]
    assert torch.equal(nxt, torch.argmax(logits, -1))

    def rel(a, b):
        return (a - b).norm(dim=-1) / b.norm(dim=-1)

    err_bf16, err_fp32, noise = rel(logits, ref), rel(logits, exact), rel(ref, exact)
    print(f"\n7B geometry, 2 layers, context {ctx}, batch {batch}: relative logit error vs bf16 "
          f"oracle mean {float(err_bf16.mean()):.3e}; vs fp32 model mean "
          f"{float(err_fp32.mean()):.3e}; bf16 oracle vs fp32 model mean "
          f"{float(noise.mean()):.3e}", flush=True)
    assert float(err_bf16.mean()) <= 1.25 * float(noise.mean())
    assert float(err_fp32.mean()) <= 1.25 * float(noise.mean())
    assert float(err_bf16.max()) <= 1.5 * float(noise.max())
    flips = _flip_report(logits, ref, exact, nxt, torch.argmax(ref, -1))
    print(f"tokens: {batch - len(flips)}/{batch} equal to the oracle's argmax", flush=True)


def _new_kv(engine, layer, batch, pos):
    """The key and value the step wrote at position pos of every row, from the paged pools of
    cache entry layer_<layer> (key [blocks, Hkv, 64, D], value [blocks, Hkv, D, 64]):
    [B, Hkv, D] each, float32 on the host."""
    e = engine.kv_cache_entry(f"layer_{layer}")
    bs = e["block_size"]
    blocks = e["block_table"].long()[:, pos // bs]
    slot = pos % bs
    k = e["key_pool"][blocks][:, :, slot, :]
    v = e["value_pool"][blocks][:, :, :, slot]
    return k.float().cpu(), v.float().cpu()


@pytest.mark.slow
def test_qwen2_7b_shape_full_model_step_at_context_8192():
    """Config 5 at full size: all 28 Qwen2-7B-shape layers, batch 64, every row at position 8191
    over an 8191-key context in every layer (15 GB of weights, 30 GB of paged cache), through the
    large-hidden decode graph. The whole model is too large for the oracle, so the run is held to
    properties: next_ids == argmax(logits); a HIP-graph replay of the step equals the eager step
    bit for bit (logits, ids and the K/V it appended in every layer); and the K/V that layers 0
    and 1 appended equal, at the bf16 bar, those of the oracle's 2-layer slice of the same model
    on the same context (layer 1's input is layer 0's whole output, attention over 8192 keys
    included)."""
    from dataclasses import replace

    from dli_qwen2 import QWEN2_7B

    cfg, ctx, batch = QWEN2_7B, 8192, 64
    pos_i = ctx - 1
    w = random_weights(cfg, seed=97, device="cuda")
    ids = torch.randint(0, cfg.vocab, (batch,), generator=torch.Generator().manual_seed(98))
    session = DecodeSession(cfg, w, batch, max_seq_len=ctx + 8)
    pos = torch.full((batch,), pos_i, dtype=torch.int64, device="cuda")
    session.step(ids.cuda(), pos)  # creates the cache entries (the context is written next)
    torch.cuda.synchronize()
    sliced = {k: v.cpu() for k, v in w.items()
              if not k.startswith("model.layers.") or int(k.split(".")[2]) < 2}
    oracle = Qwen2Oracle(replace(cfg, layers=2), sliced)
    oracle.reset_static(batch, ctx, seed=99, fill=pos_i)
    _fill_paged_cache(session.engine, oracle, 2, batch, pos_i)
    g = torch.Generator(device="cuda").manual_seed(100)
    for i in range(2, cfg.layers):  # the other layers' context: seeded N(0, 1) bf16
        e = session.engine.kv_cache_entry(f"layer_{i}")
        for pool in (e["key_pool"], e["value_pool"]):
            pool.copy_(torch.randn(pool.shape, generator=g, device="cuda").to(pool.dtype))
    torch.cuda.synchronize()
    del sliced

    logits, nxt = session.step(ids.cuda(), pos)
    logits, nxt = logits.clone(), nxt.clone()
    torch.cuda.synchronize()
    eager_kv = [_new_kv(session.engine, i, batch, pos_i) for i in range(cfg.layers)]
    assert bool(torch.isfinite(logits).all())
    assert torch.equal(nxt, torch.argmax(logits, -1)), "next_ids != argmax(logits)"

    session.capture()  # its warm-up step rewrites position 8191 with the same values
    session.ids.copy_(ids.cuda())
    session.positions.copy_(pos)
    out = session.replay()
    torch.cuda.synchronize()
    session.check_status()
    assert torch.equal(out["logits"], logits), "graph replay logits differ from the eager step"
    assert torch.equal(out["next_ids"], nxt)
    for i in range(cfg.layers):
        k, v = _new_kv(session.engine, i, batch, pos_i)
        assert torch.equal(k, eager_kv[i][0]) and torch.equal(v, eager_kv[i][1]), f"layer {i}"

    oracle.step_static(ids, pos_i)  # writes the slice's new K/V at position 8191
    for i in range(2):
        ref_k = oracle.k_static[i][:, :, pos_i]
        ref_v = oracle.v_static[i][:, :, pos_i]
        k, v = eager_kv[i]
        for name, a, b in (("key", k, ref_k), ("value", v, ref_v)):
            rel = float((a - b).norm() / b.norm())
            print(f"\nlayer {i} {name} appended at {pos_i}: relative L2 error {rel:.3e}",
                  flush=True)
            assert rel <= 1e-2, f"layer {i} {name}: relative error {rel:.3e}"
            torch.testing.assert_close(a, b, rtol=2e-2, atol=2e-2)


def test_large_hidden_prefill_graph_then_decode_teacher_forced_parity():
    """A large-hidden model (the Qwen2-7B geometry, one layer) with its prompt through the
    prefill graph: the head is rms_norm + linear + argmax there (lm_head_argmax holds at most
    1024 columns), then greedy steps; every row scored by the oracle."""
    from dataclasses import replace

    from dli_qwen2 import QWEN2_7B

    cfg = replace(QWEN2_7B, layers=1)
    w = random_weights(cfg, seed=101, device="cuda")
    _teacher_forced_parity(cfg, w, batch=2, prompt_len=8, steps=4, seed=102, agree_min=0.75,
                           prefill=True)
