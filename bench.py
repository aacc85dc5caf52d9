"""Decode throughput of the gfx950 operator plugin on one MI355X.

Workload: Qwen2-0.5B-shape (24 layers, hidden 896, 14/2 heads, head_dim 64, MLP 4864, vocab
151936, tied embeddings), random-init bf16, greedy decode at batch 32 with every sequence at
context 4096 (a seeded synthetic KV context fills positions 0..4094; each step writes position
4095 and attends over 4096 keys). One step = one replay of the captured dli.graph.v1 decode
step through Engine + libdli_hip_ops.so; inputs already in HBM. --graph stack (default): every
decoder layer in one persistent decoder_stack launch, then model.norm and lm_head + argmax;
--graph fused: five launches per layer.

Prints one JSON line: decode tok/s (whole job), ms/step, the step's HBM roofline fraction
(algorithmic bytes = weights + KV read + KV write + bf16 logits), the dominant kernel's roofline
(the decoder stack, or decode attention for the fused graph, timed live with HIP events on its
stream) and a CPU baseline (the same step as the reference-style graph through the dli Engine and
the ATen CPU reference plugin on this host's cores, a bounded sample of steps).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dl-inference_amd", "python"))

METRIC = "decode tok/s + % HBM roofline, Qwen2-0.5B-shape bf16 b=32 ctx4096"
METRIC_7B = "decode tok/s + % HBM roofline, Qwen2-7B-shape bf16 b=64 ctx8192"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=("decode", "alexnet", "prefill", "linear"),
                    default="decode",
                    help="decode (default): the Qwen2 decode step; alexnet: the AlexNet-style "
                         "fp32 CNN forward (batch 64) on the MFMA GEMM operators; prefill: the "
                         "operators of one Qwen2 decoder layer at batch 4 x 2048 tokens; linear: "
                         "the single fp32 linear layer [64,1024] x [4096,1024]^T + b")
    ap.add_argument("--model", choices=("0.5b", "7b"), default="0.5b",
                    help="decode model shape: 0.5b (Qwen2-0.5B, batch 32, context 4096) or 7b "
                         "(Qwen2-7B, batch 64, context 8192: the large-hidden decode graph)")
    ap.add_argument("--batch", type=int, default=None, help="decode 32 (7b: 64), alexnet 64")
    ap.add_argument("--context", type=int, default=None, help="decode 4096 (7b: 8192)")
    ap.add_argument("--layers", type=int, default=None, help="override (for quick local checks)")
    ap.add_argument("--cpu-baseline-steps", type=int, default=8)
    ap.add_argument("--cpu-baseline-warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--splits", default=None, help="split-K per projection, e.g. o=2,down=4")
    ap.add_argument("--eager", action="store_true", help="run the step without graph capture")
    ap.add_argument("--steps-per-graph", type=int, default=0,
                    help="decode: chained greedy steps per captured HIP graph (0: the largest "
                         "of 5, 4, 2, 1 that divides both --steps and --warmup)")
    ap.add_argument("--graph", choices=("stack", "fused"), default="stack",
                    help="stack: all decoder layers in one persistent launch; fused: five "
                         "launches per layer")
    ap.add_argument("--profile", default=None, metavar="PATH",
                    help="after timing, run --profile-steps eager steps under a dli.ProfileSession "
                         "and write its dli.profile.v1 JSON to PATH (per-node CPU and GPU time; "
                         "summary: python -m dli.profile summarize PATH)")
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after timing, copy this many MiB device-to-device 3 times (a plain copy "
                         "of known size that scales rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# (graph, batch, context) -> the committed PMC summary of that workload's dominant kernel
TRAFFIC_PROFILES = {
    ("stack", 32, 4096): os.path.join(ROOT, "profiles",
                                      "decoder_stack_pmc_qwen2-0.5b_b32_ctx4096.txt"),
    ("fused", 32, 4096): os.path.join(ROOT, "profiles",
                                      "decode_attention_pmc_qwen2-0.5b_b32_ctx4096.txt"),
    ("large", 64, 8192): os.path.join(ROOT, "profiles",
                                      "decode_attention_d128_pmc_qwen2-7b_b64_ctx8192.txt"),
}


def profiled_traffic(graph, batch, context):
    """HBM bytes per launch of the dominant kernel measured by two rocprofv3 --pmc runs
    (FETCH_SIZE, WRITE_SIZE) scaled by a copy kernel of known size; recorded in the committed
    profile of the same workload (None for a workload without one)."""
    path = TRAFFIC_PROFILES.get((graph, batch, context))
    if path is None:
        return None
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":")[1].split()[0]))
    except OSError:
        pass
    return None


def step_bytes(cfg, batch, context):
    weights = cfg.weight_bytes()
    kv_read = batch * context * cfg.kv_bytes_per_token()
    kv_write = batch * cfg.kv_bytes_per_token()
    logits = batch * cfg.vocab * 2
    return weights + kv_read + kv_write, weights, kv_read, kv_write, logits


def cpu_description():
    """Core count and CPU model of this host (recorded with every CPU baseline)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo", encoding="utf-8"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return os.cpu_count(), model


def cpu_engine_decode_baseline(cfg, weights, B, ctx, ids, steps, warmup):
    """The same decode step on the host: the reference-style dli.graph.v1 decode graph (the
    exporter's 19 nodes per layer, python/dli_export/export.py:272-446) run through the dli
    Engine with the ATen CPU reference plugin (lib/libdli_aten_ops.so) on all host cores, in
    fp32 (the reference's precision) with the bf16 weights' values. The host KV cache holds a
    synthetic context of ctx - 1 keys per layer; every step writes position ctx - 1 and attends
    over ctx keys. Median wall time per step over `steps` steps after `warmup`."""
    import statistics

    import torch

    import dli
    from dli_qwen2 import DecodeSession

    cores, model = cpu_description()
    torch.set_num_threads(cores)
    w32 = {k: v.detach().to("cpu", torch.float32) for k, v in weights.items()}
    engine = dli.Engine().load_aten_plugin()
    session = DecodeSession(cfg, w32, B, max_seq_len=ctx, fused=False, engine=engine,
                            device="cpu")
    ids = ids.cpu()
    pos = torch.full((B,), ctx - 1, dtype=torch.int64)
    session.step(ids, pos)  # creates the host cache entries
    g = torch.Generator().manual_seed(3)
    for i in range(cfg.layers):  # synthetic context: a seeded 64-key block, repeated
        e = engine.kv_cache_entry(f"layer_{i}")
        for pool, axis in ((e["key_pool"], 2), (e["value_pool"], 3)):
            shape = list(pool.shape)
            shape[axis] = 64
            block = torch.randn(shape, generator=g)
            reps = [1, 1, 1, 1]
            reps[axis] = pool.shape[axis] // 64
            pool.copy_(block.repeat(*reps))
    for _ in range(warmup):
        session.step(ids, pos)
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        session.step(ids, pos)
        times.append(time.perf_counter() - t0)
    step_s = statistics.median(times)
    return {"value": round(B / step_s, 2), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"median of {steps} decode steps after {warmup} warm-ups of the same "
                      f"batch-{B}, context-{ctx} step: the reference-style dli.graph.v1 graph "
                      f"through the dli Engine + ATen CPU reference plugin, fp32 with the bf16 "
                      f"weights' values; {step_s * 1000:.1f} ms/step; {cores} cores ({model})"}


def time_decode_attention(session, cfg, B, ctx, pos, g, stream, hip, reps=200):
    """Decode attention of one layer (same cache, fresh q) alone, timed with HIP events on the
    stream it is launched on. Returns (kernel, average us, algorithmic bytes per launch)."""
    import torch

    e = session.engine.kv_cache_entry("layer_0")
    q = torch.randn(B, cfg.heads, 1, cfg.head_dim, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    ws_bytes = hip.lib().dli_hip_paged_attention_workspace(B, cfg.heads, 1, cfg.head_dim,
                                                            e["max_blocks"] * e["block_size"])
    ws = torch.zeros((ws_bytes + 3) // 4, dtype=torch.float32, device="cuda")  # counters at 0
    s_ptr = stream.cuda_stream

    def attn():
        hip.call("dli_hip_paged_attention", hip.BF16, q.data_ptr(), e["key_pool"].data_ptr(),
                 e["value_pool"].data_ptr(), e["block_table"].data_ptr(), out.data_ptr(), B, cfg.heads,
                 cfg.kv_heads, 1, cfg.head_dim, e["block_size"], e["max_blocks"], 0,
                 pos.data_ptr(), hip.I64, 1, cfg.head_dim ** -0.5, 0, ws.data_ptr(), ws_bytes,
                 s_ptr)

    us = _time_launches(attn, stream, reps)
    nbytes = B * ctx * cfg.kv_heads * cfg.head_dim * 2 * 2 + 2 * B * cfg.heads * cfg.head_dim * 2
    return f"decode attention (decode_attention_d{cfg.head_dim})", us, nbytes


STACK_OPTIONS = None  # DliStackOptions for time_decoder_stack's launches (None: defaults)


def time_decoder_stack(session, cfg, B, ctx, pos, g, stream, hip, down_splits, reps=20):
    """The persistent decoder stack (every layer in one launch) alone, on the session's weights
    and caches, timed with HIP events on the stream it is launched on. Algorithmic bytes per
    launch: every layer's weights once, the K/V context read once, the new K/V written."""
    import ctypes

    import torch

    L = cfg.layers
    layers = (hip.DecoderLayer * L)()
    layer_bytes = 0
    for i in range(L):
        p = f"model.layers.{i}"
        names = [f"{p}.input_layernorm.weight", f"{p}.self_attn.qkv_proj.weight",
                 f"{p}.self_attn.qkv_proj.bias", f"{p}.self_attn.o_proj.weight",
                 f"{p}.post_attention_layernorm.weight", f"{p}.mlp.gate_up_proj.weight",
                 f"{p}.mlp.down_proj.weight"]
        t = [session.inputs[n] for n in names]
        layer_bytes += sum(x.numel() * x.element_size() for x in t)
        e = session.engine.kv_cache_entry(f"layer_{i}")
        layers[i] = hip.DecoderLayer(*[x.data_ptr() for x in t], e["key_pool"].data_ptr(),
                                     e["value_pool"].data_ptr(), e["block_table"].data_ptr())
    e0 = session.engine.kv_cache_entry("layer_0")
    ws_bytes = hip.lib().dli_hip_decoder_stack_workspace(L, B, cfg.hidden, cfg.heads,
                                                          cfg.kv_heads, cfg.head_dim, cfg.ffn,
                                                          e0["max_blocks"], down_splits, 0)
    ws = torch.zeros((ws_bytes + 3) // 4, dtype=torch.int32, device="cuda")
    x = (torch.randn(B, cfg.hidden, generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    out = torch.empty_like(x)
    cos, sin = session.inputs["rotary_cos"], session.inputs["rotary_sin"]
    s_ptr = stream.cuda_stream

    def stack():
        hip.call("dli_hip_decoder_stack", layers, L, x.data_ptr(), out.data_ptr(),
                 pos.data_ptr(), hip.I64, cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                 e0["block_size"], e0["max_blocks"], B, cfg.hidden, cfg.heads, cfg.kv_heads,
                 cfg.head_dim, cfg.ffn, cfg.eps, down_splits, ws.data_ptr(), ws_bytes, None,
                 ctypes.byref(STACK_OPTIONS) if STACK_OPTIONS is not None else None, s_ptr)

    us = _time_launches(stack, stream, reps)
    aborted = ctypes.c_int()
    hip.call("dli_hip_decoder_stack_status", ws.data_ptr(), ctypes.byref(aborted), s_ptr)
    if aborted.value:
        raise RuntimeError("decoder_stack: a workgroup gave up waiting")
    kv = cfg.kv_bytes_per_token()
    nbytes = layer_bytes + B * ctx * kv + B * kv
    return "decoder stack (decoder_stack_m2, all layers in one launch)", us, nbytes


def _time_launches(fn, stream, reps):
    import torch

    for _ in range(5):
        fn()
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a0.record(stream)
    for _ in range(reps):
        fn()
    a1.record(stream)
    torch.cuda.synchronize()
    return a0.elapsed_time(a1) * 1000.0 / reps


FP32_MFMA_PEAK_TFLOPS = 157.3


def bench_alexnet(args):
    """AlexNet-style fp32 CNN forward (conv 64/192/384/256/256 3x3, FC 4096-4096-10) at batch 64
    on 3x32x32 inputs: one step = one replay of the captured dli.graph.v1 forward. Reports
    images/s, the step's fp32 MFMA roofline, the slowest node's roofline (per-node HIP events of
    dli.ProfileSession over eager runs), parity against ATen on the CPU, and the ATen CPU forward
    timed on this host."""
    import torch

    import dli
    import dli_alexnet as net

    B = args.batch or 64
    dev = "cuda"
    weights = net.random_weights(seed=0, device=dev)
    g = torch.Generator().manual_seed(1)
    x = torch.randn((B,) + net.IMAGE, generator=g).to(dev)
    engine = dli.Engine().load_plugin()
    graph = net.build_graph(B, fused=True)
    inputs = {"x": x, **weights}
    out = engine.run(graph, inputs)["logits"]
    torch.cuda.synchronize()
    # parity on the benchmark batch: ATen fp32 on the CPU, same inputs
    ref = net.torch_forward(x.cpu(), {k: v.cpu() for k, v in weights.items()})
    rel_err = float((out.cpu() - ref).norm() / ref.norm())
    hip_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hip_graph):
        out = engine.run(graph, inputs)["logits"]
    for _ in range(args.warmup):
        hip_graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        hip_graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    flops = net.flops_per_image() * B
    tflops = flops / (ms * 1e-3) / 1e12

    # slowest node (HIP event pairs per node, eager runs)
    prof = dli.ProfileSession()
    for _ in range(6):
        engine.run(graph, inputs, profile=prof)
    prof.finalize()
    doc = json.loads(prof.to_json())
    per = {}
    for e in doc["events"]:
        if e["run_id"] > 0 and e["gpu_duration_ns"] is not None:
            per.setdefault(e["node_name"], []).append(e["gpu_duration_ns"])
    med = {k: sorted(v)[(len(v) - 1) // 2] for k, v in per.items()}
    node_flops = {}
    hw = net.IMAGE[1] * net.IMAGE[2]
    for i, (cin, cout) in enumerate(net.CONVS):
        node_flops[f"features.conv{i}"] = 2 * B * hw * cout * cin * 9
        if i in net.POOL_AFTER:
            hw //= 4
    for i, (fin, fout) in enumerate(net.FCS):
        node_flops[f"classifier.fc{i}"] = 2 * B * fin * fout
    top = max(med, key=med.get)
    top_tflops = node_flops.get(top, 0) / (med[top] * 1e-9) / 1e12

    cpu = None
    if not args.no_cpu_baseline and args.cpu_baseline_steps > 0:
        xc, wc = x.cpu(), {k: v.cpu() for k, v in weights.items()}
        net.torch_forward(xc, wc)
        t1 = time.perf_counter()
        for _ in range(args.cpu_baseline_steps):
            net.torch_forward(xc, wc)
        cpu_s = (time.perf_counter() - t1) / args.cpu_baseline_steps
        cpu = {"value": round(B / cpu_s, 2), "unit": "images/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{args.cpu_baseline_steps} forwards (after 1 warm-up) of the same "
                         f"batch-{B} network with ATen fp32 CPU ops (the ops the reference's "
                         f"CPU path runs); {cpu_s * 1000:.1f} ms/forward"}
    print(json.dumps({
        "metric": "AlexNet-style fp32 CNN images/s + % fp32 MFMA peak, batch 64",
        "value": round(B / (ms * 1e-3), 1), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "AlexNet-style CNN fp32 forward, batch 64, 3x32x32 input: conv "
                               "64/192/384/256/256 3x3 (fused ReLU), max_pool 2 after conv 1-2, "
                               "FC 4096-4096-10", "global_batch": B,
                   "graph": "dli.graph.v1 forward, HIP-graph replay"},
        "roofline": {"bound": "mfma", "kernel": top, "achieved": round(top_tflops, 2),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(top_tflops / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "avg_us": round(med[top] / 1000, 2), "flops_per_launch": node_flops.get(top)},
        "step_roofline": {"bound": "mfma", "flops_per_step": flops, "achieved": round(tflops, 2),
                          "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4)},
        "node_us": {k: round(v / 1000, 2) for k, v in med.items()},
        "parity": {"relative_l2_vs_aten_cpu": rel_err},
        "cpu_baseline": cpu, "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(0)}), flush=True)


BF16_MFMA_PEAK_TFLOPS = 2500.0


def bench_prefill(args):
    """Config 3: one Qwen2 decoder layer of prefill in bf16 at batch 4 x 2048 tokens (hidden 896,
    14 / 2 heads, head_dim 64, MLP 4864; activations ~N(0, 1), weights ~N(0, 0.02)) as the
    chained dli.graph.v1 prefill graph in its fused form (build_prefill_graph fused=True:
    RMSNorm, q/k/v tiled bf16 MFMA linears, the [B,S,H,D] <-> [B,H,S,D] transposes, RoPE,
    KV-cache append and causal GQA flash attention, o_proj and down_proj with the residual add in
    their GEMM epilogue, gate/up as one GEMM with SwiGLU in its epilogue) through the Engine and
    the gfx950 plugin. One step = one replay of the captured layer; value = 274.4 GFLOP per layer over the
    step time. The per-node GPU times (dli.ProfileSession, eager runs) name the dominant kernel
    for the roofline. CPU baseline: the same graph through the Engine and the ATen CPU reference
    plugin on this host's cores (bf16, one run after one warm-up)."""
    import torch

    import dli
    from dataclasses import replace

    from dli_qwen2 import QWEN2_0_5B, build_prefill_graph, pack_fused_weights, random_weights

    cfg = QWEN2_0_5B
    B, S = args.batch or 4, 2048
    H, Hq, Hkv, D, F = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ffn
    T = B * S
    node_flops = {
        "q_proj": 2 * T * H * Hq * D, "k_proj": 2 * T * H * Hkv * D, "v_proj": 2 * T * H * Hkv * D,
        "attention": 2 * 2 * B * Hq * D * (S * (S + 1) // 2), "o_proj": 2 * T * Hq * D * H,
        "gate_up": 2 * 2 * T * H * F, "down_proj": 2 * T * F * H}
    flops = sum(node_flops.values())
    # the fused layer's one q|k|v GEMM (with RoPE and the head layout in its epilogue)
    node_flops["qkv_rope_heads"] = sum(node_flops[f"{x}_proj"] for x in "qkv")
    w = {k: v for k, v in random_weights(cfg, seed=0, device="cuda").items()
         if k.startswith("model.layers.0.") or k.startswith("rotary")}
    w = pack_fused_weights(replace(cfg, layers=1), w)  # + packed q|k|v and gate/up weights
    g = torch.Generator().manual_seed(1)
    h = torch.randn(B, S, H, generator=g).to(torch.bfloat16).cuda()
    engine = dli.Engine().load_plugin()
    engine.configure_kv_cache(block_size=64, max_seq_len=S)
    # the fused layer (q|k|v with RoPE and the head layout in one GEMM, o_proj and down_proj with
    # their residual adds, gate/up with SwiGLU in one GEMM); the CPU baseline runs the reference's
    # node sequence (same values up to rounding)
    graph = build_prefill_graph(cfg, B, S, layers=1, from_hidden=True, fused=True)
    ref_graph = build_prefill_graph(cfg, B, S, layers=1, from_hidden=True)
    inputs = {**w, "hidden_states": h}

    def run(profile=None):
        engine.set_kv_cache_length(0)  # the prompt starts at position 0 of an empty cache
        return engine.run(graph, inputs, profile=profile)["output"]

    run()
    torch.cuda.synchronize()
    hip_graph = torch.cuda.CUDAGraph()
    engine.set_kv_cache_length(0)
    with torch.cuda.graph(hip_graph):
        engine.run(graph, inputs)
    for _ in range(args.warmup):
        hip_graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        hip_graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    tflops = flops / (ms * 1e-3) / 1e12

    prof = dli.ProfileSession()
    for _ in range(4):
        run(profile=prof)
    prof.finalize()
    doc = json.loads(prof.to_json())
    per = {}
    for e in doc["events"]:
        if e["run_id"] > 0 and e["gpu_duration_ns"] is not None:
            per.setdefault(e["node_name"].rsplit(".", 1)[-1], []).append(e["gpu_duration_ns"])
    med = {k: sorted(v)[(len(v) - 1) // 2] / 1000.0 for k, v in per.items()}
    top = max((k for k in med if k in node_flops), key=med.get)
    top_tflops = node_flops[top] / (med[top] * 1e-6) / 1e12
    nodes = {k: {"us": round(v, 2), "tflops": round(node_flops[k] / (v * 1e-6) / 1e12, 1)
                 if k in node_flops else None} for k, v in sorted(med.items(), key=lambda x: -x[1])}

    cpu = None
    if not args.no_cpu_baseline:
        cores, model = cpu_description()
        torch.set_num_threads(cores)
        cpu_engine = dli.Engine().load_aten_plugin()
        cpu_engine.configure_kv_cache(block_size=64, max_seq_len=S)
        cpu_inputs = {k: v.cpu() for k, v in inputs.items()}
        cpu_engine.set_kv_cache_length(0)
        ref = cpu_engine.run(ref_graph, cpu_inputs)["output"]  # warm-up, and the parity reference
        cpu_engine.set_kv_cache_length(0)
        t1 = time.perf_counter()
        cpu_engine.run(ref_graph, cpu_inputs)
        cpu_s = time.perf_counter() - t1
        got = run().float().cpu()
        rel = float((got - ref.float()).norm() / ref.float().norm())
        cpu = {"value": round(flops / cpu_s / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
               "kind": "port",
               "sample": f"one run (after one warm-up) of the same one-layer prefill graph through "
                         f"the dli Engine + ATen CPU reference plugin, bf16 data with fp32 "
                         f"compute; {cpu_s * 1000:.0f} ms/layer; {cores} cores ({model}); GPU vs "
                         f"CPU output relative L2 {rel:.2e}"}
    print(json.dumps({
        "metric": "Qwen2 decoder-layer prefill bf16 TFLOP/s (chained layer graph)",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"Qwen2 decoder layer prefill, batch {B} x {S} tokens, hidden 896, "
                               "14/2 heads, head_dim 64, MLP 4864, chained dli.graph.v1 layer "
                               "(HIP-graph replay)", "flops_per_layer": flops},
        "roofline": {"bound": "mfma", "kernel": top, "achieved": round(top_tflops, 1),
                     "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(top_tflops / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "avg_us": round(med[top], 2), "flops_per_launch": node_flops[top]},
        "step_roofline": {"bound": "mfma", "flops_per_step": flops, "achieved": round(tflops, 1),
                          "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)},
        "nodes": nodes, "cpu_baseline": cpu, "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(0)}), flush=True)


FP32_LINEAR = (64, 1024, 4096)  # config 1: x [64, 1024], W [4096, 1024], b [4096]


def linear_inputs(seed=0):
    """x ~ N(0, 1); W and b ~ U(-1/32, 1/32) (Kaiming-uniform bound 1/sqrt(1024)); seeded on the
    host, so every device sees the same bits."""
    import torch

    m, k, n = FP32_LINEAR
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    w = torch.rand(n, k, generator=g) * (2 / 32) - 1 / 32
    b = torch.rand(n, generator=g) * (2 / 32) - 1 / 32
    return x, w, b


def bench_linear(args):
    """Config 1, the single fp32 linear layer y = x W^T + b at [64, 1024] x [4096, 1024]^T: the
    gfx950 fp32 MFMA linear (dli_hip_linear_act with its split-K workspace) timed with HIP events
    over --steps launches, against the reference's CPU path on this host: one "aten" node
    (aten::linear through the c10 dispatcher, src/aten_operator.cc:65-106) run by the dli Engine,
    median of >= 20 calls, bit-compared with torch.nn.functional.linear. Roofline: 536,870,912
    flop per call against the fp32 MFMA peak (the call's 18,104,320 bytes take 2.3 us at 8 TB/s,
    its flops 3.4 us at 157.3 TFLOP/s)."""
    import statistics

    import torch
    import torch.nn.functional as F

    import dli
    from dli import hip

    m, k, n = FP32_LINEAR
    flops = 2 * m * n * k
    nbytes = 4 * (m * k + n * k + n + m * n)
    x, w, b = linear_inputs()
    expect = F.linear(x, w, b)
    xd, wd, bd = x.cuda(), w.cuda(), b.cuda()
    out = torch.empty(m, n, device="cuda")
    ws_bytes = hip.lib().dli_hip_linear_workspace(hip.F32, m, n, k)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def launch():
        hip.call("dli_hip_linear_act", hip.F32, hip.F32, xd.data_ptr(), wd.data_ptr(),
                 bd.data_ptr(), out.data_ptr(), m, n, k, 0, ws.data_ptr() if ws_bytes else None,
                 ws_bytes, stream.cuda_stream)

    us = _time_launches(launch, stream, max(args.steps, 20))
    got = out.cpu()
    rel_l2 = float((got - expect).norm() / expect.norm())
    max_abs = float((got - expect).abs().max())
    close = bool(torch.allclose(got, expect, rtol=1e-4, atol=1e-5))
    # the reference's CPU path: Engine + "aten" node
    cores, model = cpu_description()
    torch.set_num_threads(cores)
    engine = dli.Engine()
    graph = dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "single_linear", "inputs": ["x", "w", "b"],
        "outputs": ["y"], "nodes": [{"name": "fc", "op": "aten", "inputs": ["x", "w", "b"],
                                     "outputs": ["y"], "attrs": {"name": "aten::linear"}}]}))
    feeds = {"x": x, "w": w, "b": b}
    y = engine.run(graph, feeds)["y"]
    for _ in range(3):
        engine.run(graph, feeds)
    times = []
    for _ in range(max(args.cpu_baseline_steps, 20)):
        t0 = time.perf_counter()
        engine.run(graph, feeds)
        times.append(time.perf_counter() - t0)
    cpu_us = statistics.median(times) * 1e6
    tflops = flops / (us * 1e-6) / 1e12
    print(json.dumps({
        "metric": "single linear fp32 [64,1024]x[4096,1024]^T+b us/call", "value": round(us, 2),
        "unit": "us/call", "n_gpus": 1, "steps": max(args.steps, 20), "warmup": 5,
        "ms_per_step": round(us / 1000, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "single linear layer fp32, x [64,1024] ~N(0,1), W [4096,1024] and "
                               "b [4096] ~U(-1/32,1/32), y = x W^T + b"},
        "roofline": {"bound": "mfma", "kernel": "dli_hip_linear_act fp32 (16x16x4 f32 MFMA)",
                     "achieved": round(tflops, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": None, "avg_us": round(us, 2), "flops_per_launch": flops,
                     "bytes_per_launch": nbytes},
        "parity": {"relative_l2_vs_torch_cpu": rel_l2, "max_abs_error": max_abs,
                   "allclose_rtol_1e-4_atol_1e-5": close,
                   "cpu_aten_node_bit_identical_to_F_linear": bool(torch.equal(y, expect))},
        "cpu_baseline": {"value": round(cpu_us, 2), "unit": "us/call", "cores": cores,
                         "kind": "port",
                         "sample": f"median of {len(times)} calls after 4 warm-ups: one \"aten\" "
                                   f"node (aten::linear) through the dli Engine on the host; "
                                   f"{cores} cores ({model})"},
        "device": torch.cuda.get_device_name(0)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU decode would be data-parallel by batch: each GPU its own "
                                   "sequences and KV cache, no per-step collective)"}))
        sys.exit(2)
    if args.workload == "alexnet":
        bench_alexnet(args)
        return
    if args.workload == "prefill":
        bench_prefill(args)
        return
    if args.workload == "linear":
        bench_linear(args)
        return

    import torch

    import dli
    from dli import hip
    from dli_qwen2 import QWEN2_0_5B, QWEN2_7B, DecodeSession, random_weights
    from dataclasses import replace

    large = args.model == "7b"
    base = QWEN2_7B if large else QWEN2_0_5B
    cfg = base if args.layers is None else replace(base, layers=args.layers)
    B = args.batch or (64 if large else 32)
    ctx = args.context or (8192 if large else 4096)
    from dli_qwen2.graph import DEFAULT_SPLITS, STACK_SPLITS, large_splits

    graph_kind = "large" if large else args.graph
    splits = dict({"stack": STACK_SPLITS, "fused": DEFAULT_SPLITS,
                   "large": large_splits(B)}[graph_kind])
    if args.splits:
        splits.update({k: int(v) for k, v in (item.split("=") for item in args.splits.split(","))})
    dev = "cuda"
    torch.manual_seed(0)
    weights = random_weights(cfg, seed=0, device=dev)
    session = DecodeSession(cfg, weights, batch=B, max_seq_len=ctx + 64, fused=True,
                            splits=splits, logits_dtype="bfloat16", stack=args.graph == "stack")
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, cfg.vocab, (B,), generator=g, device=dev)
    pos = torch.full((B,), ctx - 1, dtype=torch.int64, device=dev)
    session.ids.copy_(ids)
    session.positions.copy_(pos)
    session.run_eager()  # reserves the paged caches
    torch.cuda.synchronize()
    # seeded synthetic context: positions [0, ctx-1) of every layer's K/V pools
    for i in range(cfg.layers):
        e = session.engine.kv_cache_entry(f"layer_{i}")
        for pool in (e["key_pool"], e["value_pool"]):
            pool.copy_(torch.randn(pool.shape, generator=g, device=dev, dtype=torch.float32)
                       .to(pool.dtype))
    torch.cuda.synchronize()
    # Graph mode: one captured graph holds `spg` chained greedy steps (each step reads the
    # previous step's next_ids, every step at the same position: the steady state of a context
    # of ctx tokens), so a replay is spg steps and the ~8 us a graph launch costs, and the copy
    # that chains one replay's tokens into the next, are paid once per spg steps.
    spg = 1
    if not args.eager:
        spg = args.steps_per_graph or next(
            k for k in (5, 4, 2, 1) if args.steps % k == 0 and args.warmup % k == 0)
        if spg < 1 or args.steps % spg or args.warmup % spg:
            raise SystemExit("--steps and --warmup must be multiples of --steps-per-graph")
        session.capture(chain_ids=True, steps=spg)  # each replay feeds its tokens to the next

    def one_step():  # spg steps
        if args.eager:
            out = session.run_eager()
            session.ids.copy_(out["next_ids"])
            return out
        return session.replay()

    for _ in range(args.warmup // spg):
        one_step()
    torch.cuda.synchronize()
    session.check_status()  # a decoder_stack wait that gave up invalidates the steps: exit non-zero
    stream = torch.cuda.current_stream()
    start_ev, stop_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start_ev.record(stream)
    for _ in range(args.steps // spg):
        one_step()
    stop_ev.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    session.check_status()
    ms_per_step = start_ev.elapsed_time(stop_ev) / args.steps
    tok_s = B * 1000.0 / ms_per_step
    total, w_bytes, kv_read, kv_write, logit_bytes = step_bytes(cfg, B, ctx)
    total += logit_bytes
    step_gbs = total / (ms_per_step * 1e-3) / 1e9

    if graph_kind == "stack":
        kernel, dom_us, dom_bytes = time_decoder_stack(session, cfg, B, ctx, pos, g, stream, hip,
                                                       splits["down"])
    else:
        kernel, dom_us, dom_bytes = time_decode_attention(session, cfg, B, ctx, pos, g, stream, hip)
    dom_gbs = dom_bytes / (dom_us * 1e-6) / 1e9

    if args.profile:
        prof_session = dli.ProfileSession()
        for _ in range(args.profile_steps):
            session.run_eager(profile=prof_session)
        prof_session.finalize()
        prof_session.write_json(args.profile)
        del prof_session

    if args.calibration_copy_mib > 0:
        src = torch.empty(args.calibration_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if not args.no_cpu_baseline and args.cpu_baseline_steps > 0 and not large:
        cpu = cpu_engine_decode_baseline(cfg, weights, B, ctx, ids, args.cpu_baseline_steps,
                                         args.cpu_baseline_warmup)

    graph_desc = {"stack": "decoder_stack (one persistent launch for the embedding gather and "
                           "all layers) + lm_head_argmax + argmax_finalize",
                  "fused": "fused (five launches per layer)",
                  "large": "large-hidden graph (per layer: q|k|v + RoPE + KV append, "
                           "head_dim-128 MFMA decode attention, o_proj and down_proj each with "
                           "their residual add and the RMSNorm after it, gate_up + SwiGLU)"}[graph_kind]
    shape = "Qwen2-7B" if large else "Qwen2-0.5B"
    result = {
        # the headline metric names its batch and context; other decode sizes name theirs
        "metric": (METRIC_7B if large else METRIC) if (B, ctx) == ((64, 8192) if large else (32, 4096))
        else f"decode tok/s + % HBM roofline, {shape}-shape bf16 b={B} ctx{ctx}",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{shape}-shape bf16 greedy decode, batch {B}, context {ctx}",
                   "model": f"{shape.lower()}-shape (random init)", "global_batch": B,
                   "seq_len": ctx, "layers": cfg.layers, "parallelism": "none (1 GPU)",
                   "graph": graph_desc + " dli.graph.v1 decode step, "
                            + ("eager" if args.eager else
                               f"HIP-graph replay, {spg} chained steps per captured graph"),
                   "steps_per_graph": spg, "splits": splits},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(graph_kind, B, ctx),
                     "avg_us": round(dom_us, 2), "bytes_per_launch": dom_bytes},
        "step_roofline": {"bound": "hbm", "bytes_per_step": total, "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                          "bytes": {"weights": w_bytes, "kv_read": kv_read, "kv_write": kv_write,
                                    "logits_bf16": logit_bytes}},
        "cpu_baseline": cpu if not large else {
            "value": None, "unit": "tok/s", "cores": None, "kind": "port",
            "sample": "not run for this shape: one host step would hold 30 GB of fp32 weights "
                      "and a 60 GB fp32 cache; the 0.5B line carries the Engine + ATen CPU "
                      "baseline"},
        "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
