"""dli.graph.v1 builders for one Qwen2 decode step (one new token per sequence).

reference-style graph (fused=False): the node sequence of the reference exporter
(python/dli_export/export.py:272-446; 19 nodes per layer) with the extensions a batched decode
needs — a `positions` input feeding rotary_embedding (5th input) and attention (4th input),
grouped KV heads, fp32 logits and an `argmax` node.

fused graph (fused=True): 5 launches per layer on the fused operators of the gfx950 plugin
(qkv_rope_append and gate_up_silu with their RMSNorm inside, paged_attention, and
linear_residual for o_proj and for down_proj), then one lm_head_argmax node that also applies
model.norm.
Same rounding points, same tensor names for inputs and outputs.

stack graph (fused=True, stack=True): the embedding and the decoder layers of the fused graph
as one decoder_stack node (one persistent launch for all layers, which gathers the token rows of
the embedding table itself), bit-identical to the fused graph. It
has a third output, `status` (int32 [1], the launch status the decoder_stack node accumulates:
non-zero when a wait in the persistent launch gave up and the step's outputs are invalid), which
the decode drivers check where they synchronize anyway.
"""
from __future__ import annotations

import json

import torch

import dli

from .config import Qwen2Config

INPUTS = ["input_ids", "positions"]
OUTPUTS = ["logits", "next_ids"]


def _node(nodes, name, op, inputs, outputs, attrs=None):
    nodes.append({"name": name, "op": op, "inputs": list(inputs), "outputs": list(outputs),
                  "attrs": attrs or {}})


def _reference_nodes(cfg: Qwen2Config, batch: int, nodes: list):
    h = "hidden_states"
    q_w = cfg.heads * cfg.head_dim
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        t = f"layers_{i}"
        _node(nodes, f"{p}.input_layernorm", "rms_norm", [h, f"{p}.input_layernorm.weight"],
              [f"{t}_input_norm"], {"eps": cfg.eps})
        for proj in ("q", "k", "v"):
            _node(nodes, f"{p}.self_attn.{proj}_proj", "linear",
                  [f"{t}_input_norm", f"{p}.self_attn.{proj}_proj.weight", f"{p}.self_attn.{proj}_proj.bias"],
                  [f"{t}_{proj}"])
        _node(nodes, f"{p}.self_attn.q_reshape", "reshape", [f"{t}_q"], [f"{t}_q_heads"],
              {"shape": [batch, cfg.heads, 1, cfg.head_dim]})
        _node(nodes, f"{p}.self_attn.k_reshape", "reshape", [f"{t}_k"], [f"{t}_k_heads"],
              {"shape": [batch, cfg.kv_heads, 1, cfg.head_dim]})
        _node(nodes, f"{p}.self_attn.v_reshape", "reshape", [f"{t}_v"], [f"{t}_v_heads"],
              {"shape": [batch, cfg.kv_heads, 1, cfg.head_dim]})
        _node(nodes, f"{p}.self_attn.rotary_embedding", "rotary_embedding",
              [f"{t}_q_heads", f"{t}_k_heads", "rotary_cos", "rotary_sin", "positions"],
              [f"{t}_q_rotary", f"{t}_k_rotary"])
        _node(nodes, f"{p}.self_attn.attention", "attention",
              [f"{t}_q_rotary", f"{t}_k_rotary", f"{t}_v_heads", "positions"], [f"{t}_attention"],
              {"causal": True, "kv_cache": f"layer_{i}"})
        _node(nodes, f"{p}.self_attn.merge", "reshape", [f"{t}_attention"], [f"{t}_attention_merged"],
              {"shape": [batch, q_w]})
        _node(nodes, f"{p}.self_attn.o_proj", "linear",
              [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight"], [f"{t}_attention_proj"])
        _node(nodes, f"{p}.attention_residual", "add", [h, f"{t}_attention_proj"], [f"{t}_after_attention"])
        _node(nodes, f"{p}.post_attention_layernorm", "rms_norm",
              [f"{t}_after_attention", f"{p}.post_attention_layernorm.weight"],
              [f"{t}_post_attention_norm"], {"eps": cfg.eps})
        _node(nodes, f"{p}.mlp.gate_proj", "linear",
              [f"{t}_post_attention_norm", f"{p}.mlp.gate_proj.weight"], [f"{t}_gate"])
        _node(nodes, f"{p}.mlp.up_proj", "linear",
              [f"{t}_post_attention_norm", f"{p}.mlp.up_proj.weight"], [f"{t}_up"])
        _node(nodes, f"{p}.mlp.act_fn", "silu", [f"{t}_gate"], [f"{t}_silu"])
        _node(nodes, f"{p}.mlp.mul", "mul", [f"{t}_silu", f"{t}_up"], [f"{t}_gated"])
        _node(nodes, f"{p}.mlp.down_proj", "linear", [f"{t}_gated", f"{p}.mlp.down_proj.weight"],
              [f"{t}_mlp_down"])
        _node(nodes, f"{p}.mlp_residual", "add", [f"{t}_after_attention", f"{t}_mlp_down"], [f"{t}_output"])
        h = f"{t}_output"
    _node(nodes, "model.norm", "rms_norm", [h, "model.norm.weight"], ["norm_hidden"], {"eps": cfg.eps})
    _node(nodes, "lm_head", "linear", ["norm_hidden", "lm_head.weight"], ["logits"],
          {"out_dtype": "float32"})
    _node(nodes, "greedy", "argmax", ["logits"], ["next_ids"])


def _large_nodes(cfg: Qwen2Config, batch: int, nodes: list, splits: dict, fused: bool = False):
    """Decode step for hidden sizes the fused norm-prologue kernels do not hold in registers
    (hidden > 1024, e.g. the Qwen2-7B shape). Attention over the paged cache runs on the MFMA
    decode kernel for head_dim 64 or 128.
    fused=False: the reference node sequence with o_proj and down_proj each fused with their
    residual add (linear_residual), which the ATen CPU plugin also runs.
    fused=True (the GPU plugin's operators, same rounding points): per layer
    qkv_rope_append (q|k|v projection over the packed self_attn.qkv_proj.{weight,bias}, bias,
    RoPE, q out, k and v into the cache) -> paged_attention -> linear_residual_norm (o_proj +
    residual + post_attention_layernorm) -> gate_up_silu (over the interleaved
    mlp.gate_up_proj.weight) -> linear_residual_norm (down_proj + residual + the next layer's
    input_layernorm, or model.norm after the last layer); the first layer's input_layernorm is
    one rms_norm node (pack_large_weights packs the weights)."""
    h = "hidden_states"
    q_w = cfg.heads * cfg.head_dim
    if fused:
        _node(nodes, "model.layers.0.input_layernorm", "rms_norm",
              [h, "model.layers.0.input_layernorm.weight"], ["layers_0_input_norm"],
              {"eps": cfg.eps})
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        t = f"layers_{i}"
        if fused:
            last = i + 1 == cfg.layers
            next_norm = "model.norm.weight" if last else \
                f"model.layers.{i + 1}.input_layernorm.weight"
            next_xn = "norm_hidden" if last else f"layers_{i + 1}_input_norm"
            _node(nodes, f"{p}.self_attn.qkv_rope_append", "qkv_rope_append",
                  [f"{t}_input_norm", f"{p}.self_attn.qkv_proj.weight",
                   f"{p}.self_attn.qkv_proj.bias", "rotary_cos", "rotary_sin", "positions"],
                  [f"{t}_q_rotary"],
                  {"kv_cache": f"layer_{i}", "q_heads": cfg.heads, "kv_heads": cfg.kv_heads,
                   "head_dim": cfg.head_dim, "eps": cfg.eps})
            _node(nodes, f"{p}.self_attn.attention", "paged_attention",
                  [f"{t}_q_rotary", "positions"], [f"{t}_attention"],
                  {"kv_cache": f"layer_{i}", "attention_splits": splits.get("attn", 0)})
            _node(nodes, f"{p}.self_attn.merge", "reshape", [f"{t}_attention"],
                  [f"{t}_attention_merged"], {"shape": [batch, q_w]})
            _node(nodes, f"{p}.self_attn.o_proj", "linear_residual_norm",
                  [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight", h,
                   f"{p}.post_attention_layernorm.weight"],
                  [f"{t}_after_attention", f"{t}_post_attention_norm"],
                  {"splits": splits.get("o", 1), "eps": cfg.eps})
            _node(nodes, f"{p}.mlp.gate_up", "gate_up_silu",
                  [f"{t}_post_attention_norm", f"{p}.mlp.gate_up_proj.weight"], [f"{t}_gated"])
            _node(nodes, f"{p}.mlp.down_proj", "linear_residual_norm",
                  [f"{t}_gated", f"{p}.mlp.down_proj.weight", f"{t}_after_attention", next_norm],
                  [f"{t}_output", next_xn], {"splits": splits.get("down", 1), "eps": cfg.eps})
            h = f"{t}_output"
            continue
        _node(nodes, f"{p}.input_layernorm", "rms_norm", [h, f"{p}.input_layernorm.weight"],
              [f"{t}_input_norm"], {"eps": cfg.eps})
        for proj, heads in (("q", cfg.heads), ("k", cfg.kv_heads), ("v", cfg.kv_heads)):
            _node(nodes, f"{p}.self_attn.{proj}_proj", "linear",
                  [f"{t}_input_norm", f"{p}.self_attn.{proj}_proj.weight",
                   f"{p}.self_attn.{proj}_proj.bias"], [f"{t}_{proj}"])
            _node(nodes, f"{p}.self_attn.{proj}_reshape", "reshape", [f"{t}_{proj}"],
                  [f"{t}_{proj}_heads"], {"shape": [batch, heads, 1, cfg.head_dim]})
        _node(nodes, f"{p}.self_attn.rotary_embedding", "rotary_embedding",
              [f"{t}_q_heads", f"{t}_k_heads", "rotary_cos", "rotary_sin", "positions"],
              [f"{t}_q_rotary", f"{t}_k_rotary"])
        _node(nodes, f"{p}.self_attn.attention", "attention",
              [f"{t}_q_rotary", f"{t}_k_rotary", f"{t}_v_heads", "positions"], [f"{t}_attention"],
              {"causal": True, "kv_cache": f"layer_{i}"})
        _node(nodes, f"{p}.self_attn.merge", "reshape", [f"{t}_attention"],
              [f"{t}_attention_merged"], {"shape": [batch, q_w]})
        _node(nodes, f"{p}.self_attn.o_proj", "linear_residual",
              [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight", h],
              [f"{t}_after_attention"], {"splits": splits.get("o", 1)})
        _node(nodes, f"{p}.post_attention_layernorm", "rms_norm",
              [f"{t}_after_attention", f"{p}.post_attention_layernorm.weight"],
              [f"{t}_post_attention_norm"], {"eps": cfg.eps})
        _node(nodes, f"{p}.mlp.gate_proj", "linear",
              [f"{t}_post_attention_norm", f"{p}.mlp.gate_proj.weight"], [f"{t}_gate"])
        _node(nodes, f"{p}.mlp.up_proj", "linear",
              [f"{t}_post_attention_norm", f"{p}.mlp.up_proj.weight"], [f"{t}_up"])
        _node(nodes, f"{p}.mlp.act_fn", "silu", [f"{t}_gate"], [f"{t}_silu"])
        _node(nodes, f"{p}.mlp.mul", "mul", [f"{t}_silu", f"{t}_up"], [f"{t}_gated"])
        _node(nodes, f"{p}.mlp.down_proj", "linear_residual",
              [f"{t}_gated", f"{p}.mlp.down_proj.weight", f"{t}_after_attention"],
              [f"{t}_output"], {"splits": splits.get("down", 1)})
        h = f"{t}_output"
    if not fused:
        _node(nodes, "model.norm", "rms_norm", [h, "model.norm.weight"], ["norm_hidden"],
              {"eps": cfg.eps})
    _node(nodes, "lm_head", "linear", ["norm_hidden", "lm_head.weight"], ["logits"],
          {"out_dtype": "float32"})
    _node(nodes, "greedy", "argmax", ["logits"], ["next_ids"])


def _fused_nodes(cfg: Qwen2Config, batch: int, nodes: list, splits: dict, logits_dtype: str):
    h = "hidden_states"
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        t = f"layers_{i}"
        _node(nodes, f"{p}.self_attn.qkv_rope_append", "qkv_rope_append",
              [h, f"{p}.input_layernorm.weight", f"{p}.self_attn.qkv_proj.weight",
               f"{p}.self_attn.qkv_proj.bias", "rotary_cos", "rotary_sin", "positions"],
              [f"{t}_q_rotary"],
              {"kv_cache": f"layer_{i}", "q_heads": cfg.heads, "kv_heads": cfg.kv_heads,
               "head_dim": cfg.head_dim, "eps": cfg.eps})
        _node(nodes, f"{p}.self_attn.attention", "paged_attention", [f"{t}_q_rotary", "positions"],
              [f"{t}_attention"],
              {"kv_cache": f"layer_{i}", "attention_splits": splits.get("attn", 0)})
        _node(nodes, f"{p}.self_attn.merge", "reshape", [f"{t}_attention"], [f"{t}_attention_merged"],
              {"shape": [batch, cfg.heads * cfg.head_dim]})
        _node(nodes, f"{p}.self_attn.o_proj", "linear_residual",
              [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight", h],
              [f"{t}_after_attention"], {"splits": splits.get("o", 1)})
        _node(nodes, f"{p}.mlp.gate_up", "gate_up_silu",
              [f"{t}_after_attention", f"{p}.post_attention_layernorm.weight",
               f"{p}.mlp.gate_up_proj.weight"], [f"{t}_gated"], {"eps": cfg.eps})
        _node(nodes, f"{p}.mlp.down_proj", "linear_residual",
              [f"{t}_gated", f"{p}.mlp.down_proj.weight", f"{t}_after_attention"],
              [f"{t}_output"], {"splits": splits.get("down", 1)})
        h = f"{t}_output"
    _head_nodes(cfg, nodes, h, logits_dtype)


def _head_nodes(cfg: Qwen2Config, nodes: list, h: str, logits_dtype: str):
    """model.norm + lm_head + greedy choice as one lm_head_argmax node: the final RMSNorm runs
    in registers inside the lm_head kernel (its third input is model.norm's weight)."""
    _node(nodes, "lm_head", "lm_head_argmax", [h, "lm_head.weight", "model.norm.weight"], OUTPUTS,
          {"logits_dtype": logits_dtype, "eps": cfg.eps})


def _stack_nodes(cfg: Qwen2Config, nodes: list, splits: dict, logits_dtype: str,
                 check_status: bool = False, stack_trace: bool = False):
    """Every decoder layer in one decoder_stack node (one persistent launch), then the head
    (model.norm inside lm_head_argmax) as in the fused graph. Same rounding points and values as
    the fused graph with o split 1 and the same attention split count (splits["attn"], 0 = each
    path's own choice). stack_trace: the node also reads graph input "stack_trace", an int64
    buffer that receives the launch's stage timeline. The node takes the token ids and the
    embedding table itself (model.embed_tokens folded into the launch: no embedding node)."""
    inputs = ["input_ids", "positions", "rotary_cos", "rotary_sin"]
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        inputs += [f"{p}.input_layernorm.weight", f"{p}.self_attn.qkv_proj.weight",
                   f"{p}.self_attn.qkv_proj.bias", f"{p}.self_attn.o_proj.weight",
                   f"{p}.post_attention_layernorm.weight", f"{p}.mlp.gate_up_proj.weight",
                   f"{p}.mlp.down_proj.weight"]
    inputs.append("model.embed_tokens.weight")
    if stack_trace:
        inputs.append("stack_trace")
    _node(nodes, "model.layers", "decoder_stack", inputs, ["layers_output", "status"],
          {"layers": cfg.layers, "q_heads": cfg.heads, "kv_heads": cfg.kv_heads,
           "head_dim": cfg.head_dim, "eps": cfg.eps,
           "down_splits": splits.get("down", STACK_SPLITS["down"]),
           "attention_splits": splits.get("attn", 0),
           "kv_cache_prefix": "layer_", "check_status": int(check_status)})
    _head_nodes(cfg, nodes, "layers_output", logits_dtype)


# split-K per projection (down_proj's K over 4 workgroups per tile in the fused graph, 3 in the
# decoder stack, whose q|k|v workgroups take no down_proj unit)
DEFAULT_SPLITS = {"o": 1, "down": 4}
STACK_SPLITS = {"o": 1, "down": 3}
# K splits of o_proj and down_proj in the large-hidden graph. From 9 rows they run on the tiled
# MFMA GEMM, which splits K into the node's workspace as far as these counts size it (it picks 4
# for both at hidden 3584); up to 8 rows the skinny split-K kernels take them (at most 8).
LARGE_SPLITS = {"o": 1, "down": 2}
LARGE_SPLITS_TILED = {"o": 4, "down": 4}


def large_splits(batch: int) -> dict:
    return dict(LARGE_SPLITS_TILED if batch > 8 else LARGE_SPLITS)
FUSED_MAX_HIDDEN = 1024  # the fused kernels keep a tile's activation rows in registers


def uses_large_graph(cfg: Qwen2Config, fused: bool) -> bool:
    """True when a fused decode graph is requested for a hidden size above what the fused
    kernels hold (the step is then the large-hidden graph, _large_nodes)."""
    return fused and cfg.hidden > FUSED_MAX_HIDDEN


def build_decode_graph(cfg: Qwen2Config, batch: int, fused: bool = True,
                       splits: dict | None = None, logits_dtype: str = "float32",
                       stack: bool = False, check_status: bool = False,
                       large_fused: bool = False, stack_trace: bool = False) -> "dli.Graph":
    """fused=False: the reference's node sequence; fused=True: five launches per layer;
    stack=True (with fused): all layers in one decoder_stack node (check_status: the node waits
    for its launch and fails if a workgroup gave up waiting; for tests, not for capture). With
    fused=True and a hidden size above 1024 (the Qwen2-7B shape) the step is the large-hidden
    graph instead (_large_nodes; large_fused selects its GPU form), whatever `stack` says.
    splits: {"o", "down": K splits, "attn": attention key-range splits, 0 = each call's own
    choice}; stack_trace: the decoder_stack node records its stage timeline into graph input
    "stack_trace" (int64, layers x CUs x 24)."""
    nodes: list = []
    if not (fused and stack) or uses_large_graph(cfg, fused):  # the stack gathers it itself
        _node(nodes, "model.embed_tokens", "embedding", ["input_ids", "model.embed_tokens.weight"],
              ["hidden_states"])
    if uses_large_graph(cfg, fused):
        _large_nodes(cfg, batch, nodes, splits or large_splits(batch), large_fused)
        graph = {"format": "dli.graph.v1", "model_type": "qwen2_decode_large",
                 "inputs": INPUTS, "outputs": OUTPUTS, "nodes": nodes}
        return dli.Graph.from_json(json.dumps(graph))
    if fused and stack:
        _stack_nodes(cfg, nodes, splits or STACK_SPLITS, logits_dtype, check_status, stack_trace)
    elif fused:
        _fused_nodes(cfg, batch, nodes, splits or DEFAULT_SPLITS, logits_dtype)
    else:
        _reference_nodes(cfg, batch, nodes)
    model_type = "qwen2_decode" if not fused else ("qwen2_decode_stack" if stack else "qwen2_decode_fused")
    outputs = OUTPUTS + ["status"] if fused and stack else OUTPUTS
    inputs = INPUTS + ["stack_trace"] if fused and stack and stack_trace else INPUTS
    graph = {"format": "dli.graph.v1", "model_type": model_type,
             "inputs": inputs, "outputs": outputs, "nodes": nodes}
    return dli.Graph.from_json(json.dumps(graph))


def _prefill_layer_nodes(cfg: Qwen2Config, batch: int, seq: int, i: int, h: str, nodes: list,
                         fused: bool = False) -> str:
    """One decoder layer over [B, S, H] activations (the exporter's node sequence,
    python/dli_export/export.py:272-424, with the [B, S, H, D] <-> [B, H, S, D] transposes a
    prompt of S tokens needs around rotary and attention). With fused, q/k/v_proj, their
    reshapes and transposes and rotary_embedding are one qkv_rope_heads node over the packed
    self_attn.qkv_proj.{weight,bias}, attention writes [B, S, H, D] itself (output_layout
    "bshd", no transpose node), o_proj + residual and
    down_proj + residual are linear_residual nodes and gate_proj, up_proj, act_fn and mul one
    gate_up_silu node over the interleaved mlp.gate_up_proj.weight (pack_fused_weights): the
    same values (each fused kernel rounds where the nodes it replaces round). Returns the layer's
    output name."""
    p, t = f"model.layers.{i}", f"layers_{i}"
    q_w = cfg.heads * cfg.head_dim
    _node(nodes, f"{p}.input_layernorm", "rms_norm", [h, f"{p}.input_layernorm.weight"],
          [f"{t}_input_norm"], {"eps": cfg.eps})
    if fused:
        _node(nodes, f"{p}.self_attn.qkv_rope_heads", "qkv_rope_heads",
              [f"{t}_input_norm", f"{p}.self_attn.qkv_proj.weight",
               f"{p}.self_attn.qkv_proj.bias", "rotary_cos", "rotary_sin"],
              [f"{t}_q_rotary", f"{t}_k_rotary", f"{t}_v_heads"],
              {"q_heads": cfg.heads, "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
               "start_pos": 0})
    else:
        for proj in ("q", "k", "v"):
            _node(nodes, f"{p}.self_attn.{proj}_proj", "linear",
                  [f"{t}_input_norm", f"{p}.self_attn.{proj}_proj.weight",
                   f"{p}.self_attn.{proj}_proj.bias"], [f"{t}_{proj}"])
        for proj, heads in (("q", cfg.heads), ("k", cfg.kv_heads), ("v", cfg.kv_heads)):
            _node(nodes, f"{p}.self_attn.{proj}_reshape", "reshape", [f"{t}_{proj}"],
                  [f"{t}_{proj}_bshd"], {"shape": [batch, seq, heads, cfg.head_dim]})
            _node(nodes, f"{p}.self_attn.{proj}_transpose", "transpose", [f"{t}_{proj}_bshd"],
                  [f"{t}_{proj}_heads"], {"perm": [0, 2, 1, 3]})
        _node(nodes, f"{p}.self_attn.rotary_embedding", "rotary_embedding",
              [f"{t}_q_heads", f"{t}_k_heads", "rotary_cos", "rotary_sin"],
              [f"{t}_q_rotary", f"{t}_k_rotary"], {"start_pos": 0})
    if fused:  # the attention kernel writes [B, S, H, D] itself
        _node(nodes, f"{p}.self_attn.attention", "attention",
              [f"{t}_q_rotary", f"{t}_k_rotary", f"{t}_v_heads"], [f"{t}_attention_bshd"],
              {"causal": True, "kv_cache": f"layer_{i}", "output_layout": "bshd"})
    else:
        _node(nodes, f"{p}.self_attn.attention", "attention",
              [f"{t}_q_rotary", f"{t}_k_rotary", f"{t}_v_heads"], [f"{t}_attention"],
              {"causal": True, "kv_cache": f"layer_{i}"})
        _node(nodes, f"{p}.self_attn.attention_transpose", "transpose", [f"{t}_attention"],
              [f"{t}_attention_bshd"], {"perm": [0, 2, 1, 3]})
    _node(nodes, f"{p}.self_attn.merge", "reshape", [f"{t}_attention_bshd"],
          [f"{t}_attention_merged"], {"shape": [batch, seq, q_w]})
    if fused:
        _node(nodes, f"{p}.self_attn.o_proj", "linear_residual",
              [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight", h],
              [f"{t}_after_attention"])
    else:
        _node(nodes, f"{p}.self_attn.o_proj", "linear",
              [f"{t}_attention_merged", f"{p}.self_attn.o_proj.weight"], [f"{t}_attention_proj"])
        _node(nodes, f"{p}.attention_residual", "add", [h, f"{t}_attention_proj"],
              [f"{t}_after_attention"])
    _node(nodes, f"{p}.post_attention_layernorm", "rms_norm",
          [f"{t}_after_attention", f"{p}.post_attention_layernorm.weight"],
          [f"{t}_post_attention_norm"], {"eps": cfg.eps})
    if fused:
        _node(nodes, f"{p}.mlp.gate_up", "gate_up_silu",
              [f"{t}_post_attention_norm", f"{p}.mlp.gate_up_proj.weight"], [f"{t}_gated"])
        _node(nodes, f"{p}.mlp.down_proj", "linear_residual",
              [f"{t}_gated", f"{p}.mlp.down_proj.weight", f"{t}_after_attention"],
              [f"{t}_output"])
        return f"{t}_output"
    _node(nodes, f"{p}.mlp.gate_proj", "linear",
          [f"{t}_post_attention_norm", f"{p}.mlp.gate_proj.weight"], [f"{t}_gate"])
    _node(nodes, f"{p}.mlp.up_proj", "linear",
          [f"{t}_post_attention_norm", f"{p}.mlp.up_proj.weight"], [f"{t}_up"])
    _node(nodes, f"{p}.mlp.act_fn", "silu", [f"{t}_gate"], [f"{t}_silu"])
    _node(nodes, f"{p}.mlp.mul", "mul", [f"{t}_silu", f"{t}_up"], [f"{t}_gated"])
    _node(nodes, f"{p}.mlp.down_proj", "linear", [f"{t}_gated", f"{p}.mlp.down_proj.weight"],
          [f"{t}_mlp_down"])
    _node(nodes, f"{p}.mlp_residual", "add", [f"{t}_after_attention", f"{t}_mlp_down"],
          [f"{t}_output"])
    return f"{t}_output"


def build_prefill_graph(cfg: Qwen2Config, batch: int, seq: int, layers: int | None = None,
                        from_hidden: bool = False, fused_head: bool = True,
                        fused: bool = False) -> "dli.Graph":
    """Prefill of a `seq`-token prompt per sequence (every sequence starts at position 0 of an
    empty KV cache; the cache entries layer_0.. are filled with the prompt's keys and values, so
    decode-step graphs continue at position `seq`).

    from_hidden=False: input_ids int64 [B, S] -> embedding -> the decoder layers -> the last
    token's hidden state (an "aten" select node) -> model.norm + lm_head + greedy choice
    (lm_head_argmax; with fused_head=False the reference's rms_norm, linear and argmax nodes);
    outputs logits [B, V] and next_ids [B] (the first generated token).
    from_hidden=True: hidden_states [B, S, H] -> the decoder layers (the first `layers`) ->
    output hidden [B, S, H] (one decoder layer of prefill, the config-3 workload).
    fused: the layers' fused form (_prefill_layer_nodes), which reads mlp.gate_up_proj.weight."""
    n_layers = cfg.layers if layers is None else layers
    nodes: list = []
    h = "hidden_states"
    if not from_hidden:
        _node(nodes, "model.embed_tokens", "embedding",
              ["input_ids", "model.embed_tokens.weight"], [h])
    for i in range(n_layers):
        h = _prefill_layer_nodes(cfg, batch, seq, i, h, nodes, fused)
    if from_hidden:
        _node(nodes, "output", "reshape", [h], ["output"], {"shape": [batch, seq, cfg.hidden]})
        graph = {"format": "dli.graph.v1", "model_type": "qwen2_prefill_layers",
                 "inputs": ["hidden_states"], "outputs": ["output"], "nodes": nodes}
        return dli.Graph.from_json(json.dumps(graph))
    _node(nodes, "last_token", "aten", [h], ["last_hidden"],
          {"name": "aten::select", "overload": "int", "dim": 1, "index": seq - 1,
           "attr_order": ["dim", "index"]})
    if fused_head:
        _head_nodes(cfg, nodes, "last_hidden", "float32")
    else:
        _node(nodes, "model.norm", "rms_norm", ["last_hidden", "model.norm.weight"],
              ["norm_hidden"], {"eps": cfg.eps})
        _node(nodes, "lm_head", "linear", ["norm_hidden", "lm_head.weight"], ["logits"],
              {"out_dtype": "float32"})
        _node(nodes, "greedy", "argmax", ["logits"], ["next_ids"])
    graph = {"format": "dli.graph.v1", "model_type": "qwen2_prefill",
             "inputs": ["input_ids"], "outputs": OUTPUTS, "nodes": nodes}
    return dli.Graph.from_json(json.dumps(graph))


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor, block: int = 16) -> torch.Tensor:
    """[F, H] x 2 -> [2F, H]: rows [2*block*i, +block) gate block i, then up block i."""
    f, hsz = gate.shape
    g = gate.reshape(f // block, block, hsz)
    u = up.reshape(f // block, block, hsz)
    return torch.stack([g, u], dim=1).reshape(2 * f, hsz).contiguous()


def pack_large_weights(cfg: Qwen2Config, weights: dict) -> dict:
    """The packed tensors of the large-hidden graph's GPU form, in place of the ones they join:
    self_attn.qkv_proj.{weight,bias} ([q|k|v] rows) and mlp.gate_up_proj.weight (16-row
    interleave of gate and up)."""
    out = dict(weights)
    for i in range(cfg.layers):
        a = f"model.layers.{i}.self_attn"
        out[f"{a}.qkv_proj.weight"] = torch.cat(
            [out.pop(f"{a}.{x}_proj.weight") for x in "qkv"], 0).contiguous()
        out[f"{a}.qkv_proj.bias"] = torch.cat(
            [out.pop(f"{a}.{x}_proj.bias") for x in "qkv"], 0).contiguous()
        p = f"model.layers.{i}.mlp"
        out[f"{p}.gate_up_proj.weight"] = interleave_gate_up(out.pop(f"{p}.gate_proj.weight"),
                                                              out.pop(f"{p}.up_proj.weight"))
    return out


def pack_fused_weights(cfg: Qwen2Config, weights: dict, drop_unfused: bool = False) -> dict:
    """Adds the packed tensors the fused graph reads: qkv_proj.{weight,bias} ([q|k|v] rows) and
    mlp.gate_up_proj.weight (16-row interleave)."""
    out = dict(weights)
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        a = f"{p}.self_attn"
        out[f"{a}.qkv_proj.weight"] = torch.cat(
            [weights[f"{a}.{x}_proj.weight"] for x in "qkv"], 0).contiguous()
        out[f"{a}.qkv_proj.bias"] = torch.cat([weights[f"{a}.{x}_proj.bias"] for x in "qkv"], 0).contiguous()
        out[f"{p}.mlp.gate_up_proj.weight"] = interleave_gate_up(
            weights[f"{p}.mlp.gate_proj.weight"], weights[f"{p}.mlp.up_proj.weight"])
        if drop_unfused:
            for x in "qkv":
                out.pop(f"{a}.{x}_proj.weight")
                out.pop(f"{a}.{x}_proj.bias")
            out.pop(f"{p}.mlp.gate_proj.weight")
            out.pop(f"{p}.mlp.up_proj.weight")
    return out
