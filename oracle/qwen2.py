"""Qwen2 decoder oracle on the CPU (test infrastructure; see oracle/__init__.py).

torch float32 on the CPU with the bf16 rounding points of the dli.graph.v1 decode graph
(every node's output is rounded to bf16, except the fp32 logits): the same per-node math as
oracle/ops.py (rms_norm/kernel.py, linear/kernel.py, rotary/kernel.py, attention/kernel.py,
silu/kernel.py, mul/kernel.py, add/kernel.py), vectorised over positions so that a whole prompt
is one forward pass. Weights are the bf16 values as float32.
"""
from __future__ import annotations

import math

import torch


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def _rms_norm(x, w, eps):
    return x * (1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)) * w


def _rotary(x, cos, sin, pos):
    """x [B, H, S, D]; pos [B, S] absolute positions; interleaved pairs (rotary/kernel.py)."""
    c = cos[pos][:, None]  # [B, 1, S, D/2]
    s = sin[pos][:, None]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


class Qwen2Oracle:
    """Greedy decoding of a few sequences with a float32 KV cache of bf16 values."""

    def __init__(self, cfg, weights: dict, threads: int | None = None, round_bf16: bool = True):
        if threads:
            torch.set_num_threads(threads)
        self.cfg = cfg
        # round_bf16=False gives the plain fp32 model (used to pin the oracle against an
        # independent implementation of Qwen2).
        self.rnd = _bf16 if round_bf16 else (lambda t: t)
        self.w = {k: v.detach().to("cpu", torch.float32) for k, v in weights.items()}
        self.k_cache = None
        self.v_cache = None

    def reset(self, batch: int):
        self.k_cache = [None] * self.cfg.layers
        self.v_cache = [None] * self.cfg.layers
        self.length = 0
        self.batch = batch

    def forward(self, ids: torch.Tensor, last_only: bool = False,
                logits_last: int | None = None) -> torch.Tensor:
        """ids [B, S] int64: the next S tokens of every sequence (all at the same position).
        Returns fp32 logits [B, S, V] ([B, 1, V] with last_only, [B, n, V] for the last n
        positions with logits_last=n)."""
        w = self.w
        h = w["model.embed_tokens.weight"][ids]  # [B, S, H]
        h = self.forward_hidden(h, range(self.cfg.layers))
        if last_only:
            h = h[:, -1:]
        elif logits_last is not None:
            h = h[:, h.shape[1] - logits_last:]
        x = self.rnd(_rms_norm(h, w["model.norm.weight"], self.cfg.eps))
        return x @ w["lm_head.weight"].T

    def forward_hidden(self, h: torch.Tensor, layers) -> torch.Tensor:
        """The decoder layers `layers` (indices) applied to hidden states h [B, S, H] at the
        next S positions of every sequence (the cache grows by S); returns the residual stream
        after them (one layer of prefill when layers = [i] and the cache is fresh)."""
        cfg, w, _bf16 = self.cfg, self.w, self.rnd
        h = h.detach().to("cpu", torch.float32)
        b, s = h.shape[:2]
        pos = torch.arange(self.length, self.length + s)[None].expand(b, s)
        scale = 1.0 / math.sqrt(cfg.head_dim)
        group = cfg.heads // cfg.kv_heads
        for i in layers:
            p = f"model.layers.{i}"
            x = _bf16(_rms_norm(h, w[f"{p}.input_layernorm.weight"], cfg.eps))
            q = _bf16(x @ w[f"{p}.self_attn.q_proj.weight"].T + w[f"{p}.self_attn.q_proj.bias"])
            k = _bf16(x @ w[f"{p}.self_attn.k_proj.weight"].T + w[f"{p}.self_attn.k_proj.bias"])
            v = _bf16(x @ w[f"{p}.self_attn.v_proj.weight"].T + w[f"{p}.self_attn.v_proj.bias"])
            q = q.view(b, s, cfg.heads, cfg.head_dim).transpose(1, 2)
            k = k.view(b, s, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
            v = v.view(b, s, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
            q = _bf16(_rotary(q, w["rotary_cos"], w["rotary_sin"], pos))
            k = _bf16(_rotary(k, w["rotary_cos"], w["rotary_sin"], pos))
            kc = k if self.k_cache[i] is None else torch.cat([self.k_cache[i], k], 2)
            vc = v if self.v_cache[i] is None else torch.cat([self.v_cache[i], v], 2)
            self.k_cache[i], self.v_cache[i] = kc, vc
            kk = kc.repeat_interleave(group, dim=1)
            vv = vc.repeat_interleave(group, dim=1)
            scores = (q @ kk.transpose(-1, -2)) * scale  # [B, Hq, S, L]
            total = kc.shape[2]
            allowed = torch.arange(total)[None, :] <= (self.length + torch.arange(s))[:, None]
            scores = scores.masked_fill(~allowed, float("-inf"))
            attn = _bf16(torch.softmax(scores, dim=-1) @ vv)  # [B, Hq, S, D]
            attn = attn.transpose(1, 2).reshape(b, s, cfg.heads * cfg.head_dim)
            o = _bf16(attn @ w[f"{p}.self_attn.o_proj.weight"].T)
            h = _bf16(h + o)
            x2 = _bf16(_rms_norm(h, w[f"{p}.post_attention_layernorm.weight"], cfg.eps))
            g = _bf16(x2 @ w[f"{p}.mlp.gate_proj.weight"].T)
            u = _bf16(x2 @ w[f"{p}.mlp.up_proj.weight"].T)
            a = _bf16(_bf16(g / (1.0 + torch.exp(-g))) * u)
            d = _bf16(a @ w[f"{p}.mlp.down_proj.weight"].T)
            h = _bf16(h + d)
        self.length += s
        return h

    # -- preallocated cache (CPU baseline timing) ------------------------------------------------
    def reset_static(self, batch: int, capacity: int, seed: int = 0, fill: int = 0):
        """Preallocated float32 caches [B, Hkv, capacity, D]; the first `fill` positions get
        seeded N(0, 1) bf16 values (a synthetic context of that length)."""
        cfg = self.cfg
        g = torch.Generator().manual_seed(seed)
        shape = (batch, cfg.kv_heads, capacity, cfg.head_dim)
        self.k_static = [torch.zeros(shape) for _ in range(cfg.layers)]
        self.v_static = [torch.zeros(shape) for _ in range(cfg.layers)]
        for i in range(cfg.layers):
            if fill:
                self.k_static[i][:, :, :fill] = _bf16(torch.randn(batch, cfg.kv_heads, fill, cfg.head_dim, generator=g))
                self.v_static[i][:, :, :fill] = _bf16(torch.randn(batch, cfg.kv_heads, fill, cfg.head_dim, generator=g))

    def step_static(self, ids: torch.Tensor, pos: int) -> torch.Tensor:
        """One decode step of ids [B] at position `pos` (same for every row) over the
        preallocated caches; returns fp32 logits [B, V]."""
        cfg, w, rnd = self.cfg, self.w, self.rnd
        b = ids.shape[0]
        h = w["model.embed_tokens.weight"][ids]  # [B, H]
        scale = 1.0 / math.sqrt(cfg.head_dim)
        group = cfg.heads // cfg.kv_heads
        c, s_ = w["rotary_cos"][pos], w["rotary_sin"][pos]

        def rope(x):
            out = torch.empty_like(x)
            out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s_
            out[..., 1::2] = x[..., 0::2] * s_ + x[..., 1::2] * c
            return out

        for i in range(cfg.layers):
            p = f"model.layers.{i}"
            x = rnd(_rms_norm(h, w[f"{p}.input_layernorm.weight"], cfg.eps))
            q = rnd(x @ w[f"{p}.self_attn.q_proj.weight"].T + w[f"{p}.self_attn.q_proj.bias"])
            k = rnd(x @ w[f"{p}.self_attn.k_proj.weight"].T + w[f"{p}.self_attn.k_proj.bias"])
            v = rnd(x @ w[f"{p}.self_attn.v_proj.weight"].T + w[f"{p}.self_attn.v_proj.bias"])
            q = rnd(rope(q.view(b, cfg.heads, cfg.head_dim)))
            k = rnd(rope(k.view(b, cfg.kv_heads, cfg.head_dim)))
            self.k_static[i][:, :, pos] = k
            self.v_static[i][:, :, pos] = v.view(b, cfg.kv_heads, cfg.head_dim)
            kc = self.k_static[i][:, :, :pos + 1]  # [B, Hkv, L, D]
            vc = self.v_static[i][:, :, :pos + 1]
            qg = q.view(b, cfg.kv_heads, group, cfg.head_dim)
            scores = (qg @ kc.transpose(-1, -2)) * scale  # [B, Hkv, group, L]
            attn = rnd(torch.softmax(scores, -1) @ vc).reshape(b, cfg.heads * cfg.head_dim)
            h = rnd(h + rnd(attn @ w[f"{p}.self_attn.o_proj.weight"].T))
            x2 = rnd(_rms_norm(h, w[f"{p}.post_attention_layernorm.weight"], cfg.eps))
            gt = rnd(x2 @ w[f"{p}.mlp.gate_proj.weight"].T)
            up = rnd(x2 @ w[f"{p}.mlp.up_proj.weight"].T)
            a = rnd(rnd(gt / (1.0 + torch.exp(-gt))) * up)
            h = rnd(h + rnd(a @ w[f"{p}.mlp.down_proj.weight"].T))
        x = rnd(_rms_norm(h, w["model.norm.weight"], cfg.eps))
        return x @ w["lm_head.weight"].T

    def generate(self, prompt: torch.Tensor, steps: int):
        """Greedy tokens [B, steps] plus the top-1 / top-2 logit margins [B, steps]."""
        self.reset(prompt.shape[0])
        logits = self.forward(prompt, last_only=True)[:, -1]
        tokens, margins = [], []
        for _ in range(steps):
            top = torch.topk(logits, 2, dim=-1)
            nxt = torch.argmax(logits, dim=-1)
            tokens.append(nxt)
            margins.append(top.values[:, 0] - top.values[:, 1])
            logits = self.forward(nxt[:, None])[:, -1]
        return torch.stack(tokens, 1), torch.stack(margins, 1)

    def teacher_forced(self, prompt: torch.Tensor, continuation: torch.Tensor):
        """Logits after every prefix of prompt + continuation[:, :-1]: one forward pass.
        Returns argmax ids [B, T] and margins [B, T] for the T continuation positions."""
        self.reset(prompt.shape[0])
        full = torch.cat([prompt, continuation[:, :-1]], 1)
        logits = self.forward(full, logits_last=continuation.shape[1])
        top = torch.topk(logits, 2, dim=-1)
        return torch.argmax(logits, -1), top.values[..., 0] - top.values[..., 1], logits
