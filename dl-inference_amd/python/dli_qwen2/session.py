"""Greedy decode driver: one dli.graph.v1 decode step run through Engine + the gfx950 plugin,
optionally captured once into a HIP graph (torch.cuda.CUDAGraph) and replayed per step.

Static input buffers (input_ids, positions) are updated in place before every step, so the
captured graph reads the new token ids and per-sequence positions without any host work in
the graph itself.
"""
from __future__ import annotations

import torch

import dli

from .config import Qwen2Config
from .graph import (build_decode_graph, build_prefill_graph, pack_fused_weights,
                    pack_large_weights, uses_large_graph)


class DecodeSession:
    def __init__(self, cfg: Qwen2Config, weights: dict, batch: int, max_seq_len: int,
                 fused: bool = True, engine: "dli.Engine | None" = None, splits: dict | None = None,
                 block_size: int = 64, logits_dtype: str = "float32", device: str = "cuda",
                 stack: bool = False, check_status: bool = False, prefill: bool = False,
                 stack_trace: "torch.Tensor | None" = None):
        self.cfg = cfg
        self.batch = batch
        self.fused = fused
        self.stack = fused and stack and not uses_large_graph(cfg, fused)
        self.engine = engine or dli.Engine().load_plugin()
        self.engine.configure_kv_cache(block_size=block_size, max_seq_len=max_seq_len)
        # the large-hidden graph's GPU form (fused q|k|v, residual + RMSNorm and MLP nodes of
        # the GPU plugin; the ATen CPU plugin runs the reference's nodes)
        large_fused = uses_large_graph(cfg, fused) and device != "cpu" and not prefill
        # stack_trace: int64 device buffer (layers x CUs x 24) for the decoder stack's stage
        # timeline, written by every step
        if stack_trace is not None and not self.stack:
            raise ValueError("stack_trace needs the decoder stack graph")
        self.graph = build_decode_graph(cfg, batch, fused=fused, splits=splits,
                                        logits_dtype=logits_dtype, stack=stack,
                                        check_status=check_status, large_fused=large_fused,
                                        stack_trace=stack_trace is not None)
        # prefill=True: generate() runs the prompt through one prefill graph (the layers over
        # [B, S] tokens at once), which reads the unpacked q/k/v and gate/up weights
        self.prefill = prefill
        self._prefill_graphs: dict = {}
        if fused and not uses_large_graph(cfg, fused):
            tensors = pack_fused_weights(cfg, weights, drop_unfused=not prefill)
        elif large_fused:
            tensors = pack_large_weights(cfg, weights)
        else:
            tensors = dict(weights)
        self.ids = torch.zeros(batch, dtype=torch.int64, device=device)
        self.positions = torch.zeros(batch, dtype=torch.int64, device=device)
        tensors["input_ids"] = self.ids
        tensors["positions"] = self.positions
        if stack_trace is not None:
            tensors["stack_trace"] = stack_trace
        self.inputs = tensors
        self.max_seq_len = max_seq_len
        self._graph = None
        self._graph_steps = 1
        self.step_positions = None
        self._out = None
        self._status = None

    # -- one step ---------------------------------------------------------------------------
    def run_eager(self, profile=None):
        """One step without graph capture; profile: a dli.ProfileSession timing every node."""
        return self._keep_status(self.engine.run(self.graph, self.inputs, profile=profile))

    def capture(self, chain_ids: bool = False, steps: int = 1):
        """Warm up once (loads kernels, allocates caches and scratch), then capture a step.
        With chain_ids the captured step also copies its next_ids into the input ids, so
        replays continue greedy decoding with no host work.

        steps > 1 (needs chain_ids): the graph holds `steps` greedy steps, step i + 1 reading
        step i's next_ids directly and step i its positions from row i of `step_positions`
        ([steps, B] int64, static; capture fills every row with the current positions, the
        caller rewrites it before a replay, e.g. positions + i to decode consecutive tokens).
        One graph launch then covers `steps` steps: each launch of a captured graph costs about
        8 us on top of its kernels, and the chaining copy about 4 us more. replay() returns the
        last step's outputs; step() refuses such a graph."""
        if steps < 1 or (steps > 1 and not chain_ids):
            raise ValueError("steps must be >= 1, and steps > 1 needs chain_ids")
        self.run_eager()
        torch.cuda.synchronize()
        self.step_positions = self.positions.unsqueeze(0).repeat(steps, 1) if steps > 1 else None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            inputs = dict(self.inputs)
            for i in range(steps):
                if steps > 1:
                    inputs["positions"] = self.step_positions[i]
                out = self.engine.run(self.graph, inputs)
                inputs["input_ids"] = out["next_ids"]
            if chain_ids:
                self.ids.copy_(out["next_ids"])
        self._graph = graph
        self._graph_steps = steps
        self._out = out
        self._keep_status(out)
        return self

    def check_status(self):
        """Raises if a step since the last check reported a failed launch: the stack graph's
        `status` output is non-zero when a wait in the persistent decoder_stack launch gave up
        (the step's outputs are then invalid). Clears the word. Synchronizes with the device."""
        status = self._status
        if status is None or int(status.item()) == 0:
            return
        status.zero_()
        raise RuntimeError("decode step failed: a decoder_stack workgroup gave up waiting "
                           "(its outputs are invalid)")

    def _keep_status(self, out):
        if "status" in out:
            self._status = out["status"]
        return out

    def step(self, ids: torch.Tensor, positions: torch.Tensor):
        """Runs one decode step for ids [B] at positions [B]; returns (logits, next_ids). A
        failed launch of an earlier step raises here (the position check synchronizes)."""
        if int(positions.max()) >= self.max_seq_len:
            raise ValueError("position exceeds the KV cache capacity")
        if self._graph is not None and self._graph_steps != 1:
            raise ValueError("the captured graph holds several steps: run it with replay()")
        self.check_status()
        self.ids.copy_(ids)
        self.positions.copy_(positions)
        if self._graph is not None:
            self._graph.replay()
            out = self._out
        else:
            out = self.run_eager()
        self._keep_status(out)
        return out["logits"], out["next_ids"]

    def replay(self):
        """Replays the captured step (or steps) on the current static inputs; returns the
        outputs of the graph's last step."""
        self._graph.replay()
        return self._out

    # -- greedy generation ----------------------------------------------------------------------
    def run_prefill(self, prompt: torch.Tensor):
        """Runs the prompt [B, S] (positions 0..S-1 of every sequence) through the prefill graph
        (build_prefill_graph): the cache entries receive the prompt's keys and values and the
        first greedy token comes back. Returns (logits [B, V], next_ids [B])."""
        b, s = prompt.shape
        if b != self.batch:
            raise ValueError("prompt batch differs from the session's")
        if s > self.max_seq_len:
            raise ValueError("prompt exceeds the KV cache capacity")
        graph = self._prefill_graphs.get(s)
        if graph is None:
            on_gpu = prompt.is_cuda and self.fused and not uses_large_graph(self.cfg, self.fused)
            # lm_head_argmax holds a tile's rows in registers (hidden <= 1024): larger hiddens
            # take rms_norm + linear + argmax
            fused_head = prompt.is_cuda and not uses_large_graph(self.cfg, True)
            graph = build_prefill_graph(self.cfg, b, s, fused_head=fused_head, fused=on_gpu)
            self._prefill_graphs[s] = graph
        self.engine.set_kv_cache_length(0)  # the prompt starts every sequence at position 0
        inputs = dict(self.inputs)
        inputs["input_ids"] = prompt.contiguous()
        out = self.engine.run(graph, inputs)
        return out["logits"], out["next_ids"]

    def generate(self, prompt: torch.Tensor, steps: int, start: int = 0):
        """prompt [B, S] int64 (device). Feeds the prompt, then decodes `steps` greedy tokens.
        Returns [B, steps] int64. The prompt goes through the prefill graph in one run when the
        session was built with prefill=True (start must then be 0), else one position per decode
        step."""
        b, s = prompt.shape
        pos = torch.full((b,), start, dtype=torch.int64, device=prompt.device)
        next_ids = None
        if self.prefill:
            if start != 0:
                raise ValueError("a prefill graph starts at position 0")
            _, next_ids = self.run_prefill(prompt)
            pos += s
        else:
            for t in range(s):
                _, next_ids = self.step(prompt[:, t], pos)
                pos += 1
        generated = []
        for _ in range(steps):
            generated.append(next_ids.clone())
            _, next_ids = self.step(next_ids.clone(), pos)
            pos += 1
        out = torch.stack(generated, dim=1)
        if out.is_cuda:
            torch.cuda.synchronize()
        self.check_status()
        return out
