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
from .graph import build_decode_graph, pack_fused_weights


class DecodeSession:
    def __init__(self, cfg: Qwen2Config, weights: dict, batch: int, max_seq_len: int,
                 fused: bool = True, engine: "dli.Engine | None" = None, splits: dict | None = None,
                 block_size: int = 64, logits_dtype: str = "float32", device: str = "cuda",
                 stack: bool = False, check_status: bool = False):
        self.cfg = cfg
        self.batch = batch
        self.fused = fused
        self.stack = fused and stack
        self.engine = engine or dli.Engine().load_plugin()
        self.engine.configure_kv_cache(block_size=block_size, max_seq_len=max_seq_len)
        self.graph = build_decode_graph(cfg, batch, fused=fused, splits=splits,
                                        logits_dtype=logits_dtype, stack=stack,
                                        check_status=check_status)
        tensors = pack_fused_weights(cfg, weights, drop_unfused=True) if fused else dict(weights)
        self.ids = torch.zeros(batch, dtype=torch.int64, device=device)
        self.positions = torch.zeros(batch, dtype=torch.int64, device=device)
        tensors["input_ids"] = self.ids
        tensors["positions"] = self.positions
        self.inputs = tensors
        self.max_seq_len = max_seq_len
        self._graph = None
        self._out = None
        self._status = None

    # -- one step ---------------------------------------------------------------------------
    def run_eager(self, profile=None):
        """One step without graph capture; profile: a dli.ProfileSession timing every node."""
        return self._keep_status(self.engine.run(self.graph, self.inputs, profile=profile))

    def capture(self, chain_ids: bool = False):
        """Warm up once (loads kernels, allocates caches and scratch), then capture a step.
        With chain_ids the captured step also copies its next_ids into the input ids, so
        replays continue greedy decoding with no host work."""
        self.run_eager()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self.engine.run(self.graph, self.inputs)
            if chain_ids:
                self.ids.copy_(out["next_ids"])
        self._graph = graph
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
        """Replays the captured step on the current static inputs (for timing)."""
        self._graph.replay()
        return self._out

    # -- greedy generation ----------------------------------------------------------------------
    def generate(self, prompt: torch.Tensor, steps: int, start: int = 0):
        """prompt [B, S] int64 (device). Feeds the prompt one position per step (prefill through
        the decode step), then decodes `steps` greedy tokens. Returns [B, steps] int64."""
        b, s = prompt.shape
        pos = torch.full((b,), start, dtype=torch.int64, device=prompt.device)
        next_ids = None
        for t in range(s):
            _, next_ids = self.step(prompt[:, t], pos)
            pos += 1
        generated = []
        for _ in range(steps):
            generated.append(next_ids.clone())
            _, next_ids = self.step(next_ids.clone(), pos)
            pos += 1
        out = torch.stack(generated, dim=1)
        torch.cuda.synchronize()
        self.check_status()
        return out
