"""The reference's Qwen2-tiny end-to-end case on the GPU (tests/e2e/test_models.py:61-71): the
one-layer model of examples/qwen2/qwen2.py:22-44 with its deterministic weights, run in fp32
through the reference-style dli.graph.v1 decode graph on the gfx950 plugin. Its logits must
match transformers' (recorded in tests/golden/qwen2_tiny_e2e.json by
tests/golden/make_qwen2_tiny.py) at the reference's rtol = atol = 1e-3, and also at the fp32
bar (1e-4 relative), for the reference's prompt [2] and at every position of [2, 5, 1, 7]."""
from __future__ import annotations

import json
import os

import pytest
import torch

from dli_qwen2 import DecodeSession
from dli_qwen2.reference_tiny import REFERENCE_TINY, reference_tiny_weights
from oracle.qwen2 import Qwen2Oracle

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "qwen2_tiny_e2e.json")


@pytest.mark.parametrize("case", ["reference", "extended"])
def test_reference_qwen2_tiny_e2e(case):
    fixture = json.load(open(FIXTURE, encoding="utf-8"))
    spec = fixture["cases"][case]
    ids = torch.tensor(spec["input_ids"], dtype=torch.int64)
    expect = torch.tensor(spec["logits"], dtype=torch.float64)
    w = reference_tiny_weights(device="cuda")
    session = DecodeSession(REFERENCE_TINY, w, batch=1, max_seq_len=REFERENCE_TINY.max_pos,
                            fused=False)
    oracle = Qwen2Oracle(REFERENCE_TINY, w, round_bf16=False)
    oracle.reset(1)
    ref = oracle.forward(ids[None])[0].double()
    for t in range(ids.numel()):
        logits, next_ids = session.step(ids[t:t + 1].cuda(),
                                        torch.tensor([t], dtype=torch.int64, device="cuda"))
        got = logits.double().cpu()[0]
        print(f"position {t}: logits {got.tolist()}", flush=True)
        torch.testing.assert_close(got, expect[t], rtol=fixture["rtol"], atol=fixture["atol"])
        torch.testing.assert_close(got, expect[t], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(got, ref[t], rtol=1e-4, atol=1e-5)
        assert int(next_ids[0]) == int(torch.argmax(expect[t]))
