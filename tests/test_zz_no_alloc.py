"""dli_hip_lm_head_argmax_norm_noalloc (the lm_head + greedy argmax entry point that allocates
nothing: its per-tile partials live in a static device array of the library) against
dli_hip_lm_head_argmax_norm with a caller workspace, through the C ABI. Two calls in a row, the
second smaller, must both match bit for bit: the static array keeps the first call's contents,
and every partial the second call reads must be its own."""
from __future__ import annotations

import ctypes

import pytest
import torch

from dli import hip

pytestmark = pytest.mark.gpu


def _case(m, vocab, hidden, seed, with_norm):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, hidden, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(vocab, hidden, generator=g) * 0.05).to(torch.bfloat16).cuda()
    nw = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).cuda() if with_norm else None
    return x, w, nw


def _run(entry, x, w, nw, logits_dtype):
    m, hidden = x.shape
    vocab = w.shape[0]
    code = hip.F32 if logits_dtype == torch.float32 else hip.BF16
    logits = torch.full((m, vocab), float("nan"), dtype=logits_dtype, device="cuda")
    ids = torch.full((m,), -1, dtype=torch.int64, device="cuda")
    stream = hip.current_stream()
    nw_ptr = nw.data_ptr() if nw is not None else None
    if entry == "noalloc":
        hip.call("dli_hip_lm_head_argmax_norm_noalloc", x.data_ptr(), nw_ptr, 1e-6, w.data_ptr(),
                 logits.data_ptr(), code, ids.data_ptr(), m, vocab, hidden, stream)
    else:
        ws_bytes = hip.lib().dli_hip_lm_head_argmax_workspace(m, vocab)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        hip.call("dli_hip_lm_head_argmax_norm", x.data_ptr(), nw_ptr, 1e-6, w.data_ptr(),
                 logits.data_ptr(), code, ids.data_ptr(), m, vocab, hidden, ws.data_ptr(),
                 ws_bytes, stream)
    torch.cuda.synchronize()
    return logits, ids


def test_noalloc_matches_workspace_entry_on_two_calls():
    calls = [  # (rows, vocab, hidden, seed, final norm, logits dtype): the second call smaller
        (32, 151936, 896, 1, True, torch.float32),
        (5, 20000, 896, 2, False, torch.bfloat16),
    ]
    for m, vocab, hidden, seed, with_norm, dt in calls:
        print(f"no-alloc lm_head m={m} vocab={vocab} hidden={hidden} norm={with_norm}", flush=True)
        x, w, nw = _case(m, vocab, hidden, seed, with_norm)
        got_logits, got_ids = _run("noalloc", x, w, nw, dt)
        ref_logits, ref_ids = _run("workspace", x, w, nw, dt)
        assert torch.equal(got_ids, ref_ids)
        assert torch.equal(got_logits, ref_logits)
        assert torch.equal(got_ids, got_logits.float().argmax(dim=1))


def test_noalloc_rejects_sizes_beyond_its_scratch():
    x = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    ids = torch.zeros(64, dtype=torch.int64, device="cuda")
    # 64 rows over 600,000 vocab rows need 8 * 64 * 18,750 bytes of partials (> 4 MiB)
    rc = hip.lib().dli_hip_lm_head_argmax_norm_noalloc(x.data_ptr(), None, ctypes.c_float(1e-6),
                                                       x.data_ptr(), None, hip.F32,
                                                       ids.data_ptr(), 64, 600000, 64,
                                                       hip.current_stream())
    assert rc == -1
    assert b"above its 4194304-byte maximum" in hip.lib().dli_hip_last_error()
