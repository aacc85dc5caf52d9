"""Flash-style bf16 attention (csrc/kernels/flash_attention.hip), the path of the `attention`
op for bf16 with head_dim 64: against the CPU oracle (oracle/ops.py attention, float64 on the
same bf16 inputs) on ragged, causal / non-causal, GQA and Sq != Sk shapes, and at the Qwen2
prefill size (batch 4 x 2048 tokens, 14 / 2 heads) against a plain PyTorch fp32 reference on the
GPU. Tolerance: the bf16 parity contract (2e-2)."""
from __future__ import annotations

import pytest
import torch

from oracle import ops
from support import assert_close, run_op, to_np

pytestmark = pytest.mark.gpu


def rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).cuda()


CASES = [  # B, Hq, Hkv, Sq, Sk
    (1, 1, 1, 1, 1),
    (2, 14, 2, 64, 64),
    (2, 14, 2, 100, 100),
    (1, 4, 2, 37, 200),    # fewer queries than keys (cache prefix)
    (1, 2, 2, 130, 70),    # more queries than keys: the first queries see no key when causal
    (3, 6, 3, 257, 257),
    (2, 16, 4, 2000, 2000),  # long, ragged last query tile
    (4, 16, 2, 1000, 1100),  # long, with a cache prefix
]


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_flash_attention_matches_oracle(case, causal):
    b, hq, hkv, sq, sk = case
    q, k, v = rand((b, hq, sq, 64), 1), rand((b, hkv, sk, 64), 2), rand((b, hkv, sk, 64), 3)
    out = run_op("attention", {"q": q, "k": k, "v": v}, attrs={"causal": causal})["output"]
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (b, hq, sq, 64)
    assert_close(out, ops.attention(to_np(q), to_np(k), to_np(v), causal=causal), "bfloat16")


@pytest.mark.parametrize("case", [(2, 14, 2, 100, 100), (1, 4, 2, 37, 200), (2, 16, 4, 2000, 2000)],
                         ids=str)
def test_flash_attention_bshd_output(case):
    """output_layout "bshd": the same values as the [B, H, S, D] output, transposed."""
    b, hq, hkv, sq, sk = case
    q, k, v = rand((b, hq, sq, 64), 7), rand((b, hkv, sk, 64), 8), rand((b, hkv, sk, 64), 9)
    bhsd = run_op("attention", {"q": q, "k": k, "v": v}, attrs={"causal": True})["output"]
    bshd = run_op("attention", {"q": q, "k": k, "v": v},
                  attrs={"causal": True, "output_layout": "bshd"})["output"]
    assert tuple(bshd.shape) == (b, sq, hq, 64)
    assert torch.equal(bshd, bhsd.transpose(1, 2).contiguous())


def test_flash_attention_qwen2_prefill_size():
    b, hq, hkv, s = 4, 14, 2, 2048
    q, k, v = rand((b, hq, s, 64), 4), rand((b, hkv, s, 64), 5), rand((b, hkv, s, 64), 6)
    out = run_op("attention", {"q": q, "k": k, "v": v}, attrs={"causal": True})["output"]
    qf = q.float()
    kf = k.float().repeat_interleave(hq // hkv, dim=1).contiguous()
    vf = v.float().repeat_interleave(hq // hkv, dim=1).contiguous()
    ref = torch.empty_like(qf)
    mask = torch.ones(s, s, dtype=torch.bool, device="cuda").tril()
    for i in range(b):  # one batch row at a time keeps the fp32 score matrix at 0.2 GB
        sc = torch.matmul(qf[i], kf[i].transpose(-1, -2).contiguous()) / 8.0
        sc = sc.masked_fill(~mask, float("-inf"))
        ref[i] = torch.matmul(torch.softmax(sc, -1), vf[i])
    torch.cuda.synchronize()
    assert_close(out, ref.cpu().double().numpy(), "bfloat16")
