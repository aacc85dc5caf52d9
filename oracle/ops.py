"""numpy restatement of the reference operators (test infrastructure; see oracle/__init__.py).

Every function computes in float64 from the given inputs and returns float64 (callers round
to the output dtype with round_bf16 / round_f16 / np.float32). Each cites the reference
kernel it restates. Pinned by tests/test_oracle.py against the reference's own known-answer
literals (tests/golden/kat_ops.json) and against independent library routines.
"""
from __future__ import annotations

import numpy as np


# --- rounding -----------------------------------------------------------------------------

def round_bf16(x) -> np.ndarray:
    """float -> bfloat16 -> float with round-to-nearest-even on the float32 bit pattern.

    NaNs stay NaN. The result is returned as float32 values exactly representable in bf16.
    """
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(f), np.float32(np.nan), out).astype(np.float32)


def round_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return round_bf16(x)
    if dtype == "float16":
        return round_f16(x)
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


# --- elementwise --------------------------------------------------------------------------

def add(a, b):
    """add/kernel.py:6-11: out[i] = a[i] + b[i % numel(b)]."""
    a = np.asarray(a, np.float64)
    flat_b = np.asarray(b, np.float64).reshape(-1)
    idx = np.arange(a.size) % flat_b.size
    return (a.reshape(-1) + flat_b[idx]).reshape(a.shape)


def mul(a, b):
    """mul/kernel.py:6-11: out[i] = a[i] * b[i % numel(b)]."""
    a = np.asarray(a, np.float64)
    flat_b = np.asarray(b, np.float64).reshape(-1)
    idx = np.arange(a.size) % flat_b.size
    return (a.reshape(-1) * flat_b[idx]).reshape(a.shape)


def silu(x):
    """silu/kernel.py:6-10: x / (1 + exp(-x))."""
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def relu(x):
    """relu/kernel.py:6-10: max(x, 0)."""
    return np.maximum(np.asarray(x, np.float64), 0.0)


def rms_norm(x, w, eps=1e-6):
    """rms_norm/kernel.py:6-14: x * rsqrt(sum(x^2)/hidden + eps) * w, per row."""
    x = np.asarray(x, np.float64)
    ms = np.sum(x * x, axis=-1, keepdims=True) / x.shape[-1]
    return x * (1.0 / np.sqrt(ms + eps)) * np.asarray(w, np.float64)


def softmax(x):
    """softmax/kernel.py:6-14: exp(x - max) / sum over the last dim."""
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def transpose(x):
    """transpose/kernel.py:6-20: out[c, r] = x[r, c] (2-D)."""
    x = np.asarray(x, np.float64)
    out = np.empty((x.shape[1], x.shape[0]))
    for r in range(x.shape[0]):
        out[:, r] = x[r, :]
    return out


def batch_norm2d(x, w, b, mean, var, eps=1e-5):
    """batch_norm2d/kernel.py:6-28, channel = (i // spatial) % C."""
    x = np.asarray(x, np.float64)
    c = x.shape[1]
    shape = (1, c, 1, 1)
    inv = 1.0 / np.sqrt(np.asarray(var, np.float64).reshape(shape) + eps)
    return ((x - np.asarray(mean, np.float64).reshape(shape)) * inv
            * np.asarray(w, np.float64).reshape(shape) + np.asarray(b, np.float64).reshape(shape))


def embedding(ids, table):
    """embedding/kernel.py:6-23: out[t, :] = table[ids[t], :]."""
    ids = np.asarray(ids, np.int64)
    return np.asarray(table, np.float64)[ids.reshape(-1)].reshape(ids.shape + (table.shape[1],))


def argmax(x):
    """First index of the row maximum (torch.argmax rule)."""
    return np.argmax(np.asarray(x, np.float64), axis=-1)


# --- GEMMs --------------------------------------------------------------------------------

def linear(x, w, b=None):
    """linear/kernel.py:6-44: y[m, n] = sum_k x[m, k] * w[n, k] (+ b[n]), w is [n, k]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    y = np.einsum("mk,nk->mn", x2, w)
    if b is not None:
        y = y + np.asarray(b, np.float64)[None, :]
    return y.reshape(lead + (w.shape[0],))


def matmul(a, b):
    """matmul/kernel.py:6-40: out = a[m, k] @ b[k, n]."""
    return np.einsum("mk,kn->mn", np.asarray(a, np.float64), np.asarray(b, np.float64))


# --- convolution / pooling ----------------------------------------------------------------

def conv2d(x, w, b=None, stride=(1, 1), padding=(0, 0)):
    """conv2d/kernel.py:6-49: direct NCHW convolution with zero padding."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    n, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    sh, sw = stride
    ph, pw = padding
    oh = (h + 2 * ph - kh) // sh + 1
    ow = (wd + 2 * pw - kw) // sw + 1
    xp = np.zeros((n, c, h + 2 * ph, wd + 2 * pw))
    xp[:, :, ph:ph + h, pw:pw + wd] = x
    out = np.zeros((n, oc, oh, ow))
    for dy in range(kh):
        for dx in range(kw):
            patch = xp[:, :, dy:dy + sh * (oh - 1) + 1:sh, dx:dx + sw * (ow - 1) + 1:sw]
            out += np.einsum("nchw,oc->nohw", patch, w[:, :, dy, dx])
    if b is not None:
        out += np.asarray(b, np.float64).reshape(1, oc, 1, 1)
    return out


def max_pool2d(x, kernel_size=(2, 2), stride=None, padding=(0, 0)):
    """max_pool2d/kernel.py:6-41: window max, padded cells are -inf."""
    x = np.asarray(x, np.float64)
    stride = stride or kernel_size
    n, c, h, w = x.shape
    kh, kw = kernel_size
    sh, sw = stride
    ph, pw = padding
    oh = (h + 2 * ph - kh) // sh + 1
    ow = (w + 2 * pw - kw) // sw + 1
    xp = np.full((n, c, h + 2 * ph, w + 2 * pw), -np.inf)
    xp[:, :, ph:ph + h, pw:pw + w] = x
    out = np.full((n, c, oh, ow), -np.inf)
    for dy in range(kh):
        for dx in range(kw):
            out = np.maximum(out, xp[:, :, dy:dy + sh * (oh - 1) + 1:sh, dx:dx + sw * (ow - 1) + 1:sw])
    return out


# --- rotary / attention -------------------------------------------------------------------

def rotary(x, cos, sin, start_pos=0, positions=None):
    """rotary/kernel.py:6-35 on one tensor [B, H, S, D]: interleaved pairs (2p, 2p+1),
    c = cos[pos, p], s = sin[pos, p], pos = start_pos + token (+ positions[b])."""
    x = np.asarray(x, np.float64)
    cos = np.asarray(cos, np.float64)
    sin = np.asarray(sin, np.float64)
    b_, h_, s_, d_ = x.shape
    pairs = cos.shape[1]
    out = x.copy()
    for b in range(b_):
        base = start_pos + (0 if positions is None else int(positions[b]))
        for t in range(s_):
            pos = base + t
            if pos < 0 or pos >= cos.shape[0]:
                continue
            c = cos[pos, :pairs]
            s = sin[pos, :pairs]
            x0 = x[b, :, t, 0:2 * pairs:2]
            x1 = x[b, :, t, 1:2 * pairs:2]
            out[b, :, t, 0:2 * pairs:2] = x0 * c - x1 * s
            out[b, :, t, 1:2 * pairs:2] = x0 * s + x1 * c
    return out


def attention(q, k, v, causal=False, scale=None, past=None):
    """attention/kernel.py:6-62 with grouped KV heads: q [B, Hq, Sq, D], k/v [B, Hkv, Sk, D].
    Query i may see key j when j <= past + i (causal); past defaults to Sk - Sq. `past` may
    be a per-sequence list (paged cache)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    b_, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    group = hq // hkv
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    out = np.zeros_like(q)
    for b in range(b_):
        past_b = (sk - sq) if past is None else (past[b] if np.ndim(past) else past)
        for h in range(hq):
            kk = k[b, h // group]
            vv = v[b, h // group]
            for i in range(sq):
                limit = min(past_b + i + 1, sk) if causal else min(past_b + sq, sk)
                if limit <= 0:
                    continue
                s = (kk[:limit] @ q[b, h, i]) * scale
                p = np.exp(s - s.max())
                out[b, h, i] = (p / p.sum()) @ vv[:limit]
    return out
