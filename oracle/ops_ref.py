"""Oracle for the non-matmul backend protocols -- TEST INFRASTRUCTURE ONLY.

numpy float64 restatements of the CPU paths that TinyBrain falls back to when
no GPU backend takes an op, used by tests as the checker of
tbh_softmax / tbh_rmsnorm / tbh_silu / tbh_gelu / tbh_attention.  Nothing in
the product imports it.

Follows (vivekptnk/tinybrain):
  * softmax    Sources/TinyBrainRuntime/Tensor.swift:1271-1330 (softmaxCPU:
               exp(x - max) / (sum + epsilon), epsilon 1e-7, per last-dim row)
  * rmsnorm    Tensor.swift:1538-1556 (rmsNormCPU: x * (1/sqrt(ss/H + eps)) * w)
  * silu       Tensor.swift:1135-1141 (x / (1 + exp(-x)))
  * gelu       Tensor.swift:1107-1121 (0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))))
  * attention  Sources/TinyBrainMetal/Shaders/FlashAttention.metal (scores
               q.k * 1/sqrt(headDim) + mask[kv], GQA head / (nh / nkv),
               output / (sum + 1e-7)); the softmax over all positions is
               that of cpuAttention in Tests/TinyBrainMetalTests/
               FlashAttentionTests.swift:65-134, whose all-masked rows come
               out NaN.

Parity pins for each function (known answers, closed forms, an independent
library routine) are in tests/test_ops_oracle.py.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

SOFTMAX_EPS = 1e-7
ATTN_EPS = 1e-7


def softmax(x: np.ndarray, eps: float = SOFTMAX_EPS) -> np.ndarray:
    x = np.asarray(x, np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / (np.sum(e, axis=-1, keepdims=True) + eps)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.asarray(x, np.float64)
    ss = np.sum(x * x, axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(ss / x.shape[-1] + eps)
    return x * inv * np.asarray(w, np.float64)


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    inner = np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)
    return 0.5 * x * (1.0 + np.tanh(inner))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: Optional[np.ndarray], head_dim: int,
              num_heads: int, num_kv_heads: int, eps: float = ATTN_EPS) -> np.ndarray:
    """q [B?, S, nh*hd], k/v [B?, T, nkv*hd], mask [T] or None -> like q."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    squeeze = q.ndim == 2
    if squeeze:
        q, k, v = q[None], k[None], v[None]
    B, S, _ = q.shape
    T = k.shape[1]
    rep = num_heads // num_kv_heads
    out = np.zeros_like(q)
    if T == 0:
        return out[0] if squeeze else out
    qh = q.reshape(B, S, num_heads, head_dim)
    kh = k.reshape(B, T, num_kv_heads, head_dim)
    vh = v.reshape(B, T, num_kv_heads, head_dim)
    scale = 1.0 / np.sqrt(head_dim)
    for h in range(num_heads):
        kvh = h // rep
        sc = np.einsum("bsd,btd->bst", qh[:, :, h], kh[:, :, kvh]) * scale   # [B, S, T]
        if mask is not None:
            sc = sc + np.asarray(mask, np.float64).reshape(1, 1, T)
        with np.errstate(invalid="ignore"):
            e = np.exp(sc - sc.max(axis=-1, keepdims=True))
        o = np.einsum("bst,btd->bsd", e, vh[:, :, kvh]) / (e.sum(axis=-1, keepdims=True) + eps)
        out.reshape(B, S, num_heads, head_dim)[:, :, h] = o
    return out[0] if squeeze else out
