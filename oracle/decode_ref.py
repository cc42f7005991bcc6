"""Decode-step oracle -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of TinyBrain's ModelRunner.step for the pre-norm LLaMA
architecture, used by tests and by bench.py's CPU baseline as the checker of
the GPU decode step.  Nothing in the product imports it.

Follows (vivekptnk/tinybrain):
  * step                 Sources/TinyBrainRuntime/ModelRunner.swift:168-208
  * applyLayer (LLaMA)   ModelRunner.swift:418-459
  * applyRoPE            ModelRunner.swift:470-494 (interleaved pairs,
                         theta = 10000^(-i/rDims), angle = Float(pos)*theta)
  * attention            ModelRunner.swift:496-592 (GQA kvHead = head/repeats,
                         scores * 1/sqrt(headDim), max-subtracted softmax)
  * rmsNorm              Tensor.swift:1538-1556 (x * invRMS * w, eps 1e-5)
  * silu                 Tensor.swift:1135-1141 (x / (1 + exp(-x)))

Projections multiply by the dequantized weights (the bit-exact fp32 values
QuantizedTensor.dequantize() yields) in float64; everything else is float64
as well, except the RoPE angle, which the reference forms in Float and which
is formed here the same way.  It is an fp64 oracle of the same computation,
not a bit-for-bit Swift replica.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import numpy as np


@dataclass
class RefLayer:
    input_norm: np.ndarray            # [hidden]
    post_norm: np.ndarray             # [hidden]
    weights: Sequence[np.ndarray]     # q, k, v, o, gate, up, down as dequantized [K, N]


class RefDecoder:
    def __init__(self, num_layers, hidden, num_heads, num_kv_heads, intermediate, vocab,
                 embeddings: np.ndarray, final_norm: np.ndarray, lm_head: np.ndarray,
                 layers: List[RefLayer], rms_eps: float = 1e-5, rope_base: float = 10000.0):
        self.L, self.H, self.nh, self.nkv = num_layers, hidden, num_heads, num_kv_heads
        self.I, self.V = intermediate, vocab
        self.hd = hidden // num_heads
        self.emb = np.asarray(embeddings, np.float64)
        self.final_norm = np.asarray(final_norm, np.float64)
        self.lm = np.asarray(lm_head, np.float64)
        self.layers = [RefLayer(np.asarray(l.input_norm, np.float64), np.asarray(l.post_norm, np.float64),
                                [np.asarray(w, np.float64) for w in l.weights]) for l in layers]
        self.eps, self.base = rms_eps, rope_base
        self.reset()

    def reset(self):
        self.pos = 0
        self.kc = [[] for _ in range(self.L)]
        self.vc = [[] for _ in range(self.L)]

    def _rms(self, x, w):
        inv = 1.0 / np.sqrt(np.sum(x * x) / x.size + self.eps)
        return x * inv * w

    def _rope(self, v, heads):
        out = v.copy()
        r = self.hd
        i = np.arange(0, r, 2)
        theta = np.power(np.float32(self.base), -(i.astype(np.float32) / np.float32(r)), dtype=np.float32)
        ang = (np.float32(self.pos) * theta).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        for h in range(heads):
            o = h * self.hd
            x0, x1 = v[o + i], v[o + i + 1]
            out[o + i] = x0 * c - x1 * s
            out[o + i + 1] = x0 * s + x1 * c
        return out

    def step(self, token: int, logits: bool = True):
        """One ModelRunner.step; with logits=False the LM head is skipped
        (the caches and position advance the same) and None is returned."""
        self.ctx_trace = []                    # attention context of each layer
        h = self.emb[token].copy()
        for li, lw in enumerate(self.layers):
            wq, wk, wv, wo, wg, wu, wd = lw.weights
            x = self._rms(h, lw.input_norm)
            q = self._rope(x @ wq, self.nh)
            k = self._rope(x @ wk, self.nkv)
            v = x @ wv
            self.kc[li].append(k)
            self.vc[li].append(v)
            K = np.stack(self.kc[li])          # [t, kv_dim]
            Vv = np.stack(self.vc[li])
            rep = self.nh // self.nkv
            ctx = np.empty(self.H)
            for hh in range(self.nh):
                kvh = hh // rep
                qh = q[hh * self.hd:(hh + 1) * self.hd]
                kh = K[:, kvh * self.hd:(kvh + 1) * self.hd]
                vh = Vv[:, kvh * self.hd:(kvh + 1) * self.hd]
                sc = (kh @ qh) * (1.0 / np.sqrt(self.hd))
                e = np.exp(sc - sc.max())
                w = e / e.sum()
                ctx[hh * self.hd:(hh + 1) * self.hd] = w @ vh
            self.ctx_trace.append(ctx)
            h = h + ctx @ wo
            x = self._rms(h, lw.post_norm)
            g = x @ wg
            u = x @ wu
            h = h + ((g / (1.0 + np.exp(-g))) * u) @ wd
        self.pos += 1
        return self._rms(h, self.final_norm) @ self.lm if logits else None
