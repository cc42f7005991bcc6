"""Decoder: the GPU decode step (tbh_decoder) for LLaMA-style models.

Mirrors ModelRunner.step / reset for the pre-norm LLaMA architecture
(Sources/TinyBrainRuntime/ModelRunner.swift:168-216, :392-592): the caller
provides ModelWeights-shaped arrays -- fp32 token embeddings [vocab, hidden],
RMSNorm weights, and per layer the seven projections as QuantizedTensor
[K, N] -- and calls step(token) for the logits of the next token.  All
compute runs in libtinybrain_hip.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _abi
from .backend import HIPBackend, _check
from .quantized import PreconditionFailure, QuantizedTensor


@dataclass
class DecoderConfig:
    """ModelConfig (ModelRunner.swift:26-100) fields the LLaMA step uses."""
    num_layers: int
    hidden: int
    num_heads: int
    num_kv_heads: int
    intermediate: int
    vocab: int
    max_seq: int = 2048
    rms_eps: float = 1e-5        # Tensor.rmsNorm default (Tensor.swift:1512)
    rope_base: float = 10000.0   # ModelRunner.applyRoPE (ModelRunner.swift:478)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.num_heads

    @property
    def kv_dim(self) -> int:
        return self.head_dim * self.num_kv_heads

    def _c(self) -> _abi.DecoderConfig:
        return _abi.DecoderConfig(self.num_layers, self.hidden, self.num_heads, self.num_kv_heads,
                                  self.intermediate, self.vocab, self.max_seq, self.rms_eps,
                                  self.rope_base)


class Decoder:
    def __init__(self, backend: HIPBackend, config: DecoderConfig, embeddings: np.ndarray,
                 final_norm: np.ndarray, lm_head: QuantizedTensor):
        self._lib = _abi.lib()
        self.backend = backend
        self.config = config
        emb = np.ascontiguousarray(embeddings, np.float32)
        fn = np.ascontiguousarray(final_norm, np.float32)
        if emb.shape != (config.vocab, config.hidden) or fn.shape != (config.hidden,):
            raise PreconditionFailure("embeddings / final norm shape does not match the config")
        if tuple(lm_head.shape) != (config.hidden, config.vocab):
            raise PreconditionFailure("lm_head must be [hidden, vocab]")
        self._h = ctypes.c_void_p()
        cfg = config._c()
        desc = lm_head.desc()
        _check(self._lib.tbh_decoder_create(backend._dev, ctypes.byref(cfg), emb.ctypes.data,
                                            fn.ctypes.data, ctypes.byref(desc), ctypes.byref(self._h)))
        backend._own(self)

    @classmethod
    def _adopt(cls, backend: HIPBackend, config: DecoderConfig, handle: ctypes.c_void_p) -> "Decoder":
        """Wrap a decoder the library built (tbh_tbf_load_decoder)."""
        d = cls.__new__(cls)
        d._lib = _abi.lib()
        d.backend = backend
        d.config = config
        d._h = handle
        backend._own(d)
        return d

    def set_layer(self, layer: int, input_norm: np.ndarray, post_attention_norm: np.ndarray,
                  projections: Sequence[QuantizedTensor]) -> None:
        """projections: q, k, v, o, gate, up, down (TransformerLayerWeights)."""
        if len(projections) != 7:
            raise PreconditionFailure("need q, k, v, o, gate, up, down")
        gi = np.ascontiguousarray(input_norm, np.float32)
        gp = np.ascontiguousarray(post_attention_norm, np.float32)
        descs = [p.desc() for p in projections]
        _check(self._lib.tbh_decoder_set_layer(self._h, layer, gi.ctypes.data, gp.ctypes.data,
                                               *[ctypes.byref(d) for d in descs]))

    def reset(self) -> None:
        """ModelRunner.reset (ModelRunner.swift:213-216)."""
        self.set_position(0)

    def set_position(self, position: int) -> None:
        _check(self._lib.tbh_decoder_set_position(self._h, position))

    @property
    def position(self) -> int:
        v = ctypes.c_int32()
        _check(self._lib.tbh_decoder_get_position(self._h, ctypes.byref(v)))
        return v.value

    def step(self, token: int) -> np.ndarray:
        """ModelRunner.step (ModelRunner.swift:168-208): logits [vocab]."""
        out = np.empty(self.config.vocab, np.float32)
        _check(self._lib.tbh_decoder_step(self._h, int(token), out.ctypes.data))
        return out

    def step_device(self, token: int, logits=None, stream=None) -> None:
        """Enqueue one step on a torch stream; logits: float32 cuda [vocab] or None."""
        import torch

        s = stream if stream is not None else torch.cuda.current_stream()
        ptr = logits.data_ptr() if logits is not None else None
        _check(self._lib.tbh_decoder_step_device(self._h, int(token), ptr,
                                                 ctypes.c_void_p(s.cuda_stream)))

    def close(self) -> None:
        if self._h:
            self._lib.tbh_decoder_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
