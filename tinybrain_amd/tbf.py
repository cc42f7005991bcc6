"""TBFFile: the .tbf v1 model-file reader (tbh_tbf_* in libtinybrain_hip.so).

Mirrors ModelWeights.load (Sources/TinyBrainRuntime/ModelWeights.swift:496-798):
the file's ModelConfig, its fp32 tensors (embeddings, norms) and its
quantized tensors as QuantizedTensor, plus load_decoder(), which repacks every
projection once into a GPU decoder (ModelWeights.load + ModelRunner).  The
file is memory-mapped by the library; arrays returned here are copies.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List

import numpy as np

from . import _abi
from .backend import HIPBackend, _check
from .decoder import Decoder, DecoderConfig
from .quantized import Layout, QuantizationMode, QuantizationPrecision, QuantizedTensor


class TBFFile:
    def __init__(self, path: str):
        self._lib = _abi.lib()
        self._h = ctypes.c_void_p()
        _check(self._lib.tbh_tbf_open(str(path).encode(), ctypes.byref(self._h)))
        c = _abi.TBFConfig()
        _check(self._lib.tbh_tbf_get_config(self._h, ctypes.byref(c)))
        # ModelConfig (ModelRunner.swift:26-120), keys as the file's JSON
        self.config: Dict = {
            "numLayers": c.num_layers, "hiddenDim": c.hidden, "numHeads": c.num_heads,
            "numKVHeads": c.num_kv_heads, "vocabSize": c.vocab, "maxSeqLen": c.max_seq,
            "intermediateDim": c.intermediate, "partialRotaryFactor": c.partial_rotary_factor,
            "architecture": c.architecture.decode(),
        }
        self._index: Dict[str, int] = {}
        self._info: List[_abi.TBFTensor] = []
        for i in range(self._lib.tbh_tbf_tensor_count(self._h)):
            t = _abi.TBFTensor()
            _check(self._lib.tbh_tbf_tensor(self._h, i, ctypes.byref(t)))
            self._info.append(t)
            self._index[t.name.decode()] = i

    @property
    def names(self) -> List[str]:
        return list(self._index)

    def shape(self, name: str):
        t = self._info[self._index[name]]
        return tuple(t.dims[d] for d in range(t.ndim))

    def is_quantized(self, name: str) -> bool:
        return bool(self._info[self._index[name]].quantized)

    def floats(self, name: str) -> np.ndarray:
        p = ctypes.c_void_p()
        n = ctypes.c_int64()
        _check(self._lib.tbh_tbf_floats(self._h, self._index[name], ctypes.byref(p), ctypes.byref(n)))
        buf = (ctypes.c_float * n.value).from_address(p.value)
        return np.array(buf, dtype=np.float32).reshape(self.shape(name))

    def quantized(self, name: str) -> QuantizedTensor:
        d = _abi.QTensorDesc()
        _check(self._lib.tbh_tbf_qtensor(self._h, self._index[name], ctypes.byref(d)))
        data = np.array((ctypes.c_int8 * d.data_bytes).from_address(d.data), dtype=np.int8)
        scales = np.array((ctypes.c_float * d.n_scales).from_address(d.scales), dtype=np.float32)
        zp = None
        if d.zero_points:
            zp = np.array((ctypes.c_int8 * d.n_zero_points).from_address(d.zero_points), dtype=np.int8)
        return QuantizedTensor((d.K, d.N), data, scales, QuantizationMode(d.mode),
                               QuantizationPrecision(d.precision), d.group_size, zp, Layout(d.layout))

    def load_decoder(self, backend: HIPBackend, max_seq: int = 0) -> Decoder:
        h = ctypes.c_void_p()
        _check(self._lib.tbh_tbf_load_decoder(backend._dev, self._h, max_seq, ctypes.byref(h)))
        c = self.config
        cfg = DecoderConfig(c["numLayers"], c["hiddenDim"], c["numHeads"], c["numKVHeads"],
                            c["intermediateDim"], c["vocabSize"], max_seq or c["maxSeqLen"])
        return Decoder._adopt(backend, cfg, h)

    def close(self) -> None:
        if self._h:
            self._lib.tbh_tbf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
