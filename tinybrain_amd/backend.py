"""HIPBackend: the QuantizedMatMulBackend of TinyBrainHIP.

Mirrors the reference operator interface
``protocol QuantizedMatMulBackend { func matmulQuantized(_ input: Tensor<Float>,
_ quantized: QuantizedTensor) throws -> Tensor<Float> }``
(Sources/TinyBrainRuntime/Backend.swift:173-175) and the way MetalBackend
implements it (Sources/TinyBrainMetal/MetalBackend.swift:894-1048):

  * shape violations are preconditions (traps in Swift; PreconditionFailure
    here), checked before anything else (MetalBackend.swift:895-897);
  * every backend failure raises HIPBackendError -- the Swift wrapper's
    `throw`, on which the unchanged runtime falls back to its CPU path
    (QuantizedTensor.swift:630-642);
  * weights are uploaded once per QuantizedTensor.identifier and kept for the
    backend's lifetime, under a lock (MetalBackend.swift:1282-1308) -- for
    INT4 too, where the reference re-uploads on every call (:1322-1359);
  * results are returned host-resident (numpy), because the reference's
    TensorStorage can only sync from an MTLBuffer (TensorStorage.swift:82-97).

All compute runs in libtinybrain_hip.so; nothing here computes a product.
"""
from __future__ import annotations

import ctypes
import threading
import uuid
from typing import Dict, Optional

import numpy as np

from . import _abi
from .quantized import PreconditionFailure, QuantizedTensor


class HIPBackendError(RuntimeError):
    """A non-zero tbh_status (the reference backend's `throws`)."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{_abi.status_name(status)}: {message}")


def _check(st: int) -> None:
    if st != _abi.OK:
        raise HIPBackendError(st, _abi.last_error())


class DeviceWeight:
    """A weight uploaded and repacked on the device (tbh_weight)."""

    def __init__(self, backend: "HIPBackend", quantized: QuantizedTensor):
        self._lib = _abi.lib()
        self._h = ctypes.c_void_p()
        desc = quantized.desc()
        _check(self._lib.tbh_weight_create(backend._dev, ctypes.byref(desc), ctypes.byref(self._h)))
        self.backend = backend
        self.K, self.N = quantized.shape
        info = _abi.WeightInfo()
        _check(self._lib.tbh_weight_get_info(self._h, ctypes.byref(info)))
        self.path = _abi.PATH_NAMES[info.path]
        self.device_bytes = info.device_bytes
        self.stream_bytes = info.stream_bytes
        self.has_zero_points = bool(info.has_zero_points)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            self._lib.tbh_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HIPBackend:
    """QuantizedMatMulBackend on one gfx950 device."""

    def __init__(self, device: int = 0):
        self._lib = _abi.lib()
        self._dev = ctypes.c_void_p()
        _check(self._lib.tbh_device_open(int(device), ctypes.byref(self._dev)))
        ordinal, cus = ctypes.c_int32(), ctypes.c_int32()
        _check(self._lib.tbh_device_get_info(self._dev, ctypes.byref(ordinal), ctypes.byref(cus)))
        self.device = ordinal.value
        self.cu_count = cus.value
        self._cache: Dict[uuid.UUID, DeviceWeight] = {}
        self._lock = threading.Lock()

    @staticmethod
    def isAvailable(device: int = 0) -> bool:
        """MetalBackend.isAvailable: a gfx950 device can be opened."""
        try:
            L = _abi.lib()
        except OSError:
            return False
        h = ctypes.c_void_p()
        if L.tbh_device_open(int(device), ctypes.byref(h)) != _abi.OK:
            return False
        L.tbh_device_close(h)
        return True

    # -- weights ------------------------------------------------------------
    def weight(self, quantized: QuantizedTensor) -> DeviceWeight:
        """Upload-once cache keyed by QuantizedTensor.identifier."""
        with self._lock:
            w = self._cache.get(quantized.identifier)
            if w is None:
                w = DeviceWeight(self, quantized)
                self._cache[quantized.identifier] = w
            return w

    def evict(self, quantized: QuantizedTensor) -> None:
        with self._lock:
            w = self._cache.pop(quantized.identifier, None)
        if w is not None:
            w.close()

    # -- QuantizedMatMulBackend ----------------------------------------------
    def matmulQuantized(self, input: np.ndarray, quantized: QuantizedTensor) -> np.ndarray:
        """y[M, N] = input[M, K] . dequantize(quantized)[K, N], fp32."""
        x = np.asarray(input)
        if x.ndim != 2:
            raise PreconditionFailure("Input must be 2D")
        if len(quantized.shape) != 2:
            raise PreconditionFailure("Weights must be 2D")
        if x.shape[1] != quantized.shape[0]:
            raise PreconditionFailure("Dimensions must match")
        x = np.ascontiguousarray(x, np.float32)       # makeContiguousCopy
        w = self.weight(quantized)
        m = x.shape[0]
        y = np.empty((m, quantized.shape[1]), np.float32)
        _check(self._lib.tbh_matmul(self._dev, x.ctypes.data, m, x.shape[1], w.handle, y.ctypes.data))
        return y

    def dequantize(self, quantized: QuantizedTensor) -> np.ndarray:
        """The uploaded weight as fp32 [K, N] (see tbh_dequantize)."""
        w = self.weight(quantized)
        out = np.empty(quantized.shape, np.float32)
        _check(self._lib.tbh_dequantize(self._dev, w.handle, out.ctypes.data))
        return out

    # -- device-resident entry (torch tensors on this device) -----------------
    def matmul_device(self, x, weight: DeviceWeight, out=None, stream=None):
        """Enqueue y = x . W on a HIP stream with GPU-resident torch tensors.

        x: float32 [M, K] contiguous cuda tensor; returns float32 [M, N]."""
        import torch

        if x.dim() != 2 or x.shape[1] != weight.K:
            raise PreconditionFailure("Dimensions must match")
        if x.dtype != torch.float32 or not x.is_contiguous() or not x.is_cuda:
            raise PreconditionFailure("x must be a contiguous float32 device tensor")
        if out is None:
            out = torch.empty((x.shape[0], weight.N), dtype=torch.float32, device=x.device)
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        _check(self._lib.tbh_matmul_device(weight.handle, x.data_ptr(), x.shape[0], x.shape[1],
                                           out.data_ptr(), ctypes.c_void_p(s.cuda_stream)))
        return out

    def matmul_bf16_device(self, x, weight: DeviceWeight, out=None, stream=None):
        """Prefill: enqueue y = x . W for bf16 activations on bf16 MFMA.

        x: bfloat16 [M, K] contiguous cuda tensor (K % 8 == 0); returns
        float32 [M, N].  See tbh_matmul_bf16_device."""
        import torch

        if x.dim() != 2 or x.shape[1] != weight.K:
            raise PreconditionFailure("Dimensions must match")
        if x.dtype != torch.bfloat16 or not x.is_contiguous() or not x.is_cuda:
            raise PreconditionFailure("x must be a contiguous bfloat16 device tensor")
        if out is None:
            out = torch.empty((x.shape[0], weight.N), dtype=torch.float32, device=x.device)
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        _check(self._lib.tbh_matmul_bf16_device(weight.handle, x.data_ptr(), x.shape[0], x.shape[1],
                                                out.data_ptr(), ctypes.c_void_p(s.cuda_stream)))
        return out

    def dequantize_device(self, weight: DeviceWeight, out=None, stream=None):
        import torch

        if out is None:
            out = torch.empty((weight.K, weight.N), dtype=torch.float32,
                              device=torch.device("cuda", self.device))
        s = stream if stream is not None else torch.cuda.current_stream(out.device)
        _check(self._lib.tbh_dequantize_device(weight.handle, out.data_ptr(),
                                               ctypes.c_void_p(s.cuda_stream)))
        return out

    def close(self) -> None:
        with self._lock:
            ws = list(self._cache.values())
            self._cache.clear()
        for w in ws:
            w.close()
        if self._dev:
            self._lib.tbh_device_close(self._dev)
            self._dev = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
