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

The same class also implements the reference's other backend protocols
(Backend.swift:177-228) -- SoftmaxBackend.softmax, RMSNormBackend.rmsnorm,
ActivationBackend.silu / gelu and AttentionBackend.attention -- with the
shape rules of MetalBackend's implementations (MetalBackend.swift:1062-1260,
1362-1525).

All compute runs in libtinybrain_hip.so; nothing here computes a product.
"""
from __future__ import annotations

import ctypes
import threading
import uuid
import weakref
from typing import Dict, Optional, Sequence

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

    def __init__(self, backend: "HIPBackend", quantized: Optional[QuantizedTensor], _handle=None):
        self._lib = _abi.lib()
        self._h = ctypes.c_void_p()
        if _handle is None:
            desc = quantized.desc()
            _check(self._lib.tbh_weight_create(backend._dev, ctypes.byref(desc), ctypes.byref(self._h)))
        else:
            self._h = _handle
        self.backend = backend
        backend._own(self)
        info = _abi.WeightInfo()
        _check(self._lib.tbh_weight_get_info(self._h, ctypes.byref(info)))
        self.K, self.N = info.K, info.N
        self.path = _abi.PATH_NAMES[info.path]
        self.device_bytes = info.device_bytes
        self.stream_bytes = info.stream_bytes
        self.has_zero_points = bool(info.has_zero_points)

    @classmethod
    def concat(cls, backend: "HIPBackend", parts: Sequence[QuantizedTensor]) -> "DeviceWeight":
        """One weight computing every part's outputs side by side
        (tbh_weight_create_concat): x . [W_0 | W_1 | ...] in one launch, for
        projections that read the same input (q, k, v; gate, up)."""
        lib = _abi.lib()
        descs = [p.desc() for p in parts]
        arr = (ctypes.POINTER(_abi.QTensorDesc) * len(descs))(*[ctypes.pointer(d) for d in descs])
        h = ctypes.c_void_p()
        _check(lib.tbh_weight_create_concat(backend._dev, len(descs), arr, ctypes.byref(h)))
        return cls(backend, None, _handle=h)

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
        # every weight and decoder made on this device: closed before the
        # device, whose handle their own teardown reads.  A lock of its own:
        # weight() holds _lock while it builds the DeviceWeight that registers.
        self._children = weakref.WeakSet()
        self._children_lock = threading.Lock()

    def _own(self, child) -> None:
        with self._children_lock:
            self._children.add(child)

    def set_option(self, option: int, value: int) -> None:
        """tbh_device_set_option: a launch-rule override (e.g.
        ``_abi.OPT_SGEMV_MIN_ROWS``; 0 restores the rule)."""
        _check(self._lib.tbh_device_set_option(self._dev, int(option), int(value)))

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

    def matmul_device_noalloc(self, x, weight: DeviceWeight, out=None, stream=None):
        """matmul_device through tbh_matmul_device_noalloc: no device memory
        is allocated by the call (for code under graph capture); `out` must
        then be given.  Calls overlapping on one GPU race on its scratch."""
        import torch

        if x.dim() != 2 or x.shape[1] != weight.K:
            raise PreconditionFailure("Dimensions must match")
        if x.dtype != torch.float32 or not x.is_contiguous() or not x.is_cuda:
            raise PreconditionFailure("x must be a contiguous float32 device tensor")
        if out is None or tuple(out.shape) != (x.shape[0], weight.N) or not out.is_contiguous():
            raise PreconditionFailure("out must be a contiguous float32 [M, N] device tensor")
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        _check(self._lib.tbh_matmul_device_noalloc(weight.handle, x.data_ptr(), x.shape[0], x.shape[1],
                                                   out.data_ptr(), ctypes.c_void_p(s.cuda_stream)))
        return out

    def linear_device(self, x, weight: DeviceWeight, bias=None, out=None, stream=None):
        """Enqueue y = x . W (+ bias[n] on every row) on a HIP stream
        (tbh_linear_device; LinearLayerWeights.apply(toRow:),
        ModelWeights.swift:47-68).  bias: None or a float32 [N] cuda tensor."""
        import torch

        if x.dim() != 2 or x.shape[1] != weight.K:
            raise PreconditionFailure("Dimensions must match")
        if x.dtype != torch.float32 or not x.is_contiguous() or not x.is_cuda:
            raise PreconditionFailure("x must be a contiguous float32 device tensor")
        if bias is not None:
            if tuple(bias.shape) != (weight.N,):
                raise PreconditionFailure("Bias must match output dimension")
            if bias.dtype != torch.float32 or not bias.is_contiguous() or not bias.is_cuda:
                raise PreconditionFailure("bias must be a contiguous float32 device tensor")
        if out is None:
            out = torch.empty((x.shape[0], weight.N), dtype=torch.float32, device=x.device)
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        _check(self._lib.tbh_linear_device(weight.handle, x.data_ptr(), x.shape[0], x.shape[1],
                                           None if bias is None else bias.data_ptr(), out.data_ptr(),
                                           ctypes.c_void_p(s.cuda_stream)))
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

    # -- SoftmaxBackend / RMSNormBackend / ActivationBackend / AttentionBackend --
    def softmax(self, input: np.ndarray) -> np.ndarray:
        """Softmax along the last dimension, rows summing to 1
        (MetalBackend.swift:1073-1134; empty input is returned as is)."""
        x = np.ascontiguousarray(input, np.float32)
        if x.size == 0:
            return x
        if x.ndim == 0:
            raise PreconditionFailure("Cannot apply softmax to empty tensor")
        y = np.empty_like(x)
        cols = x.shape[-1]
        _check(self._lib.tbh_softmax(self._dev, x.ctypes.data, x.size // cols, cols, y.ctypes.data))
        return y

    def rmsnorm(self, input: np.ndarray, weight: np.ndarray, eps: float = 1e-5) -> np.ndarray:
        """x / rms(x) * weight per row of a [tokens, hidden] tensor
        (MetalBackend.swift:1146-1207)."""
        x = np.ascontiguousarray(input, np.float32)
        g = np.ascontiguousarray(weight, np.float32).reshape(-1)
        if x.ndim != 2:
            raise PreconditionFailure("rmsnorm input must be 2-D [tokens, hidden]")
        if g.size != x.shape[1]:
            raise PreconditionFailure("weight size must equal hiddenDim")
        y = np.empty_like(x)
        _check(self._lib.tbh_rmsnorm(self._dev, x.ctypes.data, x.shape[0], x.shape[1], g.ctypes.data,
                                     float(eps), y.ctypes.data))
        return y

    def _elementwise(self, fn, input: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(input, np.float32)
        if x.size == 0:
            return x
        y = np.empty_like(x)
        _check(fn(self._dev, x.ctypes.data, x.size, y.ctypes.data))
        return y

    def silu(self, input: np.ndarray) -> np.ndarray:
        """out = x * sigmoid(x) (MetalBackend.swift:1214-1216)."""
        return self._elementwise(self._lib.tbh_silu, input)

    def gelu(self, input: np.ndarray) -> np.ndarray:
        """GELU, tanh approximation (MetalBackend.swift:1221-1223)."""
        return self._elementwise(self._lib.tbh_gelu, input)

    @staticmethod
    def _attention_shape(q, k, v, mask, headDim, numHeads, numKVHeads):
        if not (numHeads >= numKVHeads and numKVHeads > 0 and numHeads % numKVHeads == 0):
            raise PreconditionFailure("numHeads must be a multiple of numKVHeads")
        if q.ndim == 3:
            batch, seq, kv = q.shape[0], q.shape[1], k.shape[1]
        else:
            batch, seq, kv = 1, q.shape[0], k.shape[0]
        if (q.shape[-1] != numHeads * headDim or k.shape[-1] != numKVHeads * headDim
                or tuple(v.shape) != tuple(k.shape) or k.ndim != q.ndim
                or (q.ndim == 3 and k.shape[0] != batch)):
            raise PreconditionFailure("attention: query/keys/values shapes do not match the heads")
        if mask is not None and (mask.numel() if hasattr(mask, "numel") else mask.size) != kv:
            raise PreconditionFailure("attention: mask must have kvSeqLen elements")
        return _abi.AttentionShape(batch, seq, kv, headDim, numHeads, numKVHeads)

    def attention(self, query: np.ndarray, keys: np.ndarray, values: np.ndarray,
                  mask: Optional[np.ndarray], headDim: int, numHeads: int, numKVHeads: int) -> np.ndarray:
        """softmax(Q K^T / sqrt(headDim) + mask) V per head with GQA
        (MetalBackend.swift:1381-1525); returns an array shaped like query."""
        q = np.ascontiguousarray(query, np.float32)
        k = np.ascontiguousarray(keys, np.float32)
        v = np.ascontiguousarray(values, np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, np.float32).reshape(-1)
        sh = self._attention_shape(q, k, v, m, headDim, numHeads, numKVHeads)
        out = np.empty_like(q)
        _check(self._lib.tbh_attention(self._dev, ctypes.byref(sh), q.ctypes.data, k.ctypes.data,
                                       v.ctypes.data, None if m is None else m.ctypes.data, out.ctypes.data))
        return out

    # device-resident variants: contiguous float32 torch tensors on this device
    def _stream(self, t, stream):
        import torch

        return ctypes.c_void_p((stream if stream is not None else torch.cuda.current_stream(t.device)).cuda_stream)

    @staticmethod
    def _dev_tensor(t):
        import torch

        if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise PreconditionFailure("expected a contiguous float32 device tensor")
        return t

    def softmax_device(self, x, out=None, stream=None):
        import torch

        x = self._dev_tensor(x)
        out = torch.empty_like(x) if out is None else self._dev_tensor(out)
        if x.numel():
            cols = x.shape[-1]
            _check(self._lib.tbh_softmax_device(self._dev, x.data_ptr(), x.numel() // cols, cols,
                                                out.data_ptr(), self._stream(x, stream)))
        return out

    def rmsnorm_device(self, x, weight, eps: float = 1e-5, out=None, stream=None):
        import torch

        x, weight = self._dev_tensor(x), self._dev_tensor(weight)
        if x.dim() != 2 or weight.numel() != x.shape[1]:
            raise PreconditionFailure("rmsnorm: x [tokens, hidden] and weight [hidden]")
        out = torch.empty_like(x) if out is None else self._dev_tensor(out)
        _check(self._lib.tbh_rmsnorm_device(self._dev, x.data_ptr(), x.shape[0], x.shape[1], weight.data_ptr(),
                                            float(eps), out.data_ptr(), self._stream(x, stream)))
        return out

    def silu_device(self, x, out=None, stream=None):
        import torch

        x = self._dev_tensor(x)
        out = torch.empty_like(x) if out is None else self._dev_tensor(out)
        _check(self._lib.tbh_silu_device(self._dev, x.data_ptr(), x.numel(), out.data_ptr(),
                                         self._stream(x, stream)))
        return out

    def gelu_device(self, x, out=None, stream=None):
        import torch

        x = self._dev_tensor(x)
        out = torch.empty_like(x) if out is None else self._dev_tensor(out)
        _check(self._lib.tbh_gelu_device(self._dev, x.data_ptr(), x.numel(), out.data_ptr(),
                                         self._stream(x, stream)))
        return out

    def attention_device(self, query, keys, values, mask, headDim: int, numHeads: int, numKVHeads: int,
                         out=None, stream=None):
        import torch

        q, k, v = self._dev_tensor(query), self._dev_tensor(keys), self._dev_tensor(values)
        m = None if mask is None else self._dev_tensor(mask)
        sh = self._attention_shape(q, k, v, m, headDim, numHeads, numKVHeads)
        out = torch.empty_like(q) if out is None else self._dev_tensor(out)
        _check(self._lib.tbh_attention_device(self._dev, ctypes.byref(sh), q.data_ptr(), k.data_ptr(),
                                              v.data_ptr(), None if m is None else m.data_ptr(),
                                              out.data_ptr(), self._stream(q, stream)))
        return out

    def close(self) -> None:
        with self._lock:
            cached = list(self._cache.values())
            self._cache.clear()
        with self._children_lock:
            children = list(self._children) + cached
            self._children.clear()
        for c in children:
            c.close()
        if self._dev:
            self._lib.tbh_device_close(self._dev)
            self._dev = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
