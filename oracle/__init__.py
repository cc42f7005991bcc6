"""CPU oracle for TinyBrain's INT8/INT4 quantized-matmul path.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package; the product (``tinybrain_amd``) never does, and fails
loudly when its HIP library is missing instead of falling back here.

The arithmetic lives in ``tbh_oracle.c`` (a C restatement of the reference's
Swift ``QuantizedTensor`` / ``Tensor.matmulCPU`` code, each function citing the
reference file:line it follows).  This module is a thin numpy/ctypes shim over
``_build/libtbh_oracle.so``; build it with ``make -C oracle``.

Parity pins (what checks each function beyond retyping it) are in
``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import time
import os
import subprocess
from dataclasses import dataclass
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB: another build of the same source (the sanitizer build of
# `make -C oracle asan`)
_LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "_build", "libtbh_oracle.so")

# QuantizationMode (QuantizedTensor.swift:31-37) and precision codes
MODE_SYMMETRIC, MODE_ASYMMETRIC, MODE_PER_CHANNEL, MODE_INT4, MODE_INT4_PER_CHANNEL = range(5)
PREC_INT8, PREC_INT4 = 1, 2
ROUND_SWIFT, ROUND_NUMPY = 0, 1
OK, E_INVALID, E_TRAP = 0, 1, 2


class _QT(ctypes.Structure):
    _fields_ = [
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 2),
        ("data", ctypes.c_void_p),
        ("data_count", ctypes.c_int64),
        ("scales", ctypes.c_void_p),
        ("n_scales", ctypes.c_int64),
        ("zero_points", ctypes.c_void_p),
        ("n_zero_points", ctypes.c_int64),
        ("mode", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("group_size", ctypes.c_int64),
    ]


def build() -> str:
    """Compile the oracle library with its Makefile; returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i64, i32, f32p = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
        L.orc_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_double, ctypes.c_double, vp, i64]
        L.orc_pack_int4.argtypes = [ctypes.c_int8, ctypes.c_int8]
        L.orc_pack_int4.restype = ctypes.c_int8
        L.orc_unpack_int4.argtypes = [ctypes.c_int8, vp, vp]
        L.orc_int4_at.argtypes = [vp, i64]
        L.orc_int4_at.restype = i32
        L.orc_quantize_per_channel.argtypes = [vp, i64, i64, vp, vp, i32]
        L.orc_quantize_symmetric.argtypes = [vp, i64, vp, vp, i32]
        L.orc_quantize_asymmetric.argtypes = [vp, i64, vp, vp, vp, i32]
        L.orc_quantize_asymmetric.restype = i32
        L.orc_quantize_int4.argtypes = [vp, i64, i64, vp, vp, vp, i32]
        L.orc_quantize_int4_per_channel.argtypes = [vp, i64, i64, vp, vp, i32]
        L.orc_convert_int8_per_channel.argtypes = [vp, i64, i64, vp, vp]
        L.orc_validate.argtypes = [ctypes.POINTER(_QT)]
        L.orc_validate.restype = i32
        L.orc_dequantize.argtypes = [ctypes.POINTER(_QT), vp]
        L.orc_dequantize.restype = i32
        L.orc_sgemm.argtypes = [i64, i64, i64, vp, vp, vp, i32]
        L.orc_gemm_f64.argtypes = [i64, i64, i64, vp, vp, vp, i32]
        L.orc_matmul_quantized_cpu.argtypes = [vp, i64, ctypes.POINTER(_QT), vp, i32,
                                               ctypes.POINTER(ctypes.c_double),
                                               ctypes.POINTER(ctypes.c_double)]
        L.orc_matmul_quantized_cpu.restype = i32
        L.orc_matmul_quantized_fused.argtypes = [vp, i64, ctypes.POINTER(_QT), vp, i32, i32]
        L.orc_matmul_quantized_fused.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


@dataclass
class QTensor:
    """Oracle-side mirror of struct QuantizedTensor (QuantizedTensor.swift:62-166)."""
    shape: tuple
    data: np.ndarray            # int8
    scales: np.ndarray          # float32
    zero_points: Optional[np.ndarray]  # int8 or None
    mode: int
    precision: int
    group_size: int = 0

    def _c(self) -> _QT:
        q = _QT()
        q.rank = len(self.shape)
        q.dims[0] = self.shape[0]
        q.dims[1] = self.shape[1] if len(self.shape) > 1 else 0
        self._keep = [np.ascontiguousarray(self.data, np.int8),
                      np.ascontiguousarray(self.scales, np.float32)]
        q.data = _p(self._keep[0])
        q.data_count = self._keep[0].size
        q.scales = _p(self._keep[1])
        q.n_scales = self._keep[1].size
        if self.zero_points is not None:
            self._keep.append(np.ascontiguousarray(self.zero_points, np.int8))
            q.zero_points = _p(self._keep[2])
            q.n_zero_points = self._keep[2].size
        else:
            q.zero_points = None
            q.n_zero_points = 0
        q.mode = self.mode
        q.precision = self.precision
        q.group_size = self.group_size
        return q


def fill_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(seed, mean, std, _p(out), n)
    return out


def pack_int4(v1: int, v2: int) -> int:
    return int(lib().orc_pack_int4(v1, v2))


def unpack_int4(b: int) -> tuple:
    a = ctypes.c_int8()
    c = ctypes.c_int8()
    lib().orc_unpack_int4(ctypes.c_int8(b), ctypes.byref(a), ctypes.byref(c))
    return a.value, c.value


def quantize_per_channel(w: np.ndarray, rounding: int = ROUND_SWIFT) -> QTensor:
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty(w.shape, np.int8)
    s = np.empty(cols, np.float32)
    lib().orc_quantize_per_channel(_p(w), rows, cols, _p(q), _p(s), rounding)
    return QTensor(w.shape, q.reshape(-1), s, None, MODE_PER_CHANNEL, PREC_INT8)


def quantize_symmetric(w: np.ndarray, rounding: int = ROUND_SWIFT) -> QTensor:
    w = np.ascontiguousarray(w, np.float32)
    q = np.empty(w.size, np.int8)
    s = np.empty(1, np.float32)
    lib().orc_quantize_symmetric(_p(w), w.size, _p(q), _p(s), rounding)
    return QTensor(w.shape, q, s, None, MODE_SYMMETRIC, PREC_INT8)


def quantize_asymmetric(w: np.ndarray, rounding: int = ROUND_SWIFT) -> Optional[QTensor]:
    w = np.ascontiguousarray(w, np.float32)
    q = np.empty(w.size, np.int8)
    s = np.empty(1, np.float32)
    z = np.empty(1, np.int8)
    st = lib().orc_quantize_asymmetric(_p(w), w.size, _p(q), _p(s), _p(z), rounding)
    if st != OK:
        return None
    return QTensor(w.shape, q, s, z, MODE_ASYMMETRIC, PREC_INT8)


def quantize_int4(w: np.ndarray, group_size: int = 32, rounding: int = ROUND_SWIFT,
                  shape: Optional[tuple] = None) -> QTensor:
    """Flat per-group INT4 over w's C-order flattening.  ``shape`` is the
    shape recorded in the tensor (default w.shape)."""
    w = np.ascontiguousarray(w, np.float32)
    n = w.size
    groups = (n + group_size - 1) // group_size
    packed = np.empty((n + 1) // 2, np.int8)
    s = np.empty(groups, np.float32)
    z = np.empty(groups, np.int8)
    lib().orc_quantize_int4(_p(w), n, group_size, _p(packed), _p(s), _p(z), rounding)
    return QTensor(tuple(shape or w.shape), packed, s, z, MODE_INT4, PREC_INT4, group_size)


def quantize_int4_per_channel(w: np.ndarray, rounding: int = ROUND_SWIFT) -> QTensor:
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    packed = np.empty((w.size + 1) // 2, np.int8)
    s = np.empty(cols, np.float32)
    lib().orc_quantize_int4_per_channel(_p(w), rows, cols, _p(packed), _p(s), rounding)
    return QTensor(w.shape, packed, s, None, MODE_INT4_PER_CHANNEL, PREC_INT4, 0)


def convert_int8_per_channel(w_nk: np.ndarray) -> tuple:
    """Converter INT8 (convert_model.py:383-395) on a PyTorch [N, K] weight;
    returns (q_nk int8, scales float32)."""
    w = np.ascontiguousarray(w_nk, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().orc_convert_int8_per_channel(_p(w), n, k, _p(q), _p(s))
    return q, s


def validate(qt: QTensor) -> int:
    c = qt._c()
    return int(lib().orc_validate(ctypes.byref(c)))


def dequantize(qt: QTensor) -> np.ndarray:
    """QuantizedTensor.dequantize() -> float32 array of qt.shape."""
    c = qt._c()
    count = int(np.prod(qt.shape))
    out = np.empty(count, np.float32)
    st = lib().orc_dequantize(ctypes.byref(c), _p(out))
    if st != OK:
        raise ValueError(f"oracle dequantize status {st}")
    return out.reshape(qt.shape)


def sgemm(a: np.ndarray, b: np.ndarray, threads: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().orc_sgemm(m, n, k, _p(a), _p(b), _p(c), threads)
    return c


def gemm_f64(a: np.ndarray, b: np.ndarray, threads: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float64)
    lib().orc_gemm_f64(m, n, k, _p(a), _p(b), _p(c), threads)
    return c


def matmul_quantized_cpu(x: np.ndarray, qt: QTensor, threads: int = 0):
    """Reference CPU path (QuantizedTensor.swift:640-642): dequantize() then
    matmulCPU.  Returns (y, dequant_seconds, gemm_seconds)."""
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    n = qt.shape[1]
    y = np.empty((m, n), np.float32)
    c = qt._c()
    td = ctypes.c_double()
    tg = ctypes.c_double()
    st = lib().orc_matmul_quantized_cpu(_p(x), m, ctypes.byref(c), _p(y), threads,
                                        ctypes.byref(td), ctypes.byref(tg))
    if st != OK:
        raise ValueError(f"oracle matmul status {st}")
    return y, td.value, tg.value


def matmul_quantized_fused(x: np.ndarray, qt: QTensor, threads: int = 0, nk: bool = False):
    """Best-effort CPU fused dequant-GEMV (not a reference function: the host
    upper bound reported beside the reference path).  nk: the weight's flat
    data holds element (k, n) at n*K + k (the converter's INT4 storage).
    Returns (y, seconds)."""
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    y = np.empty((m, qt.shape[1]), np.float32)
    c = qt._c()
    t0 = time.perf_counter()
    st = lib().orc_matmul_quantized_fused(_p(x), m, ctypes.byref(c), _p(y), threads, int(nk))
    dt = time.perf_counter() - t0
    if st != OK:
        raise ValueError(f"oracle fused matmul status {st}")
    return y, dt


def parity_errors(y_hat: np.ndarray, y64: np.ndarray) -> dict:
    """Error figures of a GPU result against the float64 oracle.

    gated:  max|y^ - y| / max(|y|, 1e-3 * max_row|y|)   (must be <= 1e-3)
    also:   unfloored max relative error, L2 relative error (the reference's
            relativeError, QuantizationTests.swift:236-252)."""
    y_hat = np.asarray(y_hat, np.float64)
    y64 = np.asarray(y64, np.float64)
    diff = np.abs(y_hat - y64)
    row_inf = np.max(np.abs(y64), axis=-1, keepdims=True) if y64.size else y64
    floor = np.maximum(np.abs(y64), 1e-3 * row_inf)
    with np.errstate(divide="ignore", invalid="ignore"):
        gated = np.where(floor > 0, diff / floor, np.where(diff > 0, np.inf, 0.0))
        unfloored = np.where(np.abs(y64) > 0, diff / np.abs(y64), np.where(diff > 0, np.inf, 0.0))
    l2 = float(np.linalg.norm(y_hat - y64) / max(np.linalg.norm(y64), np.finfo(np.float32).tiny))
    return {
        "gated": float(gated.max()) if gated.size else 0.0,
        "unfloored": float(unfloored.max()) if unfloored.size else 0.0,
        "l2": l2,
    }
