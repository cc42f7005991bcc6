"""Host-side mirror of TinyBrain's quantized tensor API.

``QuantizedTensor`` carries the fields of the Swift struct
(Sources/TinyBrainRuntime/QuantizedTensor.swift:62-166) plus the flat-array
``layout`` this backend needs to tell the converter's INT4 order apart
(Scripts/convert_model.py:489-502 records a reversed shape over untransposed
data).  ``quantize`` restates ``Tensor.quantize(mode:groupSize:)``
(QuantizedTensor.swift:359-606) with numpy, bit for bit, so callers outside
Swift can produce the same arrays.
"""
from __future__ import annotations

import enum
import uuid
from dataclasses import dataclass, field
from typing import Optional, Tuple

import numpy as np

from . import _abi


class QuantizationMode(enum.IntEnum):
    """QuantizationMode, QuantizedTensor.swift:31-37."""
    symmetric = _abi.MODE_SYMMETRIC
    asymmetric = _abi.MODE_ASYMMETRIC
    perChannel = _abi.MODE_PER_CHANNEL
    int4 = _abi.MODE_INT4
    int4PerChannel = _abi.MODE_INT4_PER_CHANNEL


class QuantizationPrecision(enum.IntEnum):
    """QuantizationPrecision, QuantizedTensor.swift:40-57 (TBF codes)."""
    int8 = _abi.PREC_INT8
    int4 = _abi.PREC_INT4

    @property
    def bits(self) -> int:
        return 8 if self is QuantizationPrecision.int8 else 4

    @property
    def maxValue(self) -> int:
        return 127 if self is QuantizationPrecision.int8 else 7


class Layout(enum.IntEnum):
    """Order of the flat element array of a [K, N] weight."""
    KN_FLAT = _abi.LAYOUT_KN_FLAT   # runtime: i = k*N + n
    NK_FLAT = _abi.LAYOUT_NK_FLAT   # converter INT4: i = n*K + k


class PreconditionFailure(AssertionError):
    """A Swift `precondition` of the reference failed (a trap there)."""


@dataclass
class QuantizedTensor:
    shape: Tuple[int, int]                 # [K, N] = [in, out]
    data: np.ndarray                       # int8; packed nibbles for INT4
    scales: np.ndarray                     # float32
    mode: QuantizationMode
    precision: QuantizationPrecision = QuantizationPrecision.int8
    groupSize: int = 0
    zeroPoints: Optional[np.ndarray] = None
    layout: Layout = Layout.KN_FLAT
    identifier: uuid.UUID = field(default_factory=uuid.uuid4)

    def __post_init__(self):
        self.data = np.ascontiguousarray(self.data, dtype=np.int8).reshape(-1)
        self.scales = np.ascontiguousarray(self.scales, dtype=np.float32).reshape(-1)
        if self.zeroPoints is not None:
            self.zeroPoints = np.ascontiguousarray(self.zeroPoints, dtype=np.int8).reshape(-1)
        self.mode = QuantizationMode(self.mode)
        self.precision = QuantizationPrecision(self.precision)
        self.layout = Layout(self.layout)
        self.shape = tuple(int(d) for d in self.shape)
        # QuantizedTensor.init preconditions, QuantizedTensor.swift:124-155
        count = int(np.prod(self.shape))
        if self.precision is QuantizationPrecision.int8:
            _require(self.data.size == count, "INT8: data count must match shape")
        else:
            _require(self.data.size == (count + 1) // 2,
                     "INT4: data count should be ceil(shape.count / 2)")
        if self.mode in (QuantizationMode.perChannel, QuantizationMode.int4PerChannel):
            ch = self.shape[1] if len(self.shape) >= 2 else self.shape[0]
            _require(self.scales.size == ch, "Per-channel: need one scale per output channel")
        elif self.mode in (QuantizationMode.symmetric, QuantizationMode.asymmetric):
            _require(self.scales.size == 1, "Per-tensor: need single scale")
        elif self.groupSize > 0:
            _require(self.scales.size == (count + self.groupSize - 1) // self.groupSize,
                     "INT4 per-group: need one scale per group")
        else:
            _require(self.scales.size == 1, "INT4 per-tensor: need single scale")
        if self.zeroPoints is not None:
            _require(self.zeroPoints.size == self.scales.size, "Zero points must match scales")

    @property
    def byteSize(self) -> int:
        """QuantizedTensor.byteSize, QuantizedTensor.swift:288-292."""
        zp = 0 if self.zeroPoints is None else self.zeroPoints.size
        return self.data.size + 4 * self.scales.size + zp

    def desc(self) -> "_abi.QTensorDesc":
        """The C descriptor (pointers borrow this object's arrays)."""
        _require(len(self.shape) == 2, "Weights must be 2D")
        d = _abi.QTensorDesc()
        d.K, d.N = self.shape
        d.precision = int(self.precision)
        d.mode = int(self.mode)
        d.layout = int(self.layout)
        d.group_size = int(self.groupSize)
        d.data = self.data.ctypes.data
        d.data_bytes = self.data.size
        d.scales = self.scales.ctypes.data
        d.n_scales = self.scales.size
        if self.zeroPoints is not None:
            d.zero_points = self.zeroPoints.ctypes.data
            d.n_zero_points = self.zeroPoints.size
        return d


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise PreconditionFailure(msg)


# ---------------------------------------------------------------------------
# INT4 nibbles (QuantizedTensor.swift:314-331)
# ---------------------------------------------------------------------------
def packInt4(value1: int, value2: int) -> int:
    v1 = max(-7, min(7, int(value1))) & 0x0F
    v2 = max(-7, min(7, int(value2))) & 0x0F
    return int(np.uint8((v1 << 4) | v2).view(np.int8))


def unpackInt4(packed: int) -> Tuple[int, int]:
    b = int(np.int8(packed).view(np.uint8))
    hi, lo = (b >> 4) & 0x0F, b & 0x0F
    return (hi - 16 if hi > 7 else hi, lo - 16 if lo > 7 else lo)


def unpack_int4_array(data: np.ndarray, count: int) -> np.ndarray:
    """Flat INT4 decode of `count` elements (even index = high nibble)."""
    b = np.ascontiguousarray(data, np.int8).view(np.uint8)
    nib = np.empty(b.size * 2, np.int8)
    nib[0::2] = (b >> 4).astype(np.int8)
    nib[1::2] = (b & 0x0F).astype(np.int8)
    nib = nib[:count]
    return np.where(nib > 7, nib - 16, nib).astype(np.int8)


def pack_int4_array(q: np.ndarray) -> np.ndarray:
    """Pack int values (clamped to [-7, 7]) two per byte, even -> high."""
    q = np.clip(np.asarray(q, np.int32).reshape(-1), -7, 7)
    if q.size % 2:
        q = np.concatenate([q, np.zeros(1, np.int32)])
        hi, lo = q[0::2], q[1::2]
        out = ((hi & 0xF) << 4) | (lo & 0xF)
        out[-1] = (hi[-1] & 0xF) << 4
    else:
        hi, lo = q[0::2], q[1::2]
        out = ((hi & 0xF) << 4) | (lo & 0xF)
    return out.astype(np.uint8).view(np.int8)


# ---------------------------------------------------------------------------
# Quantizers (QuantizedTensor.swift:359-606)
# ---------------------------------------------------------------------------
_LEAST_NONZERO = np.float32(np.finfo(np.float32).smallest_subnormal)


def _round_swift(v: np.ndarray) -> np.ndarray:
    """Swift Float.round(): half away from zero, exact in fp32."""
    t = np.trunc(v)
    f = v - t
    return (t + np.where(np.abs(f) >= np.float32(0.5), np.sign(v), np.float32(0))).astype(np.float32)


def _scale(abs_max: np.ndarray, levels: float) -> np.ndarray:
    abs_max = np.asarray(abs_max, np.float32)
    return np.where(abs_max < _LEAST_NONZERO, np.float32(1.0),
                    abs_max / np.float32(levels)).astype(np.float32)


def quantize(w: np.ndarray, mode: QuantizationMode = QuantizationMode.perChannel,
             groupSize: int = 32) -> QuantizedTensor:
    """Tensor.quantize(mode:groupSize:), QuantizedTensor.swift:359-372, for a
    2-D fp32 weight w of shape [K, N] (runtime layout)."""
    w = np.ascontiguousarray(w, np.float32)
    mode = QuantizationMode(mode)
    if mode is QuantizationMode.perChannel:
        return _quantize_per_channel(w)
    if mode is QuantizationMode.int4:
        return quantize_int4_flat(w, groupSize, shape=w.shape, layout=Layout.KN_FLAT)
    if mode is QuantizationMode.symmetric:
        return _quantize_symmetric(w)
    if mode is QuantizationMode.asymmetric:
        return _quantize_asymmetric(w)
    return _quantize_int4_per_channel(w)


def _quantize_per_channel(w):
    # QuantizedTensor.swift:379-424
    _require(w.ndim == 2, "Per-channel quantization requires 2D tensor")
    s = _scale(np.abs(w).max(axis=0), 127.0)
    q = np.clip(_round_swift(w / s[None, :]), -127, 127).astype(np.int8)
    return QuantizedTensor(w.shape, q.reshape(-1), s, QuantizationMode.perChannel)


def _quantize_symmetric(w):
    # QuantizedTensor.swift:427-449
    flat = w.reshape(-1)
    abs_max = np.float32(max(abs(flat.min()), abs(flat.max()))) if flat.size else np.float32(0)
    s = np.float32(abs_max / np.float32(127)) if abs_max > _LEAST_NONZERO else np.float32(1)
    q = np.clip(_round_swift(flat / s), -127, 127).astype(np.int8)
    return QuantizedTensor(w.shape, q, np.array([s], np.float32), QuantizationMode.symmetric)


def _quantize_asymmetric(w):
    # QuantizedTensor.swift:452-476 (traps where Int8(zeroPoint) overflows)
    flat = w.reshape(-1)
    mn = np.float32(flat.min()) if flat.size else np.float32(0)
    mx = np.float32(flat.max()) if flat.size else np.float32(0)
    rng = np.float32(mx - mn)
    s = np.float32(rng / np.float32(255)) if rng > _LEAST_NONZERO else np.float32(1)
    zf = _round_swift(np.array([np.float32(-mn / s) - np.float32(128)], np.float32))[0]
    _require(-128 <= zf <= 127, "Int8(zeroPoint) out of range")
    zp = np.int8(zf)
    qv = _round_swift(flat / s) + np.float32(zp)
    q = np.clip(qv, -128, 127).astype(np.int8)
    return QuantizedTensor(w.shape, q, np.array([s], np.float32), QuantizationMode.asymmetric,
                           zeroPoints=np.array([zp], np.int8))


def quantize_int4_flat(w: np.ndarray, groupSize: int = 32, shape=None,
                       layout: Layout = Layout.KN_FLAT) -> QuantizedTensor:
    """quantizeINT4, QuantizedTensor.swift:502-560, over w's C-order
    flattening (groups of `groupSize` consecutive flat elements).

    For the BASELINE / converter INT4 layout pass the PyTorch [N, K] weight,
    shape=(K, N) and layout=NK_FLAT: groups then run along K."""
    w = np.ascontiguousarray(w, np.float32)
    flat = w.reshape(-1)
    n = flat.size
    gs = int(groupSize)
    groups = (n + gs - 1) // gs
    padded = np.zeros(groups * gs, np.float32)
    padded[:n] = flat
    blocks = padded.reshape(groups, gs)
    s = _scale(np.abs(blocks).max(axis=1), 7.0)
    q = np.clip(_round_swift(blocks / s[:, None]), -7, 7).astype(np.int32).reshape(-1)[:n]
    shape = tuple(shape) if shape is not None else w.shape
    return QuantizedTensor(shape, pack_int4_array(q), s, QuantizationMode.int4,
                           QuantizationPrecision.int4, gs, np.zeros(groups, np.int8), layout)


def _quantize_int4_per_channel(w):
    # QuantizedTensor.swift:563-606
    _require(w.ndim == 2, "Per-channel quantization requires 2D tensor")
    s = _scale(np.abs(w).max(axis=0), 7.0)
    q = np.clip(_round_swift(w / s[None, :]), -7, 7).astype(np.int32)
    return QuantizedTensor(w.shape, pack_int4_array(q), s, QuantizationMode.int4PerChannel,
                           QuantizationPrecision.int4, 0)
