"""TinyBrainHIP: MI355X (gfx950) INT8/INT4 weight-only quantized matmul.

The drop-in boundary is the C ABI in include/tinybrain_hip.h
(libtinybrain_hip.so, built by ``python -m tinybrain_amd.build``); this
package is the host-side mirror of the reference's operator API over it:

  * ``QuantizedTensor`` / ``quantize``       -- QuantizedTensor.swift
  * ``HIPBackend.matmulQuantized``            -- QuantizedMatMulBackend
                                                 (Backend.swift:173-175)
  * ``LinearLayerWeights.apply``              -- ModelWeights.swift:47-68
"""
from .quantized import (Layout, PreconditionFailure, QuantizationMode,  # noqa: F401
                        QuantizationPrecision, QuantizedTensor, packInt4,
                        quantize, quantize_int4_flat, unpackInt4,
                        unpack_int4_array, pack_int4_array)
from .backend import DeviceWeight, HIPBackend, HIPBackendError  # noqa: F401
from .decoder import Decoder, DecoderConfig  # noqa: F401
from .linear import LinearLayerWeights  # noqa: F401
from .tbf import TBFFile  # noqa: F401

__all__ = [
    "HIPBackend", "HIPBackendError", "DeviceWeight", "QuantizedTensor", "LinearLayerWeights", "Decoder", "DecoderConfig", "TBFFile",
    "QuantizationMode", "QuantizationPrecision", "Layout", "PreconditionFailure",
    "quantize", "quantize_int4_flat", "packInt4", "unpackInt4",
]
