"""LinearLayerWeights: a quantized projection with an optional bias.

Mirrors ``LinearLayerWeights`` (Sources/TinyBrainRuntime/ModelWeights.swift:
33-69): ``apply(toRow:)`` multiplies a row matrix by the quantized weights
and then adds the bias to every output row.  Here the product and the bias
add both run on the GPU (tbh_linear_device); the reference adds the bias in
a host loop after reading the product back.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from .quantized import PreconditionFailure, QuantizedTensor


class LinearLayerWeights:
    def __init__(self, weights: QuantizedTensor, bias: Optional[np.ndarray] = None):
        self.weights = weights
        self.bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)

    def apply(self, toRow: np.ndarray, backend) -> np.ndarray:
        """y = toRow . dequantize(weights) (+ bias), fp32 [M, N] (ModelWeights.swift:48-68)."""
        K, N = self.weights.shape
        if self.bias is not None and self.bias.shape != (N,):
            raise PreconditionFailure("Bias must match output dimension")   # :53-54
        x = np.ascontiguousarray(toRow, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != K:
            raise PreconditionFailure("Dimensions must match")
        import torch

        dev = torch.device("cuda", backend.device)
        xd = torch.from_numpy(x).to(dev)
        bd = None if self.bias is None else torch.from_numpy(self.bias).to(dev)
        y = backend.linear_device(xd, backend.weight(self.weights), bd)
        torch.cuda.synchronize(dev)
        return y.cpu().numpy()
