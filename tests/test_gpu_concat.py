"""tbh_weight_create_concat: one weight computing the outputs of several
weights that read the same x, side by side (the q|k|v and gate|up
projections of a layer, ModelRunner.swift:418-452, each its own
apply(toRow:) call in the reference, ModelWeights.swift:47-68).

Gates: the concatenated weight dequantizes bit for bit to the parts'
dequantized matrices side by side (dequantize(), QuantizedTensor.swift:182-286),
and its product is within the matmul gate of the float64 product of those
matrices at decode and prefill row counts."""
import ctypes

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi

pytestmark = pytest.mark.gpu

GATE = 1e-3


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


def _part(kind, seed, K, N):
    """(product QuantizedTensor, dequantized [K, N] fp32)."""
    if kind == "int8":
        qt = O.quantize_per_channel(O.fill_normal(seed, K * N, std=0.02).reshape(K, N))
        return T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision), O.dequantize(qt)
    if kind == "int8_zp":
        qt = O.quantize_per_channel(O.fill_normal(seed, K * N, std=0.02).reshape(K, N))
        qt.zero_points = ((np.arange(N) % 7) - 3).astype(np.int8)
        return (T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, 0, qt.zero_points),
                O.dequantize(qt))
    if kind == "int4kn":
        qt = O.quantize_int4(O.fill_normal(seed, K * N, std=0.02).reshape(K, N), 32, O.ROUND_SWIFT)
        return (T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, 32, qt.zero_points,
                                  T.Layout.KN_FLAT), O.dequantize(qt))
    qt = O.quantize_int4(O.fill_normal(seed, N * K, std=0.02).reshape(N, K), 32, O.ROUND_SWIFT)
    flat = O.QTensor((N, K), qt.data, qt.scales, qt.zero_points, qt.mode, qt.precision, 32)
    return (T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, 32, qt.zero_points,
                              T.Layout.NK_FLAT), np.ascontiguousarray(O.dequantize(flat).T))


def _dequant(backend, w):
    out = np.empty((w.K, w.N), np.float32)
    assert _abi.lib().tbh_dequantize(backend._dev, w.handle, out.ctypes.data) == _abi.OK, _abi.last_error()
    return out


@pytest.mark.parametrize("kind,K,Ns", [
    ("int8", 2048, (2048, 256, 256)),          # the 1.1B q|k|v
    ("int8_zp", 1000, (300, 44)),              # zero points, ragged widths
    ("int4", 4096, (4096, 4096, 4096)),         # the 7B q|k|v
    ("int4", 2048, (5632, 5632)),               # the 1.1B gate|up
    ("int4kn", 2048, (1024, 512)),              # runtime layout, groups along N
])
def test_concat_equals_parts_side_by_side(backend, kind, K, Ns):
    import torch

    parts = [_part(kind, 0xC0 + 13 * i + K, K, N) for i, N in enumerate(Ns)]
    w = T.DeviceWeight.concat(backend, [p for p, _ in parts])
    assert (w.K, w.N) == (K, sum(Ns))
    Wcat = np.concatenate([W for _, W in parts], axis=1)
    np.testing.assert_array_equal(_dequant(backend, w).view(np.uint32), Wcat.view(np.uint32))
    for M in (1, 4, 8, 64):
        xh = O.fill_normal(0xD0 + M, M * K).reshape(M, K)
        y = backend.matmul_device(torch.from_numpy(xh).cuda(), w).cpu().numpy()
        assert O.parity_errors(y, O.gemm_f64(xh, Wcat))["gated"] <= GATE, (kind, K, Ns, M)


def test_concat_rejects_mismatched_parts(backend):
    a, _ = _part("int8", 1, 256, 64)
    b, _ = _part("int8", 2, 128, 64)      # another K
    with pytest.raises(T.HIPBackendError) as e:
        T.DeviceWeight.concat(backend, [a, b])
    assert e.value.status == _abi.E_INVALID
    c, _ = _part("int4kn", 3, 256, 64)    # another precision
    with pytest.raises(T.HIPBackendError) as e:
        T.DeviceWeight.concat(backend, [a, c])
    assert e.value.status == _abi.E_INVALID
    d, _ = _part("int4", 4, 256, 64)      # INT4 layouts mixed
    with pytest.raises(T.HIPBackendError) as e:
        T.DeviceWeight.concat(backend, [c, d])
    assert e.value.status in (_abi.E_UNSUPPORTED, _abi.E_INVALID)
    h = ctypes.c_void_p()
    assert _abi.lib().tbh_weight_create_concat(backend._dev, 0, None, ctypes.byref(h)) == _abi.E_INVALID
