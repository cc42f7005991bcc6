"""CPU tests of the host side: the C-ABI library surface, the Python mirror of
QuantizedTensor / quantize(), and error behaviour without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    syms = set()
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            syms |= set(re.findall(r"\b(tbh_[a-z0-9_]+)\s*\(", text))
    return syms


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    declared = _declared_symbols()
    assert declared, "no declarations found"
    assert declared == set(_abi.EXPORTS)
    for s in declared:
        assert hasattr(lib, s), s


def test_abi_version_and_status_strings():
    lib = _abi.lib()
    assert lib.tbh_abi_version() == 1
    assert _abi.status_name(_abi.E_UNSUPPORTED) == "TBH_E_UNSUPPORTED"


def _has_gpu():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_no_device_is_a_backend_error():
    assert not T.HIPBackend.isAvailable()
    with pytest.raises(T.HIPBackendError) as e:
        T.HIPBackend()
    assert e.value.status == _abi.E_NODEVICE


def test_null_arguments_are_invalid():
    lib = _abi.lib()
    assert lib.tbh_device_open(0, None) == _abi.E_INVALID
    assert lib.tbh_weight_create(None, None, None) == _abi.E_INVALID
    assert lib.tbh_matmul(None, None, 1, 1, None, None) == _abi.E_INVALID
    assert "NULL" in _abi.last_error()
    assert lib.tbh_weight_destroy(None) == _abi.OK
    assert lib.tbh_device_close(None) == _abi.OK


# ---------------------------------------------------------------------------
# quantize() mirror vs the oracle (bit-exact)
# ---------------------------------------------------------------------------
def _w(seed, shape, std=0.02):
    return O.fill_normal(seed, int(np.prod(shape)), std=std).reshape(shape)


@pytest.mark.parametrize("shape", [(64, 96), (33, 47), (1, 5), (7, 1)])
def test_quantize_per_channel_matches_oracle(shape):
    w = _w(100 + shape[0], shape)
    w.reshape(-1)[3] = 0.0
    ours = T.quantize(w, T.QuantizationMode.perChannel)
    ref = O.quantize_per_channel(w)
    np.testing.assert_array_equal(ours.data, ref.data)
    np.testing.assert_array_equal(ours.scales.view(np.uint32), ref.scales.view(np.uint32))


@pytest.mark.parametrize("gs", [32, 64, 128, 7])
@pytest.mark.parametrize("shape", [(64, 96), (5, 7), (3, 33)])
def test_quantize_int4_matches_oracle(shape, gs):
    w = _w(200 + gs, shape)
    ours = T.quantize(w, T.QuantizationMode.int4, gs)
    ref = O.quantize_int4(w, gs)
    np.testing.assert_array_equal(ours.data, ref.data)
    np.testing.assert_array_equal(ours.scales.view(np.uint32), ref.scales.view(np.uint32))
    assert ours.groupSize == gs and ours.precision == T.QuantizationPrecision.int4


def test_quantize_ties_and_zeros_match_oracle():
    t = np.array([[7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5]] * 4, np.float32)
    t[2] = 0.0
    for gs in (8, 32):
        ours = T.quantize(t, T.QuantizationMode.int4, gs)
        ref = O.quantize_int4(t, gs)
        np.testing.assert_array_equal(ours.data, ref.data)
        np.testing.assert_array_equal(ours.scales, ref.scales)
    t8 = np.array([[127.0, 2.5, -2.5, 126.5, -126.5, 0.5]], np.float32).T.copy()
    np.testing.assert_array_equal(T.quantize(t8).data, O.quantize_per_channel(t8).data)


def test_quantize_symmetric_asymmetric_match_oracle():
    w = _w(300, (16, 24), std=1.0)
    a = T.quantize(w, T.QuantizationMode.symmetric)
    b = O.quantize_symmetric(w)
    np.testing.assert_array_equal(a.data, b.data)
    np.testing.assert_array_equal(a.scales, b.scales)
    a = T.quantize(w, T.QuantizationMode.asymmetric)
    b = O.quantize_asymmetric(w)
    np.testing.assert_array_equal(a.data, b.data)
    np.testing.assert_array_equal(a.scales, b.scales)
    np.testing.assert_array_equal(a.zeroPoints, b.zero_points)
    with pytest.raises(T.PreconditionFailure):
        T.quantize(np.linspace(1, 2, 8, dtype=np.float32).reshape(2, 4), T.QuantizationMode.asymmetric)


def test_quantize_int4_per_channel_matches_oracle():
    w = _w(301, (6, 10))
    a = T.quantize(w, T.QuantizationMode.int4PerChannel)
    b = O.quantize_int4_per_channel(w)
    np.testing.assert_array_equal(a.data, b.data)
    np.testing.assert_array_equal(a.scales, b.scales)


def test_converter_layout_quantizer_matches_golden():
    # The NK (converter) layout groups along K; the Swift rounding differs from
    # np.round only on exact ties, which N(0, 0.02) data never hits.
    g = np.load(os.path.join(ROOT, "tests", "golden", "converter_vectors.npz"), allow_pickle=False)
    w = g["rand__w"]                                  # PyTorch [N, K]
    qt = T.quantize_int4_flat(w, 32, shape=(w.shape[1], w.shape[0]), layout=T.Layout.NK_FLAT)
    np.testing.assert_array_equal(qt.data, g["rand__int4_g32_p"])
    np.testing.assert_array_equal(qt.scales, g["rand__int4_g32_s"])


# ---------------------------------------------------------------------------
# nibble helpers and preconditions
# ---------------------------------------------------------------------------
def test_pack_unpack_reference_table():
    # INT4QuantizationTests.swift:37-58
    for v1, v2 in [(0, 0), (7, -7), (-7, 7), (3, -3), (1, 2), (-1, -2), (5, -3)]:
        assert T.unpackInt4(T.packInt4(v1, v2)) == (v1, v2)
    assert T.unpackInt4(T.packInt4(10, -10)) == (7, -7)
    assert T.packInt4(5, -3) == 93
    for b in range(-128, 128):
        assert T.unpackInt4(b) == O.unpack_int4(b)


def test_unpack_int4_array_matches_oracle():
    data = np.arange(-128, 128, dtype=np.int8)
    vals = T.unpack_int4_array(data, 511)
    for i in range(511):
        assert vals[i] == O.lib().orc_int4_at(data.ctypes.data, i)


def test_quantized_tensor_preconditions():
    with pytest.raises(T.PreconditionFailure):
        T.QuantizedTensor((4, 6), np.zeros(23, np.int8), np.ones(6, np.float32), T.QuantizationMode.perChannel)
    with pytest.raises(T.PreconditionFailure):
        T.QuantizedTensor((4, 6), np.zeros(24, np.int8), np.ones(5, np.float32), T.QuantizationMode.perChannel)
    with pytest.raises(T.PreconditionFailure):
        T.QuantizedTensor((5, 7), np.zeros(18, np.int8), np.ones(2, np.float32), T.QuantizationMode.int4,
                          T.QuantizationPrecision.int4, 32, zeroPoints=np.zeros(1, np.int8))
    qt = T.QuantizedTensor((5, 7), np.zeros(18, np.int8), np.ones(2, np.float32), T.QuantizationMode.int4,
                           T.QuantizationPrecision.int4, 32)
    assert qt.byteSize == 18 + 8
    d = qt.desc()
    assert (d.K, d.N, d.data_bytes, d.n_scales, d.group_size) == (5, 7, 18, 2, 32)
    assert ctypes.sizeof(_abi.QTensorDesc) == 80


def test_linear_bias_precondition():
    # ModelWeights.swift:53-54: "Bias must match output dimension", checked
    # before anything reaches the GPU
    import oracle as O

    K, N = 64, 24
    q = O.quantize_per_channel(O.fill_normal(3, K * N).reshape(K, N))
    pq = T.QuantizedTensor((K, N), q.data, q.scales, T.QuantizationMode.perChannel)
    with pytest.raises(T.PreconditionFailure):
        T.LinearLayerWeights(pq, np.zeros(N + 1, np.float32)).apply(np.zeros((1, K), np.float32), None)
    with pytest.raises(T.PreconditionFailure):
        T.LinearLayerWeights(pq, np.zeros(N, np.float32)).apply(np.zeros((1, K + 1), np.float32), None)


def test_bench_reads_every_committed_traffic_record():
    # bench.py puts these per-launch HBM byte counts into roofline.traffic:
    # the default GEMV line's dominant shape and every prefill workload
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    assert bench.profiled_traffic("int4", 32000, 2048, 1) > 0
    for name, (prec, gs, (N, K), M) in bench.PREFILL.items():
        t = bench.profiled_traffic(prec, N, K, M, "prefill")
        alg = bench.prefill_bytes(prec, gs, N, K, M)
        assert t is not None, name
        assert alg <= t <= 8 * alg, (name, t, alg)   # counted bytes cover at least the algorithmic ones
    assert bench.profiled_traffic("int8", 7, 7, 7, "prefill") is None
