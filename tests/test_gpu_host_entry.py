"""The host-pointer entry (tbh_matmul, which HIPBackend.matmulQuantized and the
Swift drop-in call) in each of its transfer and wait modes
(TBH_OPT_HOST_ENTRY 0, 1, 2 x TBH_OPT_HOST_WAIT 0, 1), against the device
entry tbh_matmul_device on the same input: bit-identical, since every mode
runs the same kernels on the same x and only moves x and y differently, and
within the matmul gate of the float64 product of the bit-exact dequantized
weights (reference: MetalBackend.matmulQuantized, MetalBackend.swift:894-974,
which commits and waits).  Row counts 1..9 and 16 cover the rows read in
place (1), the copy launch (2..8) and the DMA path past 8 rows."""
import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi

pytestmark = pytest.mark.gpu

GATE = 1e-3
ROWS = (1, 2, 3, 4, 5, 8, 9, 16)


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.set_option(_abi.OPT_HOST_ENTRY, 2)
    b.set_option(_abi.OPT_HOST_WAIT, 1)
    b.close()


def _weights():
    """(product QuantizedTensor, dequantized [K, N]) per route: INT4 K-groups
    (burst GEMV; the matrix-core GEMV from 4 rows at K = 4096), INT8 with zero
    points (VALU GEMV), runtime-layout INT4, ragged N."""
    out = []
    w = O.fill_normal(0xE1, 1000 * 2048, std=0.02).reshape(1000, 2048)          # [N, K]
    q = O.quantize_int4(w, 32, O.ROUND_SWIFT)
    pq = T.QuantizedTensor((2048, 1000), q.data, q.scales, q.mode, q.precision, 32, q.zero_points,
                           T.Layout.NK_FLAT)
    deq = O.dequantize(O.QTensor((1000, 2048), q.data, q.scales, q.zero_points, q.mode, q.precision, 32))
    out.append((pq, np.ascontiguousarray(deq.T)))
    w = O.fill_normal(0xE2, 520 * 4096, std=0.02).reshape(520, 4096)
    q = O.quantize_int4(w, 32, O.ROUND_SWIFT)
    pq = T.QuantizedTensor((4096, 520), q.data, q.scales, q.mode, q.precision, 32, q.zero_points,
                           T.Layout.NK_FLAT)
    deq = O.dequantize(O.QTensor((520, 4096), q.data, q.scales, q.zero_points, q.mode, q.precision, 32))
    out.append((pq, np.ascontiguousarray(deq.T)))
    q = O.quantize_per_channel(O.fill_normal(0xE3, 1000 * 300, std=0.02).reshape(1000, 300))
    q.zero_points = ((np.arange(300) % 9) - 4).astype(np.int8)
    pq = T.QuantizedTensor((1000, 300), q.data, q.scales, q.mode, q.precision, q.group_size, q.zero_points)
    out.append((pq, O.dequantize(q)))
    q = O.quantize_int4(O.fill_normal(0xE4, 2048 * 1024, std=0.02).reshape(2048, 1024), 32, O.ROUND_SWIFT)
    pq = T.QuantizedTensor((2048, 1024), q.data, q.scales, q.mode, q.precision, 32, q.zero_points,
                           T.Layout.KN_FLAT)
    out.append((pq, O.dequantize(q)))
    return out


@pytest.mark.parametrize("entry,wait", [(0, 0), (1, 0), (1, 1), (2, 0), (2, 1)])
def test_host_entry_modes_equal_the_device_entry(backend, entry, wait):
    import torch

    backend.set_option(_abi.OPT_HOST_ENTRY, entry)
    backend.set_option(_abi.OPT_HOST_WAIT, wait)
    try:
        for pq, W in _weights():
            K, N = pq.shape
            w = backend.weight(pq)
            for M in ROWS:
                xh = O.fill_normal(0xF00 + 7 * M + K, M * K).reshape(M, K)
                y = backend.matmulQuantized(xh, pq)
                yd = backend.matmul_device(torch.from_numpy(xh).cuda(), w)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(y.view(np.uint32), yd.cpu().numpy().view(np.uint32),
                                              err_msg=f"entry {entry} wait {wait} K {K} N {N} M {M}")
                assert O.parity_errors(y, O.gemm_f64(xh, W))["gated"] <= GATE, (entry, wait, K, N, M)
    finally:
        backend.set_option(_abi.OPT_HOST_ENTRY, 2)
        backend.set_option(_abi.OPT_HOST_WAIT, 1)


def test_host_entry_consecutive_calls_see_fresh_x(backend):
    # the locked staging is reused by every call: a call must read the x it
    # was given and return its own y, also when consecutive calls differ only
    # in x (same weight, same shape) and alternate between in-place and
    # copied x (1 and 2 rows)
    pq, W = _weights()[0]
    K = pq.shape[0]
    backend.set_option(_abi.OPT_HOST_ENTRY, 2)
    backend.set_option(_abi.OPT_HOST_WAIT, 1)
    for i in range(40):
        M = 1 + i % 2
        xh = O.fill_normal(0xA000 + i, M * K).reshape(M, K)
        y = backend.matmulQuantized(xh, pq)
        assert O.parity_errors(y, O.gemm_f64(xh, W))["gated"] <= GATE, i


def test_host_entry_options_are_validated(backend):
    for opt, bad in ((_abi.OPT_HOST_ENTRY, 3), (_abi.OPT_HOST_ENTRY, -1), (_abi.OPT_HOST_WAIT, 2)):
        with pytest.raises(T.HIPBackendError) as e:
            backend.set_option(opt, bad)
        assert e.value.status == _abi.E_INVALID
