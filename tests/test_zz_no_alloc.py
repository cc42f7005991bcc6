"""tbh_matmul_device_noalloc against tbh_matmul_device, through the C ABI.

The no-allocation entry point runs the same kernels as tbh_matmul_device;
only the split-K partial sums (of the matrix-core small-M GEMV and of the
fp32 MFMA GEMM route for more rows) and, past 64 rows, the GEMM's per-row
exponents of x go to a fixed per-GPU scratch array instead of a per-stream
workspace.  So every result is
bit-identical to tbh_matmul_device's on the same input, and within the matmul
gate (floored max relative error <= 1e-3) of the float64 product of the
bit-exact dequantized weights.
"""
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


def _int4_nk(seed, K, N, gs=32):
    w_nk = O.fill_normal(seed, N * K, std=0.02).reshape(N, K)
    qt = O.quantize_int4(w_nk, gs, O.ROUND_SWIFT)
    pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, gs, qt.zero_points,
                           T.Layout.NK_FLAT)
    flat = O.QTensor((N, K), qt.data, qt.scales, qt.zero_points, qt.mode, qt.precision, gs)
    return pq, np.ascontiguousarray(O.dequantize(flat).T)


def _int8_pc(seed, K, N):
    qt = O.quantize_per_channel(O.fill_normal(seed, K * N, std=0.02).reshape(K, N))
    pq = T.QuantizedTensor((K, N), qt.data, qt.scales, T.QuantizationMode.perChannel)
    return pq, O.dequantize(qt)


def _int4_kn(seed, K, N, gs=32):
    # the runtime layout Tensor.quantize(.int4) writes: groups along N
    qt = O.quantize_int4(O.fill_normal(seed, K * N, std=0.02).reshape(K, N), gs)
    pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, gs, qt.zero_points,
                           T.Layout.KN_FLAT)
    return pq, O.dequantize(qt)


def _noalloc(w, x, y, stream):
    """tbh_matmul_device_noalloc through ctypes; returns the status."""
    L = _abi.lib()
    return L.tbh_matmul_device_noalloc(w.handle, x.data_ptr(), x.shape[0], x.shape[1], y.data_ptr(),
                                       ctypes.c_void_p(stream.cuda_stream))


def test_noalloc_matches_device_entry_point(backend):
    import torch

    s = torch.cuda.Stream()
    # first call: 8 rows on [4096 -> 11008], the matrix-core GEMV split along
    # K 8 ways (2.8 MB of scratch); second, smaller: 3 rows on [2048 -> 1024]
    # with the matrix-core path forced from 2 rows (4 K splits, 48 KB of
    # scratch over what the first call left there); third: INT8 on the VALU
    # GEMV (no scratch); fourth: 16 rows on [5632 -> 2048], the fp32 MFMA
    # GEMM route with K split over the CUs (2 MB of scratch); fifth: 96 rows
    # there, x as two f16 pieces (the row exponents ahead of the partials);
    # sixth: 80 rows of a runtime-layout weight on the weight-side kernel
    cases = [(_int4_nk(901, 4096, 11008), 8, 0), (_int4_nk(902, 2048, 1024), 3, 2),
             (_int8_pc(903, 2048, 512), 1, 0), (_int4_nk(905, 5632, 2048), 16, 0),
             (_int4_nk(906, 5632, 2048), 96, 0), (_int4_kn(907, 2048, 1024), 80, 0)]
    try:
        for (pq, W), M, min_rows in cases:
            backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, min_rows)
            w = backend.weight(pq)
            xh = O.fill_normal(904 + M, M * pq.shape[0]).reshape(M, pq.shape[0])
            x = torch.from_numpy(xh).cuda()
            y_ref = torch.empty((M, pq.shape[1]), dtype=torch.float32, device="cuda")
            y = torch.full((M, pq.shape[1]), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()          # the fills above ran on torch's current stream
            with torch.cuda.stream(s):
                backend.matmul_device(x, w, out=y_ref, stream=s)
                assert _noalloc(w, x, y, s) == _abi.OK, _abi.last_error()
            torch.cuda.synchronize()
            got, ref = y.cpu().numpy(), y_ref.cpu().numpy()
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
            assert O.parity_errors(got, O.gemm_f64(xh, W))["gated"] <= GATE
    finally:
        backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)


def test_noalloc_under_graph_capture(backend):
    # Captured on a fresh stream, where tbh_matmul_device has no workspace
    # yet, the no-allocation call still splits K (its scratch needs no
    # allocation); every replay, with eager work and synchronisation in
    # between, equals the eager no-allocation result bit for bit.
    import torch

    pq, W = _int4_nk(911, 4096, 4096)
    w = backend.weight(pq)
    M = 8
    xh = O.fill_normal(912, M * 4096).reshape(M, 4096)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty((M, 4096), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        assert _noalloc(w, x, y, s) == _abi.OK, _abi.last_error()
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    assert O.parity_errors(eager, O.gemm_f64(xh, W))["gated"] <= GATE
    s2 = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s2):
        assert _noalloc(w, x, y, s2) == _abi.OK, _abi.last_error()
    # 5 rows: the matrix-core GEMV with its own K split, through the same scratch
    other = torch.empty((5, 4096), dtype=torch.float32, device="cuda")
    x2 = torch.from_numpy(O.fill_normal(913, 5 * 4096).reshape(5, 4096)).cuda()
    torch.cuda.synchronize()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s2):
            g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        with torch.cuda.stream(s):         # eager work on the same scratch between replays
            assert _noalloc(w, x2, other, s) == _abi.OK, _abi.last_error()
        torch.cuda.synchronize()
    del g


def test_noalloc_rejects_scratch_beyond_the_limit(backend):
    # With the limit lowered below what the split needs, the call is rejected
    # before anything is enqueued: y keeps its contents.
    import torch

    pq, _ = _int4_nk(921, 4096, 11008)
    w = backend.weight(pq)
    x = torch.from_numpy(O.fill_normal(922, 8 * 4096).reshape(8, 4096)).cuda()
    y = torch.full((8, 11008), 7.0, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    backend.set_option(_abi.OPT_NOALLOC_SCRATCH_BYTES, 4096)
    try:
        st = _noalloc(w, x, y, s)
        torch.cuda.synchronize()
        assert st == _abi.E_INVALID
        assert "scratch" in _abi.last_error()
        assert bool(torch.all(y == 7.0))
    finally:
        backend.set_option(_abi.OPT_NOALLOC_SCRATCH_BYTES, 0)
    with pytest.raises(T.HIPBackendError):
        backend.set_option(_abi.OPT_NOALLOC_SCRATCH_BYTES, (16 << 20) + 1)


def test_noalloc_rejects_a_later_piece_beyond_the_limit(backend):
    # x runs in pieces of up to 8 rows, and the pieces of one call can take
    # different routes: with the matrix-core GEMV forced from 2 rows, 10 rows
    # on INT4 [2048 -> 1024] run 8 rows on the burst GEMV (no scratch), then
    # the last 2 on the matrix-core GEMV split along K (32 KB of scratch).
    # With the limit at 4 KB the second launch is refused: the call returns
    # TBH_E_INVALID (y unspecified), and with the limit restored the same
    # call equals tbh_matmul_device bit for bit.
    import torch

    pq, W = _int4_nk(931, 2048, 1024)
    w = backend.weight(pq)
    xh = O.fill_normal(932, 10 * 2048).reshape(10, 2048)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty((10, 1024), dtype=torch.float32, device="cuda")
    y_ref = torch.empty_like(y)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 2)
    try:
        backend.set_option(_abi.OPT_NOALLOC_SCRATCH_BYTES, 4096)
        try:
            st = _noalloc(w, x, y, s)
            torch.cuda.synchronize()
            assert st == _abi.E_INVALID
            assert "scratch" in _abi.last_error()
        finally:
            backend.set_option(_abi.OPT_NOALLOC_SCRATCH_BYTES, 0)
        with torch.cuda.stream(s):
            backend.matmul_device(x, w, out=y_ref, stream=s)
            assert _noalloc(w, x, y, s) == _abi.OK, _abi.last_error()
        torch.cuda.synchronize()
    finally:
        backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)
    got = y.cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), y_ref.cpu().numpy().view(np.uint32))
    assert O.parity_errors(got, O.gemm_f64(xh, W))["gated"] <= GATE
