"""GPU parity sweep across the dispatch boundaries of the matmul path.

Every weight below runs at row counts on both sides of each routing
threshold of tbh_matmul* (burst GEMV at 1, 2, 4 rows; the VALU GEMV at 3;
the matrix-core GEMV from 2..5 rows up to 8 per launch; the exact-split
MFMA GEMM from 8..64 rows) and of the prefill tile rules
(tbh_matmul_bf16_device: 64 / 128 / 256 rows), with ragged N and K, every
INT8 mode, zero points, and INT4 in both flat layouts (runtime-layout INT4
with N-blocks of 16, 32, 48, 128 rows).  Each result is held
to the same bars as the other parity tests: dequantize() bit-exact against
the oracle (QuantizedTensor.swift:182-246 restated), and the product within
GATE (floored max relative error) of a float64 oracle over the same
dequantized weights.
"""
import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T

pytestmark = pytest.mark.gpu

GATE = 1e-3


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


def _oracle_weight(qt, layout):
    """Logical [K, N] fp32 weight: dequantize() in the stored flat order."""
    if layout == T.Layout.KN_FLAT:
        return O.dequantize(qt)
    K, N = qt.shape
    flat = O.QTensor((N, K), qt.data, qt.scales, qt.zero_points, qt.mode, qt.precision, qt.group_size)
    return np.ascontiguousarray(O.dequantize(flat).T)


def _weight(kind, K, N, seed):
    """(oracle QTensor, product QuantizedTensor) for one weight kind."""
    layout = T.Layout.KN_FLAT
    if kind in ("int8", "int8_zp"):
        qt = O.quantize_per_channel(O.fill_normal(seed, K * N, std=0.02).reshape(K, N))
        if kind == "int8_zp":
            qt.zero_points = ((np.arange(N) % 9) - 4).astype(np.int8)
    elif kind == "int8_sym":
        qt = O.quantize_symmetric(O.fill_normal(seed, K * N).reshape(K, N))
    elif kind == "int8_asym":
        w = O.fill_normal(seed, K * N).reshape(K, N)
        qt = O.quantize_asymmetric(w - w.min() * 0.5)
    elif kind.startswith("int4_nk"):          # converter layout, groups along K
        gs = int(kind.split("_g")[1].split("_")[0])
        qt = O.quantize_int4(O.fill_normal(seed, N * K, std=0.02).reshape(N, K), gs, O.ROUND_SWIFT)
        qt.shape = (K, N)
        if kind.endswith("_zp"):
            qt.zero_points = ((np.arange(qt.scales.size) % 7) - 3).astype(np.int8)
        layout = T.Layout.NK_FLAT
    elif kind.startswith("int4_kn"):          # runtime layout, groups along N
        gs = int(kind.split("_g")[1])
        qt = O.quantize_int4(O.fill_normal(seed, K * N, std=0.02).reshape(K, N), gs)
    else:
        raise ValueError(kind)
    pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                           qt.zero_points, layout)
    return qt, pq


FP32_MS = (1, 2, 3, 4, 5, 8, 9, 12, 16, 33, 65)

FP32_CASES = [
    ("int8", 2048, 1003),        # ragged N, burst GEMV / MFMA GEMM
    ("int8", 1000, 777),         # K off every chunk multiple
    ("int8", 4096, 300),
    ("int8", 96, 5000),
    ("int8_zp", 512, 333),
    ("int8_sym", 300, 129),
    ("int8_asym", 300, 129),
    ("int4_nk_g32", 2048, 1003),
    ("int4_nk_g32", 4096, 300),  # matrix-core GEMV with a K split
    ("int4_nk_g32", 5632, 257),
    ("int4_nk_g64", 1024, 100),
    ("int4_nk_g128", 4096, 77),
    ("int4_nk_g32_zp", 512, 90),
    ("int4_kn_g32", 2048, 1024),  # runtime layout on the burst GEMV / MFMA GEMM (two N-blocks per tile)
    ("int4_kn_g32", 512, 96),
    ("int4_kn_g16", 256, 96),     # N-blocks of 16 rows: four per GEMM tile
    ("int4_kn_g128", 1000, 384),  # one N-block per GEMM tile
    ("int4_kn_g48", 256, 96),     # N-blocks the GEMM tiles cannot hold: GEMV kernels at every M
    ("int4_kn_g64", 256, 100),    # groups that do not tile N: generic kernel
]


@pytest.mark.parametrize("kind,K,N", FP32_CASES)
def test_fp32_rows_across_thresholds(backend, kind, K, N):
    qt, pq = _weight(kind, K, N, seed=1000 + K + N)
    W = _oracle_weight(qt, pq.layout)
    deq = backend.dequantize(pq)
    np.testing.assert_array_equal(deq.view(np.uint32), W.view(np.uint32))
    for M in FP32_MS:
        x = O.fill_normal(7 * K + M, M * K).reshape(M, K)
        y = backend.matmulQuantized(x, pq)
        err = O.parity_errors(y, O.gemm_f64(x, W))
        assert err["gated"] <= GATE, (kind, K, N, M, err)


BF16_MS = (64, 65, 127, 128, 129, 255, 256, 257, 513)

BF16_CASES = [
    ("int8", 1000, 777),
    ("int8", 2048, 1003),
    ("int8_zp", 512, 333),
    ("int4_nk_g32", 2048, 1003),
    ("int4_nk_g128", 4096, 300),
    ("int4_nk_g32_zp", 512, 90),
    ("int4_kn_g32", 2048, 1003 // 32 * 32),   # runtime layout
    ("int4_kn_g16", 512, 80),
]


@pytest.mark.parametrize("kind,K,N", BF16_CASES)
def test_bf16_rows_across_tile_rules(backend, kind, K, N):
    import torch

    qt, pq = _weight(kind, K, N, seed=2000 + K + N)
    W = _oracle_weight(qt, pq.layout)
    w = backend.weight(pq)
    for M in BF16_MS:
        xb = torch.from_numpy(O.fill_normal(11 * K + M, M * K).reshape(M, K)).to(torch.bfloat16)
        y = backend.matmul_bf16_device(xb.cuda(), w)
        torch.cuda.synchronize()
        err = O.parity_errors(y.cpu().numpy(), O.gemm_f64(xb.float().numpy(), W))
        assert err["gated"] <= GATE, (kind, K, N, M, err)


EXTREME_CASES = [
    ("int8", 8, 1),               # one output column, one 8-wide K piece
    ("int8", 16, 3),
    ("int8", 40, 7),
    ("int8", 8192, 8),
    ("int8", 32768, 16),          # long K: many chunks per lane
    ("int4_nk_g32", 32, 1),
    ("int4_nk_g32", 64, 5),
    ("int4_nk_g32", 16384, 64),
    ("int4_nk_g128", 32768, 9),
    ("int4_kn_g32", 96, 32),      # runtime layout, a single N-block
    ("int8_zp", 16384, 16),       # long K with zero points: the MFMA GEMM
    ("int4_nk_g32_zp", 16384, 9),
    ("int4_kn_g32", 16384, 32),   # long K, runtime layout: the generic kernel
]


@pytest.mark.parametrize("kind,K,N", EXTREME_CASES)
def test_fp32_extreme_shapes(backend, kind, K, N):
    qt, pq = _weight(kind, K, N, seed=3000 + K + N)
    W = _oracle_weight(qt, pq.layout)
    deq = backend.dequantize(pq)
    np.testing.assert_array_equal(deq.view(np.uint32), W.view(np.uint32))
    for M in (1, 2, 3, 5, 8, 13, 64, 300):
        x = O.fill_normal(13 * K + M, M * K).reshape(M, K)
        y = backend.matmulQuantized(x, pq)
        err = O.parity_errors(y, O.gemm_f64(x, W))
        assert err["gated"] <= GATE, (kind, K, N, M, err)


@pytest.mark.parametrize("kind,K,N", [("int8", 8, 1), ("int8", 40, 7), ("int8", 8192, 8),
                                      ("int4_nk_g32", 32, 1), ("int4_nk_g32", 16384, 64)])
def test_bf16_extreme_shapes(backend, kind, K, N):
    import torch

    qt, pq = _weight(kind, K, N, seed=4000 + K + N)
    W = _oracle_weight(qt, pq.layout)
    w = backend.weight(pq)
    for M in (64, 129, 300):
        xb = torch.from_numpy(O.fill_normal(17 * K + M, M * K).reshape(M, K)).to(torch.bfloat16)
        y = backend.matmul_bf16_device(xb.cuda(), w)
        torch.cuda.synchronize()
        err = O.parity_errors(y.cpu().numpy(), O.gemm_f64(xb.float().numpy(), W))
        assert err["gated"] <= GATE, (kind, K, N, M, err)


def test_long_k_without_an_mfma_route_is_unsupported(backend):
    # K past the GEMV kernels' staged x and not a multiple of 8 (which the MFMA
    # GEMM needs): the call says so instead of failing a launch
    from tinybrain_amd import _abi
    from tinybrain_amd.backend import HIPBackendError

    K, N = 16388, 4
    qt, pq = _weight("int8", K, N, seed=5000)
    x = O.fill_normal(5, 2 * K).reshape(2, K)
    with pytest.raises(HIPBackendError) as e:
        backend.matmulQuantized(x, pq)
    assert e.value.status == _abi.E_UNSUPPORTED, str(e.value)
    assert "too long" in str(e.value)


@pytest.mark.parametrize("kind,K,N", [("int8", 2048, 1003), ("int8_zp", 512, 333), ("int4_nk_g32", 2048, 1003),
                                      ("int4_kn_g32", 512, 96)])
def test_device_x_4_byte_aligned(backend, kind, K, N):
    # tbh_matmul_device on an x that is a contiguous view 4 bytes into its
    # buffer: the kernels that need 16-byte aligned rows are skipped, the
    # rest read x element by element
    import torch

    qt, pq = _weight(kind, K, N, seed=6000 + K + N)
    W = _oracle_weight(qt, pq.layout)
    w = backend.weight(pq)
    for M in (1, 2, 4, 5, 8, 12, 65):
        x = O.fill_normal(19 * K + M, M * K).reshape(M, K)
        buf = torch.zeros(M * K + 4, dtype=torch.float32, device="cuda")
        xv = buf[1:1 + M * K].view(M, K)
        xv.copy_(torch.from_numpy(x))
        assert xv.data_ptr() % 16 == 4
        y = backend.matmul_device(xv, w)
        torch.cuda.synchronize()
        err = O.parity_errors(y.cpu().numpy(), O.gemm_f64(x, W))
        assert err["gated"] <= GATE, (kind, K, N, M, err)
