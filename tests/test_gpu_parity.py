"""GPU parity: libtinybrain_hip vs the CPU oracle, through the C ABI.

Bars (from the task's correctness contract):
  * dequantize: bit-exact fp32 (bit patterns) vs QuantizedTensor.dequantize()
    restated in the oracle;
  * matmul: max|y^ - y| / max(|y|, 1e-3 * max_row|y|) <= 1e-3 against a float64
    oracle over the same dequantized weights (GATE below), and L2 relative
    error <= 1e-3 against the restated reference CPU path
    (dequantize() + sgemm, QuantizedTensor.swift:640-642).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi

pytestmark = pytest.mark.gpu

GATE = 1e-3          # floored max relative error vs float64
CPU_PATH_L2 = 1e-3   # L2 relative error vs the reference CPU path


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _product(qt: O.QTensor, shape_kn, layout=T.Layout.KN_FLAT) -> T.QuantizedTensor:
    return T.QuantizedTensor(shape_kn, qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                             qt.zero_points, layout)


def _oracle_weight(qt: O.QTensor, layout) -> np.ndarray:
    """Logical [K, N] fp32 weight: dequantize() in the stored flat order."""
    if layout == T.Layout.KN_FLAT:
        return O.dequantize(qt)
    K, N = qt.shape
    flat = O.QTensor((N, K), qt.data, qt.scales, qt.zero_points, qt.mode, qt.precision, qt.group_size)
    return np.ascontiguousarray(O.dequantize(flat).T)


def _check(backend, pq: T.QuantizedTensor, oq: O.QTensor, Ms=(1,), seed=1, cpu_path=True):
    W = _oracle_weight(oq, pq.layout)
    deq = backend.dequantize(pq)
    np.testing.assert_array_equal(deq.view(np.uint32), W.view(np.uint32))
    K = pq.shape[0]
    for M in Ms:
        x = O.fill_normal(seed * 1000 + M, M * K).reshape(M, K)
        y = backend.matmulQuantized(x, pq)
        y64 = O.gemm_f64(x, W)
        err = O.parity_errors(y, y64)
        assert err["gated"] <= GATE, (M, err)
        if cpu_path:
            y_ref = O.sgemm(x, W)
            l2 = np.linalg.norm(y.astype(np.float64) - y_ref) / max(np.linalg.norm(y_ref), 1e-30)
            assert l2 <= CPU_PATH_L2, (M, l2)
    return backend.weight(pq)


def _int8_pc(seed, K, N, std=0.02):
    w = O.fill_normal(seed, K * N, std=std).reshape(K, N)
    return O.quantize_per_channel(w)


def _int4_nk(seed, K, N, gs, std=0.02):
    """BASELINE / converter layout: PyTorch [N, K] quantized flat, groups along K."""
    w_nk = O.fill_normal(seed, N * K, std=std).reshape(N, K)
    qt = O.quantize_int4(w_nk, gs, O.ROUND_SWIFT)
    qt.shape = (K, N)
    return qt


def _int4_kn(seed, K, N, gs, std=0.02):
    """Runtime layout: Tensor.quantize(.int4) on [K, N]."""
    return O.quantize_int4(O.fill_normal(seed, K * N, std=std).reshape(K, N), gs)


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("K,N", [(128, 64), (100, 37), (2048, 256), (17, 8), (4096, 24)])
def test_int8_per_channel(backend, K, N):
    qt = _int8_pc(K * 7 + N, K, N)
    w = _check(backend, _product(qt, (K, N)), qt, Ms=(1, 2, 3, 4, 5, 8))
    assert w.path == "int8_row"


def test_int8_baseline_config0(backend):
    # W [5632 x 2048] (out x in) -> reference [K=2048, N=5632]
    qt = _int8_pc(0x7B1A0000, 2048, 5632)
    _check(backend, _product(qt, (2048, 5632)), qt, Ms=(1, 8))


def test_int8_symmetric_and_asymmetric(backend):
    w = O.fill_normal(77, 256 * 96).reshape(256, 96)
    for qt in (O.quantize_symmetric(w), O.quantize_asymmetric(w - w.min() * 0.5)):
        assert qt is not None
        _check(backend, _product(qt, (256, 96)), qt, Ms=(1, 3))


def test_int8_zero_points(backend):
    qt = _int8_pc(78, 192, 40)
    qt.zero_points = ((np.arange(40) % 9) - 4).astype(np.int8)
    w = _check(backend, _product(qt, (192, 40)), qt, Ms=(1, 4))
    assert w.has_zero_points


def test_int8_reference_matmul_tolerance(backend):
    # QuantizationTests.swift:117-135: INT8 matmul within 1% L2 of fp32
    x = O.fill_normal(31, 128 * 256).reshape(128, 256)
    w = O.fill_normal(32, 256 * 512).reshape(256, 512)
    qt = O.quantize_per_channel(w)
    y = backend.matmulQuantized(x, _product(qt, (256, 512)))
    fp32 = O.sgemm(x, w)
    assert np.linalg.norm(y - fp32) / np.linalg.norm(fp32) < 0.01


# ---------------------------------------------------------------------------
# INT4
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("K,N,gs", [(2048, 256, 32), (256, 40, 64), (512, 24, 128),
                                    (96, 8, 32), (48, 10, 48), (100, 9, 0)])
def test_int4_converter_layout(backend, K, N, gs):
    qt = _int4_nk(K + N + gs, K, N, gs if gs else K * N)
    if gs == 0:
        qt.group_size = 0
    w = _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(1, 2, 3, 4, 5, 8))
    assert w.path == "int4_kgroup"


@pytest.mark.parametrize("K,N", [(2048, 2048), (2048, 5632), (5632, 2048), (2048, 32000)])
def test_int4_baseline_config1(backend, K, N):
    # INT4 g32 along K, shapes [N x K], M in {1, 4, 8}
    qt = _int4_nk(0x7B1A0010 + K + N, K, N, 32)
    _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(1, 4, 8))


# Burst GEMV (M in {1, 2, 4}; no zero points, 16-byte aligned x, K % 4 == 0):
# one case per chunk-iteration count I = ceil(chunks / 64) = 1..6 and across
# the rows per wave U the launch picks from N, M and the CU count (256 on
# MI355X): 2 or 4 at M = 1, up to 16 at M = 2.  The matrix-core kernel is
# switched off here (large-K INT4 weights take it from 2 rows on by default),
# so M = 8 runs as two M = 4 launches.
@pytest.mark.parametrize("prec,K,N", [
    ("int4", 2048, 40960),   # I=1, U=16
    ("int4", 2048, 20000),   # I=1, U=8
    ("int4", 4096, 9000),    # I=2, U=4
    ("int4", 5632, 3001),    # I=3, ragged N
    ("int4", 8192, 1000),    # I=4
    ("int4", 10240, 520),    # I=5
    ("int4", 11008, 2048),   # I=6 (7B down projection)
    ("int8", 1024, 40000),   # I=1, U=8
    ("int8", 2048, 5632),    # I=2, U=2
    ("int8", 5632, 2048),    # I=6 (1.1B down projection)
    ("int8", 4000, 777),     # I=4, ragged N
])
def test_burst_shapes(backend, prec, K, N):
    if prec == "int8":
        oq = _int8_pc(41 + K, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(43 + K, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 9)
    try:
        _check(backend, pq, oq, Ms=(1, 2, 4, 8), cpu_path=False)
    finally:
        backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)


# One x row with rows of five or six chunk iterations (or four, on at least
# 8192 rows) and at least 4096 rows: each row is split between two waves of
# its block, whose totals meet in LDS.  Ragged K leaves the upper half's last
# iterations partly or wholly past the row (lanes there re-read the last
# chunk and add nothing); ragged N leaves row groups of the last block idle.
@pytest.mark.parametrize("prec,K,N", [
    ("int4", 9024, 4100),    # 282 chunks: I = 3 per half, the upper half's last iteration empty
    ("int4", 8192, 8192),    # I = 4 over 8192 rows
    ("int8", 4104, 8200),    # 257 chunks: one chunk in the upper half's second iteration
    ("int8", 4096, 8192),    # I = 4 over 8192 rows
])
def test_burst_k_split(backend, prec, K, N):
    if prec == "int8":
        oq = _int8_pc(47 + K + N, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(53 + K + N, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    _check(backend, pq, oq, Ms=(1, 2), cpu_path=False)


@pytest.mark.parametrize("kind,K,N", [
    ("int8", 2048, 5632),     # INT8 under 16384 outputs: 8 rows on one burst launch, the GEMM from 9
    ("int8", 2048, 1003),     # ragged N
    ("int8", 1000, 64),       # K off the chunk multiple
    ("int4", 2048, 2048),     # configs[1] shape the matrix-core GEMV never takes
    ("int4", 4096, 520),      # two chunk iterations per row: eight staged x rows would need 144 KB
                              # of LDS, so 8 rows run as two 4-row launches (matrix-core GEMV off)
    ("int4kn", 2048, 5632),   # runtime layout (groups along N)
])
def test_burst_eight_rows(backend, kind, K, N):
    # eight x rows in one burst GEMV launch: each row's chunk unpacked once,
    # the x rows taken one at a time; five to seven rows on the same launch
    # and three on the four-row one, the rows past M masked; M = 9 and 16
    # add the tails
    if kind == "int8":
        oq = _int8_pc(0x8B + K + N, K, N)
        pq = _product(oq, (K, N))
    elif kind == "int4":
        oq = _int4_nk(0x8C + K + N, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    else:
        oq = _int4_kn(0x8D + K + N, K, N, 32)
        pq = _product(oq, (K, N))
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 9)
    try:
        _check(backend, pq, oq, Ms=(3, 5, 6, 7, 8, 9, 11, 16), cpu_path=False)
    finally:
        backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)


def _extreme_rows(seed, K):
    """Eight x rows of unusual ranges: huge, tiny, a third zero, all zero,
    one huge 32-element chunk, one tiny chunk, all positive (as after a
    ReLU or SiLU) and all positive with a large common offset."""
    x = O.fill_normal(seed, 8 * K).reshape(8, K)
    x[0] *= 1e6
    x[1] *= 1e-7
    x[2, ::3] = 0.0
    x[3, :] = 0.0
    x[4, :32] *= 1e20
    x[5, 32:64] *= 1e-20
    x[6] = np.abs(x[6])
    x[7] = 100.0 + np.abs(x[7])
    return x


@pytest.mark.parametrize("kind,K,N", [
    ("int8", 2048, 1000),
    ("int8_zp", 1000, 300),
    ("int4", 2048, 1000),
    ("int4", 5632, 300),     # three chunk iterations per row
    ("int4kn", 2048, 1024),  # runtime layout: x times the N-block's scale row in LDS
])
def test_burst_x_range_extremes(backend, kind, K, N):
    # the burst GEMV keeps x in fp32 and the weights exact in f16, so huge,
    # tiny and all-positive activations (no cancellation to hide rounding)
    # stay within the gate, one row at a time and on the 2-, 4- and 8-row
    # launches; an all-zero row gives exactly zero
    if kind.startswith("int8"):
        oq = _int8_pc(0xE1 + K, K, N)
        if kind == "int8_zp":
            oq.zero_points = ((np.arange(N) % 9) - 4).astype(np.int8)
        pq = _product(oq, (K, N))
    elif kind == "int4":
        oq = _int4_nk(0xE2 + K, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    else:
        oq = _int4_kn(0xE3 + K, K, N, 32)
        pq = _product(oq, (K, N))
    W = _oracle_weight(oq, pq.layout)
    x = _extreme_rows(0xE4 + K + N, K)
    y64 = O.gemm_f64(x, W)
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 9)
    try:
        outs = [backend.matmulQuantized(x[m:m + 1], pq) for m in range(8)]
        outs.append(backend.matmulQuantized(x[:2], pq))
        outs.append(backend.matmulQuantized(x[4:], pq))
        outs.append(backend.matmulQuantized(x, pq))
    finally:
        backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)
    rows = [[m] for m in range(8)] + [[0, 1], [4, 5, 6, 7], list(range(8))]
    for y, ms in zip(outs, rows):
        for i, m in enumerate(ms):
            if m == 3:
                assert np.all(y[i] == 0.0), (kind, len(ms))
            else:
                err = O.parity_errors(y[i:i + 1], y64[m:m + 1])
                assert err["gated"] <= GATE, (kind, m, len(ms), err)


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)])
def test_int4_7b_projection_shapes(backend, K, N):
    # the 7B projection set (q/k/v/o, gate/up, down, LM
    # head), INT4 g32 along K, batch M in {1, 8}; M = 2..4 cross the default
    # VALU / matrix-core thresholds of these shapes
    qt = _int4_nk(0x7B1A0070 + K + N, K, N, 32)
    _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(1, 2, 3, 4, 8), cpu_path=False)


@pytest.mark.parametrize("K,N,gs,path", [(256, 512, 32, "int4_ngroup"), (2048, 2048, 32, "int4_ngroup"),
                                         (128, 64, 128, "int4_ngroup"), (64, 96, 96, "int4_ngroup"),
                                         (40, 48, 48, "int4_ngroup"), (50, 40, 48, "generic"),
                                         (33, 7, 16, "generic")])
def test_int4_runtime_layout(backend, K, N, gs, path):
    qt = _int4_kn(K * 3 + N + gs, K, N, gs)
    w = _check(backend, _product(qt, (K, N)), qt, Ms=(1, 2, 4, 5))
    assert w.path == path


@pytest.mark.parametrize("K,N,gs", [
    (2048, 32000, 32),    # configs[1] shapes in the runtime layout, I = 1, U = 4
    (2048, 5632, 32), (5632, 2048, 32),   # I = 3
    (2048, 2048, 64),
    (11008, 4096, 32),    # I = 6 (7B down projection)
    (4096, 11008, 128),
    (1024, 64, 128),      # group spans two k rows: every output shares each k-block's scale
    (160, 96, 32),        # one chunk iteration, ragged
])
def test_int4_runtime_layout_burst(backend, K, N, gs):
    # Tensor.quantize(.int4) weights (groups along N) on the burst GEMV: each
    # block stages x times its N-block's per-k scale row
    qt = _int4_kn(K + N + gs, K, N, gs)
    w = _check(backend, _product(qt, (K, N)), qt, Ms=(1, 2, 4), cpu_path=False)
    assert w.path == "int4_ngroup"


def test_int4_zero_points(backend):
    qt = _int4_nk(91, 256, 24, 32)
    qt.zero_points = ((np.arange(qt.scales.size) % 7) - 3).astype(np.int8)
    w = _check(backend, _product(qt, (256, 24), T.Layout.NK_FLAT), qt, Ms=(1, 3))
    assert w.path == "int4_kgroup" and w.has_zero_points
    qk = _int4_kn(92, 64, 32, 32)
    qk.zero_points = ((np.arange(qk.scales.size) % 5) - 2).astype(np.int8)
    w = _check(backend, _product(qk, (64, 32)), qk, Ms=(1, 2))
    assert w.path == "generic"


def test_int4_nibble_minus_eight(backend):
    # nibble 0x8 decodes to -8 (QuantizedTensor.swift:207-212) although the
    # quantizers never write it
    K, N = 64, 16
    data = np.full(K * N // 2, np.uint8(0x8F).view(np.int8), np.int8)  # (-8, -1) pairs
    scales = np.linspace(0.5, 2.0, K * N // 32).astype(np.float32)
    qt = O.QTensor((K, N), data, scales, None, O.MODE_INT4, O.PREC_INT4, 32)
    _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(1, 2))
    _check(backend, _product(qt, (K, N)), qt, Ms=(1, 2))


def test_int4_reference_metal_vs_cpu_consistency(backend):
    # INT4QuantizationTests.swift:233-254: 8x128 @ 128x64, gs=128, GPU vs CPU <1% L2
    x = O.fill_normal(51, 8 * 128).reshape(8, 128)
    qt = O.quantize_int4(O.fill_normal(52, 128 * 64).reshape(128, 64), 128)
    y = backend.matmulQuantized(x, _product(qt, (128, 64)))
    y_cpu, _, _ = O.matmul_quantized_cpu(x, qt)
    assert np.linalg.norm(y - y_cpu) / np.linalg.norm(y_cpu) < 0.01
    assert O.parity_errors(y, O.gemm_f64(x, O.dequantize(qt)))["gated"] <= GATE


# ---------------------------------------------------------------------------
# boundary behaviour
# ---------------------------------------------------------------------------
def test_shape_mismatch_is_a_precondition(backend):
    qt = _int8_pc(5, 64, 16)
    pq = _product(qt, (64, 16))
    with pytest.raises(T.PreconditionFailure):
        backend.matmulQuantized(np.zeros((2, 63), np.float32), pq)
    with pytest.raises(T.PreconditionFailure):
        backend.matmulQuantized(np.zeros(64, np.float32), pq)
    # the C ABI reports it as TBH_E_INVALID
    w = backend.weight(pq)
    x = np.zeros((1, 63), np.float32)
    y = np.zeros((1, 16), np.float32)
    st = _abi.lib().tbh_matmul(backend._dev, x.ctypes.data, 1, 63, w.handle, y.ctypes.data)
    assert st == _abi.E_INVALID


def test_int4_per_channel_is_unsupported(backend):
    qt = O.quantize_int4_per_channel(O.fill_normal(6, 16 * 32).reshape(16, 32))
    with pytest.raises(T.HIPBackendError) as e:
        backend.matmulQuantized(np.zeros((1, 16), np.float32), _product(qt, (16, 32)))
    assert e.value.status == _abi.E_UNSUPPORTED


def test_dimension_above_limit_is_unsupported(backend):
    # K or N above 2^30 is refused before any array is read (the kernels hold
    # row and column indices in 32-bit integers); the caller's CPU path takes it
    one = np.zeros(16, np.uint8)
    s = np.ones(1, np.float32)
    for K, N in (((1 << 30) + 1, 1), (1, (1 << 30) + 1)):
        d = _abi.QTensorDesc(K=K, N=N, precision=_abi.PREC_INT8, mode=_abi.MODE_SYMMETRIC,
                             layout=_abi.LAYOUT_KN_FLAT, group_size=0, data=one.ctypes.data,
                             data_bytes=K * N, scales=s.ctypes.data, n_scales=1)
        h = ctypes.c_void_p()
        st = _abi.lib().tbh_weight_create(backend._dev, ctypes.byref(d), ctypes.byref(h))
        assert st == _abi.E_UNSUPPORTED and not h.value, (K, N)


@pytest.mark.parametrize("kind", ["int8", "int4", "int4kn"])
def test_rows_beyond_one_gemm_launch(backend, kind):
    # 2^18 + 37 rows: the GEMM takes x in chunks of 2^18 rows, one launch
    # after the other, through the fp32 entry and the bf16 entry
    import torch

    K, N, M = 64, 32, (1 << 18) + 37
    if kind == "int8":
        oq = _int8_pc(0xB1, K, N)
        pq = _product(oq, (K, N))
    elif kind == "int4":
        oq = _int4_nk(0xB2, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    else:
        oq = _int4_kn(0xB3, K, N, 16)      # N-blocks of 16 rows
        pq = _product(oq, (K, N))
    W = _oracle_weight(oq, pq.layout)
    x = O.fill_normal(0xB4, M * K).reshape(M, K)
    y = backend.matmulQuantized(x, pq)
    err = O.parity_errors(y, O.gemm_f64(x, W))
    assert err["gated"] <= GATE, (kind, err)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    yb = backend.matmul_bf16_device(xb.cuda(), backend.weight(pq))
    torch.cuda.synchronize()
    errb = O.parity_errors(yb.cpu().numpy(), O.gemm_f64(xb.float().numpy(), W))
    assert errb["gated"] <= GATE, (kind, "bf16", errb)


def test_empty_input(backend):
    qt = _int8_pc(8, 32, 8)
    y = backend.matmulQuantized(np.zeros((0, 32), np.float32), _product(qt, (32, 8)))
    assert y.shape == (0, 8)


def test_backend_close_closes_its_weights_and_decoders_first():
    # tbh_weight_destroy and tbh_decoder_destroy read their device handle, so
    # HIPBackend.close() destroys every weight and decoder made on it (cached
    # or not) before it closes the device; their own close is then a no-op
    b = T.HIPBackend(0)
    qt = _int8_pc(97, 64, 32)
    direct = T.DeviceWeight(b, _product(qt, (64, 32)))
    cached = b.weight(_product(qt, (64, 32)))
    H, V = 64, 128
    cfg = T.DecoderConfig(num_layers=1, hidden=H, num_heads=4, num_kv_heads=2, intermediate=128, vocab=V,
                          max_seq=8)
    lm = O.quantize_per_channel(O.fill_normal(98, H * V, std=0.02).reshape(H, V))
    dec = T.Decoder(b, cfg, O.fill_normal(99, V * H).reshape(V, H), np.ones(H, np.float32), _product(lm, (H, V)))
    b.close()
    assert not direct.handle.value and not cached.handle.value and not dec._h.value
    direct.close()
    dec.close()
    del direct, cached, dec


def test_weight_cached_by_identifier_and_deterministic(backend):
    qt = _int4_nk(9, 512, 64, 32)
    pq = _product(qt, (512, 64), T.Layout.NK_FLAT)
    x = O.fill_normal(10, 3 * 512).reshape(3, 512)
    y1 = backend.matmulQuantized(x, pq)
    w1 = backend.weight(pq)
    y2 = backend.matmulQuantized(x, pq)
    assert backend.weight(pq) is w1
    np.testing.assert_array_equal(y1, y2)


def test_device_resident_entry_point(backend):
    import torch

    qt = _int4_nk(12, 2048, 512, 32)
    pq = _product(qt, (2048, 512), T.Layout.NK_FLAT)
    w = backend.weight(pq)
    W = _oracle_weight(qt, T.Layout.NK_FLAT)
    stream = torch.cuda.Stream()
    for M in (1, 4, 8):
        x = O.fill_normal(13 + M, M * 2048).reshape(M, 2048)
        xd = torch.from_numpy(x).cuda()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            yd = backend.matmul_device(xd, w, stream=stream)
        stream.synchronize()
        err = O.parity_errors(yd.cpu().numpy(), O.gemm_f64(x, W))
        assert err["gated"] <= GATE
    deq = backend.dequantize_device(w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(deq.cpu().numpy().view(np.uint32), W.view(np.uint32))


# ---------------------------------------------------------------------------
# 2..8 rows of x on the matrix cores (tbh_sgemv.hip): row-layout INT4 K-group
# weights without zero points; small N splits K over blocks
# ---------------------------------------------------------------------------
@pytest.fixture
def sgemv_from_two_rows(backend):
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 2)   # the MFMA path for every M >= 2
    backend.set_option(_abi.OPT_MFMA_MIN_ROWS, 1 << 30)   # and never the GEMM: M = 16 as two 8-row launches
    yield
    backend.set_option(_abi.OPT_SGEMV_MIN_ROWS, 0)
    backend.set_option(_abi.OPT_MFMA_MIN_ROWS, 0)


@pytest.mark.parametrize("M", [2, 3, 4, 5, 6, 7, 9, 16])
@pytest.mark.parametrize("K,N,gs", [(1024, 96, 32), (2048, 1000, 64), (4096, 300, 128), (160, 24, 32),
                                    (5632, 2048, 32)])
def test_sgemv_every_m(backend, sgemv_from_two_rows, M, K, N, gs):
    qt = _int4_nk(600 + M + K + gs, K, N, gs)
    _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(M,), cpu_path=False)


def test_sgemv_x_range_extremes(backend, sgemv_from_two_rows):
    # per-row power-of-two rescaling: huge, tiny and zero rows, and rows with
    # one huge or one tiny 32-element chunk
    K, N = 1024, 200
    qt = _int4_nk(701, K, N, 32)
    pq = _product(qt, (K, N), T.Layout.NK_FLAT)
    W = _oracle_weight(qt, T.Layout.NK_FLAT)
    x = O.fill_normal(702, 6 * K).reshape(6, K)
    x[0] *= 1e6
    x[1] *= 1e-7
    x[2, ::3] = 0.0
    x[3, :] = 0.0
    x[4, :32] *= 1e20               # one huge chunk, the rest ordinary
    x[5, 32:64] *= 1e-20            # one tiny chunk
    y = backend.matmulQuantized(x, pq)
    y64 = O.gemm_f64(x, W)
    for m in (0, 1, 2, 4, 5):
        assert O.parity_errors(y[m:m + 1], y64[m:m + 1])["gated"] <= GATE, m
    assert np.all(y[3] == 0.0)


def test_sgemv_split_k_determinism_and_graphs(backend, sgemv_from_two_rows):
    # N = 2048 gives 16 blocks of 128 rows, so K is split over blocks and the
    # splits are summed in a fixed order by a second kernel.  Captured on a
    # stream with no workspace yet, the launch runs unsplit or falls back to
    # the VALU kernel; captured after an eager call, the split launch.
    import torch

    K, N, M = 2048, 2048, 8
    oq = _int4_nk(801, K, N, 32)
    w = backend.weight(_product(oq, (K, N), T.Layout.NK_FLAT))
    xh = O.fill_normal(802, M * K).reshape(M, K)
    ref = O.gemm_f64(xh, _oracle_weight(oq, T.Layout.NK_FLAT))
    x = torch.from_numpy(xh).cuda()
    a = backend.matmul_device(x, w)
    b = backend.matmul_device(x, w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert O.parity_errors(a.cpu().numpy(), ref)["gated"] <= GATE
    s = torch.cuda.Stream()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    for phase in range(2):
        if phase == 1:
            with torch.cuda.stream(s):
                backend.matmul_device(x, w, out=y, stream=s)
            torch.cuda.synchronize()
            eager = y.cpu().numpy().copy()
            np.testing.assert_array_equal(eager, a.cpu().numpy())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            backend.matmul_device(x, w, out=y, stream=s)
        first = None
        for _ in range(3):
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            assert O.parity_errors(got, ref)["gated"] <= GATE, phase
            if first is None:
                first = got.copy()
            np.testing.assert_array_equal(got, first)
        if phase == 1:
            np.testing.assert_array_equal(first, eager)
        del g


def test_workspace_growth_keeps_captured_graphs_valid(backend, sgemv_from_two_rows):
    # A graph captured with a split launch holds its stream's workspace.  A
    # larger eager split launch on the same stream then grows that workspace:
    # the old buffer must stay allocated (it is retired, not freed), so the
    # graph still replays to the product, also after torch has allocated and
    # filled memory in between.  Covers the matrix-core GEMV (tbh_matmul_device)
    # and the prefill GEMM (tbh_matmul_bf16_device).
    import torch

    s = torch.cuda.Stream()
    # small: 2 x [2048 -> 1024] splits K 4 ways (32 KiB of partials, the
    # first 1 MiB workspace); large: 8 x [8192 -> 4096] splits K 16 ways (2 MiB)
    qs = _int4_nk(811, 2048, 1024, 32)
    ws = backend.weight(_product(qs, (2048, 1024), T.Layout.NK_FLAT))
    ql = _int4_nk(812, 8192, 4096, 32)
    wl = backend.weight(_product(ql, (8192, 4096), T.Layout.NK_FLAT))
    xs_h = O.fill_normal(813, 2 * 2048).reshape(2, 2048)
    xl_h = O.fill_normal(814, 8 * 8192).reshape(8, 8192)
    ref_s = O.gemm_f64(xs_h, _oracle_weight(qs, T.Layout.NK_FLAT))
    ref_l = O.gemm_f64(xl_h, _oracle_weight(ql, T.Layout.NK_FLAT))
    # prefill, M = 64: [5632 -> 2048] splits K 15 ways (7.9 MB of partials,
    # an 8 MiB workspace); [5632 -> 6000] 6 ways (9.2 MB, more than 8 MiB)
    qp = _int4_nk(815, 5632, 2048, 32)
    wp = backend.weight(_product(qp, (5632, 2048), T.Layout.NK_FLAT))
    qp2 = _int4_nk(816, 5632, 6000, 32)
    wp2 = backend.weight(_product(qp2, (5632, 6000), T.Layout.NK_FLAT))
    xp_b = torch.from_numpy(O.fill_normal(817, 64 * 5632).reshape(64, 5632)).to(torch.bfloat16)
    xp2_b = torch.from_numpy(O.fill_normal(818, 64 * 5632).reshape(64, 5632)).to(torch.bfloat16)
    ref_p = O.gemm_f64(xp_b.float().numpy(), _oracle_weight(qp, T.Layout.NK_FLAT))
    ref_p2 = O.gemm_f64(xp2_b.float().numpy(), _oracle_weight(qp2, T.Layout.NK_FLAT))

    xs, xl = torch.from_numpy(xs_h).cuda(), torch.from_numpy(xl_h).cuda()
    xp, xp2 = xp_b.cuda(), xp2_b.cuda()
    ys = torch.empty((2, 1024), dtype=torch.float32, device="cuda")
    yl = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
    yp = torch.empty((64, 2048), dtype=torch.float32, device="cuda")
    yp2 = torch.empty((64, 6000), dtype=torch.float32, device="cuda")
    for small, large, ref_small, ref_large, y_small, y_large in (
        (lambda: backend.matmul_device(xs, ws, out=ys, stream=s),
         lambda: backend.matmul_device(xl, wl, out=yl, stream=s), ref_s, ref_l, ys, yl),
        (lambda: backend.matmul_bf16_device(xp, wp, out=yp, stream=s),
         lambda: backend.matmul_bf16_device(xp2, wp2, out=yp2, stream=s), ref_p, ref_p2, yp, yp2),
    ):
        with torch.cuda.stream(s):
            small()                       # sizes the stream's workspace for the small call
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            small()                       # the split launch, on that workspace
        with torch.cuda.stream(s):
            large()                       # grows the workspace: a new buffer
        torch.cuda.synchronize()
        assert O.parity_errors(y_large.cpu().numpy(), ref_large)["gated"] <= GATE
        junk = [torch.full((1 << 18,), float("nan"), device="cuda") for _ in range(16)]
        for _ in range(3):
            y_small.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert O.parity_errors(y_small.cpu().numpy(), ref_small)["gated"] <= GATE
        del g, junk


# ---------------------------------------------------------------------------
# many rows of fp32 x on the MFMA GEMM: each row split exactly into three bf16
# pieces (tbh_matmul / tbh_matmul_device from the per-weight row threshold)
# ---------------------------------------------------------------------------
@pytest.fixture
def mfma_from(backend):
    def set_rows(rows):
        backend.set_option(_abi.OPT_MFMA_MIN_ROWS, rows)
    yield set_rows
    backend.set_option(_abi.OPT_MFMA_MIN_ROWS, 0)


def test_fp32_mfma_reference_shapes(backend, mfma_from):
    # QuantizationTests.swift:117-135 (128 x 256 @ 256 x 512) and :137-151
    # (10 x 768 @ 768 x 3072), INT8 per channel: through the rule (M = 128)
    # and with the GEMM forced from one row (M = 10)
    for (M, K, N), rows in (((128, 256, 512), 0), ((10, 768, 3072), 1)):
        mfma_from(rows)
        qt = _int8_pc(151 + K, K, N)
        _check(backend, _product(qt, (K, N)), qt, Ms=(M,), seed=3)
        # the reference's own bound: within 1% (L2) of the fp32 product
        x = O.fill_normal(152 + M, M * K).reshape(M, K)
        w = O.fill_normal(151 + K, K * N, std=0.02).reshape(K, N)
        y = backend.matmulQuantized(x, _product(qt, (K, N)))
        ref = x.astype(np.float64) @ w.astype(np.float64)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.01


@pytest.mark.parametrize("prec,K,N,M", [
    ("int8", 2048, 5632, 16), ("int8", 2048, 5632, 128), ("int8", 1000, 777, 33), ("int8", 64, 40, 300),
    ("int4", 5632, 2048, 17), ("int4", 2048, 5632, 64), ("int4", 4096, 1000, 200), ("int4", 96, 24, 70),
])
def test_fp32_mfma_shapes(backend, prec, K, N, M):
    # ragged M (the last row quad of a tile partly past M), ragged K and N,
    # K-split and unsplit launches
    if prec == "int8":
        oq = _int8_pc(161 + K + M, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(163 + K + M, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    _check(backend, pq, oq, Ms=(M,), seed=7)


def test_fp32_mfma_every_small_m(backend, mfma_from):
    # forced from one row: M = 1 .. 9 as whole and ragged row quads
    mfma_from(1)
    qt = _int4_nk(171, 1024, 300, 64)
    pq = _product(qt, (1024, 300), T.Layout.NK_FLAT)
    _check(backend, pq, qt, Ms=(1, 2, 3, 4, 5, 7, 9), seed=9)


def test_fp32_mfma_exact_split(backend, mfma_from):
    # x values whose 24 significant bits all matter, across the exponent
    # range, and zero rows: the three bf16 pieces carry x exactly, so the
    # result stays within the matmul gate of the float64 product
    mfma_from(1)
    K, N, M = 512, 256, 8
    qt = _int8_pc(181, K, N)
    pq = _product(qt, (K, N))
    W = O.dequantize(qt)
    rng = np.random.default_rng(182)
    mant = rng.integers(1 << 23, 1 << 24, size=(M, K)).astype(np.float64) / (1 << 23)
    sign = np.where(rng.random((M, K)) < 0.5, -1.0, 1.0)
    expo = rng.integers(-60, 60, size=(M, 1)).astype(np.float64)
    expo[6], expo[7] = 100, -100
    x = (sign * mant * np.exp2(expo)).astype(np.float32)
    x[3] = 0.0
    x[5, ::2] = 0.0
    y = backend.matmulQuantized(x, pq)
    y64 = O.gemm_f64(x, W)
    for m in range(M):
        assert O.parity_errors(y[m:m + 1], y64[m:m + 1])["gated"] <= GATE, m
    assert np.all(y[3] == 0.0)
    # error against sum_k |x_k w_kn|: fp32 accumulation gives about
    # sqrt(K) 2^-24 (at most K 2^-24 = 3e-5); a split that kept only the
    # upper 16 bits of x would give about 2^-9
    mag = np.abs(x.astype(np.float64)) @ np.abs(W.astype(np.float64))
    with np.errstate(invalid="ignore"):
        rel = np.where(mag > 0, np.abs(y - y64) / mag, 0.0)
    assert float(rel.max()) < 3e-5


@pytest.mark.parametrize("kind", ["int8", "int4", "int8_zp"])
def test_fp32_mfma_f16_pieces(backend, kind):
    # past 64 rows fp32 x goes to the GEMM as two f16 pieces scaled by a
    # power of two per row: rows across the exponent range with all 24
    # significant bits in use, a row mixing magnitudes 2^-30..2^30, zero rows
    # and rows holding infinities or NaN (whose NaN and signed-infinity
    # pattern must equal the float64 product's)
    K, N, M = 512, 256, 80
    if kind == "int4":
        qt = _int4_nk(183, K, N, 32)
        pq = _product(qt, (K, N), T.Layout.NK_FLAT)
    else:
        qt = _int8_pc(183, K, N)
        if kind == "int8_zp":
            qt.zero_points = ((np.arange(N) % 9) - 4).astype(np.int8)
        pq = _product(qt, (K, N))
    W = _oracle_weight(qt, pq.layout)
    rng = np.random.default_rng(184)
    mant = rng.integers(1 << 23, 1 << 24, size=(M, K)).astype(np.float64) / (1 << 23)
    sign = np.where(rng.random((M, K)) < 0.5, -1.0, 1.0)
    expo = rng.integers(-60, 60, size=(M, 1)).astype(np.float64) * np.ones((1, K))
    expo[6], expo[7] = 100, -100
    expo[8] = rng.integers(-30, 31, size=K)
    x = (sign * mant * np.exp2(expo)).astype(np.float32)
    x[3] = 0.0
    x[5, ::2] = 0.0
    x[10, 17] = np.inf
    x[11, 3], x[11, 40] = -np.inf, 2.5e38
    x[12, 9] = np.nan
    y = backend.matmulQuantized(x, pq)
    with np.errstate(invalid="ignore", over="ignore"):
        y64 = O.gemm_f64(x, W)
    for m in (10, 11, 12):
        np.testing.assert_array_equal(np.isnan(y[m]), np.isnan(y64[m]), err_msg=str(m))
        np.testing.assert_array_equal(np.isposinf(y[m]), np.isposinf(y64[m]), err_msg=str(m))
        np.testing.assert_array_equal(np.isneginf(y[m]), np.isneginf(y64[m]), err_msg=str(m))
    fin = [m for m in range(M) if m not in (10, 11, 12)]
    for m in fin:
        assert O.parity_errors(y[m:m + 1], y64[m:m + 1])["gated"] <= GATE, m
    assert np.all(y[3] == 0.0)
    # error against sum_k |x_k w_kn|: the pieces hold x to 2^-22 of the
    # row's largest element, below fp32 accumulation's sqrt(K) 2^-24
    mag = np.abs(x[fin].astype(np.float64)) @ np.abs(W.astype(np.float64))
    with np.errstate(invalid="ignore"):
        rel = np.where(mag > 0, np.abs(y[fin] - y64[fin]) / mag, 0.0)
    assert float(rel.max()) < 3e-5


@pytest.mark.parametrize("M", [64, 96])
def test_fp32_mfma_device_and_graph(backend, M):
    # tbh_matmul_device through the rule (M = 64: three bf16 pieces; 96: two
    # f16 pieces after the row-exponent pass): bit-identical across calls
    # and graph replays, equal to the host entry point
    import torch

    K, N = 2048, 2048
    oq = _int4_nk(191, K, N, 32)
    pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    w = backend.weight(pq)
    xh = O.fill_normal(192, M * K).reshape(M, K)
    host = backend.matmulQuantized(xh, pq)
    x = torch.from_numpy(xh).cuda()
    s = torch.cuda.Stream()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        backend.matmul_device(x, w, out=y, stream=s)
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    np.testing.assert_array_equal(eager, host)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        backend.matmul_device(x, w, out=y, stream=s)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), eager)
    del g


# ---------------------------------------------------------------------------
# both HBM layouts: K-contiguous rows (VALU GEMV, default) and 1 KiB MFMA
# tiles (MFMA GEMV, TBH_LAYOUT=tiles)
# ---------------------------------------------------------------------------
@pytest.fixture
def tile_layout(monkeypatch):
    monkeypatch.setenv("TBH_LAYOUT", "tiles")
    yield


@pytest.mark.parametrize("K,N", [(2048, 512), (100, 37), (5632, 64), (2048, 5632)])
def test_int8_tile_layout(backend, tile_layout, K, N):
    qt = _int8_pc(K + 3 * N, K, N)
    _check(backend, _product(qt, (K, N)), qt, Ms=(1, 2, 3, 4, 5, 8))


@pytest.mark.parametrize("K,N,gs", [(2048, 512, 32), (256, 40, 64), (100, 9, 0), (5632, 48, 32),
                                    (2048, 32000, 32), (48, 10, 48)])
def test_int4_tile_layout(backend, tile_layout, K, N, gs):
    qt = _int4_nk(K + N + gs + 1, K, N, gs if gs else K * N)
    if gs == 0:
        qt.group_size = 0
    _check(backend, _product(qt, (K, N), T.Layout.NK_FLAT), qt, Ms=(1, 2, 3, 4, 5, 8))


def test_tile_layout_zero_points(backend, tile_layout):
    qt = _int4_nk(93, 256, 24, 32)
    qt.zero_points = ((np.arange(qt.scales.size) % 7) - 3).astype(np.int8)
    _check(backend, _product(qt, (256, 24), T.Layout.NK_FLAT), qt, Ms=(1, 3, 8))
    q8 = _int8_pc(94, 192, 40)
    q8.zero_points = ((np.arange(40) % 9) - 4).astype(np.int8)
    _check(backend, _product(q8, (192, 40)), q8, Ms=(1, 4, 8))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8, 9, 16])
def test_mfma_every_m(backend, tile_layout, M):
    qt = _int4_nk(300 + M, 1024, 96, 32)
    _check(backend, _product(qt, (1024, 96), T.Layout.NK_FLAT), qt, Ms=(M,))
    q8 = _int8_pc(400 + M, 640, 80)
    _check(backend, _product(q8, (640, 80)), q8, Ms=(M,))


def test_x_range_extremes(backend, tile_layout):
    # per-row power-of-two rescaling keeps huge and tiny activations exact
    qt = _int4_nk(501, 512, 64, 32)
    pq = _product(qt, (512, 64), T.Layout.NK_FLAT)
    W = _oracle_weight(qt, T.Layout.NK_FLAT)
    x = O.fill_normal(502, 4 * 512).reshape(4, 512)
    x[0] *= 1e6
    x[1] *= 1e-7
    x[2, ::3] = 0.0
    x[3, :] = 0.0
    y = backend.matmulQuantized(x, pq)
    y64 = O.gemm_f64(x, W)
    for m in range(3):
        assert O.parity_errors(y[m:m + 1], y64[m:m + 1])["gated"] <= GATE, m
    assert np.all(y[3] == 0.0)


# ---------------------------------------------------------------------------
# prefill: bf16 activations on bf16 MFMA (tbh_matmul_bf16_device)
# ---------------------------------------------------------------------------
def _prefill_check(backend, pq, oq, M, seed):
    import torch

    K, N = pq.shape
    W = _oracle_weight(oq, pq.layout)
    x32 = O.fill_normal(seed, M * K).reshape(M, K)
    xb = torch.from_numpy(x32).to(torch.bfloat16)          # round to nearest even
    xf = xb.float().numpy()                                 # the exact values multiplied
    y = backend.matmul_bf16_device(xb.cuda(), backend.weight(pq))
    torch.cuda.synchronize()
    err = O.parity_errors(y.cpu().numpy(), O.gemm_f64(xf, W))
    assert err["gated"] <= GATE, (M, K, N, err)
    return err


@pytest.mark.parametrize("prec,K,N,M", [
    ("int8", 2048, 5632, 64),     # BASELINE configs[3] shapes
    ("int8", 2048, 5632, 512),
    ("int4", 5632, 2048, 128),
    ("int4", 5632, 2048, 512),
    ("int8", 64, 40, 3),          # tiny, ragged tiles
    ("int8", 1000, 777, 129),     # K not a multiple of 64, ragged M and N
    ("int4", 96, 24, 70),
    ("int4", 4096, 1000, 200),
])
def test_prefill_bf16(backend, prec, K, N, M):
    if prec == "int8":
        oq = _int8_pc(61 + K + M, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(67 + K + M, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    _prefill_check(backend, pq, oq, M, seed=5 + M)


# Tile counts that fill whole rounds of resident blocks and leave at most
# half a tile's time for a last round once its tiles are split along K: the
# leftover tiles' parts are summed by a second launch (INT8 128 x 128 blocks:
# two per CU, 512 at once; INT4: one per CU, 256).  Ragged N puts split tiles
# on the output's edge.  INT8 M = 2048 (704 tiles, 192 left) stays unsplit:
# its 192 tiles already have a CU each.
@pytest.mark.parametrize("prec,K,N,M", [
    ("int8", 2048, 5632, 1536),   # 528 tiles: 16 left, 8 parts
    ("int8", 2048, 5000, 2048),   # 640 tiles: 128 left, 2 parts, the last N tile ragged
    ("int8", 1000, 5632, 3072),   # 1056 tiles: 32 left; K of 16 steps, 8 parts of 2
    ("int4", 5632, 2048, 3072),   # 384 tiles: 128 left after one round of 256, 2 parts
    ("int8", 2048, 5632, 2048),   # unsplit
])
def test_prefill_split_tail(backend, prec, K, N, M):
    if prec == "int8":
        oq = _int8_pc(71 + K + M, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(73 + K + M, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    _prefill_check(backend, pq, oq, M, seed=9 + M)


def test_prefill_split_tail_graph(backend):
    # the split tail's GEMM and sum captured in a HIP graph: every replay (with
    # eager work on the same stream between them) equals the eager call bit
    # for bit
    import torch

    K, N, M = 2048, 5632, 1536
    oq = _int8_pc(201, K, N)
    pq = _product(oq, (K, N))
    w = backend.weight(pq)
    x = torch.from_numpy(O.fill_normal(202, M * K).reshape(M, K)).to(torch.bfloat16).cuda()
    s = torch.cuda.Stream()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    other = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        backend.matmul_bf16_device(x, w, out=y, stream=s)
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        backend.matmul_bf16_device(x, w, out=y, stream=s)
    for i in range(3):
        y.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
            backend.matmul_bf16_device(x[: M // 2], w, out=other[: M // 2], stream=s)   # eager, same stream
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), eager, err_msg=f"replay {i}")
    del g


def _prefill_tile(prec, N, M, K=0, cus=256):
    """The launch rule of tbh_prefill.hip (launch_prec) for bf16 x, restated
    to show which tile family and wave count each case below reaches."""
    Np = -(-N // 8) * 8
    t128 = -(-Np // 128) * -(-M // 128)
    t64x128 = -(-Np // 128) * -(-M // 64)
    t64 = -(-Np // 64) * -(-M // 64)
    if M >= 256:
        if t128 >= cus:
            return "128x128", 8
        if t64 >= 2 * cus and (prec == "int8" or -(-K // 64) <= 48):
            return "64x64", 4
        return "128x128 split", 8
    if prec == "int4":
        return "64x128 split", 8
    if t128 >= cus:
        return "128x128", 4
    if t64x128 >= cus:
        return "64x128", 4
    return "64x64 split", 4


@pytest.mark.parametrize("K,N,M,tile", [
    (2048, 5632, 2048, ("128x128", 8)),      # BASELINE configs[3] INT8 at M = 2048
    (2048, 5632, 128, ("64x64 split", 4)),   # configs[3] INT8 at M = 128
    (2048, 32000, 129, ("128x128", 4)),      # 4-wave 128 x 128, ragged M
    (2048, 20480, 128, ("64x128", 4)),       # 64 x 128
    (4096, 520, 300, ("128x128 split", 8)),  # 8-wave 128 x 128 split along K, ragged N
])
def test_prefill_bf16_int8_tiles(backend, K, N, M, tile):
    # every INT8 tile family of the prefill launch rule under parity
    assert backend.cu_count != 256 or _prefill_tile("int8", N, M) == tile
    oq = _int8_pc(131 + K + N + M, K, N)
    _prefill_check(backend, _product(oq, (K, N)), oq, M, seed=29 + M)


def test_prefill_bf16_int4_64x64(backend):
    # INT4 on 64 x 64 tiles without a K split (M >= 256, too few 128 x 128
    # tiles for the CUs, enough 64 x 64 tiles for two per CU, short rows)
    K, N, M = 2048, 5632, 512
    assert backend.cu_count != 256 or _prefill_tile("int4", N, M, K) == ("64x64", 4)
    oq = _int4_nk(137, K, N, 32)
    _prefill_check(backend, _product(oq, (K, N), T.Layout.NK_FLAT), oq, M, seed=31)


def test_prefill_bf16_int4_128x128_split(backend):
    # INT4 with rows of more than 48 K steps where the same tile counts
    # would give INT8 64 x 64 tiles: 128 x 128 tiles split along K
    K, N, M = 5632, 2048, 1024
    assert backend.cu_count != 256 or _prefill_tile("int4", N, M, K) == ("128x128 split", 8)
    oq = _int4_nk(137, K, N, 32)
    _prefill_check(backend, _product(oq, (K, N), T.Layout.NK_FLAT), oq, M, seed=31)


def test_prefill_bf16_large_m(backend):
    # configs[3] at M = 2048 (INT4 g32, 2048 x 5632)
    oq = _int4_nk(71, 5632, 2048, 32)
    _prefill_check(backend, _product(oq, (5632, 2048), T.Layout.NK_FLAT), oq, 2048, seed=9)


def test_prefill_bf16_int4_k128_steps(backend):
    # INT4 with every CU holding a 128 x 128 tile (16 x 16 tiles on 256 CUs)
    # stages K steps of 128: ragged M and N, K = 1056 ending in a partial
    # step (1056 = 8 * 128 + 32), zero points
    K, N, M = 1056, 2000, 2000
    q4 = _int4_nk(89, K, N, 32)
    q4.zero_points = ((np.arange(q4.scales.size) % 5) - 2).astype(np.int8)
    _prefill_check(backend, _product(q4, (K, N), T.Layout.NK_FLAT), q4, M, seed=23)


def test_prefill_bf16_zero_points_and_groups(backend):
    qi = _int8_pc(73, 512, 96)
    qi.zero_points = ((np.arange(96) % 9) - 4).astype(np.int8)
    _prefill_check(backend, _product(qi, (512, 96)), qi, 65, seed=11)
    q4 = _int4_nk(79, 512, 48, 64)                         # group 64 along K
    q4.zero_points = ((np.arange(q4.scales.size) % 7) - 3).astype(np.int8)
    _prefill_check(backend, _product(q4, (512, 48), T.Layout.NK_FLAT), q4, 64, seed=13)
    q0 = _int4_nk(83, 256, 40, 256 * 40)                   # one group for the whole tensor
    _prefill_check(backend, _product(q0, (256, 40), T.Layout.NK_FLAT), q0, 64, seed=17)


def test_prefill_bf16_split_k_determinism_and_graphs(backend):
    # M = 64 gives fewer output tiles than CUs, so the launch splits K and
    # sums the splits in a second kernel, in a fixed order.
    import torch

    K, N, M = 5632, 2048, 64
    oq = _int4_nk(101, K, N, 32)
    w = backend.weight(_product(oq, (K, N), T.Layout.NK_FLAT))
    xb = torch.from_numpy(O.fill_normal(19, M * K).reshape(M, K)).to(torch.bfloat16)
    ref = O.gemm_f64(xb.float().numpy(), _oracle_weight(oq, T.Layout.NK_FLAT))
    x = xb.cuda()
    a = backend.matmul_bf16_device(x, w)
    b = backend.matmul_bf16_device(x, w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert O.parity_errors(a.cpu().numpy(), ref)["gated"] <= GATE

    # Captured on a stream that has no workspace yet: the launch runs unsplit.
    # Captured again after an eager call has sized it: the split launch.
    s = torch.cuda.Stream()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    for phase in range(2):
        if phase == 1:
            with torch.cuda.stream(s):
                backend.matmul_bf16_device(x, w, out=y)
            torch.cuda.synchronize()
            eager = y.cpu().numpy().copy()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            backend.matmul_bf16_device(x, w, out=y)
        first = None
        for _ in range(3):
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            assert O.parity_errors(got, ref)["gated"] <= GATE, phase
            if first is None:
                first = got.copy()
            np.testing.assert_array_equal(got, first)
        if phase == 1:
            np.testing.assert_array_equal(first, eager)
        del g


@pytest.mark.parametrize("K,N,gs,M", [
    (2048, 5632, 32, 512),   # configs[3] shape, Tensor.quantize(.int4): two N-blocks per 64-output tile
    (5632, 2048, 32, 64),    # split along K
    (1000, 384, 128, 129),   # N-blocks of 128 rows (one per tile), K off the 64-deep steps, ragged M
    (512, 320, 64, 300),     # N-blocks of 64 rows
    (256, 96, 16, 70),       # N-blocks of 16 rows (four per tile), last tile half past N
    (1000, 40, 80, 65),      # a group spans two k rows: all outputs share each k-block's scale
])
def test_prefill_bf16_runtime_layout(backend, K, N, gs, M):
    # INT4 with groups along N (one scale per (N-block, k)): up to 64 rows the
    # GEMM stages x times each N-block's scales as three bf16 pieces, past
    # that the dequantized weights fl(q s) as two f16 pieces
    qk = _int4_kn(149 + K + N + gs, K, N, gs)
    pq = _product(qk, (K, N))
    assert backend.weight(pq).path == "int4_ngroup"
    _prefill_check(backend, pq, qk, M, seed=37 + M)


@pytest.mark.parametrize("M", [64, 65, 96])
def test_prefill_bf16_runtime_layout_block_ranges(backend, M):
    # past 64 rows the runtime-layout GEMM scales x by a power of two per row
    # and fl(q s) by one per N-block, the latter split into two f16 pieces:
    # N-blocks whose scales differ by 2^40, rows that differ by 2^30, each
    # N-block checked on its own (M = 64 takes the three bf16 pieces of x)
    import torch

    K, N, gs = 1024, 256, 32
    src = O.fill_normal(0x5CA1 + M, K * N, std=0.02).reshape(K, N)
    for b in range(N // gs):
        src[:, b * gs:(b + 1) * gs] *= np.float32(2.0 ** (20 * ((b % 3) - 1)))
    qk = O.quantize_int4(src, gs)
    pq = _product(qk, (K, N))
    W = _oracle_weight(qk, pq.layout)
    x = O.fill_normal(0x5CA2 + M, M * K).reshape(M, K)
    x *= (np.float32(2.0) ** ((np.arange(M) % 3 - 1) * 15).astype(np.float32))[:, None]
    xb = torch.from_numpy(x).to(torch.bfloat16)
    y = backend.matmul_bf16_device(xb.cuda(), backend.weight(pq))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    y64 = O.gemm_f64(xb.float().numpy(), W)
    for r in range(3):
        for b in range(N // gs):
            cols = slice(b * gs, (b + 1) * gs)
            err = O.parity_errors(y[r::3, cols], y64[r::3, cols])
            assert err["gated"] <= GATE, (M, r, b, err)


@pytest.mark.parametrize("M", [64, 80])
def test_prefill_bf16_runtime_layout_nonfinite(backend, M):
    # infinities and NaNs in x reach the outputs as the float64 product of
    # the same dequantized weights gives them (inf * 0 = NaN, inf - inf =
    # NaN; an infinity meets both f16 pieces of a weight, which share its
    # sign), and leave the other rows' scaling alone
    import torch

    K, N, gs = 512, 256, 32
    qk = _int4_kn(0xF1 + M, K, N, gs)
    pq = _product(qk, (K, N))
    W = _oracle_weight(qk, pq.layout)
    x = O.fill_normal(0xF2 + M, M * K).reshape(M, K)
    x[0, 5] = np.inf
    x[1, 100] = -np.inf
    x[2, 7] = np.nan
    x[3, 3], x[3, 9] = np.inf, -np.inf
    x[4, 11] = np.inf
    x[4, 200] = 3.0e38                      # a finite huge value beside the infinity
    xb = torch.from_numpy(x).to(torch.bfloat16)
    y = backend.matmul_bf16_device(xb.cuda(), backend.weight(pq))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        y64 = O.gemm_f64(xb.float().numpy(), W)
    for m in range(5):
        np.testing.assert_array_equal(np.isnan(y[m]), np.isnan(y64[m]), err_msg=str(m))
        np.testing.assert_array_equal(np.isposinf(y[m]), np.isposinf(y64[m]) | (np.isfinite(y64[m]) & (y64[m] > 3.4e38)), err_msg=str(m))
        np.testing.assert_array_equal(np.isneginf(y[m]), np.isneginf(y64[m]) | (np.isfinite(y64[m]) & (y64[m] < -3.4e38)), err_msg=str(m))
    err = O.parity_errors(y[5:], y64[5:])
    assert err["gated"] <= GATE, (M, err)


@pytest.mark.parametrize("entry", ["bf16", "fp32"])
def test_prefill_runtime_layout_graphs(backend, entry):
    # runtime-layout INT4 past 64 rows (exponent pass, weight-side kernel,
    # K split): calls bit-identical to each other; a graph captured on a
    # stream without a workspace takes the three-piece form, one captured
    # after an eager call the f16 form, and its replays, with eager calls on
    # another stream between them, equal the eager call bit for bit
    import torch

    K, N, gs, M = 2048, 1024, 32, 96
    qk = _int4_kn(0xB1, K, N, gs)
    pq = _product(qk, (K, N))
    w = backend.weight(pq)
    xh = O.fill_normal(0xB2, M * K).reshape(M, K)
    if entry == "bf16":
        xt = torch.from_numpy(xh).to(torch.bfloat16)
        run = backend.matmul_bf16_device
    else:
        xt = torch.from_numpy(xh)
        run = backend.matmul_device
    ref = O.gemm_f64(xt.float().numpy(), _oracle_weight(qk, pq.layout))
    x = xt.cuda()
    a = run(x, w)
    b = run(x, w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert O.parity_errors(a.cpu().numpy(), ref)["gated"] <= GATE
    s = torch.cuda.Stream()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    for phase in range(2):
        if phase == 1:
            with torch.cuda.stream(s):
                run(x, w, out=y)
            torch.cuda.synchronize()
            eager = y.cpu().numpy().copy()
            np.testing.assert_array_equal(eager, a.cpu().numpy())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run(x, w, out=y)
        first = None
        for _ in range(3):
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            assert O.parity_errors(got, ref)["gated"] <= GATE, phase
            if first is None:
                first = got.copy()
            np.testing.assert_array_equal(got, first)
            run(x, w)                          # eager work between the replays
            torch.cuda.synchronize()
        if phase == 1:
            np.testing.assert_array_equal(first, eager)
        del g


@pytest.mark.parametrize("entry", ["bf16", "fp32"])
def test_prefill_runtime_layout_wide_scales_nonfinite(backend, entry):
    # an N-block whose scales span 2^60 (one k row of tiny weights): the
    # weight-side kernel's variant that floors tiny scales keeps every
    # nonzero weight's high f16 piece nonzero, so infinite x meets it as
    # inf * w (+-inf), as the float64 product does; finite rows stay within
    # the gate
    import torch

    K, N, gs, M = 512, 256, 32, 80
    src = O.fill_normal(0xA1, K * N, std=0.02).reshape(K, N)
    src[7, :] *= np.float32(1e-18)
    qk = O.quantize_int4(src, gs)
    pq = _product(qk, (K, N))
    W = _oracle_weight(qk, pq.layout)
    x = O.fill_normal(0xA2, M * K).reshape(M, K)
    x[0, 7] = np.inf                      # meets the tiny weights of k = 7
    x[1, 7], x[1, 8] = -np.inf, 1e30
    xin = torch.from_numpy(x)
    if entry == "bf16":
        xin = xin.to(torch.bfloat16)
        y = backend.matmul_bf16_device(xin.cuda(), backend.weight(pq))
        torch.cuda.synchronize()
        y = y.cpu().numpy()
    else:
        y = backend.matmulQuantized(x, pq)
    with np.errstate(invalid="ignore", over="ignore"):
        y64 = O.gemm_f64(xin.float().numpy(), W)
    for m in (0, 1):
        np.testing.assert_array_equal(np.isnan(y[m]), np.isnan(y64[m]), err_msg=str(m))
        np.testing.assert_array_equal(np.isposinf(y[m]), np.isposinf(y64[m]), err_msg=str(m))
        np.testing.assert_array_equal(np.isneginf(y[m]), np.isneginf(y64[m]), err_msg=str(m))
    err = O.parity_errors(y[2:], y64[2:])
    assert err["gated"] <= GATE, (entry, err)


@pytest.mark.parametrize("kind,K,N,M", [
    ("int8", 2048, 1024, 64),      # split along K
    ("int8", 2048, 5632, 512),     # one block per tile, no split
    ("int4", 5632, 2048, 64),
    ("int4", 2048, 5632, 2048),    # 128 x 128 tiles, K steps of 128
    ("int4kn", 2048, 1024, 128),   # runtime layout: three pieces of fl(x * s)
])
def test_prefill_bf16_x_range_extremes(backend, kind, K, N, M):
    # the eight extreme rows (huge, tiny, zeros, one huge or tiny chunk, all
    # positive) repeated over M rows, each copy rescaled by a power of two
    import torch

    if kind == "int8":
        oq = _int8_pc(0xE5 + K, K, N)
        pq = _product(oq, (K, N))
    elif kind == "int4":
        oq = _int4_nk(0xE6 + K, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    else:
        oq = _int4_kn(0xE7 + K, K, N, 32)
        pq = _product(oq, (K, N))
    W = _oracle_weight(oq, pq.layout)
    base = _extreme_rows(0xE8 + K + M, K)
    x = np.concatenate([base * np.float32(2.0 ** ((r % 9) - 4)) for r in range(M // 8)])
    xb = torch.from_numpy(x).to(torch.bfloat16)
    y = backend.matmul_bf16_device(xb.cuda(), backend.weight(pq))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    y64 = O.gemm_f64(xb.float().numpy(), W)
    for m in range(M):
        if m % 8 == 3:
            assert np.all(y[m] == 0.0), (kind, m)
        else:
            err = O.parity_errors(y[m:m + 1], y64[m:m + 1])
            assert err["gated"] <= GATE, (kind, m, err)


def test_prefill_bf16_unsupported(backend):
    import torch

    qk = _int4_kn(89, 256, 96, 48)                         # runtime layout, N-blocks of 48 rows
    pq = _product(qk, (256, 96))
    x = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(T.HIPBackendError) as e:
        backend.matmul_bf16_device(x, backend.weight(pq))
    assert e.value.status == _abi.E_UNSUPPORTED
    qi = _int8_pc(97, 100, 16)                             # K % 8 != 0
    x = torch.zeros((64, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(T.HIPBackendError) as e:
        backend.matmul_bf16_device(x, backend.weight(_product(qi, (100, 16))))
    assert e.value.status == _abi.E_UNSUPPORTED


# LinearLayerWeights.apply(toRow:) (ModelWeights.swift:47-68): the product,
# then one fp32 add of bias[n] to every row.
@pytest.mark.parametrize("prec,K,N,M", [("int8", 2048, 256, 1), ("int4", 2048, 5632, 4), ("int4", 4096, 1000, 8),
                                        ("int8", 1000, 777, 3)])
def test_linear_bias(backend, prec, K, N, M):
    import torch

    if prec == "int8":
        oq = _int8_pc(111 + K, K, N)
        pq = _product(oq, (K, N))
    else:
        oq = _int4_nk(113 + K, K, N, 32)
        pq = _product(oq, (K, N), T.Layout.NK_FLAT)
    W = _oracle_weight(oq, pq.layout)
    x = O.fill_normal(29 + M, M * K).reshape(M, K)
    bias = O.fill_normal(31, N, std=0.5)
    lin = T.LinearLayerWeights(pq, bias)
    y = lin.apply(x, backend)
    # the product as tbh_matmul_device computes it, plus the bias in fp32:
    # bit-identical to the reference order (product first, then the add)
    w = backend.weight(pq)
    yd = backend.matmul_device(torch.from_numpy(x).cuda(), w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y, yd.cpu().numpy() + bias[None, :])
    err = O.parity_errors(y, O.gemm_f64(x, W) + bias[None, :].astype(np.float64))
    assert err["gated"] <= GATE, err
    # no bias: the plain product
    np.testing.assert_array_equal(T.LinearLayerWeights(pq).apply(x, backend), yd.cpu().numpy())


def test_linear_zero_weights_give_the_bias(backend):
    # closed form: all-zero weights quantize to q = 0 (scale 1.0), so every
    # output row is exactly the bias
    K, N = 256, 96
    oq = O.quantize_per_channel(np.zeros((K, N), np.float32))
    bias = O.fill_normal(37, N, std=1.0)
    y = T.LinearLayerWeights(_product(oq, (K, N)), bias).apply(O.fill_normal(41, 2 * K).reshape(2, K), backend)
    np.testing.assert_array_equal(y, np.broadcast_to(bias, (2, N)))
