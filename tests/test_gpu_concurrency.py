"""Host threads sharing one device: the C ABI's concurrency contract.

tbh_weight_create / tbh_weight_destroy may run on any thread; tbh_matmul
(host pointers) is serialised per device; tbh_matmul_device runs on the
caller's stream, each stream with its own split-K workspace.  The reference
guards its weight cache with a lock (MetalBackend.swift:33-34, 1282-1308)
and tests its buffer pool from concurrent tasks (BufferPoolTests.swift:87).

Every result must equal, bit for bit, the same call made from one thread
(the kernels sum K splits in a fixed order, so a result depends on the
inputs and the route only), and be within the matmul gate of the float64
product.
"""
import threading

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T

pytestmark = pytest.mark.gpu

GATE = 1e-3
THREADS = 8
# rows of x: one-row burst GEMV, eight-row burst launch or matrix-core GEMV
# with split K, fp32 MFMA GEMM (with split K on the smaller weights)
MS = (1, 8, 64)


def _weights():
    out = []
    for j, (kind, K, N) in enumerate([("int8", 2048, 1024), ("int4", 2048, 3000), ("int4", 5632, 512),
                                      ("int4kn", 1024, 2048)]):
        if kind == "int8":
            qt = O.quantize_per_channel(O.fill_normal(0xC0 + j, K * N, std=0.02).reshape(K, N))
            layout = T.Layout.KN_FLAT
        elif kind == "int4":
            qt = O.quantize_int4(O.fill_normal(0xC0 + j, N * K, std=0.02).reshape(N, K), 32, O.ROUND_SWIFT)
            qt.shape = (K, N)
            layout = T.Layout.NK_FLAT
        else:
            qt = O.quantize_int4(O.fill_normal(0xC0 + j, K * N, std=0.02).reshape(K, N), 32)
            layout = T.Layout.KN_FLAT
        if layout == T.Layout.KN_FLAT:
            W = O.dequantize(qt)
        else:
            flat = O.QTensor((N, K), qt.data, qt.scales, qt.zero_points, qt.mode, qt.precision, qt.group_size)
            W = np.ascontiguousarray(O.dequantize(flat).T)
        pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                               qt.zero_points, layout)
        out.append((pq, W))
    return out


def _run_threads(fn):
    errors = []

    def body(t):
        try:
            fn(t)
        except BaseException as e:   # reported on the main thread
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=body, args=(t,)) for t in range(THREADS)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not errors, errors


def test_threads_share_a_device():
    import torch

    weights = _weights()
    xs = {(j, M): O.fill_normal(0xD0 + 16 * j + M, M * pq.shape[0]).reshape(M, pq.shape[0])
          for j, (pq, _) in enumerate(weights) for M in MS}
    b = T.HIPBackend(0)
    try:
        # one thread first: the expected bits
        want = {key: b.matmulQuantized(x, weights[key[0]][0]) for key, x in xs.items()}
        for (j, M), y in want.items():
            assert O.parity_errors(y, O.gemm_f64(xs[(j, M)], weights[j][1]))["gated"] <= GATE, (j, M)

        # host entry, shared cached weights, from every thread at once
        def host_calls(t):
            for r in range(3):
                for key in sorted(xs, key=lambda k: (k[0] + t + r) % len(weights)):
                    y = b.matmulQuantized(xs[key], weights[key[0]][0])
                    np.testing.assert_array_equal(y, want[key], err_msg=str((t, r, key)))

        _run_threads(host_calls)

        # each thread builds and destroys its own copies of the weights and
        # runs them on a stream of its own (device entry)
        def own_weights(t):
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):    # copies and allocations on this thread's stream
                for r in range(2):
                    ws = [T.DeviceWeight(b, pq) for pq, _ in weights]
                    for (j, M), x in sorted(xs.items()):
                        xd = torch.from_numpy(x).cuda()
                        y = b.matmul_device(xd, ws[j], stream=s)
                        got = y.cpu().numpy()
                        np.testing.assert_array_equal(got, want[(j, M)], err_msg=str((t, r, j, M)))
                    s.synchronize()
                    for w in ws:
                        w.close()

        _run_threads(own_weights)
    finally:
        b.close()
