"""Seeded random parity cases over the whole routing of the matmul path.

Each case draws a weight kind (every INT8 mode, zero points, INT4 in the
converter layout with groups along K and in the runtime layout with groups
along N, group sizes that do and do not tile the layouts), a shape (ragged K
and N, K not a multiple of 8 included) and a row count (1..9, the masked-row
counts, the GEMM thresholds and a few prefill sizes), then checks
dequantize() bit-exactly against the oracle (QuantizedTensor.swift:182-286
restated) and the fp32 product (tbh_matmul_device) and, where the weight
takes it, the bf16 prefill product (tbh_matmul_bf16_device) within GATE of a
float64 product over the same dequantized weights.  The cases are fixed by
their seeds, so a failure names a reproducible case.
"""
import os

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi
from test_gpu_sweep import _oracle_weight, _weight

pytestmark = pytest.mark.gpu

GATE = 1e-3

KINDS = ["int8", "int8_zp", "int8_sym", "int8_asym", "int4_nk_g32", "int4_nk_g64", "int4_nk_g128",
         "int4_nk_g32_zp", "int4_kn_g16", "int4_kn_g32", "int4_kn_g64", "int4_kn_g48"]
MS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 11, 13, 16, 24, 33, 64, 65, 130]


def _case(seed):
    r = np.random.RandomState(seed)
    kind = KINDS[r.randint(len(KINDS))]
    gs = int(kind.split("_g")[1].split("_")[0]) if "_g" in kind else 0
    if kind.startswith("int4_nk"):
        K = gs * r.randint(1, 6000 // gs + 1) if r.rand() < 0.8 else 8 * r.randint(1, 700)
        N = r.randint(1, 2500)
    elif kind.startswith("int4_kn"):
        K = 8 * r.randint(1, 700)
        N = gs * r.randint(1, 2500 // gs + 1) if r.rand() < 0.8 else r.randint(1, 2500)
    else:
        K = 8 * r.randint(1, 700) if r.rand() < 0.85 else r.randint(8, 5600)
        N = r.randint(1, 3000)
    while K * N > 6_000_000:
        N = max(1, N // 2)
    M = MS[r.randint(len(MS))]
    return kind, int(K), int(N), int(M)


# TBH_FUZZ_SEEDS=first:count runs another range of seeds (a longer sweep)
_range = os.environ.get("TBH_FUZZ_SEEDS")
SEEDS = (list(range(int(_range.split(":")[0]), int(_range.split(":")[0]) + int(_range.split(":")[1])))
         if _range else list(range(0xF0, 0xF0 + 160)))


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


@pytest.mark.parametrize("seed", SEEDS)
def test_random_case(backend, seed):
    _run_case(backend, *_case(seed), seed)


# Long rows over many output rows, which the draw above never reaches: one
# or two x rows, INT8 K in (3072, 6144] or INT4 K in (6144, 12288], 4096 to
# 9000 output rows -- the shapes on which the burst GEMV splits every row
# between two waves of its block at one x row.
LONG_KINDS = ["int8", "int8_sym", "int4_nk_g32", "int4_nk_g64", "int4_nk_g128", "int4_kn_g32", "int4_kn_g64"]


def _long_case(seed):
    r = np.random.RandomState(seed)
    kind = LONG_KINDS[r.randint(len(LONG_KINDS))]
    gs = int(kind.split("_g")[1]) if "_g" in kind else 0
    if kind.startswith("int8"):
        K = 8 * r.randint(3072 // 8 + 1, 6144 // 8 + 1)
    else:
        step = gs if kind.startswith("int4_nk") else 8
        K = step * r.randint(6144 // step + 1, 12288 // step + 1)
    step = gs if kind.startswith("int4_kn") else 1
    N = step * r.randint(4096 // step, 9000 // step + 1)
    M = (1, 1, 1, 2)[r.randint(4)]
    return kind, int(K), int(N), int(M)


# TBH_FUZZ_LONG_SEEDS=first:count runs another range of seeds
_long_range = os.environ.get("TBH_FUZZ_LONG_SEEDS")
LONG_SEEDS = (list(range(int(_long_range.split(":")[0]),
                         int(_long_range.split(":")[0]) + int(_long_range.split(":")[1])))
              if _long_range else list(range(0x1F0, 0x1F0 + 12)))


@pytest.mark.parametrize("seed", LONG_SEEDS)
def test_random_long_rows(backend, seed):
    _run_case(backend, *_long_case(seed), seed)


# Large prefill batches over many output rows, which neither draw above
# reaches: M 1024..3072, 4096..9000 output rows, K up to 1536 (so the float64
# products stay quick) -- grids of one or more whole rounds of resident
# blocks, whose leftover tiles the prefill GEMM may split along K.
LARGE_KINDS = ["int8", "int8_zp", "int4_nk_g32", "int4_nk_g64", "int4_nk_g128"]


def _large_case(seed):
    r = np.random.RandomState(seed)
    kind = LARGE_KINDS[r.randint(len(LARGE_KINDS))]
    gs = int(kind.split("_g")[1]) if "_g" in kind else 8
    K = gs * r.randint(max(1, 256 // gs), 1536 // gs + 1)
    N = r.randint(4096, 9001)
    M = 8 * r.randint(1024 // 8, 3072 // 8 + 1)
    return kind, int(K), int(N), int(M)


_large_range = os.environ.get("TBH_FUZZ_LARGE_SEEDS")
LARGE_SEEDS = (list(range(int(_large_range.split(":")[0]),
                          int(_large_range.split(":")[0]) + int(_large_range.split(":")[1])))
               if _large_range else list(range(0x2F0, 0x2F0 + 8)))


@pytest.mark.parametrize("seed", LARGE_SEEDS)
def test_random_large_prefill(backend, seed):
    _run_case(backend, *_large_case(seed), seed)


# Runtime-layout INT4 (groups along N) at 65..600 rows of x, where the bf16
# entry's GEMM scales x per row and the dequantized weights per N-block and
# splits the weights into two f16 pieces: group sizes that give one, two or four N-blocks per 64-output tile or a
# group spanning rows of k, ragged K, M and N.
NG_KINDS = ["int4_kn_g16", "int4_kn_g32", "int4_kn_g64", "int4_kn_g128", "int4_kn_g48"]


def _ng_case(seed):
    r = np.random.RandomState(seed)
    kind = NG_KINDS[r.randint(len(NG_KINDS))]
    gs = int(kind.split("_g")[1])
    K = 8 * r.randint(1, 2048 // 8 + 1)
    N = gs * r.randint(1, 3000 // gs + 1) if r.rand() < 0.8 else r.randint(1, 3000)
    M = r.randint(65, 601)
    return kind, int(K), int(N), int(M)


_ng_range = os.environ.get("TBH_FUZZ_NG_SEEDS")
NG_SEEDS = (list(range(int(_ng_range.split(":")[0]), int(_ng_range.split(":")[0]) + int(_ng_range.split(":")[1])))
            if _ng_range else list(range(0x3F0, 0x3F0 + 12)))


@pytest.mark.parametrize("seed", NG_SEEDS)
def test_random_runtime_prefill(backend, seed):
    _run_case(backend, *_ng_case(seed), seed)


def _run_case(backend, kind, K, N, M, seed):
    import torch

    qt, pq = _weight(kind, K, N, seed=seed)
    W = _oracle_weight(qt, pq.layout)
    deq = backend.dequantize(pq)
    np.testing.assert_array_equal(deq.view(np.uint32), W.view(np.uint32), err_msg=str((kind, K, N)))
    x = O.fill_normal(seed * 31 + M, M * K).reshape(M, K)
    y = backend.matmulQuantized(x, pq)
    err = O.parity_errors(y, O.gemm_f64(x, W))
    assert err["gated"] <= GATE, (kind, K, N, M, err)

    # device entry: the same bits as the host entry; the allocation-free
    # entry: the same bits again, or refused when its scratch is too small
    w = backend.weight(pq)
    xd = torch.from_numpy(x).cuda()
    yd = backend.matmul_device(xd, w)
    out = torch.empty_like(yd)
    try:
        backend.matmul_device_noalloc(xd, w, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, yd), (kind, K, N, M, "noalloc")
    except T.HIPBackendError as e:
        assert e.status == _abi.E_INVALID and "scratch" in str(e), (kind, K, N, M, str(e))
    np.testing.assert_array_equal(yd.cpu().numpy(), y, err_msg=str((kind, K, N, M, "device entry")))

    # bf16 prefill entry: weights and shapes it takes; the rest say so
    xb = torch.from_numpy(x).to(torch.bfloat16)
    try:
        yb = backend.matmul_bf16_device(xb.cuda(), w)
    except T.HIPBackendError as e:
        assert e.status == _abi.E_UNSUPPORTED, (kind, K, N, M, str(e))
        return
    torch.cuda.synchronize()
    errb = O.parity_errors(yb.cpu().numpy(), O.gemm_f64(xb.float().numpy(), W))
    assert errb["gated"] <= GATE, (kind, K, N, M, "bf16", errb)
