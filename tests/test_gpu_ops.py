"""GPU parity of the non-matmul backend protocols (tbh_softmax, tbh_rmsnorm,
tbh_silu, tbh_gelu, tbh_attention) against oracle/ops_ref.py (float64 on the
same fp32 inputs).  Cases mirror the reference's Phase3KernelTests.swift and
FlashAttentionTests.swift (whose gate is a 5e-4 relative tolerance) plus the
shapes of the decode path and the kernels' own edge cases (rows longer than
one wave handles, lengths that are not multiples of 4, unaligned pointers,
masked tiles).  The gates here are tighter than the reference's and are
written at each assertion."""
import ctypes

import numpy as np
import pytest

import tinybrain_amd as T
from oracle import ops_ref as R
from tinybrain_amd import _abi
from tinybrain_amd.quantized import PreconditionFailure

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


def _rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).normal(size=shape) * scale).astype(np.float32)


@pytest.mark.parametrize("shape,seed", [
    ((4,), None), ((8, 16), 1), ((256, 512), 2), ((1, 32000), 3), ((3, 1001), 4), ((5, 3001), 5),
    ((37, 7), 6), ((2, 3, 40), 7), ((1, 1), 8),
])
def test_softmax(backend, shape, seed):
    x = np.array([1, 2, 3, 4], np.float32) if seed is None else _rand(seed, shape, 3.0)
    y = backend.softmax(x)
    assert y.shape == x.shape
    # rtol 2e-6 (fp32 exp, sum and division); atol covers fp32 denormals
    np.testing.assert_allclose(y, R.softmax(x), rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(y.sum(axis=-1), 1.0, atol=1e-5)


def test_softmax_extremes(backend):
    x = np.array([1000.0, 999.0, 998.0, 0.0, -100.0, -200.0, 500.0, 501.0], np.float32)
    y = backend.softmax(x)
    assert np.all(np.isfinite(y)) and abs(float(y.sum()) - 1.0) < 1e-4
    np.testing.assert_allclose(y, R.softmax(x), rtol=2e-6, atol=1e-38)
    z = np.array([[-np.inf, 0.0, 1.0, -np.inf], [-np.inf] * 4], np.float32)
    yz = backend.softmax(z)
    np.testing.assert_allclose(yz[0], R.softmax(z[0]), rtol=2e-6)
    assert np.all(np.isnan(yz[1]))            # all -inf: x - max = NaN, as softmaxCPU


@pytest.mark.parametrize("tokens,hidden,eps,seed", [
    (1, 8, 1e-5, None), (4, 32, 1e-5, 1), (32, 256, 1e-6, 2), (7, 2048, 1e-5, 3), (3, 5632, 1e-5, 4),
    (5, 1000, 1e-5, 5), (2, 1003, 1e-6, 6), (9, 4097, 1e-5, 7),
])
def test_rmsnorm(backend, tokens, hidden, eps, seed):
    if seed is None:
        x = np.arange(1, 9, dtype=np.float32)[None]
        w = np.ones(8, np.float32)
    else:
        x = _rand(seed, (tokens, hidden))
        w = np.random.default_rng(seed + 50).uniform(0.5, 1.5, hidden).astype(np.float32)
    y = backend.rmsnorm(x, w, eps)
    np.testing.assert_allclose(y, R.rmsnorm(x, w, eps), rtol=2e-6, atol=1e-7)


def test_rmsnorm_preconditions(backend):
    with pytest.raises(PreconditionFailure):
        backend.rmsnorm(np.ones(8, np.float32), np.ones(8, np.float32))
    with pytest.raises(PreconditionFailure):
        backend.rmsnorm(np.ones((2, 8), np.float32), np.ones(7, np.float32))


@pytest.mark.parametrize("op", ["silu", "gelu"])
def test_activations(backend, op):
    ref = getattr(R, op)
    fn = getattr(backend, op)
    basic = np.array([-3.0, -1.0, 0.0, 1.0, 3.0], np.float32)
    y = fn(basic)
    assert y[2] == 0.0
    np.testing.assert_allclose(y, ref(basic), rtol=2e-6, atol=1e-7)
    for n, seed in [(4096, 1), (1000003, 2), (3, 3)]:
        x = _rand(seed, (n,), 4.0)
        np.testing.assert_allclose(fn(x), ref(x), rtol=2e-6, atol=1e-7)
    pos = (np.arange(64) * 0.1).astype(np.float32)
    yp = fn(pos)
    assert np.all(yp >= 0.0) and np.all(yp <= pos + 1e-6)


def test_ops_device_api(backend):
    # The device entries on torch tensors (including an unaligned view, which
    # takes the scalar kernels) give the host entries' bits.
    import torch

    x = _rand(11, (6, 1030), 2.0)
    w = np.random.default_rng(12).uniform(0.5, 1.5, 1030).astype(np.float32)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    np.testing.assert_array_equal(backend.softmax_device(xd).cpu().numpy(), backend.softmax(x))
    np.testing.assert_array_equal(backend.rmsnorm_device(xd, wd, 1e-5).cpu().numpy(), backend.rmsnorm(x, w))
    flat = torch.from_numpy(_rand(13, (4097,), 3.0)).cuda()
    view = flat[1:]                                  # 4-byte offset: not 16-byte aligned
    for op in ("silu", "gelu"):
        got = getattr(backend, op + "_device")(view).cpu().numpy()
        np.testing.assert_array_equal(got, getattr(backend, op)(view.cpu().numpy()))
    torch.cuda.synchronize()


ATTN_CASES = [
    # (batch, seq, kv, head_dim, heads, kv_heads) -- FlashAttentionTests.swift
    (None, 8, 8, 16, 4, 4),          # basic MHA
    (None, 16, 16, 16, 32, 8),       # GQA 32:8
    (None, 12, 12, 32, 8, 2),        # GQA small
    (None, 1, 32, 16, 4, 4),         # single-token decode over 32 cached positions
    (None, 37, 37, 16, 4, 4),        # not a multiple of the reference's 32-row tile
    (None, 16, 16, 32, 1, 1),        # single head
    (2, 8, 8, 16, 4, 4),             # batched
    (None, 256, 256, 32, 8, 4),      # larger sequence, GQA 8:4
    (None, 16, 16, 64, 4, 4),        # head_dim 64
    # decode and kernel edge cases
    (None, 1, 512, 64, 32, 4),       # TinyLlama decode at context 512
    (3, 5, 130, 128, 8, 2),          # head_dim 128, several 64-position tiles
    (None, 4, 70, 256, 2, 1),        # head_dim 256 (four elements per lane)
    (None, 6, 65, 80, 4, 2),         # head_dim 80: partial second lane group
    (None, 9, 33, 6, 3, 3),          # head_dim 6: scalar loads
    (None, 1, 4096, 64, 32, 4),      # long decode context: many key-position splits
    (2, 3, 300, 32, 32, 2),          # 16 query heads per key/value head: two head groups
    (None, 2, 200, 64, 12, 1),       # 12 query heads per key/value head: a partial group
]


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention(backend, case):
    B, S, Tk, hd, nh, nkv = case
    seed = S * 1000 + Tk + hd
    lead = () if B is None else (B,)
    q = _rand(seed, lead + (S, nh * hd))
    k = _rand(seed + 1, lead + (Tk, nkv * hd))
    v = _rand(seed + 2, lead + (Tk, nkv * hd))
    y = backend.attention(q, k, v, None, hd, nh, nkv)
    assert y.shape == q.shape
    # fp32 scores and accumulation: rtol 1e-4, atol 1e-5 (reference gate 5e-4)
    np.testing.assert_allclose(y, R.attention(q, k, v, None, hd, nh, nkv), rtol=1e-4, atol=1e-5)


def test_attention_masks(backend):
    S, Tk, hd, nh, nkv = 16, 16, 16, 4, 4
    q, k, v = _rand(1, (S, nh * hd)), _rand(2, (Tk, nkv * hd)), _rand(3, (Tk, nkv * hd))
    mask = np.zeros(Tk, np.float32)
    mask[8:] = -np.inf                                # FlashAttentionTests.testMaskedAttention
    np.testing.assert_allclose(backend.attention(q, k, v, mask, hd, nh, nkv),
                               R.attention(q, k, v, mask, hd, nh, nkv), rtol=1e-4, atol=1e-5)
    # a fully masked first 64-position tile, then attended positions
    Tk = 150
    k, v = _rand(4, (Tk, nkv * hd)), _rand(5, (Tk, nkv * hd))
    mask = np.zeros(Tk, np.float32)
    mask[:70] = -np.inf
    mask[100:110] = -0.5
    np.testing.assert_allclose(backend.attention(q, k, v, mask, hd, nh, nkv),
                               R.attention(q, k, v, mask, hd, nh, nkv), rtol=1e-4, atol=1e-5)
    # every position masked: NaN, as the reference's CPU attention; no positions: zeros
    assert np.all(np.isnan(backend.attention(q, k, v, np.full(Tk, -np.inf, np.float32), hd, nh, nkv)))
    e = np.zeros((0, nkv * hd), np.float32)
    assert np.all(backend.attention(q, e, e, None, hd, nh, nkv) == 0.0)


def test_attention_device_and_errors(backend):
    import torch

    q, k, v = _rand(7, (2, 3, 4 * 32)), _rand(8, (2, 20, 2 * 32)), _rand(9, (2, 20, 2 * 32))
    got = backend.attention_device(*(torch.from_numpy(a).cuda() for a in (q, k, v)), None, 32, 4, 2)
    np.testing.assert_array_equal(got.cpu().numpy(), backend.attention(q, k, v, None, 32, 4, 2))
    with pytest.raises(PreconditionFailure):
        backend.attention(q, k, v, None, 32, 4, 3)
    # the C entry checks on its own: heads not a multiple, head_dim too large
    sh = _abi.AttentionShape(1, 1, 1, 32, 4, 3)
    buf = np.zeros(1024, np.float32)
    p = buf.ctypes.data
    assert backend._lib.tbh_attention(backend._dev, ctypes.byref(sh), p, p, p, None, p) == _abi.E_INVALID
    sh = _abi.AttentionShape(1, 1, 1, 300, 1, 1)
    assert backend._lib.tbh_attention(backend._dev, ctypes.byref(sh), p, p, p, None, p) == _abi.E_UNSUPPORTED
