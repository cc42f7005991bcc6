"""Pins of oracle/ops_ref.py (the checker of the softmax, RMSNorm, SiLU, GELU
and attention kernels) by known answers, closed forms and independent library
routines (torch float64), chosen so that a dropped term, a wrong head
mapping or a misplaced epsilon fails.  CPU only."""
import numpy as np
import pytest

from oracle import ops_ref as R


def test_softmax_known_answer_and_epsilon():
    # softmax([1, 2, 3, 4]) = e^i / sum(e^j): published closed form
    want = np.exp([1.0, 2.0, 3.0, 4.0]) / np.exp([1.0, 2.0, 3.0, 4.0]).sum()
    got = R.softmax(np.array([1.0, 2.0, 3.0, 4.0]))
    np.testing.assert_allclose(got, [0.0320586033, 0.0871443187, 0.2368828181, 0.6439142599], atol=1e-9)
    np.testing.assert_allclose(got, want, rtol=2e-7)
    # the epsilon sits in the denominator once: a row of n equal values is 1/(n + 1e-7)
    np.testing.assert_allclose(R.softmax(np.zeros(8)), np.full(8, 1.0 / (8 + 1e-7)), rtol=1e-15)


def test_softmax_stability_and_library():
    import torch

    x = np.array([1000.0, 999.0, 998.0, 0.0, -100.0, -200.0, 500.0, 501.0])   # Phase3KernelTests
    y = R.softmax(x)
    assert np.all(np.isfinite(y)) and abs(y.sum() - 1.0) < 1e-6
    r = np.random.default_rng(0).normal(size=(7, 33)) * 4
    t = torch.softmax(torch.from_numpy(r), dim=-1).numpy()
    np.testing.assert_allclose(R.softmax(r), t, rtol=1e-6, atol=1e-12)


def test_rmsnorm_closed_form_and_library():
    import torch

    x = np.arange(1.0, 9.0)                                  # Phase3KernelTests identity case
    y = R.rmsnorm(x[None], np.ones(8), 1e-5)[0]
    np.testing.assert_allclose(y, x / np.sqrt(np.mean(x ** 2) + 1e-5), rtol=1e-15)
    r = np.random.default_rng(1).normal(size=(5, 48))
    w = np.random.default_rng(2).uniform(0.5, 1.5, 48)
    t = torch.nn.functional.rms_norm(torch.from_numpy(r), (48,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(R.rmsnorm(r, w, 1e-6), t, rtol=1e-12)


def test_activations_known_answers_and_library():
    import torch

    assert R.silu(np.array([0.0]))[0] == 0.0 and R.gelu(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(R.silu(np.array([1.0])), [1.0 / (1.0 + np.exp(-1.0))], rtol=1e-15)
    np.testing.assert_allclose(R.silu(np.array([1.0])), [0.7310585786300049], rtol=1e-14)
    x = np.linspace(-8, 8, 257)
    np.testing.assert_allclose(R.silu(x), torch.nn.functional.silu(torch.from_numpy(x)).numpy(), rtol=1e-12,
                               atol=1e-300)
    tg = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    # 1 + tanh(inner) cancels for x << 0, so the forms agree to an absolute 1e-15 there
    np.testing.assert_allclose(R.gelu(x), tg, rtol=1e-12, atol=1e-15)
    # and it is the tanh form, not the erf form: they differ by up to ~5e-4
    te = torch.nn.functional.gelu(torch.from_numpy(x)).numpy()
    assert 1e-4 < np.max(np.abs(R.gelu(x) - te)) < 1e-3


def _torch_attention(q, k, v, mask, hd, nh, nkv):
    import torch

    q, k, v = (torch.from_numpy(np.asarray(a, np.float64)) for a in (q, k, v))
    if q.dim() == 2:
        q, k, v = q[None], k[None], v[None]
    B, S, T = q.shape[0], q.shape[1], k.shape[1]
    qh = q.reshape(B, S, nh, hd).transpose(1, 2)
    kh = k.reshape(B, T, nkv, hd).transpose(1, 2).repeat_interleave(nh // nkv, dim=1)
    vh = v.reshape(B, T, nkv, hd).transpose(1, 2).repeat_interleave(nh // nkv, dim=1)
    am = None if mask is None else torch.from_numpy(np.asarray(mask, np.float64)).reshape(1, 1, 1, T)
    o = torch.nn.functional.scaled_dot_product_attention(qh.contiguous(), kh.contiguous(), vh.contiguous(),
                                                         attn_mask=am)
    return o.transpose(1, 2).reshape(B, S, nh * hd).numpy()


@pytest.mark.parametrize("B,S,T,hd,nh,nkv,masked", [
    (1, 8, 8, 16, 4, 4, False),
    (1, 12, 12, 32, 8, 2, False),       # GQA: head h reads kv head h // 4
    (2, 5, 9, 16, 4, 2, True),
    (1, 1, 40, 64, 8, 1, True),
])
def test_attention_matches_library(B, S, T, hd, nh, nkv, masked):
    rng = np.random.default_rng(B * 100 + T)
    q = rng.normal(size=(B, S, nh * hd))
    k = rng.normal(size=(B, T, nkv * hd))
    v = rng.normal(size=(B, T, nkv * hd))
    mask = None
    if masked:
        mask = np.zeros(T)
        mask[T // 2:] = -np.inf
        mask[0] = -np.inf
    got = R.attention(q, k, v, mask, hd, nh, nkv, eps=0.0)
    np.testing.assert_allclose(got, _torch_attention(q, k, v, mask, hd, nh, nkv), rtol=1e-10, atol=1e-12)
    # the 1e-7 epsilon changes the result by a relative 1e-7 at most (sum p >= 1)
    np.testing.assert_allclose(R.attention(q, k, v, mask, hd, nh, nkv), got, rtol=2e-7, atol=1e-12)


def test_attention_edge_cases():
    q = np.ones((3, 8))
    k = np.ones((4, 8))
    v = np.arange(32.0).reshape(4, 8)
    assert np.all(np.isnan(R.attention(q, k, v, np.full(4, -np.inf), 8, 1, 1)))
    assert np.all(R.attention(q, np.zeros((0, 8)), np.zeros((0, 8)), None, 8, 1, 1) == 0.0)
    # equal scores: the mean of the value rows
    np.testing.assert_allclose(R.attention(q, k, v, None, 8, 1, 1, eps=0.0), np.tile(v.mean(0), (3, 1)))
