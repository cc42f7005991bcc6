"""CPU checks that pin the decode-step oracle (oracle/decode_ref.py) by
closed forms and invariants of the reference's formulas
(ModelRunner.swift:470-592, Tensor.swift:1135-1141, :1538-1556)."""
import numpy as np

from oracle.decode_ref import RefDecoder, RefLayer


def _tiny(nh=4, nkv=2, hd=8, inter=16, vocab=5, layers=1, zero=False, seed=0):
    rng = np.random.default_rng(seed)
    H = nh * hd
    kv = nkv * hd
    shapes = [(H, H), (H, kv), (H, kv), (H, H), (H, inter), (H, inter), (inter, H)]
    lays = []
    for _ in range(layers):
        ws = [np.zeros(s) if zero else rng.normal(0, 0.1, s) for s in shapes]
        lays.append(RefLayer(rng.normal(1, 0.1, H), rng.normal(1, 0.1, H), ws))
    emb = rng.normal(0, 1, (vocab, H))
    return RefDecoder(layers, H, nh, nkv, inter, vocab, emb, rng.normal(1, 0.1, H),
                      rng.normal(0, 0.1, (H, vocab)), lays)


def test_rope_known_answer_and_position_zero():
    d = _tiny(nh=1, nkv=1, hd=4)
    v = np.array([1.0, 0.0, 0.0, 1.0])
    d.pos = 0
    np.testing.assert_array_equal(d._rope(v, 1), v)            # angle 0: identity
    d.pos = 1
    r = d._rope(v, 1)
    # pair 0: theta = 10000^0 = 1 -> (cos 1, sin 1); pair 1: theta = 10000^(-1/2) = 0.01
    np.testing.assert_allclose(r[:2], [np.cos(1.0), np.sin(1.0)], rtol=1e-7)
    np.testing.assert_allclose(r[2:], [-np.sin(np.float32(0.01)), np.cos(np.float32(0.01))], rtol=1e-6)


def test_rope_preserves_pair_norms_and_relative_position():
    d = _tiny(nh=2, nkv=2, hd=16)
    rng = np.random.default_rng(3)
    q, k = rng.normal(size=32), rng.normal(size=32)
    d.pos = 7
    rq = d._rope(q, 2)
    np.testing.assert_allclose(np.hypot(rq[0::2], rq[1::2]), np.hypot(q[0::2], q[1::2]), rtol=1e-12)
    # q(p) . k(p') depends on p - p' only (per head, per pair)
    def dot_at(p, pk):
        d.pos = p
        a = d._rope(q, 2)
        d.pos = pk
        return a @ d._rope(k, 2)
    np.testing.assert_allclose(dot_at(9, 4), dot_at(14, 9), rtol=1e-5)


def test_single_position_attention_returns_v_of_the_kv_group():
    # With one cached position the softmax weight is 1, so each query head's
    # context is v of KV head h // (num_heads / num_kv_heads).
    d = _tiny(nh=4, nkv=2, hd=8, layers=1)
    x = d._rms(d.emb[3], d.layers[0].input_norm)
    v = x @ d.layers[0].weights[2]
    d.step(3)
    ctx = d.ctx_trace[0]
    for hh in range(4):
        np.testing.assert_allclose(ctx[hh * 8:(hh + 1) * 8], v[(hh // 2) * 8:(hh // 2 + 1) * 8], rtol=1e-12)


def test_two_positions_attention_is_a_convex_combination():
    d = _tiny(nh=2, nkv=1, hd=8, layers=1, seed=2)
    d.step(1)
    d.step(4)
    ctx = d.ctx_trace[0]
    v0, v1 = d.vc[0][0], d.vc[0][1]
    for hh in range(2):
        c = ctx[hh * 8:(hh + 1) * 8]
        # c = a v0 + (1 - a) v1 for one a in (0, 1)
        a = np.dot(c - v1, v0 - v1) / np.dot(v0 - v1, v0 - v1)
        assert 0.0 < a < 1.0
        np.testing.assert_allclose(c, a * v0 + (1 - a) * v1, rtol=1e-10, atol=1e-12)


def test_zero_projections_leave_the_embedding():
    d = _tiny(zero=True)
    logits = d.step(2)
    h = d.emb[2]
    x = h / np.sqrt(np.sum(h * h) / h.size + 1e-5) * d.final_norm
    np.testing.assert_allclose(logits, x @ d.lm, rtol=1e-12)
    assert d.pos == 1


def test_softmax_weights_and_reset():
    d = _tiny(layers=2, seed=5)
    a = [d.step(t) for t in (1, 2, 3)]
    d.reset()
    b = [d.step(t) for t in (1, 2, 3)]
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_swiglu_ffn_closed_form():
    # ModelRunner.swift:445-452: h <- h + (silu(x Wg) * (x Wu)) Wd with
    # x = rmsNorm(h, post_norm).  Attention projections are zero, so h after
    # attention is the embedding row.  Gate and up are diagonal maps chosen
    # so that x Wg = g and x Wu = u for known vectors g, u; down sends entry
    # j to output column perm[j] times c[j]; the LM head is the identity, so
    # the logits are rmsNorm(h_out, final_norm).  The expectation goes
    # through torch's rms_norm and silu, not through the oracle's helpers.
    import torch
    import torch.nn.functional as F

    H, inter = 8, 4
    d = _tiny(nh=2, nkv=1, hd=4, inter=inter, vocab=H, zero=True, seed=9)
    rng = np.random.default_rng(19)
    tok = 3
    h = d.emb[tok].copy()
    post = d.layers[0].post_norm
    x = F.rms_norm(torch.tensor(h), (H,), weight=torch.tensor(post), eps=1e-5).numpy()
    g = np.array([1.5, -2.0, 0.7, 3.0])
    u = np.array([-0.5, 1.2, 2.0, -1.0])
    perm = np.array([5, 0, 7, 2])
    c = rng.normal(0, 1, inter)
    wg = np.zeros((H, inter))
    wu = np.zeros((H, inter))
    wd = np.zeros((inter, H))
    for j in range(inter):
        wg[j, j] = g[j] / x[j]
        wu[j, j] = u[j] / x[j]
        wd[j, perm[j]] = c[j]
    w = list(d.layers[0].weights)
    w[4], w[5], w[6] = wg, wu, wd
    d.layers[0].weights = w
    d.lm = np.eye(H)
    silu = F.silu(torch.tensor(g)).numpy()
    h_out = h.copy()
    h_out[perm] += silu * u * c
    want = F.rms_norm(torch.tensor(h_out), (H,), weight=torch.tensor(d.final_norm), eps=1e-5).numpy()
    logits = d.step(tok)
    np.testing.assert_allclose(logits, want, rtol=1e-10, atol=1e-12)
    # the plausible slips give a different answer: gate and up swapped
    # (silu(u) * g), or the residual dropped
    swapped = h.copy()
    swapped[perm] += F.silu(torch.tensor(u)).numpy() * g * c
    no_res = np.zeros(H)
    no_res[perm] = silu * u * c
    for bad in (swapped, no_res):
        b = F.rms_norm(torch.tensor(bad), (H,), weight=torch.tensor(d.final_norm), eps=1e-5).numpy()
        assert np.max(np.abs(b - logits)) > 1e-3
