"""GPU decode step (tbh_decoder) against the decode-step oracle
(oracle/decode_ref.py, ModelRunner.step restated in float64) on the same
dequantized weights.  Gate: max|logit - ref| / max(|ref|, 1e-3 * max|ref|)
<= 1e-3 at every step."""
import os

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from oracle.decode_ref import RefDecoder, RefLayer
from tinybrain_amd import _abi

pytestmark = pytest.mark.gpu

GATE = 1e-3


@pytest.fixture(scope="module")
def backend():
    b = T.HIPBackend(0)
    yield b
    b.close()


def _weight(prec, seed, K, N, std=0.02):
    """(product QuantizedTensor, dequantized [K, N] fp32) for one projection."""
    if prec == "int8":
        qt = O.quantize_per_channel(O.fill_normal(seed, K * N, std=std).reshape(K, N))
        pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                               qt.zero_points, T.Layout.KN_FLAT)
        return pq, O.dequantize(qt)
    if prec == "int4kn":
        # Tensor.quantize(.int4) on [K, N]: the runtime layout, groups of 32 along N
        qt = O.quantize_int4(O.fill_normal(seed, K * N, std=std).reshape(K, N), 32, O.ROUND_SWIFT)
        pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                               qt.zero_points, T.Layout.KN_FLAT)
        return pq, O.dequantize(qt)
    qt = O.quantize_int4(O.fill_normal(seed, N * K, std=std).reshape(N, K), 32, O.ROUND_SWIFT)
    pq = T.QuantizedTensor((K, N), qt.data, qt.scales, qt.mode, qt.precision, qt.group_size,
                           qt.zero_points, T.Layout.NK_FLAT)
    return pq, np.ascontiguousarray(O.dequantize(qt).T)


def _model(backend, cfg: T.DecoderConfig, prec: str, seed: int):
    H, I, V, kv = cfg.hidden, cfg.intermediate, cfg.vocab, cfg.kv_dim
    norm = lambda s: (1.0 + 0.1 * O.fill_normal(s, H)).astype(np.float32)
    emb = O.fill_normal(seed, V * H).reshape(V, H)
    fn = norm(seed + 1)
    lm, lm_w = _weight(prec, seed + 2, H, V)
    dec = T.Decoder(backend, cfg, emb, fn, lm)
    layers = []
    shapes = [(H, H), (H, kv), (H, kv), (H, H), (H, I), (H, I), (I, H)]
    for l in range(cfg.num_layers):
        ws = [_weight(prec, seed + 100 * (l + 1) + j, K, N) for j, (K, N) in enumerate(shapes)]
        gi, gp = norm(seed + 100 * (l + 1) + 50), norm(seed + 100 * (l + 1) + 51)
        dec.set_layer(l, gi, gp, [w[0] for w in ws])
        layers.append(RefLayer(gi, gp, [w[1] for w in ws]))
    ref = RefDecoder(cfg.num_layers, H, cfg.num_heads, cfg.num_kv_heads, I, V, emb, fn, lm_w, layers,
                     cfg.rms_eps, cfg.rope_base)
    return dec, ref


def _gated(y, ref):
    floor = 1e-3 * np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), floor)))


SMALL = dict(num_layers=2, hidden=256, num_heads=4, num_kv_heads=2, intermediate=512, vocab=1000,
             max_seq=32)


@pytest.mark.parametrize("prec", ["int8", "int4", "int4kn"])
def test_decode_small(backend, prec):
    # int4kn: the runtime INT4 layout (groups along N) needs a vocabulary the
    # groups tile
    cfg = T.DecoderConfig(**dict(SMALL, vocab=1024 if prec == "int4kn" else SMALL["vocab"]))
    dec, ref = _model(backend, cfg, prec, seed=11)
    for i, tok in enumerate([5, 17, 3, 999, 0, 42, 7, 7, 512, 1]):
        y = dec.step(tok)
        r = ref.step(tok)
        assert _gated(y, r) <= GATE, (i, tok, _gated(y, r))
        assert dec.position == i + 1
    dec.close()


def test_decode_tinyllama_width(backend):
    # TinyLlama-1.1B layer shapes with 2 of the 22 layers
    cfg = T.DecoderConfig(num_layers=2, hidden=2048, num_heads=32, num_kv_heads=4, intermediate=5632,
                          vocab=32000, max_seq=64)
    dec, ref = _model(backend, cfg, "int8", seed=21)
    for i, tok in enumerate([1, 31999, 450]):
        y = dec.step(tok)
        r = ref.step(tok)
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


class _Scaled:
    """x @ (W * f) for the float64 reference, without a copy of W per layer."""
    __array_ufunc__ = None    # numpy defers x @ self to __rmatmul__

    def __init__(self, w, f):
        self.w, self.f = w, f

    def __rmatmul__(self, x):
        return (x @ self.w) * self.f


def test_decode_tinyllama_full_depth(backend):
    # BASELINE configs[2] at its full depth: 22 layers, hidden 2048, 32/4
    # heads, FFN 5632, vocab 32000, INT8 per-channel.  One quantized matrix
    # per projection shape is shared by the layers, with each layer's scales
    # multiplied by 1 + 0.05 l and its own norm weights, so every layer's
    # dequantized weights and caches differ; the float64 reference applies
    # the factor to the shared dequantized matrix.
    cfg = T.DecoderConfig(num_layers=22, hidden=2048, num_heads=32, num_kv_heads=4, intermediate=5632,
                          vocab=32000, max_seq=64)
    H, I, V, kv = cfg.hidden, cfg.intermediate, cfg.vocab, cfg.kv_dim
    shapes = [(H, H), (H, kv), (H, kv), (H, H), (H, I), (H, I), (I, H)]
    base = []
    for j, (K, N) in enumerate(shapes):
        qt = O.quantize_per_channel(O.fill_normal(601 + j, K * N, std=0.02).reshape(K, N))
        base.append((qt, O.dequantize(qt).astype(np.float64)))
    norm = lambda sd: (1.0 + 0.1 * O.fill_normal(sd, H)).astype(np.float32)
    emb = O.fill_normal(611, V * H).reshape(V, H)
    fn = norm(612)
    lm, lm_w = _weight("int8", 613, H, V)
    dec = T.Decoder(backend, cfg, emb, fn, lm)
    layers, factors = [], []
    for l in range(cfg.num_layers):
        f = np.float32(1.0 + 0.05 * l)
        factors.append(float(f))
        ws = [T.QuantizedTensor((K, N), qt.data, (qt.scales * f).astype(np.float32), qt.mode, qt.precision,
                                qt.group_size, qt.zero_points, T.Layout.KN_FLAT)
              for (qt, _), (K, N) in zip(base, shapes)]
        gi, gp = norm(700 + 2 * l), norm(701 + 2 * l)
        dec.set_layer(l, gi, gp, ws)
        layers.append(RefLayer(gi, gp, [w64 for _, w64 in base]))   # the same arrays: no copies
    ref = RefDecoder(cfg.num_layers, H, cfg.num_heads, cfg.num_kv_heads, I, V, emb, fn, lm_w, layers,
                     cfg.rms_eps, cfg.rope_base)
    for l, f in enumerate(factors):
        ref.layers[l].weights = [_Scaled(w, f) for w in ref.layers[l].weights]
    for i, tok in enumerate([1, 31999, 450, 2048, 7]):
        y = dec.step(tok)
        r = ref.step(tok)
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_tinyllama_context_520(backend):
    # BASELINE configs[2]'s head layout at its own context: hidden 2048, 32
    # query heads over 4 KV heads (8 per KV head), head_dim 64, FFN 5632,
    # vocab 32000, INT8 per-channel, 2 layers, 520 steps.  Positions 511..519
    # run 16 and 17 attention ranges of 32 positions through the merge, as
    # the 1.1B bench step at context 512 does.  The caches and positions
    # advance at every step on both sides; logits are gated at the range
    # edges (the oracle skips its LM head elsewhere).
    cfg = T.DecoderConfig(num_layers=2, hidden=2048, num_heads=32, num_kv_heads=4, intermediate=5632,
                          vocab=32000, max_seq=528)
    dec, ref = _model(backend, cfg, "int8", seed=29)
    gates = (0, 63, 64, 127, 128, 511, 512, 519)
    rng = np.random.default_rng(29)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=520)):
        y = dec.step(int(tok))
        r = ref.step(int(tok), logits=i in gates)
        if i in gates:
            assert _gated(y, r) <= GATE, (i, _gated(y, r))
    assert dec.position == 520 and ref.pos == 520
    dec.close()


def test_decode_tinyllama_width_runtime_int4(backend):
    # TinyLlama-1.1B layer shapes, 2 layers, INT4 in the runtime layout that
    # Tensor.quantize(.int4) and the perplexity harness write (groups of 32
    # along N): Q|K|V concatenated, gate|up rows interleaved with one scale
    # table per part
    cfg = T.DecoderConfig(num_layers=2, hidden=2048, num_heads=32, num_kv_heads=4, intermediate=5632,
                          vocab=32000, max_seq=64)
    dec, ref = _model(backend, cfg, "int4kn", seed=27)
    for i, tok in enumerate([1, 31999, 450, 9]):
        y = dec.step(tok)
        r = ref.step(tok)
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_7b_width(backend):
    # 7B layer shapes with 2 of the 32 layers: INT4
    # group 32 along K, hidden 4096, 32 query and 32 KV heads (head_dim 128,
    # one query head per KV head), FFN 11008, vocab 32000
    cfg = T.DecoderConfig(num_layers=2, hidden=4096, num_heads=32, num_kv_heads=32, intermediate=11008,
                          vocab=32000, max_seq=64)
    dec, ref = _model(backend, cfg, "int4", seed=23)
    for i, tok in enumerate([1, 31999, 450, 7]):
        y = dec.step(tok)
        r = ref.step(tok)
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


@pytest.mark.parametrize("heads", [(4, 2), (16, 2), (8, 8)])
def test_decode_long_context(backend, heads):
    # more than two attention ranges (32 positions at head_dim 64 for 4/2,
    # 64 at head_dim 16 and 32 for 16/2 and 8/8), so the step's attention
    # combines several range partials (and, for 4/2, a quad with idle waves)
    nh, nkv = heads
    cfg = T.DecoderConfig(**dict(SMALL, num_heads=nh, num_kv_heads=nkv, max_seq=160))
    dec, ref = _model(backend, cfg, "int8", seed=61 + nh)
    rng = np.random.default_rng(nh * 7 + nkv)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=150)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


@pytest.mark.parametrize("hd,nh,nkv,prec", [
    (48, 4, 2, "int8"), (48, 4, 2, "int4"),
    (80, 2, 1, "int8"), (80, 2, 1, "int4"),
    (96, 8, 2, "int8"), (96, 8, 2, "int4"),
    (112, 4, 4, "int8"), (112, 4, 4, "int4"),
])
def test_decode_head_dims_off_powers_of_two(backend, hd, nh, nkv, prec):
    # head_dim / 4 not a power of two: attention scores one position per
    # lane with whole key rows, and the value pieces and the merge use
    # 64 / (head_dim / 4) lane groups with the lanes past them idle; 70
    # steps cross a 64-position range
    H = hd * nh
    cfg = T.DecoderConfig(num_layers=2, hidden=H, num_heads=nh, num_kv_heads=nkv, intermediate=2 * H,
                          vocab=500, max_seq=72)
    dec, ref = _model(backend, cfg, prec, seed=83 + hd + nh)
    rng = np.random.default_rng(hd * 5 + nkv)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=70)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_merge_beyond_one_load_round(backend):
    # head_dim 128: attention ranges of 32 positions; the merge kernel loads
    # 32 ranges (1024 positions) per head in its first round and loops over
    # the rest; 1100 steps reach 35 ranges, so every range past the 32nd
    # goes through that loop
    cfg = T.DecoderConfig(**dict(SMALL, num_layers=1, num_heads=2, num_kv_heads=1, max_seq=1104))
    dec, ref = _model(backend, cfg, "int8", seed=71)
    rng = np.random.default_rng(71)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=1100)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        if i % 50 == 0 or i >= 1020:
            assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_long_context_head_dim_64(backend):
    # head_dim 64 (the 1.1B model's), 1100 steps: 35 attention ranges of 32
    # positions; the merge kernel's first load round (4 lane groups x 8
    # loads for head_dim 64) takes 32 of them, its loop the rest
    cfg = T.DecoderConfig(**dict(SMALL, num_layers=1, max_seq=1104))
    dec, ref = _model(backend, cfg, "int8", seed=73)
    rng = np.random.default_rng(73)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=1100)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        if i % 50 == 0 or i in (511, 512, 513) or i >= 1020:
            assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_merge_beyond_one_load_round_head_dim_64(backend):
    # head_dim 64: the merge kernel's first load round covers 32 ranges of
    # 32 positions; 2100 steps reach 66, so 34 ranges go through its loop
    cfg = T.DecoderConfig(**dict(SMALL, num_layers=1, max_seq=2112))
    dec, ref = _model(backend, cfg, "int8", seed=79)
    rng = np.random.default_rng(79)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=2100)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        if i % 100 == 0 or i >= 2040:
            assert _gated(y, r) <= GATE, (i, _gated(y, r))
    dec.close()


def test_decode_reset_is_deterministic(backend):
    cfg = T.DecoderConfig(**SMALL)
    dec, _ = _model(backend, cfg, "int8", seed=31)
    a = [dec.step(t) for t in (4, 8, 15)]
    dec.reset()
    assert dec.position == 0
    b = [dec.step(t) for t in (4, 8, 15)]
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    dec.close()


def test_decode_full_cache_is_an_error(backend):
    cfg = T.DecoderConfig(**dict(SMALL, max_seq=3))
    dec, _ = _model(backend, cfg, "int8", seed=41)
    for t in (1, 2, 3):
        dec.step(t)
    with pytest.raises(T.HIPBackendError) as e:
        dec.step(4)
    assert e.value.status == _abi.E_INVALID
    dec.set_position(0)
    dec.step(1)                                   # usable again after a reset
    dec.close()


def test_decode_graph_replay_advances_position(backend):
    import torch

    cfg = T.DecoderConfig(**SMALL)
    eager, _ = _model(backend, cfg, "int8", seed=51)
    graphed, _ = _model(backend, cfg, "int8", seed=51)
    want = [eager.step(9) for _ in range(5)]
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    graphed.step_device(9, logits, s)             # position 0, eager
    torch.cuda.synchronize()
    np.testing.assert_array_equal(logits.cpu().numpy(), want[0])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        graphed.step_device(9, logits, s)
    graphed.set_position(1)                       # capture does not run the step
    for i in range(1, 5):
        logits.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(logits.cpu().numpy(), want[i])
    assert graphed.position == 5
    eager.close()
    graphed.close()


def test_decode_mixed_precision_qkv_is_rejected(backend):
    # Q in INT4 (runtime layout), K and V in INT8: Q|K|V cannot be one weight
    cfg = T.DecoderConfig(**dict(SMALL, num_layers=1))
    H, kv, I = cfg.hidden, cfg.kv_dim, cfg.intermediate
    lm, _ = _weight("int8", 1, H, cfg.vocab)
    dec = T.Decoder(backend, cfg, O.fill_normal(2, cfg.vocab * H).reshape(cfg.vocab, H),
                    np.ones(H, np.float32), lm)
    ws = [_weight("int8", 3 + j, K, N)[0] for j, (K, N) in
          enumerate([(H, H), (H, kv), (H, kv), (H, H), (H, I), (H, I), (I, H)])]
    qk = O.quantize_int4(O.fill_normal(9, H * H).reshape(H, H), 32, O.ROUND_SWIFT)   # groups along N
    ws[0] = T.QuantizedTensor((H, H), qk.data, qk.scales, qk.mode, qk.precision, qk.group_size,
                              qk.zero_points, T.Layout.KN_FLAT)
    with pytest.raises(T.HIPBackendError) as e:
        dec.set_layer(0, np.ones(H, np.float32), np.ones(H, np.float32), ws)
    assert e.value.status in (_abi.E_UNSUPPORTED, _abi.E_INVALID)
    dec.close()


def _dequant_kn(q: T.QuantizedTensor) -> np.ndarray:
    """Logical [K, N] fp32 weight of a product QuantizedTensor (oracle dequantize)."""
    K, N = q.shape
    if q.layout == T.Layout.NK_FLAT:
        oq = O.QTensor((N, K), q.data, q.scales, q.zeroPoints, int(q.mode), int(q.precision), q.groupSize)
        return np.ascontiguousarray(O.dequantize(oq).T)
    oq = O.QTensor((K, N), q.data, q.scales, q.zeroPoints, int(q.mode), int(q.precision), q.groupSize)
    return O.dequantize(oq)


@pytest.mark.parametrize("fname", ["converter_tiny_int8.tbf", "converter_tiny_int4.tbf"])
def test_decode_from_converter_tbf_file(backend, fname):
    # ModelWeights.load + ModelRunner.step on a file the reference converter wrote
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", fname)
    with T.TBFFile(path) as f:
        c = f.config
        dec = f.load_decoder(backend, max_seq=16)
        names = ["attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down"]
        layers = [RefLayer(f.floats(f"layer_{l}_ln_input"), f.floats(f"layer_{l}_ln_post"),
                           [_dequant_kn(f.quantized(f"layer_{l}_{n}")) for n in names])
                  for l in range(c["numLayers"])]
        ref = RefDecoder(c["numLayers"], c["hiddenDim"], c["numHeads"], c["numKVHeads"],
                         c["intermediateDim"], c["vocabSize"], f.floats("embeddings"),
                         f.floats("final_norm"), _dequant_kn(f.quantized("output")), layers)
        for i, tok in enumerate([3, 39, 0, 17, 17]):
            y, r = dec.step(tok), ref.step(tok)
            assert _gated(y, r) <= GATE, (fname, i, _gated(y, r))
        dec.close()


def _decode_case(seed):
    """A random decoder the library takes: head_dim a multiple of 16 up to
    128, 1..8 query heads per KV head, INT8, converter INT4 or runtime INT4
    (whose output widths are then multiples of 32)."""
    r = np.random.RandomState(seed)
    prec = ["int8", "int4", "int4kn"][r.randint(3)]
    while True:
        hd = 16 * r.randint(1, 9)
        rep = [1, 2, 4, 8][r.randint(4)]
        nkv = [1, 2, 4][r.randint(3)]
        H = hd * rep * nkv
        if rep * hd > 1024 or H > 2048:
            continue
        if prec != "int8" and H % 32:
            continue
        if prec == "int4kn" and (nkv * hd) % 32:
            continue
        break
    mult = 4 if prec == "int8" else 32
    inter = mult * r.randint(max(1, H // mult), 2 * H // mult + 2)
    vocab = 32 * r.randint(4, 64) if prec == "int4kn" else r.randint(100, 2000)
    steps = int(r.randint(3, 140))
    layers = int(r.randint(1, 3))
    return prec, dict(num_layers=layers, hidden=H, num_heads=rep * nkv, num_kv_heads=nkv, intermediate=int(inter),
                      vocab=int(vocab), max_seq=steps + int(r.randint(0, 9))), steps


# TBH_DECODE_FUZZ_SEEDS=first:count runs another range of seeds
_range = os.environ.get("TBH_DECODE_FUZZ_SEEDS")
DECODE_SEEDS = (list(range(int(_range.split(":")[0]), int(_range.split(":")[0]) + int(_range.split(":")[1])))
                if _range else list(range(0xDE0, 0xDE0 + 24)))


@pytest.mark.parametrize("seed", DECODE_SEEDS)
def test_decode_random_configs(backend, seed):
    # seeded random model shapes through the whole step; logits at every step
    # within the gate of the float64 restatement
    prec, kw, steps = _decode_case(seed)
    cfg = T.DecoderConfig(**kw)
    dec, ref = _model(backend, cfg, prec, seed=seed)
    rng = np.random.default_rng(seed)
    for i, tok in enumerate(rng.integers(0, cfg.vocab, size=steps)):
        y = dec.step(int(tok))
        r = ref.step(int(tok))
        assert _gated(y, r) <= GATE, (prec, kw, i, _gated(y, r))
    dec.close()
