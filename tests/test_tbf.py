"""TBF v1 reader (tbh_tbf_*): files written by the reference converter's own
writer (tests/golden/make_tbf_fixture.py), files laid out byte for byte as
ModelWeights.save writes them (ModelWeights.swift:376-488), and malformed
files.  No GPU: the reader is host code."""
import json
import os
import struct

import numpy as np
import pytest

import oracle as O
import tinybrain_amd as T
from tinybrain_amd import _abi

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SRC = os.path.join(GOLDEN, "converter_tiny_weights.npz")
PROJ = [("attn_q", "q_proj"), ("attn_k", "k_proj"), ("attn_v", "v_proj"), ("attn_o", "o_proj"),
        ("ffn_gate", "gate_proj"), ("ffn_up", "up_proj"), ("ffn_down", "down_proj")]
DIMS = {"numLayers": 1, "hiddenDim": 32, "numHeads": 2, "numKVHeads": 1, "vocabSize": 40,
        "maxSeqLen": 64, "intermediateDim": 64, "architecture": "llama", "partialRotaryFactor": 1.0}


def _common(f, src):
    assert f.config == DIMS
    np.testing.assert_array_equal(f.floats("embeddings"), src["embeddings"])
    np.testing.assert_array_equal(f.floats("final_norm"), src["final_norm"])
    np.testing.assert_array_equal(f.floats("layer_0_ln_input"), src["layer0_input_layernorm"])
    np.testing.assert_array_equal(f.floats("layer_0_ln_post"), src["layer0_post_attention_layernorm"])
    assert not f.is_quantized("embeddings") and f.is_quantized("output")


def _projections(src):
    for tname, sname in PROJ:
        yield "layer_0_" + tname, src["layer0_" + sname]
    yield "output", src["lm_head"]


def test_converter_int8_file():
    src = np.load(SRC)
    with T.TBFFile(os.path.join(GOLDEN, "converter_tiny_int8.tbf")) as f:
        _common(f, src)
        for name, w_nk in _projections(src):
            q = f.quantized(name)
            q_nk, s = O.convert_int8_per_channel(w_nk)          # convert_model.py:370-395
            assert q.shape == (w_nk.shape[1], w_nk.shape[0])    # stored [in, out]
            assert q.precision == T.QuantizationPrecision.int8
            assert q.mode == T.QuantizationMode.perChannel and q.layout == T.Layout.KN_FLAT
            np.testing.assert_array_equal(q.data.reshape(q.shape), q_nk.T)
            np.testing.assert_array_equal(q.scales, s)
            assert q.zeroPoints is not None and not q.zeroPoints.any()


def test_converter_int4_file():
    src = np.load(SRC)
    with T.TBFFile(os.path.join(GOLDEN, "converter_tiny_int4.tbf")) as f:
        _common(f, src)
        for name, w_nk in _projections(src):
            q = f.quantized(name)
            ref = O.quantize_int4(w_nk, 32, O.ROUND_NUMPY)      # convert_model.py:398-459
            assert q.shape == (w_nk.shape[1], w_nk.shape[0])
            assert q.precision == T.QuantizationPrecision.int4 and q.mode == T.QuantizationMode.int4
            assert q.layout == T.Layout.NK_FLAT and q.groupSize == 32   # groups along K
            np.testing.assert_array_equal(q.data, ref.data)
            np.testing.assert_array_equal(q.scales, ref.scales)


def _swift_save(path, cfg, float_tensors, quant_tensors):
    """The byte layout of ModelWeights.save (ModelWeights.swift:376-488):
    header, metadata (mode byte always 2), index with absolute offsets, and
    4 KiB-aligned blobs, in write order (fp32 and quantized interleaved as
    given)."""
    pad = lambda b: b + b"\0" * ((-len(b)) % 4096)
    js = json.dumps(cfg).encode()
    out = pad(b"TBFM" + struct.pack("<II", 1, len(js)) + js)
    meta = struct.pack("<I", len(quant_tensors))
    for name, q in quant_tensors.items():
        nb = name.encode()
        meta += struct.pack("<I", len(nb)) + nb
        meta += struct.pack("<BBI", 2 if q.precision == T.QuantizationPrecision.int4 else 1, 2, q.groupSize)
        meta += struct.pack("<I", q.scales.size) + q.scales.astype("<f4").tobytes()
        zp = q.zeroPoints if q.zeroPoints is not None else np.zeros(0, np.int8)
        meta += struct.pack("<I", zp.size) + zp.astype(np.int8).tobytes()
    out += pad(meta)
    entries = [(n, a.astype("<f4").tobytes(), a.shape) for n, a in float_tensors.items()]
    entries += [(n, q.data.astype(np.int8).tobytes(), q.shape) for n, q in quant_tensors.items()]
    index = struct.pack("<I", len(entries))
    index_len = len(index) + sum(4 + len(n.encode()) + 4 + 4 * len(s) + 16 for n, _, s in entries)
    data_start = len(out) + index_len + ((-index_len) % 4096)
    blobs, off = b"", data_start
    for n, blob, shape in entries:
        nb = n.encode()
        index += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
        index += b"".join(struct.pack("<i", d) for d in shape)
        index += struct.pack("<QQ", off, len(blob))
        blobs += pad(blob)
        off = data_start + len(blobs)
    out += pad(index) + blobs
    with open(path, "wb") as fh:
        fh.write(out)


def test_swift_written_file_round_trip(tmp_path):
    rng = np.random.default_rng(3)
    w8 = rng.normal(0, 0.02, size=(48, 40)).astype(np.float32)
    q8 = T.quantize(w8, T.QuantizationMode.perChannel)
    w4 = rng.normal(0, 0.02, size=(64, 24)).astype(np.float32)
    q4 = T.quantize(w4, T.QuantizationMode.int4)                 # runtime layout, groups along N
    emb = rng.normal(size=(10, 48)).astype(np.float32)
    cfg = {"numLayers": 1, "hiddenDim": 48, "numHeads": 3, "vocabSize": 10, "maxSeqLen": 16}
    path = str(tmp_path / "swift.tbf")
    _swift_save(path, cfg, {"embeddings": emb}, {"a": q8, "b": q4})
    with T.TBFFile(path) as f:
        # decodeIfPresent defaults (ModelRunner.swift:109-120)
        assert f.config["numKVHeads"] == 3 and f.config["intermediateDim"] == 4 * 48
        assert f.config["architecture"] == "llama" and f.config["partialRotaryFactor"] == 1.0
        np.testing.assert_array_equal(f.floats("embeddings"), emb)
        a, b = f.quantized("a"), f.quantized("b")
        assert a.mode == T.QuantizationMode.perChannel and a.shape == (48, 40)
        np.testing.assert_array_equal(a.data, q8.data)
        np.testing.assert_array_equal(a.scales, q8.scales)
        assert b.layout == T.Layout.KN_FLAT and b.groupSize == q4.groupSize
        np.testing.assert_array_equal(b.data, q4.data)
        np.testing.assert_array_equal(b.scales, q4.scales)


@pytest.mark.parametrize("cut", [3, 11, 12 + 50, 4096 + 2, 4096 * 2 + 30, 4096 * 3 + 100])
def test_truncated_files_are_rejected(tmp_path, cut):
    raw = open(os.path.join(GOLDEN, "converter_tiny_int8.tbf"), "rb").read()
    p = tmp_path / "cut.tbf"
    p.write_bytes(raw[:cut])
    with pytest.raises(T.HIPBackendError) as e:
        T.TBFFile(str(p))
    assert e.value.status == _abi.E_INVALID


def test_corrupt_headers_are_rejected(tmp_path):
    raw = bytearray(open(os.path.join(GOLDEN, "converter_tiny_int8.tbf"), "rb").read())
    bad = tmp_path / "bad.tbf"
    for patch, status in [((0, b"XXXX"), _abi.E_INVALID),                  # magic
                          ((4, struct.pack("<I", 2)), _abi.E_UNSUPPORTED),  # version
                          ((8, struct.pack("<I", 10 ** 8)), _abi.E_INVALID),  # config length
                          ((4096, struct.pack("<I", 10 ** 9)), _abi.E_INVALID)]:  # metadata count
        b = bytearray(raw)
        b[patch[0]:patch[0] + len(patch[1])] = patch[1]
        bad.write_bytes(bytes(b))
        with pytest.raises(T.HIPBackendError) as e:
            T.TBFFile(str(bad))
        assert e.value.status == status
