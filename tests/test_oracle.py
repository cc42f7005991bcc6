"""Pins for the CPU oracle (oracle/tbh_oracle.c) -- CPU only.

Every oracle function is checked against something other than a retyping of
its own formula:
  * the reference's known answers and tolerance tests
    (INT4QuantizationTests.swift, QuantizationTests.swift, TensorTests.swift),
  * golden vectors written by the reference converter itself
    (tests/golden/converter_vectors.npz, from Scripts/convert_model.py),
  * closed forms / exhaustive enumeration / library reductions (numpy).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "converter_vectors.npz")


# --------------------------------------------------------------------------
# packInt4 / unpackInt4 (QuantizedTensor.swift:314-331)
# --------------------------------------------------------------------------
def test_pack_unpack_reference_table():
    # INT4QuantizationTests.swift:37-50
    for v1, v2 in [(0, 0), (7, -7), (-7, 7), (3, -3), (1, 2), (-1, -2), (5, -3)]:
        assert O.unpack_int4(O.pack_int4(v1, v2)) == (v1, v2)


def test_pack_clamps_reference():
    # INT4QuantizationTests.swift:53-58
    assert O.unpack_int4(O.pack_int4(10, -10)) == (7, -7)


def test_pack_known_byte():
    # QuantizedTensor.swift:305-312 / DequantINT4.metal:10-13: 5, -3 -> 0b0101_1101 = 93
    assert O.pack_int4(5, -3) == 93


def test_unpack_exhaustive_against_arithmetic_shift():
    # All 256 bytes: sign extension via int8 arithmetic shifts (a different
    # route than the reference's raw > 7 ? raw - 16 : raw).
    for b in range(256):
        sb = np.int8(np.uint8(b).view(np.int8))
        hi = int(np.int8(sb) >> np.int8(4))
        lo = int(np.int8(np.uint8((b << 4) & 0xFF).view(np.int8)) >> np.int8(4))
        assert O.unpack_int4(int(sb)) == (hi, lo), b
    # nibble 0x8 decodes to -8 although the quantizers never emit it
    assert O.unpack_int4(np.int8(np.uint8(0x88).view(np.int8)).item()) == (-8, -8)


# --------------------------------------------------------------------------
# Converter quantizers vs golden vectors written by the converter itself
# --------------------------------------------------------------------------
@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


CASES = ["rand", "ties4", "ties8", "zeros", "ragged"]


@pytest.mark.parametrize("name", CASES)
def test_converter_int8_matches_golden(golden, name):
    w = golden[f"{name}__w"]
    q, s = O.convert_int8_per_channel(w)
    np.testing.assert_array_equal(q, golden[f"{name}__int8_q"])
    np.testing.assert_array_equal(s.view(np.uint32), golden[f"{name}__int8_s"].view(np.uint32))


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_converter_int4_matches_golden(golden, name, gs):
    w = golden[f"{name}__w"]
    qt = O.quantize_int4(w, gs, O.ROUND_NUMPY)
    np.testing.assert_array_equal(qt.data, golden[f"{name}__int4_g{gs}_p"])
    np.testing.assert_array_equal(qt.scales.view(np.uint32),
                                  golden[f"{name}__int4_g{gs}_s"].view(np.uint32))
    np.testing.assert_array_equal(qt.zero_points, golden[f"{name}__int4_g{gs}_z"])


def test_golden_ties_round_half_even(golden):
    # the golden vectors themselves show np.round's half-to-even ties:
    # 2.5 -> 2, -2.5 -> -2, 3.5 -> 4, 0.5 -> 0, 1.5 -> 2 (INT4, scale 1.0)
    p = golden["ties4__int4_g32_p"]
    vals = [O.unpack_int4(int(b)) for b in p[:4]]
    flat = [v for pair in vals for v in pair]
    assert flat == [7, 2, -2, 4, -4, 0, 0, 2]


# --------------------------------------------------------------------------
# Swift quantizers (QuantizedTensor.swift:379-606)
# --------------------------------------------------------------------------
def test_swift_rounding_half_away_from_zero():
    t = np.array([[7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5]], np.float32)
    qt = O.quantize_int4(t, 32, O.ROUND_SWIFT)
    assert qt.scales[0] == np.float32(1.0)
    flat = [v for b in qt.data for v in O.unpack_int4(int(b))]
    assert flat == [7, 3, -3, 4, -4, 1, -1, 2]
    t8 = np.array([[127.0], [2.5], [-2.5], [126.5], [-126.5], [0.5]], np.float32)  # one column
    q8 = O.quantize_per_channel(t8)
    assert q8.scales[0] == np.float32(1.0)
    assert list(q8.data) == [127, 3, -3, 127, -127, 1]


def test_per_channel_scales_reference():
    # QuantizationTests.swift:78-97: [3,4] -> 4 scales, one per column
    w = np.array([[1, 2, 3, 4], [100, 200, 300, 400], [0.01, 0.02, 0.03, 0.04]], np.float32)
    qt = O.quantize_per_channel(w)
    assert qt.scales.size == 4
    assert qt.scales[0] != qt.scales[1] and qt.scales[2] != qt.scales[3]
    # closed form: column abs-max / 127, exactly as fp32 division
    np.testing.assert_array_equal(qt.scales, np.abs(w).max(0) / np.float32(127))


def test_quantize_all_zeros_reference():
    # QuantizationTests.swift:155-169, INT4QuantizationTests.swift:258-267
    z = np.zeros((10, 10), np.float32)
    for qt in (O.quantize_per_channel(z), O.quantize_int4(z, 128)):
        assert np.all(qt.scales == 1.0)
        assert np.all(O.dequantize(qt) == 0.0)


def test_quantize_outliers_reference():
    # QuantizationTests.swift:196-215
    d = np.ones((100, 2), np.float32)
    d[99, 1] = 1000.0
    deq = O.dequantize(O.quantize_per_channel(d))
    assert abs(deq[0, 0] - 1.0) <= 0.2


def _rel(a, b):
    # relativeError, QuantizationTests.swift:236-252
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(a), 1e-45)


def test_per_channel_accuracy_reference():
    # QuantizationTests.swift:99-112
    mixed = np.concatenate([np.ones(100), np.full(100, 100.0)]).astype(np.float32).reshape(2, 100)
    assert _rel(mixed, O.dequantize(O.quantize_per_channel(mixed))) < 0.01


def test_int4_roundtrip_and_counts_reference():
    # INT4QuantizationTests.swift:62-117
    w = O.fill_normal(7, 128 * 256).reshape(128, 256)
    qt = O.quantize_int4(w, 128)
    assert qt.data.size == (128 * 256 + 1) // 2
    assert _rel(w, O.dequantize(qt)) < 0.15
    w2 = O.fill_normal(8, 64 * 128).reshape(64, 128)
    assert O.quantize_int4(w2, 32).scales.size == (64 * 128 + 31) // 32
    assert O.quantize_int4(w2, 128).scales.size == (64 * 128 + 127) // 128


def test_int4_odd_count_and_constant_reference():
    # INT4QuantizationTests.swift:281-300 and :330-338
    t = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    qt = O.quantize_int4(t, 128)
    assert qt.data.size == 5
    assert qt.data[4] & 0x0F == 0            # trailing low nibble unused
    assert _rel(t, O.dequantize(qt)) < 0.15
    c = np.full((64, 64), 5.0, np.float32)
    assert _rel(c, O.dequantize(O.quantize_int4(c, 128))) < 0.001


def test_quantizer_invariants():
    w = O.fill_normal(11, 33 * 47, std=0.02).reshape(33, 47)
    qt = O.quantize_per_channel(w)
    q = qt.data.reshape(w.shape)
    assert np.abs(q).max() <= 127
    # each column's abs-max element maps to +-127
    am = np.abs(w).argmax(0)
    assert np.all(np.abs(q[am, np.arange(47)]) == 127)
    q4 = O.quantize_int4(w, 32)
    vals = np.array([v for b in q4.data for v in O.unpack_int4(int(b))])[: w.size]
    assert np.abs(vals).max() <= 7
    flat = w.reshape(-1)
    for g in range(q4.scales.size):
        seg = slice(32 * g, min(32 * g + 32, flat.size))
        i = np.abs(flat[seg]).argmax()
        assert abs(vals[seg][i]) == 7


def test_asymmetric_traps_on_all_positive():
    # Int8(round(-min/scale - 128)) is out of range for all-positive data
    assert O.quantize_asymmetric(np.linspace(1, 2, 16, dtype=np.float32)) is None
    qt = O.quantize_asymmetric(np.linspace(-1, 2, 16, dtype=np.float32))
    assert qt is not None
    assert _rel(np.linspace(-1, 2, 16), O.dequantize(qt)) < 0.01


def test_symmetric_is_per_channel_of_one_column():
    # quantizeSymmetric (QuantizedTensor.swift:427-450) is quantizePerChannel
    # (:379-424) of the same values laid out as one column: one abs-max, one
    # scale, the same rounding and clamp.  Per-channel is pinned by its own
    # closed forms above, so this reduction pins the symmetric quantizer.
    for seed, shape in ((41, (37, 53)), (42, (1, 1000)), (43, (256, 3))):
        w = O.fill_normal(seed, int(np.prod(shape)), std=0.3).reshape(shape)
        sym = O.quantize_symmetric(w)
        col = O.quantize_per_channel(w.reshape(-1, 1))
        assert sym.scales.size == 1 and sym.zero_points is None
        np.testing.assert_array_equal(sym.scales.view(np.uint32), col.scales.view(np.uint32))
        np.testing.assert_array_equal(sym.data, col.data)
        # the abs-max element maps to +-127, every value within +-127
        i = np.abs(w.reshape(-1)).argmax()
        assert abs(int(sym.data[i])) == 127 and np.abs(sym.data.astype(int)).max() <= 127


def test_symmetric_known_answers():
    # abs-max 127 gives scale exactly 1.0, so q = round(w) with Swift's
    # half-away-from-zero rounding: 0.5 -> 1, -0.5 -> -1, 1.5 -> 2, -2.5 -> -3
    # (numpy's half-to-even would give 0, -0, 2, -2)
    w = np.array([127.0, 0.5, -0.5, 1.5, -2.5, -127.0, 3.49], np.float32)
    qt = O.quantize_symmetric(w)
    assert qt.scales[0] == np.float32(1.0)
    np.testing.assert_array_equal(qt.data, np.array([127, 1, -1, 2, -3, -127, 3], np.int8))
    assert np.array_equal(O.quantize_symmetric(w, O.ROUND_NUMPY).data,
                          np.array([127, 0, 0, 2, -2, -127, 3], np.int8))
    # all zero: scale 1.0 (absMax not above leastNonzeroMagnitude), q = 0
    z = O.quantize_symmetric(np.zeros(9, np.float32))
    assert z.scales[0] == np.float32(1.0) and not z.data.any()
    # scale = absMax / 127 in fp32: absMax 254 gives exactly 2.0
    two = O.quantize_symmetric(np.array([-254.0, 3.0, 5.0], np.float32))
    assert two.scales[0] == np.float32(2.0)
    np.testing.assert_array_equal(two.data, np.array([-127, 2, 3], np.int8))


def test_asymmetric_known_answers():
    # quantizeAsymmetric (QuantizedTensor.swift:452-476): [min, max] -> [-128, 127]
    # min -1, max 254: range 255, scale exactly 1.0, zero point
    # round(1 - 128) = -127; q = round(w / s) + zp (half away from zero)
    w = np.array([-1.0, 254.0, 0.0, 2.5, -0.5, 100.0], np.float32)
    qt = O.quantize_asymmetric(w)
    assert qt.scales[0] == np.float32(1.0)
    assert qt.zero_points.tolist() == [-127]
    np.testing.assert_array_equal(qt.data, np.array([-128, 127, -127, -124, -128, -27], np.int8))
    # min -64, max 63.5: range 127.5, scale exactly 0.5, zero point 0
    w2 = np.array([-64.0, 63.5, 0.25, -0.25, 10.0], np.float32)
    q2 = O.quantize_asymmetric(w2)
    assert q2.scales[0] == np.float32(0.5) and q2.zero_points.tolist() == [0]
    np.testing.assert_array_equal(q2.data, np.array([-128, 127, 1, -1, 20], np.int8))
    # the endpoints come back exactly: (q - zp) * s
    for qq, ww in ((qt, w), (q2, w2)):
        d = O.dequantize(qq)
        assert d[0] == ww[0] and d[1] == ww[1]
    # constant data: range 0 -> scale 1.0; zero point round(-c - 128)
    c = O.quantize_asymmetric(np.full(4, -3.0, np.float32))
    assert c.scales[0] == np.float32(1.0) and c.zero_points.tolist() == [-125]
    np.testing.assert_array_equal(c.data, np.full(4, -128, np.int8))


def test_dequant_per_tensor_closed_form():
    # dequantize() for .symmetric / .asymmetric (QuantizedTensor.swift:273-281):
    # one scale and one zero point for every element, (Float(q) - Float(zp)) * s
    # rounded once.  (q - zp) * s in float64 is exact (9-bit integer times a
    # 24-bit significand), so rounding it to fp32 gives the expected bits.
    rng = np.random.default_rng(12)
    q = rng.integers(-128, 128, size=(19, 29)).astype(np.int8)
    for mode, zp, s in ((O.MODE_SYMMETRIC, None, np.float32(0.0123)),
                        (O.MODE_ASYMMETRIC, np.array([-37], np.int8), np.float32(3.7e-3)),
                        (O.MODE_ASYMMETRIC, np.array([127], np.int8), np.float32(1.5))):
        qt = O.QTensor((19, 29), q.reshape(-1), np.array([s], np.float32), zp, mode, O.PREC_INT8)
        z = 0.0 if zp is None else float(zp[0])
        want = ((q.astype(np.float64) - z) * np.float64(s)).astype(np.float32)
        np.testing.assert_array_equal(O.dequantize(qt).view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------
# dequantize() (QuantizedTensor.swift:182-286)
# --------------------------------------------------------------------------
def test_dequant_int4_hand_bytes():
    # byte 93 = (5, -3); byte 0x88 = (-8, -8); scale 2 then 0.5 (gs = 2)
    data = np.array([93, np.uint8(0x88).view(np.int8)], np.int8)
    qt = O.QTensor((2, 2), data, np.array([2.0, 0.5], np.float32), None, O.MODE_INT4, O.PREC_INT4, 2)
    np.testing.assert_array_equal(O.dequantize(qt), np.array([[10.0, -6.0], [-4.0, -4.0]], np.float32))
    # with zero points: (q - zp) * s
    qt.zero_points = np.array([1, -2], np.int8)
    np.testing.assert_array_equal(O.dequantize(qt), np.array([[8.0, -8.0], [-3.0, -3.0]], np.float32))


def test_dequant_int4_group_zero_means_single_group():
    data = np.array([93, 93, 93], np.int8)
    qt = O.QTensor((5,), data, np.array([0.25], np.float32), None, O.MODE_INT4, O.PREC_INT4, 0)
    np.testing.assert_array_equal(O.dequantize(qt), np.array([1.25, -0.75, 1.25, -0.75, 1.25], np.float32))


def test_dequant_one_rounding_no_fma():
    # value = fp32((q - zp)) * s rounded once: compare with the float64 product
    # rounded to fp32 (exact for an 8-bit q times a 24-bit s).
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, size=(17, 23)).astype(np.int8)
    s = rng.uniform(1e-4, 2.0, size=23).astype(np.float32)
    qt = O.QTensor((17, 23), q.reshape(-1), s, None, O.MODE_PER_CHANNEL, O.PREC_INT8)
    want = (q.astype(np.float64) * s.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(O.dequantize(qt).view(np.uint32), want.view(np.uint32))


def test_dequant_int4_layouts_agree():
    # The converter layout (flat over [N, K]) decodes to the transpose of the
    # runtime layout (flat over [K, N]) for the same values.
    w = O.fill_normal(21, 8 * 64, std=0.02).reshape(8, 64)        # [N, K]
    nk = O.quantize_int4(w, 32, O.ROUND_NUMPY)                     # groups along K
    deq_nk = O.dequantize(O.QTensor((8, 64), nk.data, nk.scales, nk.zero_points,
                                    O.MODE_INT4, O.PREC_INT4, 32))
    # rebuild the same per-element values as a runtime-layout [K, N] tensor
    vals = np.array([v for b in nk.data for v in O.unpack_int4(int(b))]).reshape(8, 64)
    kn_vals = vals.T.reshape(-1)
    packed = np.array([O.pack_int4(int(kn_vals[2 * i]), int(kn_vals[2 * i + 1]))
                       for i in range(kn_vals.size // 2)], np.int8)
    # per-element scales differ in grouping; use gs = 1 to carry them exactly
    scales_kn = np.repeat(nk.scales.reshape(8, 2), 32, axis=1).T.reshape(-1)
    kn = O.QTensor((64, 8), packed, scales_kn.astype(np.float32), None, O.MODE_INT4, O.PREC_INT4, 1)
    np.testing.assert_array_equal(O.dequantize(kn), deq_nk.T)


def test_int4_per_channel_uses_dim0_and_traps():
    # QuantizedTensor.swift:218-238 indexes scales by row although the
    # quantizer writes one per column: it traps when rows > cols.
    w = O.fill_normal(5, 6 * 4).reshape(6, 4)
    qt = O.quantize_int4_per_channel(w)
    with pytest.raises(ValueError):
        O.dequantize(qt)
    w2 = O.fill_normal(5, 2 * 4).reshape(2, 4)
    qt2 = O.quantize_int4_per_channel(w2)
    out = O.dequantize(qt2)
    vals = np.array([v for b in qt2.data for v in O.unpack_int4(int(b))]).reshape(2, 4)
    np.testing.assert_array_equal(out, (vals * qt2.scales[:2, None]).astype(np.float32))


# --------------------------------------------------------------------------
# quantizeINT4PerChannel (QuantizedTensor.swift:563-606): one scale per
# column (dim 1, out_features), q = clamp(round(w / s[col]), -7, 7) with
# Swift's half-away-from-zero round, packed even flat index -> high nibble.
# --------------------------------------------------------------------------
def _nibbles_by_shift(packed: np.ndarray, n: int) -> np.ndarray:
    """Signed nibbles of a packed array by int8 arithmetic shifts (high
    nibble = byte >> 4, low = (byte << 4) >> 4): a decode independent of
    the oracle's raw > 7 ? raw - 16 : raw rule."""
    b = packed.view(np.int8).astype(np.int8)
    hi = (b >> np.int8(4)).astype(np.int64)
    lo = (np.left_shift(b.view(np.uint8), np.uint8(4)).view(np.int8) >> np.int8(4)).astype(np.int64)
    return np.stack([hi, lo], 1).reshape(-1)[:n]


def test_int4_per_channel_known_bytes():
    # Every column's abs-max is exactly 7, so every scale is exactly 1.0 and
    # q = round(w): [[7, -3], [2.5, -7]] -> flat [7, -3, 3, -7] (2.5 -> 3,
    # half away from zero) -> bytes 0x7D, 0x39 (even index in the high nibble)
    w = np.array([[7.0, -3.0], [2.5, -7.0]], np.float32)
    qt = O.quantize_int4_per_channel(w)
    assert qt.scales.tolist() == [1.0, 1.0]
    assert qt.zero_points is None and qt.mode == O.MODE_INT4_PER_CHANNEL
    assert qt.data.view(np.uint8).tolist() == [0x7D, 0x39]


def test_int4_per_channel_scale_is_column_absmax_over_7():
    # 5 x 3 (rows != cols, so a per-row scale would differ in count and
    # value): s[c] = max_r |w[r, c]| / 7 in fp32, one per column
    w = np.array([[0.1, -2.0, 0.0],
                  [0.3, 1.0, 0.0],
                  [-0.7, 0.5, 0.0],
                  [0.2, -1.5, 0.0],
                  [0.0, 0.25, 0.0]], np.float32)
    qt = O.quantize_int4_per_channel(w)
    assert qt.scales.size == 3
    assert qt.scales[0] == np.float32(0.7) / np.float32(7)
    assert qt.scales[1] == np.float32(2.0) / np.float32(7)
    assert qt.scales[2] == np.float32(1.0)          # all-zero column: scale 1.0
    q = _nibbles_by_shift(qt.data, w.size).reshape(5, 3)
    # the abs-max element of each non-zero column maps to +-7 with its sign
    assert q[2, 0] == -7 and q[0, 1] == -7
    assert not q[:, 2].any()                        # zero column stays zero
    assert qt.data.size == (15 + 1) // 2 and qt.data.view(np.uint8)[-1] & 0x0F == 0


def test_int4_per_channel_ties_round_half_away_from_zero():
    # One column with abs-max 7 (scale exactly 1.0): ties go away from zero,
    # where numpy's half-to-even would give 2, -2, 0, 0, 4 for the first five
    col = np.array([2.5, -2.5, 0.5, -0.5, 3.5, 7.0, -6.5, 8.0 / 8.0], np.float32).reshape(-1, 1)
    qt = O.quantize_int4_per_channel(col)
    assert qt.scales[0] == np.float32(1.0)
    assert _nibbles_by_shift(qt.data, 8).tolist() == [3, -3, 1, -1, 4, 7, -7, 1]
    ne = O.quantize_int4_per_channel(col, O.ROUND_NUMPY)
    assert _nibbles_by_shift(ne.data, 8).tolist() == [2, -2, 0, 0, 4, 7, -6, 1]


def test_int4_per_channel_random_invariants():
    # 37 x 29 N(0, 0.3): the error of every element is at most half its
    # column's scale (no element reaches the clamp, since |w| <= absMax),
    # every column's abs-max element gives +-7, and the packed order is the
    # flat [row, col] order (element i in byte i / 2, high nibble when even)
    w = O.fill_normal(91, 37 * 29, std=0.3).reshape(37, 29)
    qt = O.quantize_int4_per_channel(w)
    s = qt.scales.astype(np.float64)
    np.testing.assert_array_equal(qt.scales, (np.abs(w).max(0) / np.float32(7)).astype(np.float32))
    q = _nibbles_by_shift(qt.data, w.size).reshape(37, 29)
    assert np.abs(q).max() <= 7
    err = np.abs(q * s[None, :] - w.astype(np.float64))
    assert np.all(err <= 0.5 * s[None, :] * (1 + 1e-6))
    am = np.abs(w).argmax(0)
    np.testing.assert_array_equal(q[am, np.arange(29)], 7 * np.sign(w[am, np.arange(29)]).astype(int))
    # the same values quantized by the per-group quantizer with one group per
    # column (columns laid out contiguously) give the same nibbles
    for c in range(29):
        g = O.quantize_int4(np.ascontiguousarray(w[:, c]), 37)
        assert g.scales[0] == qt.scales[c]
        np.testing.assert_array_equal(_nibbles_by_shift(g.data, 37), q[:, c])


def test_validate_preconditions():
    good = O.quantize_per_channel(np.ones((4, 6), np.float32))
    assert O.validate(good) == O.OK
    bad = O.QTensor((4, 6), good.data, good.scales[:5], None, O.MODE_PER_CHANNEL, O.PREC_INT8)
    assert O.validate(bad) == O.E_INVALID
    q4 = O.quantize_int4(np.ones((5, 7), np.float32), 32)
    assert O.validate(q4) == O.OK
    short = O.QTensor((5, 7), q4.data[:-1], q4.scales, None, O.MODE_INT4, O.PREC_INT4, 32)
    assert O.validate(short) == O.E_INVALID
    zp_bad = O.QTensor((5, 7), q4.data, q4.scales, np.zeros(3, np.int8), O.MODE_INT4, O.PREC_INT4, 32)
    assert O.validate(zp_bad) == O.E_INVALID


# --------------------------------------------------------------------------
# matmul (Tensor.swift:839-861; QuantizedTensor.swift:640-642)
# --------------------------------------------------------------------------
def test_matmul_known_answer_through_int8():
    # TensorTests.swift:248-275: [[1,2,3],[4,5,6]] x [[7,8],[9,10],[11,12]]
    # = [[58,64],[139,154]].  A zero column in A and a row of 127s in B make
    # every column scale exactly 1.0, so the INT8 path reproduces it exactly.
    a = np.array([[1, 2, 3, 0], [4, 5, 6, 0]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12], [127, 127]], np.float32)
    qt = O.quantize_per_channel(b)
    assert np.all(qt.scales == 1.0)
    y, _, _ = O.matmul_quantized_cpu(a, qt)
    np.testing.assert_array_equal(y, np.array([[58, 64], [139, 154]], np.float32))


def test_gemm_f64_matches_numpy():
    a = O.fill_normal(1, 3 * 300).reshape(3, 300)
    b = O.fill_normal(2, 300 * 4100).reshape(300, 4100)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(O.gemm_f64(a, b), ref, rtol=1e-12, atol=1e-12)


def test_sgemm_fp32_accuracy():
    a = O.fill_normal(3, 5 * 700).reshape(5, 700)
    b = O.fill_normal(4, 700 * 2100).reshape(700, 2100)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    c = O.sgemm(a, b, threads=3)
    # fp32 accumulation bound ~ K * eps * sum|a b|
    bound = 700 * 2 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(c - ref) <= bound)
    np.testing.assert_array_equal(c, O.sgemm(a, b, threads=1))     # order independent of threads


def test_quantized_matmul_reference_tolerances():
    # QuantizationTests.swift:117-135 (INT8 < 1% L2) and
    # INT4QuantizationTests.swift:189-207 (INT4 < 15% L2)
    x = O.fill_normal(31, 128 * 256).reshape(128, 256)
    w = O.fill_normal(32, 256 * 512).reshape(256, 512)
    fp32 = O.sgemm(x, w)
    y8, _, _ = O.matmul_quantized_cpu(x, O.quantize_per_channel(w))
    assert _rel(fp32, y8) < 0.01
    x4 = O.fill_normal(33, 4 * 128).reshape(4, 128)
    w4 = O.fill_normal(34, 128 * 64).reshape(128, 64)
    y4, _, _ = O.matmul_quantized_cpu(x4, O.quantize_int4(w4, 128))
    assert _rel(O.sgemm(x4, w4), y4) < 0.15


def test_reference_cpu_path_is_dequant_then_sgemm():
    x = O.fill_normal(41, 3 * 96).reshape(3, 96)
    qt = O.quantize_int4(O.fill_normal(42, 96 * 40, std=0.02).reshape(96, 40), 32)
    y, td, tg = O.matmul_quantized_cpu(x, qt, threads=2)
    np.testing.assert_array_equal(y, O.sgemm(x, O.dequantize(qt)))
    assert td >= 0 and tg >= 0


def test_fill_normal_moments():
    v = O.fill_normal(123, 200001).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    np.testing.assert_array_equal(O.fill_normal(123, 10), O.fill_normal(123, 10))


def test_parity_errors_floor():
    y64 = np.array([[1.0, -2.0, 1e-9]])
    e = O.parity_errors(y64 + np.array([[1e-4, 0, 1e-7]]), y64)
    # the 1e-9 output is floored at 1e-3 * 2 = 2e-3
    assert e["gated"] == pytest.approx(max(1e-4, 1e-7 / 2e-3))


@pytest.mark.parametrize("M", [1, 3, 9])
def test_best_effort_fused_gemv_equals_reference_path(M):
    # The host upper bound reported beside the reference CPU path: fused
    # dequant-GEMV, same dequantized values and the same order over k, so the
    # same y bit for bit -- for INT8 per-channel and INT4 in the runtime flat
    # order, and for the converter's INT4 storage (element (k, n) at n*K + k)
    # against a float32 loop over k on its transposed dequantization.
    K, N = 320, 4200          # N past one 2048-column block, ragged
    rng = np.random.default_rng(M)
    x = rng.normal(size=(M, K)).astype(np.float32)
    q8 = O.quantize_per_channel(O.fill_normal(3, K * N, std=0.02).reshape(K, N))
    q4 = O.quantize_int4(O.fill_normal(4, K * N, std=0.02).reshape(K, N), 32, O.ROUND_SWIFT)
    for q in (q8, q4):
        y_ref, _, _ = O.matmul_quantized_cpu(x, q, threads=4)
        y_fused, _ = O.matmul_quantized_fused(x, q, threads=4)
        np.testing.assert_array_equal(y_fused, y_ref)
    qn = O.quantize_int4(O.fill_normal(5, N * K, std=0.02).reshape(N, K), 32, O.ROUND_SWIFT)
    qc = O.QTensor((K, N), qn.data, qn.scales, qn.zero_points, qn.mode, qn.precision, qn.group_size)
    W = np.ascontiguousarray(O.dequantize(qn).reshape(N, K).T)
    y_loop = np.zeros((M, N), np.float32)
    for k in range(K):
        y_loop += x[:, k:k + 1] * W[k]
    y_fused, _ = O.matmul_quantized_fused(x, qc, threads=4, nk=True)
    np.testing.assert_array_equal(y_fused, y_loop)
    # and against float64: the restated product, not just a self-consistent one
    y64 = x.astype(np.float64) @ W.astype(np.float64)
    assert O.parity_errors(y_fused, y64)["gated"] <= 1e-3   # the contract's gate
