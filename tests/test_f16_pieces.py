"""Error bounds of the two f16-piece decompositions the prefill GEMM uses
(tbh_prefill.hip), restated in numpy and checked over random and edge-case
values on the CPU.

- x pieces (gemm_bf16 with fp32 x, gemm_ngw with fp32 x): v scaled into
  |v| <= 2^15, hi = f16(v) and lo = f16(v - hi), both rounded to nearest:
  |v - (hi + lo)| <= max(2^-22 |v|, 2^-25).
- weight pieces (gemm_ngw): w scaled into |w| < 2^15, hi = w rounded toward
  zero, lo = lo_piece(w, w - hi) rounded to nearest, where lo_piece keeps the
  remainder at least 2^-24 in magnitude with w's sign unless w = 0:
  |w - (hi + lo)| <= max(2^-21 |w|, 2^-24), lo has w's sign, and lo = 0
  only for w = 0.  So an infinite x times the two pieces gives inf * w
  (+-inf, or NaN for w = 0) for every |w| >= 2^-24.  Below that hi would be
  0, which is why the kernel floors a scaled scale at 2^-28 for weights
  whose scales span that far (|16 q| >= 16 makes |w| >= 2^-24 for q != 0).
"""
import numpy as np
import pytest

TINY = np.float32(2.0 ** -24)


def _f16_rtz(v: np.ndarray) -> np.ndarray:
    """float32 -> float16 rounded toward zero (v_cvt_pkrtz_f16_f32)."""
    h = v.astype(np.float16)                      # round to nearest even
    over = np.abs(h.astype(np.float32)) > np.abs(v)
    h[over] = np.nextafter(h[over], np.float16(0))
    return h


def _x_pieces(v):
    hi = v.astype(np.float16)
    r = v - hi.astype(np.float32)                 # exact in fp32
    return hi, r.astype(np.float16)


def _w_pieces(w):
    hi = _f16_rtz(w)
    r = w - hi.astype(np.float32)                 # exact in fp32, w's sign or 0
    lo = np.where(w == 0, np.float32(0), np.copysign(np.maximum(np.abs(r), TINY), w)).astype(np.float32)
    return hi, lo.astype(np.float16)


def _values(seed, n=200_000):
    rng = np.random.default_rng(seed)
    mant = rng.uniform(1.0, 2.0, n)
    expo = rng.integers(-40, 15, n)               # up to the 2^15 bound, down into f16 subnormals
    v = (np.where(rng.random(n) < 0.5, -1.0, 1.0) * mant * np.exp2(expo)).astype(np.float32)
    # values exact in f16 (empty remainder), zeros and the bound itself
    v[:1000] = rng.integers(-2048, 2048, 1000).astype(np.float32) * np.float32(2.0 ** -3)
    v[1000:1010] = 0.0
    v[1010] = -0.0
    v[1011], v[1012] = 2.0 ** 15, -(2.0 ** 15) + 2.0 ** -8
    return v


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_x_pieces_bound(seed):
    v = _values(seed)
    hi, lo = _x_pieces(v)
    err = np.abs(v.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    bound = np.maximum(2.0 ** -22 * np.abs(v.astype(np.float64)), 2.0 ** -25)
    assert np.all(err <= bound)
    assert np.all(np.isfinite(hi)) and np.all(np.isfinite(lo))


@pytest.mark.parametrize("seed", [4, 5, 6])
def test_weight_pieces_bound_and_sign(seed):
    w = _values(seed)
    hi, lo = _w_pieces(w)
    w64, hi64, lo64 = w.astype(np.float64), hi.astype(np.float64), lo.astype(np.float64)
    err = np.abs(w64 - hi64 - lo64)
    assert np.all(err <= np.maximum(2.0 ** -21 * np.abs(w64), 2.0 ** -24))
    assert np.all(np.abs(hi64) <= np.abs(w64))           # toward zero
    nz = w != 0
    assert np.all(lo64[nz] != 0)                          # never an empty low piece for a weight
    assert np.all(np.sign(lo64[nz]) == np.sign(w64[nz]))
    assert np.all((hi64[nz] == 0) | (np.sign(hi64[nz]) == np.sign(w64[nz])))
    assert np.all(lo64[~nz] == 0) and np.all(hi64[~nz] == 0)


def test_infinite_x_meets_weight_pieces_like_the_product():
    # inf * hi + inf * lo against inf * w, for the weights of every kind above
    # down to 2^-24 (and zeros)
    w = _values(7, 20_000)
    w = w[(np.abs(w) >= TINY) | (w == 0)]
    hi, lo = _w_pieces(w)
    with np.errstate(invalid="ignore"):
        for xinf in (np.inf, -np.inf):
            got = xinf * hi.astype(np.float64) + xinf * lo.astype(np.float64)
            want = xinf * w.astype(np.float64)
            np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
            ok = ~np.isnan(want)
            np.testing.assert_array_equal(got[ok], want[ok])


def test_floored_scales_keep_the_high_piece():
    # |w| < 2^-24 rounds toward zero to hi = 0 (inf * 0 = NaN for an infinite
    # x); with the scale floored at 2^-28, every q != 0 gives |16 q s| >=
    # 2^-24, a nonzero high piece of w's sign, and q = 0 still gives 0
    w = np.array([2.0 ** -25, -(2.0 ** -30), 2.0 ** -40], np.float32)
    hi, lo = _w_pieces(w)
    assert np.all(hi.astype(np.float32) == 0)
    with np.errstate(invalid="ignore"):
        assert np.all(np.isnan(np.inf * hi.astype(np.float64) + np.inf * lo.astype(np.float64)))
    s = np.array([2.0 ** -50, -(2.0 ** -40), 2.0 ** -29, 0.0], np.float32)
    s_floor = np.where(s == 0, s, np.copysign(np.maximum(np.abs(s), np.float32(2.0 ** -28)), s)).astype(np.float32)
    for q16 in range(-128, 128, 16):
        w = (np.float32(q16) * s_floor).astype(np.float32)
        hi, lo = _w_pieces(w)
        nz = w != 0
        assert np.all(nz == ((q16 != 0) & (s != 0)))
        assert np.all(hi[nz] != 0) and np.all(np.sign(hi[nz].astype(np.float32)) == np.sign(w[nz]))
