"""CPU check of the division-free code tests the HIP quantizer uses (kv800_quant.hip).

The reference quantizer (kv800.py:56-76) computes code = clamp(round(fl(d / den)), 0, top) with d = fl(x - lo), an
IEEE float32 quotient and round-half-to-even. The kernels decide the same code without the division:

  * V (1-bit codes):  code >= 1  <=>  d > den / 2
  * K (2-bit codes):  code = [d > den / 2] + [fma(den, 2^-24, fma(-den, 1.5, d)) >= 0]
                             + [fma(-den, 2^-23, fma(-den, 2.5, d)) > 0]

because fl(q) > 1/2 <=> d > den / 2 for float d, fl(q) >= 3/2 <=> q >= 3/2 - 2^-24 and fl(q) > 5/2 <=>
q > 5/2 + 2^-23 (the midpoints round to the even neighbour), and near each threshold the fma residual is exact.
numpy's float32 division, subtraction and rint are the IEEE operations the reference's torch ops perform, so this test
evaluates both sides for every divisor the quantizer can produce (every fp8 e4m3fn scale byte, decoded and clamped to
>= 1e-8) against dividends walked ulp by ulp across each threshold, random dividends and the special values. fma is
formed in float64 and rounded once to float32 (exact for these operands; where d and den are 2^150 apart the double
rounding cannot move a sign).
"""
import numpy as np

F32 = np.float32


def _dens():
    vals = []
    for b in range(128):   # sign-free bytes: the scale is a max(., 1e-8) of a non-negative range
        e, m = (b >> 3) & 15, b & 7
        vals.append((1 + m / 8) * 2.0 ** (e - 7) if e else m * 2.0 ** -9)
    return np.unique(np.maximum(np.array(vals, dtype=F32), F32(1e-8)))


def _dividends(den, rng):
    out = [F32(0.0), F32(-0.0), F32(np.inf), F32(-np.inf), F32(np.nan), F32(1e-40), F32(3e38), F32(-3e38)]
    for t in (0.5, 1.5, 2.5):
        lo = hi = F32(np.float64(den) * t)
        out.append(lo)
        for _ in range(48):
            lo, hi = np.nextafter(lo, F32(-np.inf)), np.nextafter(hi, F32(np.inf))
            out += [lo, hi]
    out += list((rng.standard_normal(4000) * float(den) * 3).astype(F32))
    return np.array(out, dtype=F32)


def _fma(a, b, c):
    return (np.float64(a) * np.float64(b) + np.float64(c)).astype(F32)


def test_threshold_tests_match_division():
    rng = np.random.default_rng(7)
    checked = 0
    with np.errstate(all="ignore"):
        for den in _dens():
            den = F32(den)
            d = _dividends(den, rng)
            q = d / den
            r = np.rint(q)
            bit_ref = r >= 1
            code_ref = np.where(np.isnan(r), 0, np.clip(r, 0, 3)).astype(np.int64)
            t1 = d > den * F32(0.5)
            t2 = _fma(den, F32(2.0 ** -24), _fma(-den, F32(1.5), d)) >= 0
            t3 = _fma(-den, F32(2.0 ** -23), _fma(-den, F32(2.5), d)) > 0
            assert np.array_equal(bit_ref, t1), den
            assert np.array_equal(code_ref, t1.astype(np.int64) + t2 + t3), den
            checked += d.size
    assert checked > 400_000


def test_planted_threshold_mistakes_fail():
    """The checks above are sharp: >= for > at 1/2, or a K test without its margin, disagrees with the division."""
    rng = np.random.default_rng(8)
    with np.errstate(all="ignore"):
        den = F32(0.75)
        d = _dividends(den, rng)
        assert not np.array_equal(np.rint(d / den) >= 1, d >= den * F32(0.5))
        den = F32(1e-8)   # the clamped scale: 1.5 den and 2.5 den are not floats
        d = _dividends(den, rng)
        r = np.rint(d / den)
        assert not np.array_equal(r >= 2, _fma(-den, F32(1.5), d) >= 0)
        assert not np.array_equal(r >= 3, _fma(-den, F32(2.5), d) > 0)
