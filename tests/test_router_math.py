"""CPU check of the arithmetic identity the router kernel uses for the prefix
mean's fp32 division (model.py:172-173: h = cumsum(x) / (t+1), both fp32).

The kernel evaluates a / b for an fp32 numerator a and an integer b = t+1 as
fp32( fp64(a) * fp64(1/b) ), and falls back to the IEEE fp32 division when
that result is a nonzero subnormal.  For b <= 2^24 and a normal quotient the
product rounds correctly: a/b is then never an fp32 rounding midpoint and
stays at least 2^-50 (relative) away from every midpoint, while the fp64
product is within 2^-52 of a/b.  Subnormal quotients can be exact ties,
hence the fallback.  numpy's float32 division is IEEE round-to-nearest-even and is
the reference here.  Cases: every b up to 4096, random large b, numerators
over the whole exponent range (subnormals included), and numerators built to
put a/b as close to a midpoint as fp32 allows.
"""
import numpy as np
import pytest


def kernel_div(a, b):
    q = (a.astype(np.float64) * (1.0 / np.float64(b))).astype(np.float32)
    sub = (q != 0) & (np.abs(q) < np.finfo(np.float32).tiny)     # subnormal results: IEEE division
    return np.where(sub, a / np.float32(b), q)


def test_subnormal_ties_need_the_ieee_fallback():
    """Without the fallback, exact ties in the subnormal range round wrongly
    (a = 49 * (2k+1) * 2^-149, b = 98 gives a/b = (2k+1) * 2^-150)."""
    k = np.arange(1, 2000, dtype=np.uint32)
    a = (49 * (2 * k + 1)).astype(np.uint32).view(np.float32)
    plain = (a.astype(np.float64) * (1.0 / 98.0)).astype(np.float32)
    want = a / np.float32(98)
    assert not np.array_equal(bits(plain), bits(want))
    assert np.array_equal(bits(kernel_div(a, 98)), bits(want))


def bits(v):
    return np.ascontiguousarray(v).view(np.uint32)


def random_numerators(rng, n):
    mant = rng.uniform(1.0, 2.0, n)
    expo = rng.integers(-149, 127, n)
    a = (mant * np.exp2(expo.astype(np.float64))).astype(np.float32)
    a[: n // 16] = rng.integers(1, 1 << 23, n // 16).astype(np.uint32).view(np.float32)  # subnormals
    a[n // 16: n // 8] = rng.integers(-(1 << 20), 1 << 20, n // 8 - n // 16).astype(np.float32)  # small integers
    sign = rng.integers(0, 2, n) * 2 - 1
    return (a * sign).astype(np.float32)


def test_reciprocal_product_equals_ieee_division_all_small_b():
    rng = np.random.default_rng(0)
    a = random_numerators(rng, 20000)
    for b in range(1, 4097):
        want = a / np.float32(b)
        assert np.array_equal(bits(kernel_div(a, b)), bits(want)), f"b={b}"


def test_reciprocal_product_equals_ieee_division_large_b():
    rng = np.random.default_rng(1)
    a = random_numerators(rng, 50000)
    for b in list(rng.integers(4097, 1 << 24, 200)) + [(1 << 24) - 1, 1 << 24, 3 ** 15, 5 ** 10]:
        want = a / np.float32(b)
        assert np.array_equal(bits(kernel_div(a, b)), bits(want)), f"b={b}"


@pytest.mark.parametrize("b", [3, 5, 7, 11, 13, 1023, 2047, 2049, 4095, 65535, 65537, 1000003, (1 << 24) - 3])
def test_reciprocal_product_near_rounding_midpoints(b):
    """a = fp32 neighbours of m*b for fp32 midpoints m, the closest a/b gets to m."""
    rng = np.random.default_rng(b)
    k = rng.integers(1 << 23, 1 << 24, 20000).astype(np.float64)
    emax = 126 - 24 - int(np.ceil(np.log2(b)))                 # keep m * b finite in fp32
    e = rng.integers(-120, emax, 20000).astype(np.float64)
    m = (k + 0.5) * np.exp2(e)                      # halfway between two fp32 values
    a0 = (m * b).astype(np.float32)
    cands = [a0, np.nextafter(a0, np.float32(np.inf)), np.nextafter(a0, np.float32(-np.inf))]
    for a in cands:
        a = a[np.isfinite(a)]
        want = a / np.float32(b)
        assert np.array_equal(bits(kernel_div(a, b)), bits(want))
