"""Pins of the oracle's codebook tables and lookup.

The tables (reference src/codebook/tables.rs) are checked against an
independent restatement of the published generation algorithm (Lloyd-Max on
the Beta pdf, codebook/gen.rs:226-269: centroids initialised at the bin
centres of [-1, 1], midpoint boundaries, conditional means by composite
Simpson with 1024 steps, at most 200 iterations, relative-distortion stop
1e-12), written here in numpy, to 1e-6 as codebook_tests.rs:256-281 does.
The 2- and 3-bit tables are also the exact Lloyd-Max fixed point (closed-form
incomplete-beta moments, scipy) to 1e-6.
"""
import numpy as np
import pytest
from scipy.special import betainc, gammaln

from oracle import oracle as orc


def _pdf(x, d):
    a = (d - 3) / 2.0
    k = np.exp(gammaln(d / 2) - 0.5 * np.log(np.pi) - gammaln((d - 1) / 2))
    om = 1.0 - x * x
    return np.where(om > 0, k * np.power(np.maximum(om, 0.0), a), 0.0)


def _simpson(f, a, b, n=1024):
    x = a + np.arange(n + 1) * ((b - a) / n)
    w = np.ones(n + 1)
    w[1:-1:2] = 4.0
    w[2:-1:2] = 2.0
    return (w * f(x)).sum() * ((b - a) / n) / 3.0


def _published_generator(bits, d):
    k = 1 << bits
    c = np.array([-1.0 + 2.0 * (i + 0.5) / k for i in range(k)])
    prev = np.finfo(np.float64).max
    for _ in range(200):
        b = (c[:-1] + c[1:]) / 2
        e = np.concatenate([[-1.0], b, [1.0]])
        new = []
        for i in range(k):
            den = _simpson(lambda x: _pdf(x, d), e[i], e[i + 1])
            num = _simpson(lambda x: x * _pdf(x, d), e[i], e[i + 1])
            new.append((e[i] + e[i + 1]) / 2 if abs(den) < 1e-30 else num / den)
        c = np.array(new)
        dist = sum(_simpson(lambda x, ci=ci: (x - ci) ** 2 * _pdf(x, d), e[i], e[i + 1]) for i, ci in enumerate(c))
        if abs(prev - dist) < 1e-12 * max(abs(prev), 1e-30):
            break
        prev = dist
    return c, (c[:-1] + c[1:]) / 2


def _lloyd_fixed_point(bits, d, iters=20000):
    a = (d - 3) / 2
    kn = np.exp(gammaln(d / 2) - 0.5 * np.log(np.pi) - gammaln((d - 1) / 2))

    def cdf(x):
        return 0.5 + 0.5 * np.sign(x) * betainc(0.5, (d - 1) / 2, x * x)

    def moment(x):
        return -kn * (1 - x * x) ** (a + 1) / (2 * (a + 1))

    c = np.linspace(-0.5, 0.5, 1 << bits) * 3 / np.sqrt(d)
    for _ in range(iters):
        e = np.concatenate([[-1.0], (c[:-1] + c[1:]) / 2, [1.0]])
        cn = (moment(e[1:]) - moment(e[:-1])) / (cdf(e[1:]) - cdf(e[:-1]))
        if np.max(np.abs(cn - c)) < 1e-16:
            break
        c = cn
    return c


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [32, 64, 128, 256])
def test_tables_match_published_generator(bits, dim):
    c, b = _published_generator(bits, dim)
    tc, tb = orc.get_codebook(bits, dim)
    assert np.abs(c - tc).max() < 1e-6
    assert np.abs(b - tb).max() < 1e-6


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("dim", [32, 128])
def test_tables_are_lloyd_max_fixed_points(bits, dim):
    tc, _ = orc.get_codebook(bits, dim)
    assert np.abs(_lloyd_fixed_point(bits, dim) - tc).max() < 1e-6


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [32, 64, 128, 256])
def test_table_invariants(bits, dim):
    c, b = orc.get_codebook(bits, dim)
    assert len(c) == 1 << bits and len(b) == len(c) - 1
    assert np.all(np.diff(c) > 0) and np.all(np.diff(b) > 0)
    assert np.allclose(c, -c[::-1], atol=1e-12)
    assert b[len(b) // 2] == 0.0
    assert np.all((c[:-1] < b) & (b < c[1:]))
    assert np.allclose(b, (c[:-1] + c[1:]) / 2, atol=1e-12)


def test_unknown_dimension_is_an_error():
    with pytest.raises(ValueError):
        orc.get_codebook(3, 512)
    with pytest.raises(ValueError, match="code 2"):
        orc.get_codebook(5, 128)


def test_nearest_centroid_reference_cases():
    # codebook_tests.rs:224-250
    c, b = orc.get_codebook(3, 128)
    for i, ci in enumerate(c):
        assert orc.nearest_centroid(ci, b) == i
    c, b = orc.get_codebook(3, 64)
    for i, bi in enumerate(b):
        assert orc.nearest_centroid(bi - 1e-10, b) == i
        assert orc.nearest_centroid(bi + 1e-10, b) == i + 1
        assert orc.nearest_centroid(bi, b) == i  # strict '>': a tie goes to the lower bin
    c, b = orc.get_codebook(4, 256)
    assert orc.nearest_centroid(-1.0, b) == 0
    assert orc.nearest_centroid(1.0, b) == 15


def test_nearest_centroid_equals_searchsorted():
    rng = np.random.default_rng(0)
    _, b = orc.get_codebook(4, 128)
    v = rng.standard_normal(5000) * 0.2
    ref = np.searchsorted(b, v, side="left")
    got = np.array([orc.nearest_centroid(x, b) for x in v])
    assert np.array_equal(got, ref)


def test_pqo_codebooks():
    # precomputed/codebooks.rs:51-88
    c3, b3, o3 = orc.pqo_codebook(3)
    assert np.array_equal(c3, np.array([-2.1573, -1.3336, -0.7434, -0.2428, 0.2428, 0.7434, 1.3336, 2.1573],
                                       np.float32))
    assert np.array_equal(b3, np.array([-1.7455, -1.0385, -0.4931, 0.0, 0.4931, 1.0385, 1.7455], np.float32))
    assert o3 == np.float32(2.1573)
    c4, b4, o4 = orc.pqo_codebook(4)
    r = np.float32(2.1573)
    step = np.float32(np.float32(2) * r) / np.float32(15)
    assert np.array_equal(c4, np.array([np.float32(-r + np.float32(i) * step) for i in range(16)], np.float32))
    assert np.array_equal(b4, np.array([np.float32(-r + np.float32(np.float32(i) + np.float32(0.5)) * step)
                                        for i in range(15)], np.float32))
    assert o4 == c4.max()
    assert np.allclose(np.diff(c4), 2 * 2.1573 / 15, atol=1e-6)
    c2, b2, _ = orc.pqo_codebook(2)
    assert np.array_equal(c2, c3[[0, 2, 5, 7]])
