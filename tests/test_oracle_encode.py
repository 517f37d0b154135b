"""Pins of the device encoder's oracle (oracle/encode.py) against the mathematics: the coefficients against the
canonical-embedding sums evaluated directly in extended precision (numpy longdouble) at N = 2^10, real by the
conjugate placement, and decoded back to the slots; the split against ceil(log2) at and around powers of two; the
rounding half away from zero at ties (+-0.5, +-2.5) and the residues with their 2^split factor against Python
integers, including coefficients past 2^61 and negative ones."""
import numpy as np
import pytest

from oracle import encode as oe
from perseus_amd.encoding import decode


def test_place_is_the_orbit_of_5():
    n = 64
    z = np.arange(1, n // 2 + 1) + 1j * np.arange(n // 2)
    w = oe.place(z, n)
    for j in range(n // 2):
        t = pow(5, j, 2 * n)
        assert w[(t - 1) // 2] == z[j] and w[(2 * n - t - 1) // 2] == np.conj(z[j])
    assert np.count_nonzero(w == 0) <= 1  # every position filled (z[0] has imaginary part 0 but real part 1)


def test_coefficients_against_direct_sums():
    n = 1 << 10
    rng = np.random.default_rng(4)
    z = rng.uniform(-1, 1, n // 2) + 1j * rng.uniform(-1, 1, n // 2)
    scale = 2.0 ** 30
    c = oe.coefficients(z, n, scale)
    # c_k = scale / N sum_t m(zeta^t) zeta^(-t k) over the odd t, in extended precision
    zl = np.asarray(z, np.clongdouble)
    k = np.arange(n, dtype=np.longdouble)
    acc = np.zeros(n, np.clongdouble)
    pi = np.longdouble("3.14159265358979323846264338327950288")
    for j in range(n // 2):
        t = pow(5, j, 2 * n)
        for tt, v in ((t, zl[j]), (2 * n - t, np.conj(zl[j]))):
            ang = -pi * tt * k / n
            acc += v * (np.cos(ang) + 1j * np.sin(ang))
    exact = (acc.real / n * scale).astype(np.longdouble)
    assert np.abs(acc.imag).max() / n * scale < 1e-6, "real by the conjugate placement"
    err = float(np.abs(c.astype(np.longdouble) - exact).max())
    assert err < 1e-9 * float(np.abs(exact).max()), err
    back = decode(c, n, scale)
    assert np.abs(back - z).max() < 1e-9


@pytest.mark.parametrize("cmax,split", [(0.0, 0), (1.0, 0), (2.0 ** 61, 0), (np.nextafter(2.0 ** 61, np.inf), 1),
                                        (2.0 ** 62, 1), (2.0 ** 62 + 2.0 ** 10, 2), (3.0 * 2.0 ** 70, 11),
                                        (2.0 ** 61 - 1024.0, 0)])
def test_split(cmax, split):
    assert oe.split_of(cmax) == split


def test_rounding_ties_away_from_zero():
    for x, r in ((0.5, 1), (-0.5, -1), (2.5, 3), (-2.5, -3), (1.49999999999, 1), (-1.5, -2), (0.0, 0),
                 (2.0 ** 60 + 0.0, 2 ** 60)):
        assert oe.round_away(x) == r, x


def test_scatter_against_integers():
    primes = [1073479681, 1073184769, 1072496641]
    deg = [1, 7, 123456]
    c = np.array([0.5, -0.5, 2.5, -2.5, 1.0e6 + 0.25, -3.0e9 - 0.75, 2.0 ** 40, -(2.0 ** 45)])
    out, split = oe.scatter(c, primes, deg)
    assert split == 0
    for l, p in enumerate(primes):
        want = [((oe.round_away(x)) % p) * deg[l] % p for x in c]
        assert out[l].tolist() == want
    # past 2^61: split 2, the rounding at c / 4, then times 4
    big = np.array([2.0 ** 62 + 2.0 ** 20, -(2.0 ** 62) - 6.0, 10.0, -2.0])
    out, split = oe.scatter(big, primes, deg)
    assert split == 2
    for l, p in enumerate(primes):
        want = [(oe.round_away(x / 4) % p) * 4 * deg[l] % p for x in big]
        assert out[l].tolist() == want
    assert oe.round_away(-2.0 / 4) == -1 and oe.round_away(10.0 / 4) == 3  # ties at the split's scale
