"""The host CKKS encoder (perseus_amd/encoding.py) against what the canonical embedding fixes: the round trip, the
slot rotation as the automorphism X -> X^(5^r), the conjugation as X -> X^(2N-1), the slot-wise product as the
negacyclic product of the coefficients, and the residue conversions both ways (CRT in Python integers)."""
import numpy as np

from perseus_amd import encoding
from tests import twin
from tests.test_oracle_ks import coeff_automorph

RNG = np.random.default_rng(5)


def slots(n):
    return RNG.normal(size=n // 2) + 1j * RNG.normal(size=n // 2)


def test_round_trip():
    n, scale = 1 << 12, 2.0 ** 40
    z = slots(n)
    m = np.rint(encoding.encode(z, n, scale))
    assert np.abs(encoding.decode(m, n, scale) - z).max() < 1e-9


def test_rotation_and_conjugation_are_automorphisms():
    n, scale = 1 << 10, 2.0 ** 30
    z = slots(n)
    m = np.rint(encoding.encode(z, n, scale)).astype(np.int64)
    for r in (1, 3, 64):
        g = twin.rotation_galois(r, n)
        got = encoding.decode(coeff_automorph(m, g, n), n, scale)
        assert np.abs(got - np.roll(z, -r)).max() < 1e-6, r
    got = encoding.decode(coeff_automorph(m, 2 * n - 1, n), n, scale)
    assert np.abs(got - np.conj(z)).max() < 1e-6


def test_product_is_slotwise():
    n, scale = 1 << 8, 2.0 ** 20
    z1, z2 = slots(n), slots(n)
    m1 = np.rint(encoding.encode(z1, n, scale)).astype(np.int64)
    m2 = np.rint(encoding.encode(z2, n, scale)).astype(np.int64)
    prod = np.zeros(n, np.float64)
    for i in range(n):
        for j in range(n):
            v = float(m1[i]) * float(m2[j])
            if i + j < n:
                prod[i + j] += v
            else:
                prod[i + j - n] -= v
    assert np.abs(encoding.decode(prod, n, scale * scale) - z1 * z2).max() < 1e-4


def test_residues_round_trip():
    q = twin.descending_primes(31, 1 << 13, 4)
    c = np.array([0, 1, -1, 2 ** 62, -(2 ** 62) + 7, 12345678901234], dtype=np.float64)
    rows = encoding.to_residues(c, q)
    assert (encoding.from_residues(rows, q) == np.rint(c)).all()
