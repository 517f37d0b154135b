"""The oracle's SPRU floating-point stages (oracle/twin.cpp or_spru_fft_pass, or_spru_scatter) pinned on the CPU:
one pass against the same arithmetic done exactly in rationals (each fma rounded once, every other product and sum
rounded alone, as crates/pc-host/src/encode.rs:87-101 and spru.rs:110-140 fix them), the passes ns = 1 .. n/2 in
sequence against numpy's forward DFT, and the scatter's rounding (half to even) and residues against Python
integers, ties and negative values included.
"""
from fractions import Fraction

import numpy as np
import pytest

from tests import twin


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def tw_table(n):
    return np.exp(-1j * np.pi * np.arange(n // 2) / (n // 2))


def zt_table(n):
    return np.exp(-1j * np.pi * np.arange(n) / n)


def exact_pass(x, tw, ns):
    n = x.shape[-1]
    half = n // 2
    out = np.zeros_like(x)
    for e in range(x.shape[0]):
        for j in range(half):
            k = j % ns
            idx = (j // ns) * 2 * ns + k
            w = tw[k * (half // ns)]
            v0, v1 = x[e, j], x[e, j + half]
            tx = fma(v1.real, w.real, -(v1.imag * w.imag))
            ty = fma(v1.imag, w.real, v1.real * w.imag)
            out[e, idx] = complex(v0.real + tx, v0.imag + ty)
            out[e, idx + ns] = complex(v0.real - tx, v0.imag - ty)
    return out


@pytest.mark.parametrize("ns", [1, 2, 4, 8])
def test_fft_pass_exact(ns):
    n = 16
    rng = np.random.default_rng(ns)
    x = rng.normal(size=(2, n)) * 1e3 + 1j * rng.normal(size=(2, n)) * 1e-3
    x[0, :3] = [1.0 + 1e-17j, -0.0 + 0j, 3.0e300 - 2e-300j]
    got = twin.spru_fft_pass(x, tw_table(n), ns)
    want = exact_pass(x, tw_table(n), ns)
    assert (got.view(np.uint64) == want.view(np.uint64)).all()


def test_fft_pass_contractions_matter():
    """inputs where fma(a, b, -(c d)) differs from a b - c d in its last bit: the pin above tells the two apart"""
    rng = np.random.default_rng(11)
    n = 16
    x = rng.normal(size=(1, n)) + 1j * rng.normal(size=(1, n))
    tw = tw_table(n)
    got = twin.spru_fft_pass(x, tw, 4)
    plain = np.zeros_like(x)
    half = n // 2
    for j in range(half):
        k = j % 4
        w = tw[k * (half // 4)]
        v0, v1 = x[0, j], x[0, j + half]
        t = complex(v1.real * w.real - v1.imag * w.imag, v1.imag * w.real + v1.real * w.imag)
        idx = (j // 4) * 8 + k
        plain[0, idx], plain[0, idx + 4] = v0 + t, v0 - t
    assert (got.view(np.uint64) != plain.view(np.uint64)).any()
    assert np.abs(got - plain).max() < 1e-14


@pytest.mark.parametrize("logn", [4, 10])
def test_passes_give_the_forward_dft(logn):
    n = 1 << logn
    rng = np.random.default_rng(logn)
    x = rng.normal(size=(3, n)) + 1j * rng.normal(size=(3, n))
    y, ns = x, 1
    while ns < n:
        y = twin.spru_fft_pass(y, tw_table(n), ns)
        ns *= 2
    want = np.fft.fft(x, axis=-1)
    assert np.abs(y - want).max() < 1e-12 * n


def exact_scatter(y, zt, primes, scale):
    b, n = y.shape
    out = np.zeros((b, len(primes), n), np.uint32)
    for e in range(b):
        for k in range(n):
            re = fma(y[e, k].real, zt[k].real, -(y[e, k].imag * zt[k].imag)) * (1.0 / n)
            m = int(round(re * scale))  # Python rounds floats half to even
            for i, p in enumerate(primes):
                out[e, i, k] = m % p
    return out


def test_scatter_exact():
    n = 64
    primes = [268369921, 268361729, 3]
    rng = np.random.default_rng(4)
    y = rng.normal(size=(2, n)) * 1e9 + 1j * rng.normal(size=(2, n)) * 1e9
    zt = zt_table(n)
    # ties at scale 1 with zt = 1: re = y.x / n exactly
    zt = zt.copy()
    zt[:6] = 1.0
    y[0, :6] = np.array([2.5, 3.5, -2.5, -3.5, 0.5, -0.5]) * n + 7j
    y[1, :2] = [2.0 ** 62 * n, -(2.0 ** 62) * n]
    got = twin.spru_scatter(y, zt, primes, 1.0)
    assert [int(got[0, 0, k]) for k in range(6)] == [2, 4, primes[0] - 2, primes[0] - 4, 0, 0]
    assert (got == exact_scatter(y, zt, primes, 1.0)).all()
    got = twin.spru_scatter(y / 2.0 ** 20, zt_table(n), primes, 2.0 ** 20)
    assert (got == exact_scatter(y / 2.0 ** 20, zt_table(n), primes, 2.0 ** 20)).all()
