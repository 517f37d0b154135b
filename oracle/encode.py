"""Oracle of the device slot encoder (test infrastructure: only tests/ import it). Restates the table's `encode` entry
(crates/pc-kernels/kernels/args.cuh:595-611 EncodeArgs; encode.cuh place / fft_pass / coeffs / split_of / scatter;
crates/pc-gpu/src/encode_dev.rs fft_v):
- place(z, n): slot j at FFT position (t - 1) / 2, t = 5^j mod 2N, its conjugate at (2N - t - 1) / 2;
- coefficients(z, n, scale): c_k = scale Re(Y_k zeta^-k) / N, Y = DFT_N(place(z)), zeta = exp(i pi / N), in double;
- split_of(cmax): OpenFHE's split, ceil(log2 max |c|) - 61 when positive;
- scatter(c, primes, deg_factor): m_k = c_k / 2^split rounded half away from zero, residues (m_k mod p) deg_factor
  2^split mod p, in Python integers.
The rounding and the residues are exact integer rules; the coefficients are floating point, so a device transform's
words agree with these within the double error of the transform (the tolerance the reference states between its
host and device encoders, encode_dev.rs:1-9).
"""
import math
from fractions import Fraction

import numpy as np


def place(z, n):
    z = np.asarray(z, np.complex128)
    w = np.zeros(n, np.complex128)
    t = 1
    for j in range(n // 2):
        w[(t - 1) // 2] = z[j]
        w[(2 * n - t - 1) // 2] = np.conj(z[j])
        t = t * 5 % (2 * n)
    return w


def coefficients(z, n, scale):
    y = np.fft.fft(place(z, n))
    k = np.arange(n)
    return (y * np.exp(-1j * np.pi * k / n)).real / n * scale


def split_of(cmax):
    """0, or ceil(log2 cmax) - 61 when that is positive (cmax a non-negative double)."""
    if not cmax > 0.0:
        return 0
    f, e = math.frexp(cmax)
    logc = e - 1 if f == 0.5 else e
    return logc - 61 if logc > 61 else 0


def round_away(x):
    """x (a double, exactly) rounded to the nearest integer, halves away from zero."""
    q = Fraction(x)
    a = abs(q)
    r = int(a + Fraction(1, 2))  # floor(|x| + 1/2)
    return -r if q < 0 else r


def scatter(c, primes, deg_factor):
    """rows [len(primes)][N] of residues: round_away(c_k / 2^split) mod p times deg_factor[l] 2^split mod p."""
    c = np.asarray(c, np.float64)
    split = split_of(float(np.abs(c).max()) if len(c) else 0.0)
    m = [round_away(math.ldexp(float(x), -split)) for x in c]
    out = np.zeros((len(primes), len(c)), np.uint32)
    for l, p in enumerate(primes):
        p = int(p)
        f = int(deg_factor[l]) * pow(2, split, p) % p
        out[l] = np.array([(v % p) * f % p for v in m], np.uint64).astype(np.uint32)
    return out, split
