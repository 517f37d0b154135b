"""Host-side CKKS encoding (the canonical embedding) in double precision, for the caller that prepares plaintexts and
reads results: N/2 complex slots, slot j at the root zeta^(5^j) (zeta = exp(i pi / N)) and its conjugate at
zeta^(-5^j), so that rotating the slots left by r is the automorphism X -> X^(5^r) (crates/pc-core/src/encode.rs,
OpenFHE's slot order; crates/pc-core/src/galois.rs:35-60).

encode: coefficients m_i = round(scale Re(sum_k v_k zeta^(-i (2k+1))) / N), with v the slot values placed at the
odd powers they sit on; decode: the inverse. Both through one N-point FFT. The kernel table's `encode` entry encodes
on the device by the same mathematics (csrc/encode.hip).
"""
import numpy as np


def slot_positions(n):
    """k_j (j < N/2): the FFT position (t - 1) / 2 of slot j, t = 5^j mod 2N, and of its conjugate (2N - t - 1) / 2."""
    m = 2 * n
    t = np.empty(n // 2, np.int64)
    v = 1
    for j in range(n // 2):
        t[j] = v
        v = v * 5 % m
    return (t - 1) // 2, (m - t - 1) // 2


def encode(z, n, scale):
    """N float coefficients (not yet rounded) of the slot vector z (N/2 complex values) at `scale`."""
    z = np.asarray(z, np.complex128)
    pos, cpos = slot_positions(n)
    v = np.zeros(n, np.complex128)
    v[pos] = z
    v[cpos] = np.conj(z)
    # m_i = (1/N) sum_k v_k zeta^(-i (2k + 1)) = zeta^(-i) (1/N) sum_k v_k w^(-i k), w = exp(2 pi i / N)
    i = np.arange(n)
    m = np.exp(-1j * np.pi * i / n) * np.fft.fft(v) / n
    return m.real * scale


def decode(m, n, scale):
    """The N/2 slot values of real coefficients m (already centred integers or floats) at `scale`."""
    m = np.asarray(m, np.float64)
    i = np.arange(n)
    # v_k = sum_i m_i zeta^(i (2k + 1)) = N ifft(m_i zeta^i)_k
    v = np.fft.ifft(m * np.exp(1j * np.pi * i / n)) * n
    pos, _ = slot_positions(n)
    return v[pos] / scale


def to_residues(coef, primes):
    """Rounded coefficients (floats up to 2^63 or Python integers) as residue rows [len(primes)][N] (u32)."""
    c = np.asarray([int(x) for x in np.rint(np.asarray(coef, np.float64))], dtype=object)
    return np.stack([(c % int(p)).astype(np.uint64) for p in primes]).astype(np.uint32)


def from_residues(rows, primes):
    """The centred integers of coefficient rows [k][N] over the primes (CRT, Python integers), as floats."""
    big = 1
    for p in primes:
        big *= int(p)
    acc = np.zeros(rows.shape[1], dtype=object)
    for r, p in enumerate(primes):
        p = int(p)
        m = big // p
        acc = (acc + rows[r].astype(object) * (m * pow(m % p, -1, p))) % big
    half = big // 2
    return np.array([float(x - big) if x > half else float(x) for x in acc])
