"""Pins of the raise kernels' oracle (oracle/bts.py) and of the host tables (perseus_amd/bts.py):

- the x87 reciprocal and its rounding: the reference's own known answers (crates/pc-gpu/src/bts/raise.rs:633-662);
- small_int: the reference's known answers (raise.rs:685-697: three 28-bit sources, c = 1/4), and for random
  integers |X| < Q_k / 2 of one to four 31-bit sources the CRT value itself (no scale) and a rounding within one of
  |X| c (scale);
- small_int1: the reference's known answers (raise.rs:665-683) with the scale exact (mc 2^-sh == c) and the result
  the nearest integer to |x| c (ties up), checked with exact fractions;
- mod_raise: the output rows are the residues of ONE integer Y with Y = X (mod Q_d), X the CRT value of the sources,
  and |Y| <= d Q_d / 2 (each Garner term centred on its own prime): an uncentred term, a wrong inverse or a wrong
  Q_d / q_k breaks one of the two.
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import bts as ob
from perseus_amd import bts
from tests import twin

RNG = np.random.default_rng(99)


def test_reciprocal_and_rounding_known_answers():
    # raise.rs:633-650: (c, mantissa, shift) of round(2^192 / (1 / c)) at x87 precision
    refs = [(2.3167161361161844e-07 * 4096.0, 0xF8C16882EF368000, 118), (1.0, 0x8000000000000000, 129),
            (0.5, 0x8000000000000000, 128), (3.0, 0xC000000000000000, 130), (1e-3, 0x83126E978D4FE000, 119),
            (0.7, 0xB333333333333000, 128), (0.9489, 0xF2EB1C432CA57800, 128),
            (1.234567e-5, 0xCF203FB7BA39D000, 112)]
    for c, m, sh in refs:
        words = bts.reciprocal_words(c)
        r = sum(w << (32 * i) for i, w in enumerate(words))
        assert r == m << sh, c
        assert abs(Fraction(r, 1 << 192) - Fraction(c)) / Fraction(c) < Fraction(1, 10**15)
    # raise.rs:654-662
    assert bts.div_rn64(0, 3) == (0xAAAAAAAAAAAAAAAB, -65)
    assert bts.div_rn64(10, 1 << 20) == (1 << 63, -73)


def test_small_int_known_answers():
    # raise.rs:685-697: three sources, c = 1/4: round half up of |x| / 4 with x's sign
    q = [268042241, 265420801, 156499969]
    out = [268042241, 265420801, 156499969, 95027201]
    tab = bts.small_int_tab(q, [0, 1, 2, 3], out, 0.25)
    xs = [0, 1, -3, 1000, -1001, 123456789012345, -98765432109879]
    rows = np.array([[x % p for x in xs] for p in q], np.uint64)
    got = ob.small_int(q, rows, out, list(tab.R))
    for i, x in enumerate(xs):
        mag = (abs(x) + 2) // 4
        want = [(-mag if x < 0 else mag) % p for p in out]
        assert [int(got[o, i]) for o in range(len(out))] == want, x


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_small_int_is_the_centred_crt_value(k):
    q = twin.descending_primes(31, 1 << 17, k + 3)
    src, outs = q[:k], q
    big = 1
    for p in src:
        big *= p
    xs = [int(RNG.integers(0, 1 << 62)) * int(RNG.integers(0, 1 << 62)) % big for _ in range(300)]
    xs = [x - big if x > big // 2 else x for x in xs] + [big // 2, -(big // 2), 0, 1, -1]
    rows = np.array([[x % p for x in xs] for p in src], np.uint64)
    got = ob.small_int(src, rows, outs)
    for i, x in enumerate(xs):
        assert [int(got[o, i]) for o in range(len(outs))] == [x % p for p in outs]
    c = 3.7e-9 if k > 1 else 0.37
    tab = bts.small_int_tab(src, list(range(len(outs))), outs, c)
    got = ob.small_int(src, rows, outs, list(tab.R))
    for i, x in enumerate(xs):
        exact = abs(Fraction(x)) * Fraction(c)
        # the residues of one integer of x's sign within one of |x| c
        vals = [int(got[o, i]) for o in range(len(outs))]
        cand = [v for v in (int(exact) - 1, int(exact), int(exact) + 1, int(exact) + 2) if v >= 0]
        ok = [v for v in cand if [(-v if x < 0 else v) % p for p in outs] == vals]
        assert ok and abs(ok[0] - exact) <= 1, (x, c)


def test_small_int1_known_answers_and_rounding():
    # raise.rs:665-683: a 60-bit q0, outputs (q0, 97, 65537)
    q0 = 1152921504606584833
    for c in (2.3167161361161844e-07 * 4096.0, 1.0, 0.25, 3.0e-5, 0.7):
        mc, sh = bts.single_scale(c, q0)
        assert Fraction(mc, 1 << sh) == Fraction(c)
        for x in (0, 1, -3, 1000, -1001, 123456789012345, -98765432109879, q0 // 2, -(q0 // 2)):
            v = np.array([x % q0], np.uint64)
            got = [int(g[0]) for g in ob.small_int1(q0, mc, sh, v, [q0, 97, 65537])]
            exact = abs(Fraction(x)) * Fraction(c)
            mag = int(exact + Fraction(1, 2))  # nearest, ties up
            assert abs(mag - exact) <= Fraction(1, 2)
            assert got == [(-mag if x < 0 else mag) % p for p in (q0, 97, 65537)], (c, x)
    with pytest.raises(ValueError):
        bts.single_scale(1e30, q0)


@pytest.mark.parametrize("d", [1, 2, 3])
def test_mod_raise_is_a_small_lift(d):
    q = twin.descending_primes(31, 1 << 17, 9)
    big = 1
    for p in q[:d]:
        big *= p
    N = 400
    X = [int(RNG.integers(0, 1 << 62)) * int(RNG.integers(0, 1 << 62)) % big for _ in range(N)]
    rows = np.zeros((len(q), N), np.uint64)
    for k in range(d):
        rows[k] = [x % q[k] for x in X]
    qhatinv, qhat = bts.mod_raise_consts(q, d)
    out = ob.mod_raise(q, rows, d, d, len(q), qhatinv, qhat)
    tgt = q[d:]
    for i, x in enumerate(X):
        vals = [int(out[t, i]) for t in range(len(tgt))]
        ys = [x + u * big for u in range(-d - 1, d + 2)]
        hits = [y for y in ys if [y % p for p in tgt] == vals]
        assert len(hits) == 1, (i, hits)
        assert abs(hits[0]) <= d * big // 2
