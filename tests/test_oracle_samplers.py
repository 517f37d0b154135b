"""Pins of the oracle's samplers (the key material of every synthetic test) against the reference's rules, restated
here over raw ChaCha20 words of the RFC 8439-pinned block function, and against the mathematics:

- `uniform_below` (crates/pc-core/src/keys.rs:166-176): a 64-bit word v is accepted iff v >= 2^64 mod q, giving
  v mod q; the threshold is checked at v = rem - 1, rem, rem + 1 with Python integers, and the draw sequence is
  rebuilt from the raw DRBG words, including a stream whose first word is rejected;
- `DiscreteGaussian` (keys.rs:260-325): the CDF table against the closed-form pmf exp(-k^2 / (2 sigma^2)) (doubled for
  k > 0) summed in 50-digit decimal arithmetic; the inversion at u exactly at and just below cdf[k]; the draw order
  (one 53-bit uniform, then a sign word only when |x| > 0) rebuilt from raw words;
- `sample_sparse_ternary` (keys.rs:250-265): positions by uniform_below(n), a sign word (bit 0: 0 -> +1) drawn only
  when the position was empty, rebuilt from raw words, at sizes that force collisions.

Each check fails on the plausible slips: `>` for `>=` in the threshold, 2^64 - 1 mod q for 2^64 mod q, `<` for `<=`
in the CDF search, a dropped factor 2 or sigma^2 for 2 sigma^2 in the pmf, a sign drawn for zero or before the
collision test.
"""
import math
from decimal import Decimal, getcontext

import numpy as np
import pytest

from tests import twin

DRBG = 0x47425244


class RawDrbg:
    """The DRBG's keystream from the pinned ChaCha20 block: counter in words 12..13, stream in 14, "DRBG" in 15."""

    def __init__(self, key, stream):
        self.key, self.stream, self.ctr, self.buf = list(key), stream, 0, []

    def u32(self):
        if not self.buf:
            blk = twin.chacha_block(self.key, self.ctr & 0xFFFFFFFF, self.ctr >> 32, self.stream, DRBG, 20)
            self.buf = [int(x) for x in blk]
            self.ctr += 1
        return self.buf.pop(0)

    def u64(self):
        lo = self.u32()
        return lo | self.u32() << 32


def py_below(g, q):
    rem = (1 << 64) % q
    while True:
        v = g.u64()
        if v >= rem:
            return v % q


QS = [3, 97, 12289, 65536, 2147352577, (1 << 32) + 15, (1 << 63) + 1, (1 << 64) - 1]


@pytest.mark.parametrize("q", QS)
def test_below_threshold_exact(q):
    rem = (1 << 64) % q
    if rem:
        assert twin.below_accept(rem - 1, q) is None, "the largest rejected word"
        assert twin.below_accept(0, q) is None
    assert twin.below_accept(rem, q) == rem % q, "the smallest accepted word"
    assert twin.below_accept(rem + 1, q) == (rem + 1) % q
    assert twin.below_accept((1 << 64) - 1, q) == ((1 << 64) - 1) % q


@pytest.mark.parametrize("q", QS)
def test_below_stream_from_raw_words(q):
    key = [11, 22, 33, 44, 55, 66, 77, 88]
    g, r = twin.Prng(key, 7), RawDrbg(key, 7)
    got = [g.below(q) for _ in range(300)]
    assert got == [py_below(r, q) for _ in range(300)]
    assert g.u32() == r.u32(), "the same number of words consumed"


def test_below_first_word_rejected():
    """q = 2^63 + 1 rejects the words below 2^63 - 1 (about half): a stream whose first word is rejected returns the
    second word's residue (or a later one), never the first's."""
    q = (1 << 63) + 1
    rem = (1 << 64) % q
    assert rem == (1 << 63) - 1
    found = 0
    for s in range(64):
        key = [s, 1, 2, 3, 4, 5, 6, 7]
        r = RawDrbg(key, 0)
        w = [r.u64() for _ in range(40)]
        if w[0] >= rem:
            continue
        want = next(v % q for v in w if v >= rem)
        assert twin.Prng(key, 0).below(q) == want
        assert want != w[0] % q
        found += 1
    assert found >= 8


def exact_cdf(sigma, bound):
    getcontext().prec = 50
    s2 = Decimal(sigma) * Decimal(sigma)  # the double 3.19, exactly
    w = [Decimal(1)] + [2 * (-(Decimal(k * k)) / (2 * s2)).exp() for k in range(1, bound + 1)]
    tot = sum(w)
    acc, out = Decimal(0), []
    for x in w:
        acc += x / tot
        out.append(acc)
    return out


@pytest.mark.parametrize("sigma", [3.19, 1.0, 8.5])
def test_gauss_cdf_closed_form(sigma):
    cdf = twin.gauss_cdf(sigma)
    bound = math.ceil(14 * sigma)
    assert len(cdf) == bound + 1
    ex = exact_cdf(sigma, bound)
    for k in range(bound + 1):
        assert abs(Decimal(float(cdf[k])) - ex[k]) < Decimal("1e-15"), k
    # P(X = 0) and P(|X| = 1) from the pmf directly
    z = float(ex[0])
    assert abs(cdf[0] - z) < 1e-15
    assert abs((cdf[1] - cdf[0]) - 2 * z * math.exp(-1 / (2 * sigma * sigma))) < 1e-15


def test_gauss_inversion_boundaries():
    cdf = twin.gauss_cdf(3.19)
    last = len(cdf) - 1
    assert twin.gauss_index(0.0) == 0
    assert twin.gauss_index(1.0 - 2.0 ** -53) == min(int(np.searchsorted(cdf, 1.0 - 2.0 ** -53, "right")), last)
    n = 0
    for k in range(1, last):
        if not (cdf[k - 1] < cdf[k] < cdf[k + 1]):
            continue
        assert twin.gauss_index(float(cdf[k])) == k + 1, "u equal to cdf[k] is past k (cdf[k] <= u)"
        assert twin.gauss_index(float(np.nextafter(cdf[k], 0.0))) == k, "u just below cdf[k] stays at k"
        n += 1
    assert n >= 10
    # u at or past the table's last entry clamps to the bound
    assert twin.gauss_index(float(cdf[last])) == last


def test_gauss_draw_order_from_raw_words():
    key = [5, 4, 3, 2, 1, 0, 9, 8]
    g, r = twin.Prng(key, 2), RawDrbg(key, 2)
    got = g.gaussian(4096)
    want = []
    for _ in range(4096):
        u = (r.u64() >> 11) * 2.0 ** -53
        k = twin.gauss_index(u)
        want.append(0 if k == 0 else (k if r.u32() & 1 == 0 else -k))
    assert got.tolist() == want
    assert g.u32() == r.u32(), "a sign word only for nonzero draws"
    assert (got == 0).sum() > 300  # zeros occur, so the no-sign-word rule is exercised


@pytest.mark.parametrize("n,h", [(8, 8), (16, 5), (64, 64), (1 << 12, 192)])
def test_sparse_ternary_from_raw_words(n, h):
    key = [n, h, 3, 1, 4, 1, 5, 9]
    g, r = twin.Prng(key, 1), RawDrbg(key, 1)
    got = g.sparse_ternary(n, h)
    want = [0] * n
    placed = collisions = 0
    while placed < h:
        i = py_below(r, n)
        if want[i] == 0:
            want[i] = 1 if r.u32() & 1 == 0 else -1
            placed += 1
        else:
            collisions += 1
    assert got.tolist() == want
    assert g.u32() == r.u32()
    if n <= 64 and h == n:
        assert collisions > 0, "a full-weight draw on a small ring collides"


def test_rotation_key_draw_order_from_raw_words():
    """or_rotation_key rebuilt from its parts in the order of crates/pc-gpu/src/keygen.rs:193-262 (generate_with, a
    rotation key): the key's seed is the caller's DRBG's first 8 words and the per-digit error streams' key the next 8;
    digit d's errors are the Gaussian draws of the stream (sub, d), reduced per prime and taken to the evaluation form;
    a = KSKA(seed, d, p); b = e + [P s]_{digit d's own rows} - a sigma_{g^-1}(s). Each part is pinned by its own test
    (the DRBG words, the Gaussian's draw order, the KSKA expander, the NTT, the automorphism); this pins their order and
    the relation that joins them (a key drawn with seed and sub swapped, or its errors from one stream, fails)."""
    logn, nq, kp, dnum = 10, 6, 2, 3
    n = 1 << logn
    ps = twin.descending_primes(30, 2 * n, nq + kp)
    oc = twin.Ctx(logn, ps[:nq], ps[nq:], dnum)
    key = [11, 22, 33, 44, 55, 66, 77, 88]
    s = twin.Prng(key, 1).sparse_ternary(n, 64)
    s_eval = oc.secret_eval(s)
    gal = twin.rotation_galois(3, n)
    seed, b = oc.rotation_key(twin.Prng(key, 5), s_eval, gal)
    g = twin.Prng(key, 5)
    words = np.array([g.u32() for _ in range(16)], np.uint32)
    assert (seed == words[:8]).all()
    sub = words[8:]
    rows = oc.rows
    e = np.zeros((dnum, rows, n), np.uint32)
    for d in range(dnum):
        ev = twin.Prng(sub, d).gaussian(n, 3.19)
        assert np.abs(ev).max() < 64
        for t in range(rows):
            e[d, t] = np.mod(ev, ps[t]).astype(np.uint32)
        e[d] = oc.ntt_fwd(e[d], list(range(rows)))
    s_new = oc.automorph_rows(s_eval, twin.galois_inverse(gal, n))
    P = 1
    for x in ps[nq:]:
        P *= x
    for d in range(dnum):
        for t in range(rows):
            p = ps[t]
            a = twin.kska_row(seed, d, p, n).astype(object)
            want = e[d, t].astype(object) - a * s_new[t].astype(object)
            if t < nq and oc.digit_of(t) == d:
                want = want + (P % p) * s_eval[t].astype(object)
            assert (b[d, t].astype(object) == want % p).all(), (d, t)
