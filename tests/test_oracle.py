"""Pins of the oracle (the CPU twin) before anything is compared against it.

Each check is one the reference itself holds (a golden vector or known answer, cited) or one the mathematics fixes
(a closed form, an invariant, brute force on small inputs), chosen so that a plausible mistake in the twin (a wrong
index, sign, stride or dropped term) fails it.
"""
import json
import os

import numpy as np
import pytest

from tests import twin
from tests.twin import LIB


def fnv(v):
    """FNV-1a over u64 words (crates/pc-core/tests/kskb_frozen.rs:8-10)."""
    h = 0xCBF29CE484222325
    for x in v:
        h = ((h ^ int(x)) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")))


# ----------------------------------------------------------------------------------------------- ChaCha / expanders
def test_chacha20_rfc8439_block():
    # RFC 8439 section 2.3.2: key 00..1f, counter 1, nonce 00:00:00:09:00:00:00:4a:00:00:00:00; the state after the
    # feed-forward add
    v = GOLDEN["chacha20_rfc8439_block"]
    out = twin.chacha_block(v["key"], v["w12"], v["w13"], v["w14"], v["w15"], v["rounds"])
    assert [int(x) for x in out] == v["out"]


# crates/pc-core/tests/kskb_frozen.rs:46-52 PINNED: (p, a[0], a[1], a[n-1], FNV-1a of the row), digits 0 / 3 / 6,
# N = 2^16 (the n64 chain, crates/pc-core/src/params.rs:165-168)
KSKB = GOLDEN["kskb_frozen"]


@pytest.mark.parametrize("digit,p,a0,a1,alast,h", [tuple(r) for r in KSKB["pinned"]])
def test_kskb_frozen_vector(digit, p, a0, a1, alast, h):
    """The u64 lane's pinned keystream: it pins the ChaCha12 core, the (counter, w13, w14, tag) state layout, the block
    and retry-counter machinery (the 2^53 prime rejects ~2^-11 of its words) and the reduction, all of which the u32
    KSKA lane shares."""
    row = twin.kskb_row(KSKB["seed"], digit, p, KSKB["n"])
    assert (int(row[0]), int(row[1]), int(row[-1])) == (a0, a1, alast)
    assert fnv(row) == h


def test_kska_row_equals_slot_form():
    # crates/pc-core/src/keys.rs:466-498: the row form and the random-access slot form give the same values; at a
    # 31-bit prime near 1.5 * 2^30 a quarter of the words are rejected, so the retries are exercised
    seed = np.array([1, 2, 3, 4, 5, 6, 7, 0xDEADBEEF], np.uint32)
    n = 1 << 12
    for digit, p in [(3, 268042241), (0, 1610629121), (2, 2147352577)]:
        assert LIB.or_is_prime(p)
        row = twin.kska_row(seed, digit, p, n)
        assert (row < p).all()
        for s in list(range(0, n, 37)) + [n - 1]:
            assert int(row[s]) == LIB.or_kska_expand(seed, digit, p, s, n)


def test_kska_rejection_rule():
    """Words at or above floor((2^32-1)/p) p are rejected and retried at block + t N/16 (the spec text of
    crates/pc-core/src/keys.rs:466-481), checked by recomputing one rejected slot from raw blocks."""
    seed = np.arange(8, dtype=np.uint32) * 7 + 1
    p, n, digit = 1610629121, 1 << 10, 1
    mp = (0xFFFFFFFF // p) * p
    row = twin.kska_row(seed, digit, p, n)
    found = 0
    for b0 in range(n // 16):
        blk = twin.chacha_block(seed, b0, digit, p, 0x4B534B41, 12)
        for w in range(16):
            v = int(blk[w])
            if v < mp:
                assert int(row[16 * b0 + w]) == v % p
                continue
            found += 1
            t = 1
            while v >= mp and t < 16:
                v = int(twin.chacha_block(seed, b0 + t * (n // 16), digit, p, 0x4B534B41, 12)[w])
                t += 1
            assert int(row[16 * b0 + w]) == v % p
    assert found > 100


# ----------------------------------------------------------------------------------------------- number theory
def test_nbtheory_known_answers():
    # crates/pc-core/src/params/nbtheory.rs:170-180
    v = GOLDEN["nbtheory"]
    m, q = v["m"], v["previous_prime_of_first_prime_28"]
    assert LIB.or_previous_prime(LIB.or_first_prime(28, m), m) == q
    assert LIB.or_root_of_unity(m, q) == v["root_of_unity"]
    assert LIB.or_is_prime(q)
    assert not LIB.or_is_prime(q * 3)
    for c in v["not_prime"]:
        assert not LIB.or_is_prime(c)  # 3215031751: a strong pseudoprime to bases 2, 3, 5, 7


def test_is_prime_brute_force():
    sieve = np.ones(20000, bool)
    sieve[:2] = False
    for i in range(2, 142):
        if sieve[i]:
            sieve[i * i::i] = False
    for x in range(20000):
        assert bool(LIB.or_is_prime(x)) == bool(sieve[x]), x


def test_root_is_minimal_primitive():
    for logn, p in [(4, 97), (10, 12289), (16, 2147352577)]:
        m = 2 << logn
        r = LIB.or_root_of_unity(m, p)
        assert pow(r, m // 2, p) == p - 1
        if m <= 4096:  # brute force: no smaller primitive root
            prim = [x for x in range(2, p) if pow(x, m // 2, p) == p - 1 and pow(x, m, p) == 1]
            assert r == min(prim)


def test_descending_primes():
    m = 1 << 17
    ps = twin.descending_primes(31, m, 8)
    assert all(LIB.or_is_prime(p) and p % m == 1 and p.bit_length() == 31 for p in ps)
    assert ps == sorted(ps, reverse=True) and len(set(ps)) == 8
    # nothing skipped: every candidate between consecutive primes is composite
    for a, b in zip(ps, ps[1:]):
        for c in range(b + m, a, m):
            assert not LIB.or_is_prime(c)
    assert all(not LIB.or_is_prime(c) for c in range(ps[0] + m, 1 << 31, m))


def test_prime_const_fields():
    buf = (np.zeros(8, np.uint64))
    for p in [268042241, 1073479681, 2147352577]:
        LIB.or_prime_const(p, 32, buf.ctypes.data)
        w = buf.view(np.uint32)
        bits = p.bit_length()
        assert int(buf[0]) == p and int(buf[1]) == (1 << 64) // p and int(buf[2]) == 0
        assert int(buf[3]) == (1 << (2 * bits + 1)) // p
        assert int(w[8]) == bits and int(w[9]) == 32
        assert (int(buf[5]) * p) % (1 << 32) == (1 << 32) - 1  # -p^-1 mod 2^32
        assert int(buf[6]) == (1 << 64) % p
        r = (1 << 32) % p
        assert int(buf[7]) == r | (((r << 32) // p) << 32)


# ----------------------------------------------------------------------------------------------- galois
def test_automorph_slot_is_eval_gather_table():
    # crates/pc-core/src/galois.rs:84-100 eval_gather_table vs arith.cuh automorph_slot, and the group law
    logn, n = 6, 64
    for g in [5, 25, 2 * n - 1, 3]:
        t = [0] * n
        for j in range(n):
            idx = (((2 * j + 1) * g) % (2 * n)) >> 1
            t[int(f"{j:0{logn}b}"[::-1], 2)] = int(f"{idx:0{logn}b}"[::-1], 2)
        assert [twin.automorph_slot(g, o, logn) for o in range(n)] == t
    gi = twin.galois_inverse(25, n)
    assert (25 * gi) % (2 * n) == 1
    assert twin.rotation_galois(3, n) == pow(5, 3, 2 * n)
    assert twin.rotation_galois(-1, n) == pow(5, n // 2 - 1, 2 * n)


# ----------------------------------------------------------------------------------------------- NTT
def brev(x, bits):
    return int(f"{x:0{bits}b}"[::-1], 2)


@pytest.mark.parametrize("logn,p", [(4, 97), (6, 7681), (8, 40961), (10, 1073479681)])
def test_ntt_closed_form(logn, p):
    """out[i] = a(psi^(2 brev(i) + 1)) mod p (crates/pc-gpu/src/keys/hostref.rs:283-302, n = 16, p = 97; and larger)."""
    n = 1 << logn
    ctx = twin.Ctx(logn, [p], [], 1)
    psi = ctx.root(0)
    rng = np.random.default_rng(logn)
    a = rng.integers(0, p, n, dtype=np.uint64).astype(np.uint32)
    a[0] = p - 1
    y = ctx.ntt_fwd(a.copy()[None, :], [0])[0]
    for i in range(n):
        x = pow(psi, 2 * brev(i, logn) + 1, p)
        v = 0
        for c in reversed(a.tolist()):
            v = (v * x + c) % p
        assert int(y[i]) == v
    back = ctx.ntt_inv(y.copy()[None, :], [0])[0]
    assert (back == a).all()


def test_ntt_negacyclic_product():
    """INTT(NTT(a) NTT(b)) = a b mod (X^N + 1, p): pins the twiddle order and the negacyclic structure."""
    logn, n, p = 7, 128, 1073479681
    ctx = twin.Ctx(logn, [p], [], 1)
    rng = np.random.default_rng(7)
    a = rng.integers(0, p, n).astype(np.uint32)
    b = rng.integers(0, p, n).astype(np.uint32)
    fa = ctx.ntt_fwd(a[None, :].copy(), [0])[0].astype(object)
    fb = ctx.ntt_fwd(b[None, :].copy(), [0])[0].astype(object)
    prod = np.array([(x * y) % p for x, y in zip(fa, fb)], np.uint32)
    got = ctx.ntt_inv(prod[None, :], [0])[0]
    want = [0] * n
    al, bl = a.tolist(), b.tolist()
    for i in range(n):
        for j in range(n):
            k = i + j
            if k < n:
                want[k] = (want[k] + al[i] * bl[j]) % p
            else:
                want[k - n] = (want[k - n] - al[i] * bl[j]) % p
    assert got.tolist() == want


def test_ntt_large_roundtrip_and_twiddles():
    m = 1 << 17
    ps = twin.descending_primes(31, m, 2)
    ctx = twin.Ctx(16, ps, [], 1)
    fw, fws, iw, iws = ctx.twiddles(1)
    p, psi = ps[1], ctx.root(1)
    for i in [0, 1, 2, 3, 1000, 65535]:
        assert int(fw[i]) == pow(psi, brev(i, 16), p)
        assert int(fws[i]) == (int(fw[i]) << 32) // p
        assert (int(iw[i]) * int(fw[i])) % p == 1
    rng = np.random.default_rng(1)
    x = np.stack([rng.integers(0, p, 1 << 16) for p in ps]).astype(np.uint32)
    y = ctx.ntt_fwd(x.copy(), [0, 1])
    assert ((y < np.array(ps, np.uint64)[:, None]).all())
    assert (ctx.ntt_inv(y, [0, 1]) == x).all()


# ----------------------------------------------------------------------------------------------- bconv
def test_bconv_crt_invariant():
    """The fast conversion leaves X + u B with 0 <= u < ns (X = CRT of the sources, B their product): checked with
    Python integers against every target."""
    m = 1 << 11
    ps = twin.descending_primes(31, m, 9)
    ctx = twin.Ctx(10, ps, [], 1)
    sid, tid = [0, 1, 2, 3, 4], [5, 6, 7, 8]
    rng = np.random.default_rng(3)
    src = [rng.integers(0, ps[i], ctx.n).astype(np.uint32) for i in sid]
    src[0][:4] = [0, ps[0] - 1, 0, ps[0] - 1]
    out = ctx.bconv(src, sid, tid)
    B = 1
    for i in sid:
        B *= ps[i]
    # the fast conversion's own value, in Python integers: sum_i [y_i (B / b_i)^-1]_{b_i} (B / b_i) mod t (an exact
    # conversion, u = 0 everywhere, fails this)
    for c in range(ctx.n):
        y = [int(src[k][c]) * pow(B // ps[i], -1, ps[i]) % ps[i] for k, i in enumerate(sid)]
        for k, t in enumerate(tid):
            q = ps[t]
            assert int(out[k][c]) == sum(yi * (B // ps[i]) for yi, i in zip(y, sid)) % q, (c, t)
    for c in range(0, ctx.n, 7):
        X = 0
        for k, i in enumerate(sid):
            bi = ps[i]
            Bi = B // bi
            X += int(src[k][c]) * Bi * pow(Bi, -1, bi)
        X %= B
        us = set()
        for k, t in enumerate(tid):
            q = ps[t]
            d = (int(out[k][c]) - X) % q
            cand = [u for u in range(len(sid)) if (u * B) % q == d]
            assert len(cand) == 1
            us.add(cand[0])
        assert len(us) == 1  # the same u for every target


# ----------------------------------------------------------------------------------------------- samplers
def test_samplers():
    g = twin.Prng([9, 8, 7, 6, 5, 4, 3, 2], 5)
    s = g.sparse_ternary(1 << 12, 192)
    assert int(np.count_nonzero(s)) == 192 and set(np.unique(s).tolist()) <= {-1, 0, 1}
    e = g.gaussian(1 << 16)
    assert abs(e.mean()) < 0.1 and abs(e.std() - 3.19) < 0.05 and np.abs(e).max() <= 45
    q = 2147352577
    assert all(g.below(q) < q for _ in range(1000))
    # the DRBG keystream is ChaCha20 with the counter in words 12..13, the stream id in 14 and "DRBG" in 15
    key = [1, 2, 3, 4, 5, 6, 7, 8]
    h = twin.Prng(key, 3)
    blk0 = twin.chacha_block(key, 0, 0, 3, 0x47425244, 20)
    blk1 = twin.chacha_block(key, 1, 0, 3, 0x47425244, 20)
    assert [h.u32() for _ in range(32)] == [int(x) for x in np.concatenate([blk0, blk1])]


def test_cts_expand_rule():
    """The regenerable-ciphertext c1 lane (keys.rs:580-630): slot s reads word s & 15 of ChaCha12 block s >> 4 with
    (w13, w14, w15) = (0, p, "CTSA"); a word at or above floor((2^32 - 1)/p) p is redrawn from block s >> 4 + t N/16,
    t < 32, the last draw kept; value mod p. The reference's own checks: values below p, rows distinct per seed, per
    prime and from the KSKA lane (crates/pc-core/tests/cts_expand.rs)."""
    n = 1 << 10
    seed = [((i + 1) * 0x9E3779B9 ^ (w * 0x85EBCA6B)) & 0xFFFFFFFF for i, w in [(0, w) for w in range(8)]]
    for p in (134176769, 268369921, 1431655777):  # the last one just above 2^32 / 3: a third of the words redrawn
        row = twin.cts_expand_row(seed, p, n)
        mp = (0xFFFFFFFF // p) * p
        for s in range(0, n, 37):
            b0, w = s >> 4, s & 15
            v = 0
            for t in range(32):
                v = int(twin.chacha_block(seed, b0 + t * (n // 16), 0, p, 0x43545341, 12)[w])
                if v < mp:
                    break
            assert int(row[s]) == v % p, (p, s)
        assert (row < p).all()
    p = 134176769
    a = twin.cts_expand_row(seed, p, n)
    b = twin.cts_expand_row([x ^ 1 for x in seed], p, n)
    c = twin.cts_expand_row(seed, 132120577, n)
    k = twin.expand_row(seed, 0, p, n, twin.TAG_KSKA)
    assert (a == b).sum() < 4 and (a == c).sum() < 4 and (a == k).sum() < 4
