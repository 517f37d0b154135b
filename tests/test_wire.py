"""The wire format (perseus_amd/wire.py) on the CPU: the bit packing against Python integers, the checksum's definition,
bundles and ciphertext frames written and read back (entries in order, sizes, checksums, corruption, magic and version
refused), the regenerable frame's c1 rows against the oracle's "CTSA" expander (pinned in tests/test_oracle.py).
"""
import io
import math
from fractions import Fraction

import numpy as np
import pytest

from perseus_amd import wire
from tests import twin


def test_sum64_definition():
    off, prime, m = 0xCBF29CE484222325, 0x100000001B3, (1 << 64) - 1
    assert wire.sum64(np.zeros(0, np.uint32)) == off
    w = np.array([0x11223344, 0x55667788, 0x99AABBCC], np.uint32)
    h = ((off ^ (0x55667788 << 32 | 0x11223344)) * prime) & m
    h = ((h ^ 0x99AABBCC) * prime) & m
    assert wire.sum64(w) == h


@pytest.mark.parametrize("bits", [27, 28, 30, 31, 32])
def test_pack_row_against_python_integers(bits):
    n = 200
    rng = np.random.default_rng(bits)
    v = rng.integers(0, 1 << bits, n, dtype=np.uint64).astype(np.uint32)
    words = wire.packed_row_words(n, bits)
    # floor(n bits / 32) + 1 words padded to 16 bytes: the data fit, with a whole zero guard word when n bits is a
    # multiple of 32
    assert words % 4 == 0 and words * 32 >= n * bits + (32 if n * bits % 32 == 0 else 0)
    pk = wire.pack_row(v, bits, words)
    stream = int.from_bytes(pk.astype("<u4").tobytes(), "little")
    assert [(stream >> (bits * i)) & ((1 << bits) - 1) for i in range(n)] == [int(x) for x in v]
    assert stream >> (bits * n) == 0
    assert (wire.unpack_row(pk, bits, n) == v).all()


def bundle_bytes(entries, payloads, bits=31, n=64):
    h = {"chain": "t", "params_hash": "abc", "contract": "c", "n": n, "bits": bits,
         "row_words": wire.packed_row_words(n, bits), "entries": entries}
    f = io.BytesIO()
    bw = wire.BundleWriter(f, h)
    for p in payloads:
        bw.put(p)
    assert bw.finish() == len(f.getvalue())
    return f.getvalue(), h


def test_bundle_round_trip_and_refusals():
    n, bits = 64, 31
    rw = wire.packed_row_words(n, bits)
    rng = np.random.default_rng(5)
    shape = {"q_top": 2, "ndig": 2, "nq": 3, "kp": 1}
    b = rng.integers(0, 1 << 31, (2, 4, n)).astype(np.uint32)
    e0 = wire.ksk_entry("rot", shape, range(8), rw, step=3, galois=pow(5, 3, 2 * n))
    e1 = {"kind": "public_key", "rows": 3, "words": 2 * 3 * n}
    pk = rng.integers(0, 1 << 31, 2 * 3 * n).astype(np.uint32)
    data, h = bundle_bytes([e0, e1], [wire.pack_ksk(b, bits, rw), pk], bits, n)
    r = wire.BundleReader(io.BytesIO(data))
    assert r.header == h
    assert (r.ksk_b(0) == b).all() and (r.read(1) == pk).all()
    assert wire.galois_of(r.header["entries"][0], n) == pow(5, 3, 2 * n)
    bad = bytearray(data)
    bad[-20] ^= 1
    with pytest.raises(wire.WireError, match="checksum"):
        wire.BundleReader(io.BytesIO(bytes(bad))).read(1)
    with pytest.raises(wire.WireError, match="bytes"):
        wire.BundleReader(io.BytesIO(data[:-4]))
    with pytest.raises(wire.WireError, match="magic"):
        wire.BundleReader(io.BytesIO(b"XXXX" + data[4:]))
    with pytest.raises(wire.WireError, match="version"):
        wire.BundleReader(io.BytesIO(data[:4] + (2).to_bytes(4, "little") + data[8:]))
    f = io.BytesIO()
    bw = wire.BundleWriter(f, h)
    with pytest.raises(wire.WireError, match="declares"):
        bw.put(pk)
    with pytest.raises(wire.WireError, match="closed"):
        wire.BundleWriter(io.BytesIO(), h).finish()


def test_cts_expand_row_equals_the_oracle():
    n = 1 << 10
    rng = np.random.default_rng(2)
    for p in (134176769, 268369921, 1431655777):
        seed = rng.integers(0, 1 << 32, 8, dtype=np.uint64).astype(np.uint32)
        assert (wire.cts_expand_row(seed, p, n) == twin.cts_expand_row(seed, p, n)).all(), p


def test_ct_frames():
    n, rows, k = 64, 3, 2
    q = [268369921, 268361729, 268271617]
    rng = np.random.default_rng(3)
    meta = {"level": 4, "deg": 1, "nf": 2.0 ** 40, "slots": 32, "tag": None}
    full = np.stack([np.stack([np.stack([rng.integers(0, p, n) for p in q]) for _ in range(2)]) for _ in range(k)])
    h = {"params_hash": "x", "n": n, "k": k, "rows": rows, "meta": meta}
    f = io.BytesIO()
    wire.write_ct(f, h, full)
    f.seek(0)
    h2, d = wire.read_ct(f)
    assert h2 == h and (wire.expand_ct(h2, d, q) == full).all()
    # a regenerable seeded frame: c0 rows then 8 seed words per row, c1 drawn from the seeds
    seeds = rng.integers(0, 1 << 32, (k, rows, 8), dtype=np.uint64).astype(np.uint32)
    body = np.concatenate([np.concatenate([full[c, 0].reshape(-1), seeds[c].reshape(-1)]) for c in range(k)])
    hs = dict(h, seeded=True, regen=True)
    f = io.BytesIO()
    wire.write_ct(f, hs, body)
    raw = f.getvalue()
    h3, d3 = wire.read_ct(io.BytesIO(raw))
    got = wire.expand_ct(h3, d3, q)
    for c in range(k):
        assert (got[c, 0] == full[c, 0]).all()
        for r in range(rows):
            assert (got[c, 1, r] == twin.cts_expand_row(seeds[c, r], q[r], n)).all()
    bad = bytearray(raw)
    bad[-12] ^= 4
    with pytest.raises(wire.WireError, match="checksum"):
        wire.read_ct(io.BytesIO(bytes(bad)))
    # the same body as a DRBG-seeded frame: c1 by fill_below
    f = io.BytesIO()
    wire.write_ct(f, dict(h, seeded=True), body)
    h4, d4 = wire.read_ct(io.BytesIO(f.getvalue()))
    got = wire.expand_ct(h4, d4, q)
    assert (got[1, 1, 2] == wire.drbg_row(seeds[1, 2], q[2], n)).all()
    with pytest.raises(wire.WireError, match="needs"):
        wire.write_ct(io.BytesIO(), dict(h, bits=40), body)


# ----------------------------------------------------------------------------------------------- every frame form
META = {"level": 0, "deg": 1, "nf": 2.0 ** 30, "slots": 32, "tag": None}


@pytest.mark.parametrize("flags,ok", [
    ({}, True), ({"bits": 20}, True), ({"bits": 20, "bits1": 30}, True), ({"bits1": 30}, False),
    ({"bits": 0}, False), ({"bits": 65}, False), ({"bits": 20, "seeded": True}, False),
    ({"seeded": True}, True), ({"seeded": True, "regen": True}, True), ({"regen": True}, False),
    ({"seeded": True, "drop": 10, "bits": 40}, True), ({"seeded": True, "regen": True, "drop": 10, "bits": 40}, False),
    ({"seeded": True, "drop": 10, "bits": 127}, False), ({"seeded": True, "drop": 10}, False),
    ({"seeded": True, "drop": 10, "bits": 40, "bits1": 20}, False), ({"drop": 10, "bits": 40}, False),
    ({"bits": 20, "sub1": 4}, True), ({"sub1": 4}, False), ({"bits": 20, "sub1": 3}, False),
    ({"bits": 20, "sub1": 1}, False), ({"coeff0": True, "coeff1": True}, True), ({"sparse": True, "bits": 20}, True)])
def test_ct_header_check(flags, ok):
    h = wire.ct_header("p", 64, 2, 3, META, **flags)
    if ok:
        wire.check_ct_header(h)
    else:
        with pytest.raises(wire.WireError):
            wire.check_ct_header(h)


def test_ct_header_field_order_and_words():
    h = wire.ct_header("p", 64, 2, 3, META, coeff1=True, bits=20, sparse=False, sub1=4, bits1=30)
    assert list(h) == ["params_hash", "n", "k", "rows", "meta", "bits", "bits1", "coeff1", "sub1"]
    assert wire.ct_words(h) == 2 * (wire.packed_words(64, 20) + wire.packed_words(16, 30))
    assert wire.ct_words(wire.ct_header("p", 64, 2, 3, META)) == 2 * 2 * 3 * 64
    assert wire.ct_words(wire.ct_header("p", 64, 2, 3, META, seeded=True)) == 2 * 3 * (64 + 8)
    assert wire.ct_words(wire.ct_header("p", 64, 2, 3, META, seeded=True, drop=9, bits=77)) == \
        2 * (wire.packed_words(64, 77) + 3 * 8)


@pytest.mark.parametrize("bits", [1, 7, 22, 31, 32, 33, 48, 63, 64, 90, 126])
@pytest.mark.parametrize("n", [1, 3, 31, 33, 200])
def test_pack_bits_against_python_integers(bits, n):
    rng = np.random.default_rng(bits * 1000 + n)
    v = [int(x) for x in rng.integers(0, 1 << 62, n, dtype=np.uint64)]
    v = [(x << 64 | x * 3) & ((1 << bits) - 1) for x in v]
    w = wire.pack_bits(np.array(v, np.uint64) if bits <= 64 else v, bits)
    assert len(w) == wire.packed_words(n, bits)
    stream = int.from_bytes(w.astype("<u4").tobytes(), "little")
    assert [(stream >> (bits * i)) & ((1 << bits) - 1) for i in range(n)] == v
    assert stream >> (bits * n) == 0
    assert [int(x) for x in wire.unpack_bits(w, n, bits)] == v


def _ref_values(big, n, bits):
    """the reference's own test inputs (wire.rs pack_matches_reference): a hashed sequence, then coefficients around
    the rounding's half points (j + 1/2) Q / 2^bits, +-2"""
    x = [(i * 0x9E3779B97F4A7C15 + i * i * 0x2545F4914F6CDD1D) % big for i in range(n)]
    for k in range(min(n, 400)):
        j = (k * 0x9E3779B9) & ((1 << bits) - 1)
        x[k] = ((((2 * j + 1) * big) >> (bits + 1)) + big + (k % 5) - 2) % big
    return x


@pytest.mark.parametrize("q", [[268042241, 265420801], [268369921, 268361729], [4294828033, 2147352577],
                               [268042241, 265420801, 156499969]])
@pytest.mark.parametrize("bits", [1, 12, 16, 22, 28, 31, 32, 33, 48])
def test_pack_coeffs_rounding(q, bits):
    big = 1
    for p in q:
        big *= p
    n = 1200
    x = _ref_values(big, n, bits)
    rows = [np.array([v % p for v in x], np.uint64) for p in q]
    rows[0][800:900] = [v % q[0] + q[0] * 3 for v in x[800:900]]  # unreduced residues
    if sum(p.bit_length() for p in q) + bits > 127:
        with pytest.raises(wire.WireError):
            wire.pack_coeffs(q, rows, bits)  # past the 127-bit product the reference refuses
        return
    got = [int(v) for v in wire.pack_coeffs(q, rows, bits)]
    mask = (1 << bits) - 1
    if len(q) == 2 and big < 1 << 63 and bits <= 32:
        # the reference's two-prime rounding: f64 product by 2^bits / Q, rounded half away from zero
        # the product z rounded as a double, then z itself (exactly, as a fraction) rounded half away from zero
        scale = float(1 << bits) / float(big)
        want = [math.floor(Fraction(float(v) * scale) + Fraction(1, 2)) & mask for v in x]
    else:
        want = [(((v << bits) + big // 2) // big) & mask for v in x]
    assert got == want
    back = wire.unpack_coeffs(q, got, bits)
    for i in range(0, n, 37):
        xr = ((got[i] * big) + (1 << (bits - 1))) >> bits
        assert all(int(back[r][i]) == xr % big % p for r, p in enumerate(q))
        d = (xr - x[i]) % big
        assert min(d, big - d) <= big // (1 << (bits + 1)) + 2 + (big >> 52)
    part = wire.pack_frame_part(q, rows, bits)
    assert (part == wire.pack_bits(np.array(got, np.uint64), bits)).all()


def test_dropped_round_trip():
    """the reference's dropped_roundtrip: every residue is that of the rounded coefficient, at dropped_bits bits"""
    primes = [268042241, 265420801, 156499969, 95027201]
    n = 257
    for k in (1, 2, 3, 4):
        q = primes[:k]
        big = 1
        for p in q:
            big *= p
        xs = [((i + 1) * 0x9E3779B97F4A7C15F39CC0605CEDC835) % big for i in range(n)]
        xs[0], xs[1] = 0, big - 1
        rows = [np.array([x % p for x in xs], np.uint64).astype(np.uint32) for p in q]
        for drop in (0, 1, 9, 24, 27 * k - 2):
            w, bits = wire.pack_dropped(q, rows, drop)
            assert bits == wire.dropped_bits(q, drop) and len(w) == wire.packed_words(n, bits)
            back = wire.unpack_dropped(q, w, drop, n)
            for r, p in enumerate(q):
                want = [(((x + ((1 << drop) >> 1)) >> drop) << drop) % p for x in xs]
                assert [int(v) for v in back[r]] == want, (k, drop, r)
    with pytest.raises(wire.WireError):
        wire.dropped_bits([2 ** 31 - 1], 3)  # a prime of 31 bits
    with pytest.raises(wire.WireError):
        wire.dropped_bits(primes[:1], 28)  # every bit dropped


@pytest.mark.parametrize("q", [3, 12289, 2147352577, 4294967291, 1 << 32])
def test_drbg_row_is_the_samplers_stream(q):
    """fill_below's draws are uniform_below's in order: the oracle's pinned DRBG, seed, stream 0"""
    seed = [7, 1, 4, 1, 5, 9, 2, 6]
    g = twin.Prng(seed, 0)
    want = [g.below(q) for _ in range(700)]
    assert [int(v) for v in wire.drbg_row(seed, q, 700)] == want


def _frame(h, data):
    f = io.BytesIO()
    wire.write_ct(f, h, data)
    return f.getvalue()


def test_seeded_frames_expand():
    n, rows, primes = 64, 3, [1073479681, 1073184769, 1072496641]
    rng = np.random.default_rng(8)
    c0 = np.stack([rng.integers(0, p, n) for p in primes]).astype(np.uint32)
    seeds = rng.integers(0, 1 << 32, (rows, 8), dtype=np.uint64).astype(np.uint32)
    for regen in (False, True):
        h = wire.ct_header("p", n, 1, rows, META, seeded=True, regen=regen)
        hh, d = wire.read_ct(io.BytesIO(_frame(h, np.concatenate([c0.reshape(-1), seeds.reshape(-1)]))))
        x = wire.expand_ct(hh, d, primes)[0]
        assert (x[0] == c0).all()
        for r in range(rows):
            if regen:
                want = twin.cts_expand_row(seeds[r], primes[r], n)
            else:
                g = twin.Prng(seeds[r], 0)
                want = np.array([g.below(primes[r]) for _ in range(n)], np.uint32)
            assert (x[1, r] == want).all()
    # the DRBG rows against the pinned sampler, every value
    g = twin.Prng(seeds[1], 0)
    assert [int(v) for v in wire.drbg_row(seeds[1], primes[1], n)] == [g.below(primes[1]) for _ in range(n)]


def test_short_c0_frame_expands_to_coefficient_form():
    n, primes = 64, [268042241, 265420801]
    rng = np.random.default_rng(9)
    coef = np.stack([rng.integers(0, p, n) for p in primes]).astype(np.uint32)
    seeds = rng.integers(0, 1 << 32, (2, 8), dtype=np.uint64).astype(np.uint32)
    w, bits = wire.pack_dropped(primes, coef, 10)
    h = wire.ct_header("p", n, 1, 2, META, seeded=True, drop=10, bits=bits)
    hh, d = wire.read_ct(io.BytesIO(_frame(h, np.concatenate([w, seeds.reshape(-1)]))))
    nh, x = wire.expand_seeded(hh, d, primes)
    assert nh.get("coeff0") and "drop" not in nh and "bits" not in nh and not nh.get("seeded")
    x = x.reshape(2, 2, n)
    assert (x[0] == wire.unpack_dropped(primes, w, 10, n)).all()
    with pytest.raises(wire.WireError, match="coefficient form"):
        wire.expand_ct(hh, d, primes)
    bad = dict(h, bits=bits + 1)
    with pytest.raises(wire.WireError):
        wire.expand_seeded(bad, np.zeros(wire.ct_words(bad), np.uint32), primes)


def test_expand_refuses_what_it_cannot_return():
    n = 64
    comp = wire.ct_header("p", n, 1, 2, META, bits=20)
    with pytest.raises(wire.WireError, match="client"):
        wire.expand_ct(comp, np.zeros(wire.ct_words(comp), np.uint32), [97, 193])
    sp = wire.ct_header("p", n, 1, 2, META, sparse=True)
    d = np.zeros(wire.ct_words(sp), np.uint32)
    with pytest.raises(wire.WireError, match="sparse"):
        wire.expand_ct(sp, d, [97, 193])
    assert wire.expand_ct(sp, d, [97, 193], sparse_ok=True).shape == (1, 2, 2, n)
    for f in ("coeff0", "coeff1"):
        h = wire.ct_header("p", n, 1, 2, META, **{f: True})
        with pytest.raises(wire.WireError, match="coefficient form"):
            wire.expand_ct(h, np.zeros(wire.ct_words(h), np.uint32), [97, 193])


def test_lifted_spreads_the_coefficients():
    rng = np.random.default_rng(10)
    h = wire.ct_header("p", 16, 1, 2, dict(META, slots=8), coeff0=True, coeff1=True)
    d = rng.integers(0, 1 << 30, wire.ct_words(h), dtype=np.uint64).astype(np.uint32)
    nh, x = wire.lifted(h, d, 64)
    assert nh["n"] == 64 and nh["meta"]["slots"] == 32
    x = x.reshape(2, 2, 64)
    src = d.reshape(2, 2, 16)
    assert (x[:, :, ::4] == src).all() and (np.delete(x, np.s_[::4], axis=2) == 0).all()
    with pytest.raises(wire.WireError):
        wire.lifted(dict(h, coeff0=False), d, 64)
    with pytest.raises(wire.WireError):
        wire.lifted(h, d, 48)
