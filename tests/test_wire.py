"""The wire format (perseus_amd/wire.py) on the CPU: the bit packing against Python integers, the checksum's definition,
bundles and ciphertext frames written and read back (entries in order, sizes, checksums, corruption, magic and version
refused), the regenerable frame's c1 rows against the oracle's "CTSA" expander (pinned in tests/test_oracle.py).
"""
import io

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
    with pytest.raises(wire.WireError, match="DRBG"):
        wire.write_ct(io.BytesIO(), dict(h, seeded=True), body)
    with pytest.raises(wire.WireError, match="compressed"):
        wire.write_ct(io.BytesIO(), dict(h, bits=40), body)
