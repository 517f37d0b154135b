"""The reference's versioned wire format (crates/pc-client/src/wire.rs), host side: the key bundle ("PCKB": a JSON
header, then each entry's payload of little-endian u32 words followed by its sum64 checksum) and the ciphertext frame
("PCCT": a JSON header, the words, their checksum), so that keys and ciphertexts a reference client produced load into
this engine, and the engine's results go back in the same frames.

Key bundles: every entry read, written and checksummed; switching keys unpacked from their bit-packed b rows and loaded
into a key group. Ciphertext frames, every form CtHeader defines (wire.rs:265-308): full evaluation-form frames; seeded
frames with c1 drawn by the DRBG (keys.rs:142-208 fill_below) or by the random-access "CTSA" expander
(keys.rs:580-630); short-c0 frames (drop: c0 in coefficient form, rounded to its top bits); a subring client's
coefficient-form frames, lifted into the ring; compressed frames (bits, bits1, sub1: round(x 2^bits / Q) per
coefficient), which the engine writes for a client to decrypt and refuses to import. The arithmetic is restated here
with numpy and Python integers; import_ct and export_ct move the words through the engine, forward or inverse NTT on
the device.
"""
import io
import json
import struct

import numpy as np

VERSION = 1
BUNDLE_MAGIC = b"PCKB"
CT_MAGIC = b"PCCT"
_FNV_OFF, _FNV_PRIME = 0xCBF29CE484222325, 0x100000001B3
_M64 = (1 << 64) - 1


class WireError(ValueError):
    pass


def sum64(words):
    """FNV-1a over little-endian u64 words, a trailing odd u32 word widened (wire.rs:12-25)."""
    w = np.ascontiguousarray(words, np.uint32)
    h = _FNV_OFF
    pairs = w[: len(w) // 2 * 2].view(np.uint64) if len(w) >= 2 else np.zeros(0, np.uint64)
    for v in pairs.tolist():
        h = ((h ^ v) * _FNV_PRIME) & _M64
    if len(w) % 2:
        h = ((h ^ int(w[-1])) * _FNV_PRIME) & _M64
    return h


def packed_row_words(n, bits):
    """u32 words of one packed row of n values at `bits`: + one zero guard word, padded to 16 bytes (wire.rs:126-130)."""
    return -(-(n * bits // 32 + 1) // 4) * 4


def pack_row(vals, bits, words=None):
    """value i at bits [i bits, (i + 1) bits) of a little-endian u32 stream (wire.rs:137-150)."""
    v = np.asarray(vals, np.uint64) & np.uint64((1 << bits) - 1)
    n = len(v)
    words = words or packed_row_words(n, bits)
    out = np.zeros(words + 1, np.uint64)
    bit = np.arange(n, dtype=np.uint64) * np.uint64(bits)
    w, off = (bit >> np.uint64(5)).astype(np.int64), bit & np.uint64(31)
    x = v << off
    np.bitwise_or.at(out, w, x & np.uint64(0xFFFFFFFF))
    np.bitwise_or.at(out, w + 1, x >> np.uint64(32))
    return out[:words].astype(np.uint32)


def unpack_row(packed, bits, n):
    """inverse of pack_row (wire.rs:152-161)"""
    p = np.concatenate([np.asarray(packed, np.uint64), np.zeros(1, np.uint64)])
    bit = np.arange(n, dtype=np.uint64) * np.uint64(bits)
    w, off = (bit >> np.uint64(5)).astype(np.int64), bit & np.uint64(31)
    lo = p[w] | (p[w + 1] << np.uint64(32))
    return ((lo >> off) & np.uint64((1 << bits) - 1)).astype(np.uint32)


def _write_header(f, magic, header):
    h = json.dumps(header, separators=(",", ":")).encode()
    f.write(magic + struct.pack("<IQ", VERSION, len(h)) + h)
    return 16 + len(h)


def _read_header(f, magic):
    m = f.read(4)
    if m != magic:
        raise WireError(f"magic {m!r}, expected {magic!r}")
    ver, ln = struct.unpack("<IQ", f.read(12))
    if ver != VERSION:
        raise WireError(f"version {ver}; this library reads version {VERSION}")
    if ln > 1 << 30:
        raise WireError(f"header of {ln} bytes")
    h = f.read(ln)
    if len(h) != ln:
        raise WireError("truncated header")
    return json.loads(h), 16 + ln


def _read_words(f, n):
    b = f.read(4 * n)
    if len(b) != 4 * n:
        raise WireError("truncated payload")
    return np.frombuffer(b, "<u4").astype(np.uint32)


# ----------------------------------------------------------------------------------------------- key bundle


def ksk_rows(shape):
    """rows of a key of KeyShape {q_top, ndig, nq, kp}: Q ids 0..q_top then the kp special ids (spec.rs:63-68)"""
    return shape["q_top"] + 1 + shape["kp"]


class BundleWriter:
    """The header (dict: chain, params_hash, contract, n, bits, row_words, entries), then put() each entry's words in
    header order (wire.rs:163-198)."""

    def __init__(self, f, header):
        self.f, self.header, self.next = f, header, 0
        self.bytes = _write_header(f, BUNDLE_MAGIC, header)

    def put(self, words):
        es = self.header["entries"]
        if self.next >= len(es):
            raise WireError(f"entry {self.next} is past the header's {len(es)}")
        w = np.ascontiguousarray(words, np.uint32).reshape(-1)
        if es[self.next]["words"] != len(w):
            raise WireError(f"entry {self.next} declares {es[self.next]['words']} words, got {len(w)}")
        self.f.write(w.astype("<u4").tobytes() + struct.pack("<Q", sum64(w)))
        self.bytes += 4 * len(w) + 8
        self.next += 1

    def finish(self):
        if self.next != len(self.header["entries"]):
            raise WireError(f"bundle closed after {self.next} of {len(self.header['entries'])} entries")
        self.f.flush()
        return self.bytes


class BundleReader:
    """The header at open, any entry's payload on demand, its checksum verified (wire.rs:200-248)."""

    def __init__(self, f):
        self.f = f
        self.header, off = _read_header(f, BUNDLE_MAGIC)
        self.offsets = []
        for e in self.header["entries"]:
            self.offsets.append(off)
            off += 4 * int(e["words"]) + 8
        f.seek(0, io.SEEK_END)
        end = f.tell()
        if end != off:
            raise WireError(f"bundle is {end} bytes, its header describes {off}")

    def read(self, i):
        e = self.header["entries"][i]
        self.f.seek(self.offsets[i])
        w = _read_words(self.f, int(e["words"]))
        (c,) = struct.unpack("<Q", self.f.read(8))
        if c != sum64(w):
            raise WireError(f"entry {i} ({e['kind']}): checksum mismatch")
        return w

    def ksk_b(self, i):
        """a switching key's b as dense rows [ndig][rows][n] (its packed rows unpacked at the bundle's bits)"""
        e, h = self.header["entries"][i], self.header
        if e["kind"] != "ksk":
            raise WireError(f"entry {i} is a {e['kind']}, not a switching key")
        sh, n, bits, rw = e["shape"], int(h["n"]), int(h["bits"]), int(h["row_words"])
        rows = ksk_rows(sh)
        w = self.read(i).reshape(sh["ndig"], rows, rw)
        return np.stack([np.stack([unpack_row(w[d, r], bits, n) for r in range(rows)]) for d in range(sh["ndig"])])


def galois_of(entry, n):
    """the automorphism of a switching-key entry (spec.rs:117-124): rotations and `auto` keys carry it, conjugation
    is 2N - 1; None for the relinearization and the secret switches"""
    role = entry["role"]
    if role in ("rot", "auto", "sparse_rot"):
        return int(entry["galois"])
    if role == "conj":
        return 2 * n - 1
    return None


def ksk_entry(role, shape, seed, row_words, **fields):
    """a switching-key entry of the header: role fields flattened beside the shape (spec.rs:131-137)"""
    e = {"kind": "ksk", "role": role, **fields, "shape": dict(shape), "seed": [int(x) for x in seed]}
    e["words"] = shape["ndig"] * ksk_rows(shape) * row_words
    return e


def pack_ksk(b, bits, row_words):
    """dense b [ndig][rows][n] -> the entry's packed words [ndig][rows][row_words]"""
    return np.stack([np.stack([pack_row(r, bits, row_words) for r in d]) for d in np.asarray(b)])


def load_keys(reader, ctx, entries=None):
    """Rotation / automorphism keys of a bundle as one engine key group: each entry's b unpacked and stored at the
    bundle's packing width, `a` regenerated from its seed as the reference's. The entries must share one shape over
    the context's chain: full (q_top = nq - 1, every digit) or banded at one q_top (crates/pc-gpu/src/keys.rs:81-103
    KskShape::banded: the digits whose first prime id is <= q_top, Q rows 0..=q_top, then the special rows); a
    banded key over fewer special primes than the chain's (a LowP tier) is refused, as is a mix of bands (load each
    band's entries as its own group)."""
    from .engine import Keys, band_digits

    h = reader.header
    n = int(h["n"])
    idx = [i for i, e in enumerate(h["entries"]) if e["kind"] == "ksk" and galois_of(e, n) is not None] \
        if entries is None else list(entries)
    gal, seeds, bs, tops = [], [], [], set()
    for i in idx:
        e = h["entries"][i]
        sh = e["shape"]
        qt = int(sh["q_top"])
        if sh["nq"] != ctx.nq or sh["kp"] != ctx.kp or not 0 <= qt < ctx.nq or sh["ndig"] != band_digits(ctx, qt):
            raise WireError(f"entry {i}: a key of shape {sh} does not fit the context (nq {ctx.nq}, kp {ctx.kp}, "
                            f"dnum {ctx.dnum}; a band at q_top {qt} holds {band_digits(ctx, min(max(qt, 0), ctx.nq - 1))}"
                            f" digits)")
        tops.add(qt)
        gal.append(galois_of(e, n))
        seeds.append(np.asarray(e["seed"], np.uint32))
        bs.append(reader.ksk_b(i))
    if len(tops) > 1:
        raise WireError(f"entries of several bands {sorted(tops)}: load each band as its own group")
    bits = int(h["bits"])
    qt = tops.pop() if tops else ctx.nq - 1
    return Keys(ctx, gal, seeds=np.stack(seeds), b=bs, bits=0 if bits >= 32 else bits,
                q_top=None if qt == ctx.nq - 1 else qt), idx


# ----------------------------------------------------------------------------------------------- ciphertext frame

_CTS_TAG, _CTS_T_MAX = 0x43545341, 32
_SIGMA = (0x61707865, 0x3320646E, 0x79622D32, 0x6B206574)


def _rotl(x, r):
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def _chacha(seed, w12, w13, w14, w15, rounds=12):
    """ChaCha blocks of an 8-word key (RFC 8439's block function at `rounds` rounds) for vectors of the state words
    12 and 13 (broadcast against each other) and the constant words 14, 15, as [blocks][16] u32"""
    w12, w13 = np.broadcast_arrays(np.asarray(w12, np.uint32), np.asarray(w13, np.uint32))
    nb = w12.size
    st = [np.full(nb, v, np.uint32) for v in _SIGMA] + [np.full(nb, int(k), np.uint32) for k in seed] + \
         [w12.reshape(-1).copy(), w13.reshape(-1).copy(), np.full(nb, w14, np.uint32), np.full(nb, w15, np.uint32)]
    x = [v.copy() for v in st]

    def qr(a, b, c, d):
        x[a] += x[b]; x[d] = _rotl(x[d] ^ x[a], 16)  # noqa: E702
        x[c] += x[d]; x[b] = _rotl(x[b] ^ x[c], 12)  # noqa: E702
        x[a] += x[b]; x[d] = _rotl(x[d] ^ x[a], 8)  # noqa: E702
        x[c] += x[d]; x[b] = _rotl(x[b] ^ x[c], 7)  # noqa: E702

    with np.errstate(over="ignore"):
        for _ in range(rounds // 2):
            qr(0, 4, 8, 12), qr(1, 5, 9, 13), qr(2, 6, 10, 14), qr(3, 7, 11, 15)
            qr(0, 5, 10, 15), qr(1, 6, 11, 12), qr(2, 7, 8, 13), qr(3, 4, 9, 14)
        return np.stack([x[i] + st[i] for i in range(16)], axis=1)


def _chacha12(seed, ctr, w13, w14, w15):
    return _chacha(seed, ctr, w13, w14, w15, 12)


def cts_expand_row(seed, p, n):
    """a regenerable ciphertext's c1 row (keys.rs:606-630): slot s is word s & 15 of block s >> 4 of
    (seed, w13 = 0, p, "CTSA"); a word at or above floor((2^32 - 1) / p) p is redrawn from block s >> 4 + t n / 16
    (t < 32, the last draw kept); value mod p"""
    n16, mp = n >> 4, (0xFFFFFFFF // p) * p
    v = _chacha12(seed, np.arange(n16), 0, p, _CTS_TAG).reshape(-1).astype(np.uint64)
    bad = np.nonzero(v >= mp)[0]
    for s in bad.tolist():
        b0, w = s >> 4, s & 15
        for t in range(1, _CTS_T_MAX):
            x = int(_chacha12(seed, [(b0 + t * n16) & 0xFFFFFFFF], 0, p, _CTS_TAG)[0, w])
            v[s] = x
            if x < mp:
                break
    return (v % np.uint64(p)).astype(np.uint32)


# ----------------------------------------------------------------------------------------------- ciphertext frame
# CtHeader (wire.rs:265-308): params_hash, n, k, rows, meta, then the optional fields, each written only when set (the
# serde skip rules), in this order.
_OPT = ("bits", "seeded", "regen", "bits1", "sparse", "drop", "coeff0", "coeff1", "sub1")
_DRBG_TAG = 0x47425244  # "DRBG" (keys.rs:116-118)


def ct_header(params_hash, n, k, rows, meta, **flags):
    """a frame header with the reference's field order; flags: bits, seeded, regen, bits1, sparse, drop, coeff0,
    coeff1, sub1 (unset / False ones omitted)"""
    bad = set(flags) - set(_OPT)
    if bad:
        raise WireError(f"unknown header fields {sorted(bad)}")
    h = {"params_hash": params_hash, "n": int(n), "k": int(k), "rows": int(rows), "meta": dict(meta)}
    for f in _OPT:
        v = flags.get(f)
        if v is None or v is False:
            continue
        h[f] = bool(v) if isinstance(v, bool) else int(v)
    return h


def _opt(h, f):
    return h.get(f)


def _pow2(x):
    return x > 0 and x & (x - 1) == 0


def check_ct_header(h):
    """CtHeader::check (wire.rs:620-642): sizes in range and the flags in a combination the readers agree on"""
    n, k, rows = int(h["n"]), int(h["k"]), int(h["rows"])
    bits, bits1, sub1, drop = _opt(h, "bits"), _opt(h, "bits1"), _opt(h, "sub1"), _opt(h, "drop")
    seeded, regen = bool(h.get("seeded")), bool(h.get("regen"))
    if n == 0 or k == 0 or rows == 0 or n > 1 << 17 or not _pow2(n) or k > 64 or rows > 128:
        raise WireError(f"ciphertext header out of range: {h}")
    if (sub1 is not None and (sub1 < 2 or not _pow2(sub1) or n % sub1 != 0)) or (sub1 is not None and bits is None):
        raise WireError(f"packed frame header out of range: {h}")
    if drop is not None:
        if not (seeded and not regen and bits is not None and 1 <= bits <= 126 and bits1 is None and rows <= 4):
            raise WireError(f"short-c0 frame header out of range: {h}")
    elif (bits is not None and seeded) or any(not 1 <= b <= 64 for b in (bits, bits1) if b is not None) or \
            (bits1 is not None and bits is None):
        raise WireError(f"compressed frame header out of range: {h}")
    if regen and not seeded:
        raise WireError(f"regen frame without seeds: {h}")


def packed_words(n, bits):
    """words of n values of `bits` bits, bit-packed (wire.rs:402-405)"""
    return -(-(n * bits) // 32)


def ct_words(h):
    """CtWire::words (wire.rs:644-655)"""
    k, n, rows = int(h["k"]), int(h["n"]), int(h["rows"])
    if h.get("drop") is not None:
        return k * (packed_words(n, int(h["bits"])) + rows * 8)
    if h.get("bits") is not None:
        b0 = int(h["bits"])
        b1 = int(h["bits1"]) if h.get("bits1") is not None else b0
        return k * (packed_words(n, b0) + packed_words(n // max(int(h.get("sub1") or 1), 1), b1))
    if h.get("seeded"):
        return k * rows * (n + 8)
    return k * 2 * rows * n


def pack_bits(v, bits):
    """values of `bits` bits (<= 64, or wider Python integers), LSB first, into packed_words(len, bits) u32 words
    (wire.rs:407-436: pack_bits; pack_dropped's running word for wider values)"""
    n = len(v)
    if bits <= 64:
        x = np.asarray([int(a) for a in v] if not isinstance(v, np.ndarray) else v, np.uint64)
        mask = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(_M64)
        x = x & mask
        out = np.zeros(packed_words(n, bits) + 3, np.uint64)
        bit = np.arange(n, dtype=np.uint64) * np.uint64(bits)
        w, off = (bit >> np.uint64(5)).astype(np.int64), bit & np.uint64(31)
        lo = x << off
        np.bitwise_or.at(out, w, lo & np.uint64(0xFFFFFFFF))
        np.bitwise_or.at(out, w + 1, (lo >> np.uint64(32)) & np.uint64(0xFFFFFFFF))
        # bits shifted past the 64-bit word: x >> (64 - off) when off > 0
        hi = np.where(off > 0, x >> (np.uint64(64) - np.where(off > 0, off, np.uint64(1))), np.uint64(0))
        np.bitwise_or.at(out, w + 2, hi)
        return out[: packed_words(n, bits)].astype(np.uint32)
    acc = 0
    for i, a in enumerate(v):
        acc |= (int(a) & ((1 << bits) - 1)) << (i * bits)
    nw = packed_words(n, bits)
    return np.frombuffer(acc.to_bytes(4 * nw, "little"), "<u4").astype(np.uint32)


def unpack_bits(w, n, bits):
    """pack_bits' inverse: n values (wire.rs:543-563); numpy uint64 for bits <= 64, Python integers above"""
    w = np.asarray(w, np.uint32)
    if bits <= 64:
        p = np.concatenate([w.astype(np.uint64), np.zeros(3, np.uint64)])
        bit = np.arange(n, dtype=np.uint64) * np.uint64(bits)
        k, off = (bit >> np.uint64(5)).astype(np.int64), bit & np.uint64(31)
        lo = (p[k] | (p[k + 1] << np.uint64(32))) >> off
        hi = np.where(off > 0, p[k + 2] << (np.uint64(64) - np.where(off > 0, off, np.uint64(1))), np.uint64(0))
        mask = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(_M64)
        return (lo | hi) & mask
    acc = int.from_bytes(w.astype("<u4").tobytes(), "little")
    m = (1 << bits) - 1
    return [(acc >> (i * bits)) & m for i in range(n)]


def _crt(q, rows):
    """x in [0, Q) of residue rows (values may be unreduced), Python integers"""
    big = 1
    for p in q:
        big *= int(p)
    acc = np.zeros(len(rows[0]), dtype=object)
    for p, r in zip(q, rows):
        p = int(p)
        m = big // p
        acc = (acc + (np.asarray(r, np.uint64).astype(object) % p) * (m * pow(m % p, -1, p))) % big
    return acc, big


def pack_coeffs(q, rows, bits):
    """one `bits`-bit word (<= 64) per coefficient: round(x 2^bits / Q) mod 2^bits, x the CRT of the residues in
    [0, Q) (wire.rs:357-395). Two primes with Q < 2^63 and bits <= 32: the reference's rounding through an f64 product,
    floor(z) + (z - floor(z) >= 1/2) with z = x * (2^bits / Q) in double; otherwise the exact rounding."""
    nbits = sum(int(p).bit_length() for p in q)
    if bits == 0 or bits > 64 or nbits + bits > 127:
        raise WireError(f"pack_coeffs: {bits} bits over a {len(q)}-prime modulus")
    x, big = _crt(q, rows)
    mask = (1 << bits) - 1
    if len(q) == 2 and big < 1 << 63 and bits <= 32:
        scale = float(1 << bits) / float(big)
        z = np.array([float(int(v)) for v in x]) * scale
        f = np.floor(z)
        return ((f.astype(np.int64) + (z - f >= 0.5)).astype(np.uint64) & np.uint64(mask))
    return np.array([(((int(v) << bits) + big // 2) // big) & mask for v in x], np.uint64)


def unpack_coeffs(q, words, bits):
    """pack_coeffs' inverse up to its rounding: the residues mod each q of round(y Q / 2^bits) (wire.rs:397-400)"""
    big = 1
    for p in q:
        big *= int(p)
    xs = [((int(y) * big) + (1 << (bits - 1))) >> bits for y in words]
    return np.stack([np.array([x % big % int(p) for x in xs], np.uint64) for p in q])


def pack_frame_part(q, rows, bits):
    """a compressed frame's part: pack_bits(pack_coeffs(q, rows, bits), bits) (wire.rs:466-489)"""
    if len(rows) != len(q):
        raise WireError(f"pack_frame_part: {len(rows)} rows over a {len(q)}-prime modulus")
    return pack_bits(pack_coeffs(q, rows, bits), bits)


def dropped_bits(q, drop):
    """bits of a coefficient without its low `drop` bits over the primes q (up to 4 primes below 2^30): those of the
    largest (x + 2^(drop - 1)) >> drop, x < Q (wire.rs:491-499)"""
    big = 1
    for p in q:
        big *= int(p)
    if not q or len(q) > 4 or any(int(p) >> 30 for p in q) or drop >= big.bit_length():
        raise WireError(f"{drop} bits dropped over a {len(q)}-prime modulus")
    return max(1, ((big - 1 + ((1 << drop) >> 1)) >> drop).bit_length())


def pack_dropped(q, rows, drop):
    """coefficient-form residue rows as a short-c0 frame's words: x (the CRT value in [0, Q)) rounded to its top bits,
    (x + 2^(drop - 1)) >> drop, dropped_bits bits each (wire.rs:501-541); returns (words, bits)"""
    bits = dropped_bits(q, drop)
    x, _ = _crt(q, rows)
    half = (1 << drop) >> 1
    return pack_bits([(int(v) + half) >> drop for v in x], bits), bits


def unpack_dropped(q, words, drop, n):
    """pack_dropped's inverse up to its rounding: rows [len(q)][n] of the residues of y 2^drop (wire.rs:543-574)"""
    bits = dropped_bits(q, drop)
    ys = unpack_bits(words, n, bits)
    return np.stack([np.array([(int(y) << drop) % int(p) for y in ys], np.uint64).astype(np.uint32) for p in q])


def drbg_row(seed, q, n):
    """n values uniform below q drawn as Prng::from_seed(seed, 0).fill_below(q) draws them (keys.rs:166-208: the
    ChaCha20 "DRBG" stream with the block counter in words 12..13, stream 0 in word 14; little-endian pairs of words as
    64-bit candidates, those below 2^64 mod q rejected, the rest reduced mod q)"""
    q = int(q)
    rem = (1 << 64) % q
    out = []
    ctr = 0
    while len(out) < n:
        nb = max(1, -(-(n - len(out)) // 8) + 1)
        c = np.arange(ctr, ctr + nb, dtype=np.uint64)
        blk = _chacha(seed, (c & np.uint64(0xFFFFFFFF)).astype(np.uint32), (c >> np.uint64(32)).astype(np.uint32), 0,
                      _DRBG_TAG, 20).astype(np.uint64)
        v = (blk[:, 0::2] | (blk[:, 1::2] << np.uint64(32))).reshape(-1)
        ok = v[v >= np.uint64(rem)] if rem else v
        out.extend((ok % np.uint64(q)).tolist())
        ctr += nb
    # the stream is consumed in order: the first n accepted candidates
    return np.array(out[:n], np.uint64).astype(np.uint32 if q <= 1 << 32 else np.uint64)


def write_ct(f, header, data):
    """a ciphertext frame: header (ct_header), words (wire.rs:661-668)"""
    check_ct_header(header)
    d = np.ascontiguousarray(data, np.uint32).reshape(-1)
    if len(d) != ct_words(header):
        raise WireError(f"ciphertext data has {len(d)} words, the header needs {ct_words(header)}")
    _write_header(f, CT_MAGIC, header)
    f.write(d.astype("<u4").tobytes() + struct.pack("<Q", sum64(d)))


def read_ct(f):
    """(header, words) of a frame, its header checked and its checksum verified (wire.rs:678-688)"""
    h, _ = _read_header(f, CT_MAGIC)
    check_ct_header(h)
    d = _read_words(f, ct_words(h))
    (c,) = struct.unpack("<Q", f.read(8))
    if c != sum64(d):
        raise WireError("ciphertext checksum mismatch")
    return h, d


def expand_seeded(h, data, primes):
    """a seeded frame as a full one (wire.rs:690-732): c1's rows drawn from their seeds (regen: the "CTSA" expander;
    else the DRBG's fill_below), a short c0 unpacked into coefficient form (flagged coeff0). Other frames as they are.
    Returns (header, words)."""
    if not h.get("seeded"):
        return dict(h), np.asarray(data, np.uint32)
    k, n, rows = int(h["k"]), int(h["n"]), int(h["rows"])
    if len(primes) < rows:
        raise WireError(f"seeded frame of {rows} rows, {len(primes)} primes")
    q = [int(p) for p in primes[:rows]]
    short = None
    if h.get("drop") is not None:
        d, b = int(h["drop"]), h.get("bits")
        if b is None or dropped_bits(q, d) != int(b):
            raise WireError(f"short-c0 frame of {b} bits, {d} dropped over {rows} rows")
        short = (d, packed_words(n, int(b)))
    per = (short[1] if short else rows * n) + rows * 8
    out = np.zeros((k, 2, rows, n), np.uint32)
    data = np.asarray(data, np.uint32)
    for c in range(k):
        src = data[c * per:(c + 1) * per]
        c0, seeds = src[: per - rows * 8], src[per - rows * 8:].reshape(rows, 8)
        out[c, 0] = unpack_dropped(q, c0, short[0], n) if short else c0.reshape(rows, n)
        for r in range(rows):
            out[c, 1, r] = cts_expand_row(seeds[r], q[r], n) if h.get("regen") else drbg_row(seeds[r], q[r], n)
    nh = {f: v for f, v in h.items() if f not in ("seeded", "regen", "drop")}
    if short:
        nh.pop("bits", None)
        nh["coeff0"] = True
    return nh, out.reshape(-1)


def lifted(h, data, n):
    """a subring frame (both parts coefficient form over h.n | n coefficients) in the ring of n coefficients:
    coefficient i at i n / h.n (X -> X^(n / h.n)), every slot live (wire.rs:733-752)"""
    if h.get("seeded") or h.get("bits") is not None or not (h.get("coeff0") and h.get("coeff1")):
        raise WireError("lifted: an expanded frame with both parts in coefficient form (a subring client's)")
    hn = int(h["n"])
    if hn == 0 or n % hn or not _pow2(n // hn):
        raise WireError(f"lifted: a frame of {hn} coefficients into a ring of {n}")
    k = n // hn
    d = np.asarray(data, np.uint32).reshape(-1, hn)
    out = np.zeros((d.shape[0], n), np.uint32)
    out[:, ::k] = d
    nh = dict(h)
    nh["n"] = n
    nh["meta"] = dict(h["meta"], slots=n // 2)
    return nh, out.reshape(-1)


def expand_ct(h, data, primes, sparse_ok=False):
    """a frame's ciphertexts as [k][2][rows][n] evaluation-form words: full frames as they are, seeded ones with c1
    drawn from the seeds. Frames whose parts arrive in coefficient form (a short c0, a subring client's) need the
    forward transform (import_ct runs it on the device) and are refused here, as are compressed frames (a client's to
    decrypt) and, unless sparse_ok, frames under the client's sparse secret."""
    if h.get("bits") is not None and h.get("drop") is None:
        raise WireError("a compressed frame (bits) is for a client to decrypt")
    if h.get("sparse") and not sparse_ok:
        raise WireError("the frame is encrypted under the client's sparse secret (sparse): pass sparse_ok")
    nh, d = expand_seeded(h, data, primes)
    if nh.get("coeff0") or nh.get("coeff1"):
        raise WireError("the frame's parts are in coefficient form (coeff0 / coeff1): import it with import_ct")
    return d.reshape(int(nh["k"]), 2, int(nh["rows"]), int(nh["n"]))


def expand_frame(frame, primes, n=None):
    """A seeded frame with its c1 rows drawn from the seeds (and a short c0 unpacked: coeff0), a subring client's frame
    spread over the ring of n coefficients when n is given; returns the new frame's bytes, which import_ct reads
    (crates/pc-py/src/client.rs:963-975 expand_frame)."""
    h, data = read_ct(io.BytesIO(frame) if isinstance(frame, (bytes, bytearray)) else frame)
    h, data = expand_seeded(h, data, primes)
    if n is not None and int(h["n"]) != n and h.get("coeff1"):
        h, data = lifted(h, data, n)
    f = io.BytesIO()
    write_ct(f, h, data)
    return f.getvalue()


# ----------------------------------------------------------------------------------------------- engine import / export
def import_ct(ctx, frame, stream):
    """A ciphertext frame into the engine (the server side of crates/pc-py/src/client.rs:861-955 import_ct): frames
    carrying `bits` are refused (compressed ones are a client's to decrypt; a short-c0 frame goes through expand_frame
    first), except a subring client's; seeded frames are expanded on the host (c1 from the seeds); a subring client's
    frame is lifted into the context's ring; the words go up, and the parts in coefficient form (coeff0, coeff1) take
    the forward NTT on the device. Returns (DevBuf of k ciphertexts in the context's layout
    [k][2][rows][N], rows 0..h.rows - 1 filled, the frame's header: `sparse` tells which secret it is under)."""
    from .engine import DevBuf, Rows

    h, data = read_ct(io.BytesIO(frame) if isinstance(frame, (bytes, bytearray)) else frame)
    if h.get("bits") is not None and not (h.get("coeff1") and int(h["n"]) != ctx.n):
        raise WireError("import_ct: a compressed frame (export_ct bits=) is for a client to decrypt")
    h, data = expand_seeded(h, data, ctx.chain.q)
    if int(h["n"]) != ctx.n and h.get("coeff1"):
        h, data = lifted(h, data, ctx.n)
    k, n, rows = int(h["k"]), int(h["n"]), int(h["rows"])
    if n != ctx.n or rows > ctx.nq:
        raise WireError(f"import_ct: a frame of n {n}, {rows} rows; the context runs n {ctx.n}, {ctx.nq} Q rows")
    words = np.asarray(data, np.uint32).reshape(k, 2, rows, n)
    full = np.zeros((k, 2, ctx.rows, n), np.uint32)
    full[:, :, :rows] = words
    buf = DevBuf.from_array(full, stream)
    parts = [p for p, f in enumerate(("coeff0", "coeff1")) if h.get(f)]
    if parts:
        ids = [r for _ in range(k) for _ in parts for r in range(rows)]
        offs = [(c * 2 + p) * ctx.rows + r for c in range(k) for p in parts for r in range(rows)]
        Rows(ctx, offs, ids).ntt(buf, 1, stream)
        stream.sync()
    return buf, h


def export_ct(ctx, buf, top, meta, params_hash, stream, bits=None, k=1):
    """k ciphertexts of the context's layout as a frame (the server side of client.rs:575-640 export_ct): rows
    0..top of both parts in evaluation form, or, with `bits`, compressed: both parts through the inverse NTT on the
    device (a copy; buf is unchanged), each coefficient's CRT over q_0..q_top rounded to `bits` bits
    (pack_frame_part). Returns the frame's bytes."""
    from .engine import DevBuf, Rows

    rows, n = top + 1, ctx.n
    src = buf.download((k, 2, ctx.rows, n), stream)[:, :, :rows]
    if bits is None:
        h = ct_header(params_hash, n, k, rows, meta)
        data = src
    else:
        tmp = DevBuf.from_array(np.ascontiguousarray(src), stream)
        ids = [r for _ in range(2 * k) for r in range(rows)]
        Rows(ctx, list(range(2 * k * rows)), ids).ntt(tmp, -1, stream)
        coef = tmp.download((k, 2, rows, n), stream)
        q = ctx.chain.q[:rows]
        data = np.concatenate([pack_frame_part(q, coef[c, part], bits) for c in range(k) for part in range(2)])
        h = ct_header(params_hash, n, k, rows, meta, bits=bits)
    f = io.BytesIO()
    write_ct(f, h, data)
    return f.getvalue()
