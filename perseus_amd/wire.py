"""The reference's versioned wire format (crates/pc-client/src/wire.rs), host side: the key bundle ("PCKB": a JSON
header, then each entry's payload of little-endian u32 words followed by its sum64 checksum) and the ciphertext frame
("PCCT": a JSON header, the words, their checksum), so that keys and ciphertexts a reference client produced load into
this engine, and the engine's results go back in the same frames.

Built: every bundle entry (read, written, checksummed; switching keys unpacked from their bit-packed b rows and loaded
into a key group), the ciphertext frame's full form and its regenerable seeded form (c1 rows drawn by the "CTSA"
expander, crates/pc-core/src/keys.rs:580-630, restated here with numpy's uint32 arithmetic). Not built: the seeded
form drawn by the DRBG (`seeded` without `regen`), the compressed forms (`bits`, `bits1`, `sub1`, `drop`): reading
such a frame raises WireError.
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
        raise WireError(f"version {ver}; this build reads version {VERSION}")
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
    bundle's packing width, `a` regenerated from its seed as the reference's. The keys must be full-shape ones of the
    context's chain (q_top = nq - 1, every digit, every special prime); banded keys are refused."""
    from .engine import Keys

    h = reader.header
    n = int(h["n"])
    idx = [i for i, e in enumerate(h["entries"]) if e["kind"] == "ksk" and galois_of(e, n) is not None] \
        if entries is None else list(entries)
    gal, seeds, bs = [], [], []
    for i in idx:
        e = h["entries"][i]
        sh = e["shape"]
        if sh["q_top"] != ctx.nq - 1 or sh["nq"] != ctx.nq or sh["kp"] != ctx.kp or sh["ndig"] != ctx.dnum:
            raise WireError(f"entry {i}: a key of shape {sh} does not fit the context (nq {ctx.nq}, kp {ctx.kp}, "
                            f"dnum {ctx.dnum})")
        gal.append(galois_of(e, n))
        seeds.append(np.asarray(e["seed"], np.uint32))
        bs.append(reader.ksk_b(i))
    bits = int(h["bits"])
    return Keys(ctx, gal, seeds=np.stack(seeds), b=bs, bits=0 if bits >= 32 else bits), idx


# ----------------------------------------------------------------------------------------------- ciphertext frame

_CTS_TAG, _CTS_T_MAX = 0x43545341, 32
_SIGMA = (0x61707865, 0x3320646E, 0x79622D32, 0x6B206574)


def _rotl(x, r):
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def _chacha12(seed, ctr, w13, w14, w15):
    """ChaCha12 blocks of an 8-word key, vector of counters (RFC 8439's block function at 12 rounds, with the
    reference's nonce words: w13, w14, w15), as [len(ctr)][16] u32"""
    ctr = np.asarray(ctr, np.uint32)
    st = [np.full(len(ctr), v, np.uint32) for v in _SIGMA] + [np.full(len(ctr), int(k), np.uint32) for k in seed] + \
         [ctr, np.full(len(ctr), w13, np.uint32), np.full(len(ctr), w14, np.uint32), np.full(len(ctr), w15, np.uint32)]
    x = [s.copy() for s in st]

    def qr(a, b, c, d):
        x[a] += x[b]; x[d] = _rotl(x[d] ^ x[a], 16)  # noqa: E702
        x[c] += x[d]; x[b] = _rotl(x[b] ^ x[c], 12)  # noqa: E702
        x[a] += x[b]; x[d] = _rotl(x[d] ^ x[a], 8)  # noqa: E702
        x[c] += x[d]; x[b] = _rotl(x[b] ^ x[c], 7)  # noqa: E702

    with np.errstate(over="ignore"):
        for _ in range(6):
            qr(0, 4, 8, 12), qr(1, 5, 9, 13), qr(2, 6, 10, 14), qr(3, 7, 11, 15)
            qr(0, 5, 10, 15), qr(1, 6, 11, 12), qr(2, 7, 8, 13), qr(3, 4, 9, 14)
        return np.stack([x[i] + st[i] for i in range(16)], axis=1)


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


def ct_words(h):
    """the frame's words (wire.rs:644-655)"""
    k, n, rows = int(h["k"]), int(h["n"]), int(h["rows"])
    if h.get("drop") is not None or h.get("bits") is not None:
        raise WireError("compressed ciphertext frames are not read by this build")
    if h.get("seeded"):
        return k * rows * (n + 8)
    return k * 2 * rows * n


def check_ct_header(h):
    """sizes in range and a flag combination this build reads (wire.rs:620-642, restricted to its frames)"""
    n, k, rows = int(h["n"]), int(h["k"]), int(h["rows"])
    if n == 0 or k == 0 or rows == 0 or n > 1 << 17 or n & (n - 1) or k > 64 or rows > 128:
        raise WireError(f"ciphertext header out of range: {h}")
    if h.get("regen") and not h.get("seeded"):
        raise WireError(f"regen frame without seeds: {h}")
    if h.get("seeded") and not h.get("regen"):
        raise WireError("a seeded frame drawn by the DRBG is not read by this build (regenerable frames are)")
    for f in ("bits", "bits1", "sub1", "drop"):
        if h.get(f) is not None:
            raise WireError(f"compressed ciphertext frames ({f}) are not read by this build")


def write_ct(f, header, data):
    """a ciphertext frame: header dict (params_hash, n, k, rows, meta {level, deg, nf, slots, tag}[, seeded, regen]),
    words (wire.rs:661-668)"""
    check_ct_header(header)
    d = np.ascontiguousarray(data, np.uint32).reshape(-1)
    if len(d) != ct_words(header):
        raise WireError(f"ciphertext data has {len(d)} words, the header needs {ct_words(header)}")
    _write_header(f, CT_MAGIC, header)
    f.write(d.astype("<u4").tobytes() + struct.pack("<Q", sum64(d)))


def read_ct(f):
    """(header, words) of a frame, its checksum verified (wire.rs:678-688)"""
    h, _ = _read_header(f, CT_MAGIC)
    check_ct_header(h)
    d = _read_words(f, ct_words(h))
    (c,) = struct.unpack("<Q", f.read(8))
    if c != sum64(d):
        raise WireError("ciphertext checksum mismatch")
    return h, d


def expand_ct(h, data, primes):
    """a frame's ciphertexts as [k][2][rows][n] eval-form words: full frames as they are; regenerable seeded frames
    with c1 row r drawn from its seed at q_r (wire.rs:690-729)"""
    k, n, rows = int(h["k"]), int(h["n"]), int(h["rows"])
    if not h.get("seeded"):
        return np.asarray(data, np.uint32).reshape(k, 2, rows, n)
    per = rows * (n + 8)
    out = np.zeros((k, 2, rows, n), np.uint32)
    for c in range(k):
        src = np.asarray(data[c * per:(c + 1) * per], np.uint32)
        out[c, 0] = src[: rows * n].reshape(rows, n)
        seeds = src[rows * n:].reshape(rows, 8)
        for r in range(rows):
            out[c, 1, r] = cts_expand_row(seeds[r], int(primes[r]), n)
    return out
