"""Parity of two key-switch dot modes with the oracle, word for word, through the kernel table's C-ABI:
- ks_dot_key with KS_SUM: the R rotations of a key group summed into one output, out = sum_r sigma_r(dot_r)
  (+ out with KS_ACC), each rotation's c0 term before its automorphism (crates/pc-host/src/ks.rs:226-265);
- ks_dot_regen: one key with `a` regenerated from the args' seed, no automorphism, b through the KeyTab (dense or
  packed) or dense prime-id rows, plain outputs or the fused epilogue dst = f (alpha dst + (x - conv) binv) + k + add
  (crates/pc-host/src/ks.rs:267-340).
The key products come from the oracle's ks_dot (pinned by the decryption tests); the epilogue is stated here in
Python integers. Each test prints its case before the GPU runs.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import abi
from perseus_amd._lib import LIB
from tests import twin

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    return pa.Stream()


_CTX = {}


def contexts(name):
    if name not in _CTX:
        ch = pa.preset(name)
        _CTX[name] = (ch, pa.Context(ch, k_rot=4), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum))
    return _CTX[name]


def ext_rows(ch, top):
    return list(range(top + 1)) + [len(ch.q) + j for j in range(len(ch.p))]


def dev_ptrs(bufs):
    return pa.DevBuf.from_array(np.array([b.ptr.value for b in bufs], np.uint64).view(np.uint32))


def rand_rows(ch, rng, rows=None):
    rows = range(ch.rows) if rows is None else rows
    out = np.zeros((ch.rows, ch.n), np.uint32)
    for t in rows:
        out[t] = rng.integers(0, ch.primes[t], ch.n)
    return out


def oracle_keys(oc, ch, steps, seed):
    g = twin.Prng([seed, 2, 4, 6, 8, 10, 12, 14], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
    gals = [twin.rotation_galois(r, ch.n) for r in steps]
    keys = [oc.rotation_key(g, s_eval, x) for x in gals]
    return gals, np.stack([k[0] for k in keys]), [k[1] for k in keys]


def pack(b, bits):
    """Rows of values as little-endian bit streams of `bits` bits each, a zero guard word, padded to 16 bytes."""
    n = b.shape[-1]
    words = ((n * bits) // 32 + 1 + 3) // 4 * 4
    flat = b.reshape(-1, n).astype(np.uint64)
    out = np.zeros((flat.shape[0], words + 1), np.uint64)
    pos = np.arange(n, dtype=np.uint64) * np.uint64(bits)
    w, off = (pos >> np.uint64(5)).astype(np.int64), pos & np.uint64(31)
    for r in range(flat.shape[0]):
        x = flat[r] << off
        np.bitwise_or.at(out[r], w, x & np.uint64(0xFFFFFFFF))
        np.bitwise_or.at(out[r], w + 1, x >> np.uint64(32))
    return out[:, :words].astype(np.uint32).reshape(b.shape[:-1] + (words,)), words


class Tables:
    def __init__(self, ch, ctx, rows):
        nq, kp = len(ch.q), len(ch.p)
        big_p = 1
        for x in ch.p:
            big_p *= int(x)
        pm = [big_p % int(q) for q in ch.q] + [0] * kp
        pms = [(v << 32) // int(q) for v, q in zip(pm, ch.primes)]
        self.rows = rows
        self.b_rows = pa.DevBuf.from_array(np.array(rows, np.uint32))
        self.b_dig = pa.DevBuf.from_array(np.array([t // ch.alpha if t < nq else -1 for t in range(nq + kp)],
                                                   np.int32).view(np.uint32))
        self.b_pm = pa.DevBuf.from_array(np.array(pm, np.uint32))
        self.b_pms = pa.DevBuf.from_array(np.array(pms, np.uint32))
        self.pr = LIB.pcx_ctx_primes(ctx.h)

    def fill(self, a, ch):
        a.rows, a.digit_of = self.b_rows.ptr.value, self.b_dig.ptr.value
        a.pmod, a.pmods, a.pr = self.b_pm.ptr.value, self.b_pms.ptr.value, self.pr
        a.nq, a.nrows = len(ch.q), len(self.rows)


def inputs(ch, oc, top, K, rng):
    x = np.zeros((K, 2, ch.rows, ch.n), np.uint32)
    for c in range(K):
        x[c] = rand_rows(ch, rng, range(top + 1))[None].repeat(2, 0)
        x[c, 1] = rand_rows(ch, rng, range(top + 1))
    digits = np.stack([oc.modup(x[c, 1], top) for c in range(K)])
    return x, digits


# ----------------------------------------------------------------------------------------------- KS_SUM
@pytest.mark.parametrize("mode", ["pc0", "pc0_acc", "c0ext"])
def test_ks_dot_key_sum(stream, mode):
    say(f"[ks_sum] small K=2 R=3 {mode}")
    ch, ctx, oc = contexts("small")
    rng = np.random.default_rng({"pc0": 5, "pc0_acc": 6, "c0ext": 7}[mode])
    top, K, R = 4, 2, 3
    n, RR = ch.n, ch.rows
    x, digits = inputs(ch, oc, top, K, rng)
    rows = ext_rows(ch, top)
    # c0 in the ciphertext layout (KsArgs reads c0 and c1 at one ciphertext stride): x's own c0 for the P c0 modes;
    # for c0ext words on every row of Q u P, added as they are
    c0full = x.copy()
    if mode == "c0ext":
        for c in range(K):
            c0full[c, 0] = rand_rows(ch, rng, rows)
    c0 = c0full[:, 0]
    gals, seeds, bs = oracle_keys(oc, ch, [1, 5, 3], seed=21)
    autok = [twin.galois_inverse(g, n) for g in gals]
    prev = np.stack([rand_rows(ch, rng, rows)[None].repeat(2, 0) for _ in range(K)])
    T = Tables(ch, ctx, rows)
    bx, bc0, bmu = pa.DevBuf.from_array(x), pa.DevBuf.from_array(c0full), pa.DevBuf.from_array(digits)
    bout = pa.DevBuf.from_array(prev)
    bkb = [pa.DevBuf.from_array(b) for b in bs]
    bseed = [pa.DevBuf.from_array(np.ascontiguousarray(s, np.uint32)) for s in seeds]
    pkb, pseed = dev_ptrs(bkb), dev_ptrs(bseed)
    bautok = pa.DevBuf.from_array(np.array(autok, np.uint32))
    g = abi.KsKeyArgs()
    a = g.ks
    a.c1, a.c0, a.modup = bx.ptr.value + 4 * RR * n, bc0.ptr.value, bmu.ptr.value
    a.out0, a.out1, a.autok = bout.ptr.value, bout.ptr.value + 4 * RR * n, bautok.ptr.value
    T.fill(a, ch)
    a.ct_stride = 2 * RR * n
    a.mu_ct_stride, a.mu_digit_stride, a.out_ct_stride = ch.dnum * RR * n, RR * n, 2 * RR * n
    a.K, a.R, a.ndig = K, R, oc.live_digits(top)
    a.c0_mode = {"pc0": 1, "pc0_acc": 1 | abi.KS_ACC, "c0ext": 2}[mode] | abi.KS_SUM
    k = g.key
    k.kb, k.seed, k.row_words, k.bits, k.q_top, k.srows, k.nregen = pkb.ptr.value, pseed.ptr.value, n, 0, -1, RR, 3
    assert abi.call("ks_dot_key", g, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bout.download((K, 2, RR, n))
    for c in range(K):
        want = np.zeros((2, RR, n), object)
        for r in range(R):
            xz = x[c].copy()
            if mode == "c0ext":
                xz[0] = 0
            e = oc.ks_dot(xz, digits[c], top, seeds[r], bs[r], autok[r]).astype(object)
            if mode == "c0ext":
                e[0] = e[0] + ctx_gather(oc, c0[c], gals[r])
            want = want + e
        if mode == "pc0_acc":
            want = want + prev[c].astype(object)
        for t in rows:
            assert (got[c, :, t] == (want[:, t] % ch.primes[t]).astype(np.uint32)).all(), (c, t)


def ctx_gather(oc, rows, g):
    """rows[automorph_slot(g, o)] at every o: a scatter by g^-1."""
    return oc.automorph_rows(rows, g).astype(object)


# ----------------------------------------------------------------------------------------------- ks_dot_regen
@pytest.mark.parametrize("bsrc", ["keytab", "keytab_packed", "dense_kb"])
def test_ks_dot_regen_plain(stream, bsrc):
    say(f"[ks_dot_regen] small K=3 b from {bsrc}")
    ch, ctx, oc = contexts("small")
    rng = np.random.default_rng(31 + len(bsrc))
    top, K = 5, 3
    n, RR = ch.n, ch.rows
    x, digits = inputs(ch, oc, top, K, rng)
    rows = ext_rows(ch, top)
    _, seeds, bs = oracle_keys(oc, ch, [2], seed=33)
    seed, b = seeds[0], bs[0]
    T = Tables(ch, ctx, rows)
    bx, bmu = pa.DevBuf.from_array(x), pa.DevBuf.from_array(digits)
    bout = pa.DevBuf(K * 2 * RR * n)
    bseed = pa.DevBuf.from_array(np.ascontiguousarray(seed, np.uint32))
    g = abi.KsRegenArgs()
    a = g.ks
    a.c1, a.modup = bx.ptr.value + 4 * RR * n, bmu.ptr.value
    a.out0, a.out1 = bout.ptr.value, bout.ptr.value + 4 * RR * n
    T.fill(a, ch)
    a.ct_stride, a.mu_ct_stride, a.mu_digit_stride, a.out_ct_stride = 2 * RR * n, ch.dnum * RR * n, RR * n, 2 * RR * n
    a.key_digit_stride = RR * n
    a.K, a.R, a.ndig = K, 1, oc.live_digits(top)
    g.seed = bseed.ptr.value
    keep = []
    if bsrc == "dense_kb":
        bb = pa.DevBuf.from_array(b)
        pkb = dev_ptrs([bb])
        a.kb = pkb.ptr.value
        keep += [bb, pkb]
    else:
        bits = 30 if bsrc == "keytab_packed" else 0
        stored, words = pack(b, bits) if bits else (b, n)
        bb = pa.DevBuf.from_array(stored)
        pkb = dev_ptrs([bb])
        keep += [bb, pkb]
        k = g.key
        k.kb, k.row_words, k.bits, k.q_top, k.srows = pkb.ptr.value, words, bits, -1, RR
    assert abi.call("ks_dot_regen", g, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bout.download((K, 2, RR, n))
    for c in range(K):
        xz = x[c].copy()
        xz[0] = 0  # no c0 term
        want = oc.ks_dot(xz, digits[c], top, seed, b, 1)
        assert (got[c][:, rows] == want[:, rows]).all(), c


def test_ks_dot_regen_epilogue(stream):
    """The fused epilogue on the Q rows: dst = 2 (alpha dst + (dot - conv) binv) + k (part 0) + add."""
    say("[ks_dot_regen] small K=2 fused epilogue (alpha, dbl, k, add)")
    ch, ctx, oc = contexts("small")
    rng = np.random.default_rng(51)
    top, K = 4, 2
    n, RR = ch.n, ch.rows
    x, digits = inputs(ch, oc, top, K, rng)
    qrows = list(range(top + 1))
    _, seeds, bs = oracle_keys(oc, ch, [3], seed=35)
    seed, b = seeds[0], bs[0]
    T = Tables(ch, ctx, qrows)
    pr = [int(ch.primes[t]) for t in range(RR)]
    binv = [int(rng.integers(1, p)) for p in pr]
    alpha = [int(rng.integers(1, p)) for p in pr]
    kcon = [int(rng.integers(0, 2 * p)) for p in pr]  # the constant may come unreduced (below 2p)
    shoup_c = lambda w, p: (w << 32) // p  # noqa: E731
    dst = np.stack([np.stack([rand_rows(ch, rng, qrows) for _ in range(2)]) for _ in range(K)])
    conv = np.stack([np.stack([rand_rows(ch, rng, qrows) for _ in range(2)]) for _ in range(K)])
    add = np.stack([np.stack([rand_rows(ch, rng, qrows) for _ in range(2)]) for _ in range(K)])
    bx, bmu = pa.DevBuf.from_array(x), pa.DevBuf.from_array(digits)
    bdst, bconv, badd = pa.DevBuf.from_array(dst), pa.DevBuf.from_array(conv), pa.DevBuf.from_array(add)
    u32 = lambda v: pa.DevBuf.from_array(np.array(v, np.uint32))  # noqa: E731
    bbi, bbis = u32(binv), u32([shoup_c(w, p) for w, p in zip(binv, pr)])
    bal, bals = u32(alpha), u32([shoup_c(w, p) for w, p in zip(alpha, pr)])
    bk = u32(kcon)
    bb = pa.DevBuf.from_array(b)
    pkb = dev_ptrs([bb])
    bseed = pa.DevBuf.from_array(np.ascontiguousarray(seed, np.uint32))
    g = abi.KsRegenArgs()
    a = g.ks
    a.c1, a.modup = bx.ptr.value + 4 * RR * n, bmu.ptr.value
    T.fill(a, ch)
    a.ct_stride, a.mu_ct_stride, a.mu_digit_stride, a.out_ct_stride = 2 * RR * n, ch.dnum * RR * n, RR * n, 2 * RR * n
    a.K, a.R, a.ndig = K, 1, oc.live_digits(top)
    g.seed = bseed.ptr.value
    g.key.kb, g.key.row_words, g.key.bits, g.key.q_top, g.key.srows = pkb.ptr.value, n, 0, -1, RR
    e = g.epi
    e.dst, e.conv, e.binv, e.binvs, e.k = bdst.ptr.value, bconv.ptr.value, bbi.ptr.value, bbis.ptr.value, bk.ptr.value
    e.part_stride, e.dbl, e.alpha, e.alphas = RR * n, 1, bal.ptr.value, bals.ptr.value
    g.use_epi, g.add = 1, badd.ptr.value
    assert abi.call("ks_dot_regen", g, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bdst.download((K, 2, RR, n))
    for c in range(K):
        xz = x[c].copy()
        xz[0] = 0
        dot = oc.ks_dot(xz, digits[c], top, seed, b, 1).astype(object)
        for t in qrows:
            p = pr[t]
            for part in range(2):
                r = (alpha[t] * dst[c, part, t].astype(object) + (dot[part, t] - conv[c, part, t].astype(object))
                     * binv[t]) % p
                r = (2 * r + (kcon[t] % p if part == 0 else 0) + add[c, part, t].astype(object)) % p
                assert (got[c, part, t] == r.astype(np.uint32)).all(), (c, part, t)
