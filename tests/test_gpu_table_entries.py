"""Table entries a pc-gpu caller reaches directly, word for word against the oracle or the entry's formula in
Python integers, through the kernel table's C-ABI:
- ks_dot: dense a and b per key, K = 2 ciphertexts x R = 2 keys, c0 modes 0 / 1 / 2 / 2 | KS_ACC, outputs scattered
  by automorph_slot(autok[r], i) (the reference's own selftest, crates/pc-kernels/src/bin/selftest.rs:1108-1225), and
  the general form K = 8, R = 3, 3 digits;
- ks_dot_key at K = 2, 3, 4 (not summed), dense and bit-packed b, equal to the oracle's single-ciphertext dot run per
  ciphertext (crates/pc-gpu/tests/rotate_grid.rs: K-batched equals single);
- ksk_expand against the oracle's KSKA rows (out[d - d0][m][N]);
- ew_sub_mul, ew_scale (special rows zeroed or scaled), ew_add / ew_copy over a row set with special rows;
- ksk_unpack at 27 to 32 bits;
- bconv_wide with 17, 33 and 48 sources (the wide path: sources re-read per target), plain, prescaled, exact and
  mean-centred jobs, against the formula in Python integers (the exact job's double sum by correctly rounded
  fused multiply-adds in fractions).
Each test prints its case before the GPU runs.
"""
import math
import sys
from fractions import Fraction

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
        ch = pa.make_chain("wide52", 12, 52, 4, 1, 30) if name == "wide52" else \
            pa.make_chain("wide31", 12, 44, 4, 1, 31) if name == "wide31" else pa.preset(name)
        _CTX[name] = (ch, pa.Context(ch, k_rot=1), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum))
    return _CTX[name]


def rand_rows(ch, rng, shape_lead=()):
    p = np.array(ch.primes, np.uint64)[:, None]
    x = rng.integers(0, 1 << 62, tuple(shape_lead) + (ch.rows, ch.n), dtype=np.uint64)
    return (x % p).astype(np.uint32)


def dev_ptrs(bufs):
    return pa.DevBuf.from_array(np.array([b.ptr.value for b in bufs], np.uint64).view(np.uint32))


def scatter_index(k, logn):
    return np.array([twin.automorph_slot(k, i, logn) for i in range(1 << logn)], np.int64)


def shoup(w, p):
    return (int(w) << 32) // int(p)


def pack(b, bits):
    """Rows as little-endian bit streams of `bits` bits each, a zero guard word, padded to 16 bytes."""
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


# ----------------------------------------------------------------------------------------------- ks_dot (dense keys)
def ks_host(ch, rows, digit_of, ndig, c1, mu, c0, kb, ka, autok, pmod, mode):
    """The dot's formula (selftest.rs ks_host): s0 = sum_d x_d kb_d (+ P c0 on Q rows | + c0), s1 = sum_d x_d ka_d,
    each mod p, written at automorph_slot(autok[r], i)."""
    K, R = c1.shape[0], len(kb)
    o0 = np.zeros((K, R, ch.rows, ch.n), np.uint32)
    o1 = np.zeros_like(o0)
    idx = [scatter_index(k, ch.logn) for k in autok]
    for c in range(K):
        for r in range(R):
            for t in rows:
                p = np.uint64(ch.primes[t])
                s0 = np.zeros(ch.n, np.uint64)
                s1 = np.zeros(ch.n, np.uint64)
                for d in range(ndig):
                    x = (c1[c, t] if d == digit_of[t] else mu[c, d, t]).astype(np.uint64)
                    s0 = (s0 + x * kb[r][d, t].astype(np.uint64) % p) % p
                    s1 = (s1 + x * ka[r][d, t].astype(np.uint64) % p) % p
                if mode == 1 and t < len(ch.q):
                    s0 = (s0 + c0[c, t].astype(np.uint64) * np.uint64(pmod[t]) % p) % p
                elif mode == 2:
                    s0 = (s0 + c0[c, t].astype(np.uint64)) % p
                o0[c, r, t, idx[r]] = s0.astype(np.uint32)
                o1[c, r, t, idx[r]] = s1.astype(np.uint32)
    return o0, o1


@pytest.mark.parametrize("chain,K,R,mode", [("small31", 2, 2, 0), ("small31", 2, 2, 1), ("small31", 2, 2, 2),
                                            ("small31", 2, 2, 2 | abi.KS_ACC), ("small", 8, 3, 1),
                                            ("small", 3, 5, 2 | abi.KS_ACC)])
def test_ks_dot_dense(stream, chain, K, R, mode):
    say(f"[ks_dot] {chain} K={K} R={R} c0 mode {mode}")
    ch, ctx, oc = contexts(chain)
    rng = np.random.default_rng(100 + K * 10 + R + mode)
    n, RR, nq = ch.n, ch.rows, len(ch.q)
    ndig = ch.dnum
    digit_of = [t // ch.alpha if t < nq else -1 for t in range(RR)]
    rows = list(range(RR))
    c1, c0 = rand_rows(ch, rng, (K,)), rand_rows(ch, rng, (K,))
    mu = rand_rows(ch, rng, (K, ndig))
    kb = [rand_rows(ch, rng, (ndig,)) for _ in range(R)]
    ka = [rand_rows(ch, rng, (ndig,)) for _ in range(R)]
    autok = [1, 125, 2 * n - 1, 5, 25][:R]
    big_p = math.prod(int(x) for x in ch.p)
    pmod = [big_p % int(q) for q in ch.q] + [0] * len(ch.p)
    acc = mode & abi.KS_ACC
    prev0, prev1 = rand_rows(ch, rng, (K, R)), rand_rows(ch, rng, (K, R))
    b1, b0, bmu = pa.DevBuf.from_array(c1), pa.DevBuf.from_array(c0), pa.DevBuf.from_array(mu)
    bo0 = pa.DevBuf.from_array(prev0 if acc else np.zeros_like(prev0))
    bo1 = pa.DevBuf.from_array(prev1 if acc else np.zeros_like(prev1))
    bkb, bka = [pa.DevBuf.from_array(x) for x in kb], [pa.DevBuf.from_array(x) for x in ka]
    pkb, pka = dev_ptrs(bkb), dev_ptrs(bka)
    u32 = lambda v: pa.DevBuf.from_array(np.array(v, np.uint32))  # noqa: E731
    bauto, brows = u32(autok), u32(rows)
    bdig = pa.DevBuf.from_array(np.array(digit_of, np.int32).view(np.uint32))
    bpm, bpms = u32(pmod), u32([shoup(v, p) for v, p in zip(pmod, ch.primes)])
    a = abi.KsArgs()
    a.c1, a.modup, a.c0 = b1.ptr.value, bmu.ptr.value, b0.ptr.value
    a.out0, a.out1, a.kb, a.ka = bo0.ptr.value, bo1.ptr.value, pkb.ptr.value, pka.ptr.value
    a.autok, a.rows, a.digit_of = bauto.ptr.value, brows.ptr.value, bdig.ptr.value
    a.pmod, a.pmods, a.pr = bpm.ptr.value, bpms.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.ct_stride, a.mu_ct_stride, a.mu_digit_stride = RR * n, ndig * RR * n, RR * n
    a.out_ct_stride, a.out_rot_stride, a.key_digit_stride = R * RR * n, RR * n, RR * n
    a.K, a.R, a.ndig, a.c0_mode, a.nq, a.nrows = K, R, ndig, mode, nq, len(rows)
    assert abi.call("ks_dot", a, stream, log_n=ch.logn) == 0
    stream.sync()
    g0, g1 = bo0.download((K, R, RR, n)), bo1.download((K, R, RR, n))
    w0, w1 = ks_host(ch, rows, digit_of, ndig, c1, mu, c0, kb, ka, autok, pmod, mode & 3)
    if acc:
        p = np.array(ch.primes, np.uint64)[None, None, :, None]
        w0 = ((w0.astype(np.uint64) + prev0) % p).astype(np.uint32)
        w1 = ((w1.astype(np.uint64) + prev1) % p).astype(np.uint32)
    assert (g0 == w0).all() and (g1 == w1).all()


# ----------------------------------------------------------------------------------------------- ks_dot_key, K > 1
def oracle_keys(oc, ch, steps, seed):
    g = twin.Prng([seed, 3, 5, 7, 9, 11, 13, 15], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
    gals = [twin.rotation_galois(r, ch.n) for r in steps]
    keys = [oc.rotation_key(g, s_eval, x) for x in gals]
    return gals, np.stack([k[0] for k in keys]), [k[1] for k in keys]


@pytest.mark.parametrize("chain,K,bits,R,top", [("small", 2, 0, 2, 5), ("small31", 3, 0, 2, 5), ("small", 4, 30, 2, 5),
                                                ("rej", 2, 0, 2, 5), ("small31", 4, 31, 2, 5),
                                                ("small", 1, 30, 2, 5), ("small", 1, 30, 5, 3),
                                                ("small31", 1, 31, 2, 1), ("small31", 1, 31, 5, 5),
                                                ("small31", 1, 31, 6, 3), ("rej", 1, 31, 5, 5)])
def test_ks_dot_key_batched(stream, chain, K, bits, R, top):
    say(f"[ks_dot_key] {chain} K={K} R={R} bits={bits} top={top}: each ciphertext equals the oracle's single dot "
        "(K = 1 packed: the fast dot's packed loads, one-wave and four-wave workgroups)")
    ch, ctx, oc = contexts(chain)
    rng = np.random.default_rng(200 + K + bits + R + top)
    n, RR, nq = ch.n, ch.rows, len(ch.q)
    ndig = oc.live_digits(top)
    x = np.zeros((K, 2, RR, n), np.uint32)
    for c in range(K):
        x[c] = rand_rows(ch, rng, (2,))
        x[c, :, top + 1:] = 0
    digits = np.stack([oc.modup(x[c, 1], top) for c in range(K)])
    gals, seeds, bs = oracle_keys(oc, ch, [1, 3, 2, 7, 11, 4][:R], seed=40 + K)
    rows = list(range(top + 1)) + list(range(nq, RR))
    autok = [twin.galois_inverse(g, n) for g in gals]
    big_p = math.prod(int(v) for v in ch.p)
    pmod = [big_p % int(q) for q in ch.q] + [0] * len(ch.p)
    bx, bmu = pa.DevBuf.from_array(x), pa.DevBuf.from_array(digits)
    bout = pa.DevBuf(K * R * 2 * RR * n)
    stored = [pack(b, bits)[0] if bits else b for b in bs]
    words = pack(bs[0], bits)[1] if bits else n
    bkb = [pa.DevBuf.from_array(s) for s in stored]
    bseed = [pa.DevBuf.from_array(np.ascontiguousarray(s, np.uint32)) for s in seeds]
    pkb, pseed = dev_ptrs(bkb), dev_ptrs(bseed)
    u32 = lambda v: pa.DevBuf.from_array(np.array(v, np.uint32))  # noqa: E731
    bauto, brows = u32(autok), u32(rows)
    bdig = pa.DevBuf.from_array(np.array([t // ch.alpha if t < nq else -1 for t in range(RR)], np.int32)
                                .view(np.uint32))
    bpm, bpms = u32(pmod), u32([shoup(v, p) for v, p in zip(pmod, ch.primes)])
    g = abi.KsKeyArgs()
    a = g.ks
    a.c1, a.c0, a.modup = bx.ptr.value + 4 * RR * n, bx.ptr.value, bmu.ptr.value
    a.out0, a.out1 = bout.ptr.value, bout.ptr.value + 4 * RR * n
    a.autok, a.rows, a.digit_of = bauto.ptr.value, brows.ptr.value, bdig.ptr.value
    a.pmod, a.pmods, a.pr = bpm.ptr.value, bpms.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.ct_stride, a.mu_ct_stride, a.mu_digit_stride = 2 * RR * n, ch.dnum * RR * n, RR * n
    a.out_ct_stride, a.out_rot_stride = R * 2 * RR * n, 2 * RR * n
    a.K, a.R, a.ndig, a.c0_mode, a.nq, a.nrows = K, R, ndig, 1, nq, len(rows)
    k = g.key
    k.kb, k.seed, k.row_words, k.bits, k.q_top, k.srows, k.nregen = pkb.ptr.value, pseed.ptr.value, words, bits, -1, \
        RR, ndig
    assert abi.call("ks_dot_key", g, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bout.download((K, R, 2, RR, n))
    for c in range(K):
        for r in range(R):
            want = oc.ks_dot(x[c], digits[c], top, seeds[r], bs[r], autok[r])
            assert (got[c, r][:, rows] == want[:, rows]).all(), (c, r)


# ----------------------------------------------------------------------------------------------- ksk_expand
@pytest.mark.parametrize("chain,d0", [("small", 0), ("small31", 1), ("rej", 2)])
def test_ksk_expand(stream, chain, d0):
    say(f"[ksk_expand] {chain} digits {d0}..dnum, prime ids out of order")
    ch, ctx, _ = contexts(chain)
    rng = np.random.default_rng(300 + d0)
    seed = rng.integers(0, 1 << 32, 8, dtype=np.uint64).astype(np.uint32)
    ids = [ch.rows - 1, 0, 3, ch.rows - 2, 1]
    bseed, bids = pa.DevBuf.from_array(seed), pa.DevBuf.from_array(np.array(ids, np.int32).view(np.uint32))
    nd = ch.dnum - d0
    bout = pa.DevBuf(nd * len(ids) * ch.n)
    a = abi.KskExpandArgs()
    a.out, a.seed, a.prime_ids, a.pr = bout.ptr.value, bseed.ptr.value, bids.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.nmod, a.dnum, a.d0 = len(ids), ch.dnum, d0
    assert abi.call("ksk_expand", a, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bout.download((nd, len(ids), ch.n))
    for d in range(nd):
        for m, pid in enumerate(ids):
            assert (got[d, m] == twin.kska_row(seed, d0 + d, ch.primes[pid], ch.n)).all(), (d, m)
    a.d0 = ch.dnum
    assert abi.call("ksk_expand", a, stream, log_n=ch.logn) == -1


# ----------------------------------------------------------------------------------------------- element-wise
def rowset_ids(ch, nq, npr):
    return list(range(nq)) + [len(ch.q) + j for j in range(npr)]


@pytest.mark.parametrize("op,zero_p", [("ew_sub_mul", 0), ("ew_scale", 0), ("ew_scale", 1), ("ew_add", 0),
                                       ("ew_sub", 0), ("ew_copy", 0)])
def test_ew_entries(stream, op, zero_p):
    say(f"[{op}] small31 K=3, 2 parts, 4 Q rows + 2 special rows, zero_p={zero_p}")
    ch, ctx, _ = contexts("small31")
    rng = np.random.default_rng(400 + len(op) + zero_p)
    K, n, RR = 3, ch.n, ch.rows
    nq, npr = 4, 2
    ids = rowset_ids(ch, nq, npr)
    xa, xb = rand_rows(ch, rng, (K, 2)), rand_rows(ch, rng, (K, 2))
    sc = [int(rng.integers(0, p)) for p in ch.primes]
    prev = rand_rows(ch, rng, (K, 2))
    ba, bb, bo = pa.DevBuf.from_array(xa), pa.DevBuf.from_array(xb), pa.DevBuf.from_array(prev)
    bsc = pa.DevBuf.from_array(np.array(sc, np.uint32))
    bscs = pa.DevBuf.from_array(np.array([shoup(w, p) for w, p in zip(sc, ch.primes)], np.uint32))
    a = abi.EwArgs()
    for ref, buf in ((a.out, bo), (a.a, ba), (a.b, bb)):
        ref.base, ref.ct_stride, ref.part_stride = buf.ptr.value, 2 * RR * n, RR * n
    a.rs.nq, a.rs.np, a.rs.qmax = nq, npr, len(ch.q)
    a.sc, a.scs, a.pr = bsc.ptr.value, bscs.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.K, a.nparts, a.sub, a.zero_p = K, 2, int(op == "ew_sub"), zero_p
    name = "ew_add" if op == "ew_sub" else op
    assert abi.call(name, a, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bo.download((K, 2, RR, n))
    want = prev.copy()
    for t in ids:
        p = np.uint64(ch.primes[t])
        x, y = xa[:, :, t].astype(np.uint64), xb[:, :, t].astype(np.uint64)
        if op == "ew_sub_mul":
            r = (x + p - y) % p * np.uint64(sc[t]) % p
        elif op == "ew_scale":
            r = np.zeros_like(x) if (zero_p and t >= len(ch.q)) else x * np.uint64(sc[t]) % p
        elif op == "ew_add":
            r = (x + y) % p
        elif op == "ew_sub":
            r = (x + p - y) % p
        else:
            r = x
        want[:, :, t] = r.astype(np.uint32)
    assert (got == want).all()


# ----------------------------------------------------------------------------------------------- ksk_unpack
@pytest.mark.parametrize("bits", [27, 28, 30, 31, 32])
def test_ksk_unpack(stream, bits):
    say(f"[ksk_unpack] N=2^12 6 rows at {bits} bits")
    rng = np.random.default_rng(500 + bits)
    n, nr = 1 << 12, 6
    vals = rng.integers(0, 1 << bits, (nr, n), dtype=np.uint64).astype(np.uint32)
    packed, words = pack(vals, bits)
    bin_, bout = pa.DevBuf.from_array(packed), pa.DevBuf(nr * n)
    a = abi.KskUnpackArgs()
    a.out, a.in_, a.row_words, a.nrows, a.bits = bout.ptr.value, bin_.ptr.value, words, nr, bits
    assert abi.call("ksk_unpack", a, stream, log_n=12) == 0
    stream.sync()
    assert (bout.download((nr, n)) == vals).all()
    a.row_words = n * bits // 32  # no room for the guard word
    assert abi.call("ksk_unpack", a, stream, log_n=12) == -1


# ----------------------------------------------------------------------------------------------- bconv_wide
def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


@pytest.mark.parametrize("chain,ns,exact,prescaled", [("wide52", 17, 0, 0), ("wide52", 33, 1, 0), ("wide52", 48, 0, 1),
                                                       ("wide52", 48, 2, 0), ("wide52", 20, 1, 1),
                                                       ("wide52", 16, 0, 0), ("wide52", 16, 1, 1), ("wide31", 16, 0, 0),
                                                       ("wide31", 16, 2, 0), ("wide31", 5, 0, 0), ("wide52", 3, 0, 1)])
def test_bconv_wide(stream, chain, ns, exact, prescaled):
    say(f"[bconv] {chain} N=2^12 {ns} sources -> 6 targets, exact={exact} prescaled={prescaled}, two jobs (at most 16 "
        "sources: the LDS path, 30-bit primes without carry counts, 31-bit with)")
    ch, ctx, _ = contexts(chain)
    rng = np.random.default_rng(600 + ns + exact)
    n, RR = ch.n, ch.rows
    pr = ch.primes
    nt = 6
    jobs, pool = [], []
    # two jobs over different source / target rows of one source and one destination buffer
    specs = [(list(range(ns)), list(range(ns, ns + nt)), 0, 0), (list(range(1, ns + 1))[::-1],
                                                                  [ns + 2, ns + 3, 0, 1, 2, 3], 0, RR)]
    src = rand_rows(ch, rng)
    want = np.zeros((2 * RR, n), np.uint32)
    for (sids, tids, soff, doff) in specs:
        srow, sprime = sids, sids
        trow, tprime = list(range(len(tids))), tids
        pre = [int(rng.integers(1, pr[i])) for i in sids]
        m = [[int(rng.integers(0, pr[t])) for t in tids] for _ in sids]
        off = len(pool)
        words = srow + sprime + pre + trow + tprime + [x for row in m for x in row]
        rb = bmod = None
        if exact:
            if (off + len(words)) % 2:
                words.append(0)
            rb = [float(rng.uniform(0, 1)) / pr[i] for i in sids]  # 1 / b_i-sized: u < ns
            bmod = [int(rng.integers(0, pr[t])) for t in tids]
            words += list(np.array(rb, np.float64).view(np.uint32)) + bmod
        pool += [int(w) for w in words]
        jobs.append((soff, doff, ns, nt, off, exact, prescaled, 0))
        # the formula in Python integers
        y = [src[srow[i]].astype(object) if prescaled else src[srow[i]].astype(object) * pre[i] % pr[sids[i]]
             for i in range(ns)]
        u = None
        if exact == 1:
            u = []
            for c in range(n):
                v = 0.0
                for i in range(ns):
                    v = fma(float(int(y[i][c])), rb[i], v)
                u.append(math.floor(v + 0.5))
            u = np.array(u, dtype=object)
        elif exact == 2:
            u = np.array([(ns >> 1) + ((ns & 1) & (((c * 0x9E3779B1) & 0xFFFFFFFF) >> 31)) for c in range(n)],
                         dtype=object)
        for k, t in enumerate(tids):
            acc = sum(y[i] * m[i][k] for i in range(ns)) % pr[t]
            if exact:
                acc = (acc - u * bmod[k]) % pr[t]
            want[doff + trow[k]] = acc.astype(np.uint32)
    assert len(pool) % 2 == 0 or not exact
    bsrc = pa.DevBuf.from_array(src)
    bdst = pa.DevBuf.from_array(np.zeros((2 * RR, n), np.uint32))
    bjobs = pa.DevBuf.from_array(np.array(jobs, np.uint32).reshape(-1))
    bpool = pa.DevBuf.from_array(np.array(pool + [0], np.uint32))
    a = abi.BconvArgs()
    a.src, a.dst, a.jobs, a.pool, a.pr = bsrc.ptr.value, bdst.ptr.value, bjobs.ptr.value, bpool.ptr.value, \
        LIB.pcx_ctx_primes(ctx.h)
    a.njobs, a.max_tgt = len(jobs), nt
    assert abi.call("bconv_wide" if ns > 16 else "bconv", a, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bdst.download((2 * RR, n))
    for (sids, tids, soff, doff) in specs:
        for k in range(nt):
            assert (got[doff + k] == want[doff + k]).all(), (doff, k)
