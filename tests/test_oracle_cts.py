"""Pins of the oracle's fused CtS stage (crates/pc-host/src/cts.rs; crates/pc-kernels/kernels/cts.cuh:1-10).

The stage is checked against its unfused composition, built from independently pinned pieces:
- baby i >= 1 is the key-switch dot of key i-1 scattered by g_i^-1 (the oracle's ks_dot, pinned by the decryption
  tests). The stage instead gathers by kinv = g_i (crates/pc-core/src/galois.rs:3-12: scatter by g^-1 == gather by g);
- baby 0 is P x on the Q rows and 0 on the special rows, or x0 as stored;
- res_j = sum_i rot_i * pt_{B j + i}, with the diagonal row of special prime j at pt_prow + j and diagonals at or past
  npts skipped, under the three ptidx encodings (crates/pc-kernels/kernels/arith.cuh:242-244).
"""
import numpy as np
import pytest

from tests import twin


def small_chain(logn=10, nq=6, kp=2, dnum=3, bits=31):
    ps = twin.descending_primes(bits, 2 << logn, nq + kp)
    return twin.Ctx(logn, ps[:nq], ps[nq:], dnum)


def ptidx(o, enc):
    return o >> (enc & 0xFF) if (enc >> 24) == 0x7F else o & enc


def setup(ctx, top, K, B, npts, ptw, seed, stride=3):
    rng = np.random.default_rng(seed)
    n, R = ctx.n, ctx.rows
    pr = np.array(ctx.primes, np.int64)
    x = np.zeros((K, 2, R, n), np.uint32)
    for c in range(K):
        for t in range(top + 1):
            x[c, :, t] = rng.integers(0, pr[t], (2, n))
    digits = np.stack([ctx.modup(x[c, 1], top) for c in range(K)])
    gal = [twin.rotation_galois(stride * i, n) for i in range(1, B)]
    seeds = rng.integers(0, 2**32, (max(B - 1, 1), 8), dtype=np.uint64).astype(np.uint32)
    bs = [np.stack([np.stack([rng.integers(0, pr[t], n) for t in range(R)]) for _ in range(ctx.dnum)]).astype(np.uint32)
          for _ in range(B - 1)]
    prows = list(range(top + 1)) + [ctx.nq + j for j in range(ctx.kp)]
    pts = [np.stack([rng.integers(0, pr[t], ptw) for t in prows]).astype(np.uint32) for _ in range(npts)]
    return x, digits, gal, seeds, bs, pts


def composed(ctx, x, digits, top, B, G, gal, seeds, bs, pts, enc, x0=None, pmod=None):
    """The unfused stage: rotations as scattered key-switch dots, then the diagonal products summed in Python ints.
    pmod (per Q row) replaces P mod q_t: the dots then run on c0 = 0 and the gathered c0 times pmod is added."""
    n, R = ctx.n, ctx.rows
    K = x.shape[0]
    rows = list(range(top + 1)) + [ctx.nq + j for j in range(ctx.kp)]
    idx = np.array([ptidx(o, enc) for o in range(n)])
    res = np.zeros((K, G, 2, R, n), np.uint32)
    for c in range(K):
        rot = []
        for i in range(B):
            if i == 0:
                if x0 is not None:
                    r0 = x0[c].astype(object)
                else:
                    r0 = np.zeros((2, R, n), object)
                    for t in range(top + 1):
                        pm = ctx.pmodq[t] if pmod is None else int(pmod[t])
                        r0[:, t] = (x[c, :, t].astype(object) * pm) % ctx.primes[t]
            elif pmod is None:
                r0 = ctx.ks_dot(x[c], digits[c], top, seeds[i - 1], bs[i - 1],
                                twin.galois_inverse(gal[i - 1], n)).astype(object)
            else:
                xz = x[c].copy()
                xz[0] = 0
                r0 = ctx.ks_dot(xz, digits[c], top, seeds[i - 1], bs[i - 1],
                                twin.galois_inverse(gal[i - 1], n)).astype(object)
                g0 = ctx.automorph_rows(x[c, 0, : top + 1], gal[i - 1]).astype(object)
                for t in range(top + 1):
                    r0[0, t] = (r0[0, t] + g0[t] * int(pmod[t])) % ctx.primes[t]
            rot.append(r0)
        for j in range(G):
            for y, t in enumerate(rows):
                p = ctx.primes[t]
                acc = np.zeros((2, n), object)
                for i in range(B):
                    dg = B * j + i
                    if dg >= len(pts):
                        continue
                    w = pts[dg][y][idx].astype(object)
                    acc = acc + rot[i][:, t] * w
                res[c, j, :, t] = (acc % p).astype(np.uint32)
    return res


def rows_of(ctx, top):
    return list(range(top + 1)) + [ctx.nq + j for j in range(ctx.kp)]


@pytest.mark.parametrize("K,B,G,npts,enc", [
    (1, 4, 2, 8, 0xFFFFFFFF),         # full diagonals
    (1, 3, 2, 5, 0x7F000000 | 3),     # block-constant diagonals (o >> 3), the last diagonal past npts
    (2, 2, 1, 2, 127),                # periodic diagonals (o & 127), two ciphertexts
])
def test_cts_matches_composition(K, B, G, npts, enc):
    ctx = small_chain()
    top = 4
    ptw = ctx.n if enc == 0xFFFFFFFF else (ctx.n >> (enc & 0xFF) if enc >> 24 == 0x7F else enc + 1)
    x, digits, gal, seeds, bs, pts = setup(ctx, top, K, B, npts, ptw, seed=K * 100 + B)
    got = ctx.cts_fused(x, digits, top, B, G, pts, gal, seeds=seeds, bs=bs, enc=enc)
    want = composed(ctx, x, digits, top, B, G, gal, seeds, bs, pts, enc)
    rs = rows_of(ctx, top)
    assert (got[:, :, :, rs] == want[:, :, :, rs]).all()


def test_cts_x0_and_resident_a():
    """x0 replaces baby 0 as stored (every row); a resident `a` equal to the KSKA rows gives the regenerated result."""
    ctx = small_chain()
    top, K, B, G = 5, 1, 3, 2
    x, digits, gal, seeds, bs, pts = setup(ctx, top, K, B, 6, ctx.n, seed=7)
    rng = np.random.default_rng(8)
    x0 = np.stack([np.stack([np.stack([rng.integers(0, p, ctx.n) for p in ctx.primes]) for _ in range(2)])
                   for _ in range(K)]).astype(np.uint32)
    got = ctx.cts_fused(x, digits, top, B, G, pts, gal, seeds=seeds, bs=bs, x0=x0)
    want = composed(ctx, x, digits, top, B, G, gal, seeds, bs, pts, 0xFFFFFFFF, x0=x0)
    rs = rows_of(ctx, top)
    assert (got[:, :, :, rs] == want[:, :, :, rs]).all()
    # a for digits >= nregen read from resident rows: the KSKA rows themselves
    as_ = []
    for i in range(B - 1):
        a = np.zeros((ctx.dnum, ctx.rows, ctx.n), np.uint32)
        for d in range(ctx.dnum):
            for t in range(ctx.rows):
                a[d, t] = twin.kska_row(seeds[i], d, ctx.primes[t], ctx.n)
        as_.append(a)
    ref = ctx.cts_fused(x, digits, top, B, G, pts, gal, seeds=seeds, bs=bs)
    for nregen in (0, 1):
        alt = ctx.cts_fused(x, digits, top, B, G, pts, gal, seeds=seeds, bs=bs, as_=as_, nregen=nregen)
        assert (alt[:, :, :, rs] == ref[:, :, :, rs]).all()


def test_cts_pmod_table():
    """A caller-supplied P-factor table (the fused-rescale stages pass their own) replaces P mod q on every Q row."""
    ctx = small_chain()
    top, B, G = 3, 3, 2
    x, digits, gal, seeds, bs, pts = setup(ctx, top, 1, B, 5, ctx.n, seed=9)
    rng = np.random.default_rng(10)
    pmod = np.array([rng.integers(1, p) for p in ctx.primes[: ctx.nq]], np.uint32)
    got = ctx.cts_fused(x, digits, top, B, G, pts, gal, seeds=seeds, bs=bs, pmod=pmod)
    want = composed(ctx, x, digits, top, B, G, gal, seeds, bs, pts, 0xFFFFFFFF, pmod=pmod)
    rs = rows_of(ctx, top)
    assert (got[:, :, :, rs] == want[:, :, :, rs]).all()
