"""The one-pass transforms of N = 2^16 (one workgroup per row, taken by launches of 1024 rows or more once
pcx_ntt_one_pass_min turns them on) through the
table's ntt_fwd / ntt_inv entries: bit-exact against the oracle's transforms and against the two-pass transforms of
the same launch split into chunks of 128 rows (NttArgs.chunk), with 30-bit (lazy) and 31-bit primes, rows addressed
out of order, the forward epilogues 1-3, summed out-of-place sources and per-row inverse scales. Each test prints its
case before the GPU runs.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import abi
from perseus_amd._lib import LIB
from tests import twin

pytestmark = pytest.mark.gpu
N = 1 << 16
NR = 1024  # rows of a one-pass launch (the launcher's threshold)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    # the one-pass transform is off by default: this module turns it on from NR rows, and back off at its end
    prev = pa.ntt_one_pass_min(NR)
    yield pa.Stream()
    pa.ntt_one_pass_min(prev)


_CTX = {}


def chain(bits):
    if bits not in _CTX:
        ps = twin.descending_primes(bits, 2 * N, 21)
        ch = pa.Chain(f"ntt1_{bits}", 16, ps[:-1], ps[-1:], 1)
        _CTX[bits] = (ch, pa.Context(ch, k_rot=1), twin.Ctx(16, ps[:-1], ps[-1:], 1))
    return _CTX[bits]


class Launch:
    """NttArgs over nrows rows of a buffer: row i at roff[i] (a permutation), prime id rprime[i] (cycling)."""

    def __init__(self, ctx, ch, nrows, rng, nbuf_rows=None):
        self.nrows = nrows
        self.roff = rng.permutation(nbuf_rows or nrows).astype(np.uint32)[:nrows]
        self.ids = (np.arange(nrows) * 7 % len(ch.q)).astype(np.int32)
        self.keep = [pa.DevBuf.from_array(self.roff), pa.DevBuf.from_array(self.ids.view(np.uint32))]
        self.ctx, self.ch = ctx, ch

    def args(self, base, chunk):
        a = abi.NttArgs()
        a.base, a.roff, a.rprime = base.ptr.value, self.keep[0].ptr.value, self.keep[1].ptr.value
        a.fw, a.fws, a.iw, a.iws = (LIB.pcx_ctx_twiddle(self.ctx.h, w) for w in range(4))
        a.ninv, a.ninvs = LIB.pcx_ctx_twiddle(self.ctx.h, 4), LIB.pcx_ctx_twiddle(self.ctx.h, 5)
        a.pr, a.nrows, a.chunk = LIB.pcx_ctx_primes(self.ctx.h), self.nrows, chunk
        a.lazy = int(max(self.ch.primes) < (1 << 30))
        return a

    def primes(self):
        return np.array([self.ch.primes[i] for i in self.ids], np.uint64)[:, None]


def rand_rows(ch, ids, rng, n_rows=None):
    x = np.stack([rng.integers(0, ch.primes[i], N) for i in ids]).astype(np.uint32)
    x[0, :3] = [ch.primes[ids[0]] - 1, 0, ch.primes[ids[0]] - 1]
    return x


def scatter(L, rows, nbuf):
    """buffer contents with launch row i at roff[i]"""
    buf = np.zeros((nbuf, N), np.uint32)
    buf[L.roff] = rows
    return buf


def shoup_const(v, p):
    return (np.asarray(v, np.uint64) << np.uint64(32)) // np.asarray(p, np.uint64)


@pytest.mark.parametrize("bits", [31, 30])
def test_one_pass_against_oracle(stream, bits):
    nr = NR + 40
    say(f"[ntt1] {bits}-bit primes, {nr} rows out of order: forward, inverse, round trip")
    ch, ctx, oc = chain(bits)
    twin.set_threads(16)
    rng = np.random.default_rng(bits)
    L = Launch(ctx, ch, nr, rng)
    x = rand_rows(ch, L.ids, rng)
    buf = pa.DevBuf.from_array(scatter(L, x, nr))
    assert abi.call("ntt_fwd", L.args(buf, 0), stream, 16) == 0
    stream.sync()
    got = buf.download((nr, N))[L.roff]
    want = oc.ntt_fwd(x.copy(), list(L.ids))
    assert (got == want).all()
    assert abi.call("ntt_inv", L.args(buf, 0), stream, 16) == 0
    stream.sync()
    assert (buf.download((nr, N))[L.roff] == x).all(), "round trip"
    buf.upload(scatter(L, x, nr))
    assert abi.call("ntt_inv", L.args(buf, 0), stream, 16) == 0
    stream.sync()
    assert (buf.download((nr, N))[L.roff] == oc.ntt_inv(x.copy(), list(L.ids))).all()


@pytest.mark.parametrize("bits,epi", [(31, 1), (31, 2), (31, 3), (30, 1), (30, 2), (30, 3)])
def test_one_pass_epilogues(stream, bits, epi):
    say(f"[ntt1] {bits}-bit primes, {NR} rows, forward epilogue {epi}: one pass vs two passes vs the formula")
    ch, ctx, oc = chain(bits)
    twin.set_threads(16)
    rng = np.random.default_rng(100 * bits + epi)
    nr = NR
    L = Launch(ctx, ch, nr, rng)
    x, v, d = rand_rows(ch, L.ids, rng), rand_rows(ch, L.ids, rng), rand_rows(ch, L.ids, rng)
    s = np.array([int(rng.integers(1, p)) for p in ch.primes], np.uint64)
    ss = shoup_const(s, ch.primes)
    bes, bess = pa.DevBuf.from_array(s.astype(np.uint32)), pa.DevBuf.from_array(ss.astype(np.uint32))
    bv, bd = pa.DevBuf.from_array(scatter(L, v, nr)), pa.DevBuf.from_array(scatter(L, d, nr))
    outs = []
    for chunk in (0, 128):
        base, out = pa.DevBuf.from_array(scatter(L, x, nr)), pa.DevBuf.from_array(np.zeros((nr, N), np.uint32))
        a = L.args(base, chunk)
        a.epi, a.eout, a.ex, a.xnum = epi, out.ptr.value, bv.ptr.value, 1
        a.es, a.ess = bes.ptr.value, bess.ptr.value
        if epi == 2:
            a.ed = bd.ptr.value
        assert abi.call("ntt_fwd", a, stream, 16) == 0
        stream.sync()
        outs.append(out.download((nr, N))[L.roff])
    assert (outs[0] == outs[1]).all(), "one pass == two passes"
    X = oc.ntt_fwd(x.copy(), list(L.ids)).astype(np.uint64)
    P, sv = L.primes(), s[L.ids][:, None]
    vv = v.astype(np.uint64)
    if epi == 3:
        want = (vv * sv % P + X) % P
    else:
        want = (vv + P - X) % P * sv % P
        if epi == 2:
            want = (want + d.astype(np.uint64)) % P
    assert (outs[0] == want.astype(np.uint32)).all()


@pytest.mark.parametrize("bits", [31, 30])
def test_one_pass_sources_and_row_scales(stream, bits):
    say(f"[ntt1] {bits}-bit primes, {NR} rows: forward and inverse of two summed sources, inverse per-row scales")
    ch, ctx, oc = chain(bits)
    twin.set_threads(16)
    rng = np.random.default_rng(7 * bits)
    nr = NR
    L = Launch(ctx, ch, nr, rng)
    x0, x1 = rand_rows(ch, L.ids, rng), rand_rows(ch, L.ids, rng)
    # sources: launch row i reads rows soff[i] and soff[i] + nr of src (snum 2, sstride nr N)
    soff = rng.permutation(nr).astype(np.uint32)
    src = np.zeros((2 * nr, N), np.uint32)
    src[soff], src[soff + nr] = x0, x1
    bsrc, bso = pa.DevBuf.from_array(src), pa.DevBuf.from_array(soff)
    P = L.primes()
    xs = ((x0.astype(np.uint64) + x1) % P).astype(np.uint32)
    es = np.array([int(rng.integers(1, ch.primes[i])) for i in L.ids], np.uint64)
    ess = shoup_const(es, [ch.primes[i] for i in L.ids])
    bes, bess = pa.DevBuf.from_array(es.astype(np.uint32)), pa.DevBuf.from_array(ess.astype(np.uint32))
    for fwd in (True, False):
        outs = []
        for chunk in (0, 128):
            base = pa.DevBuf.from_array(np.zeros((nr, N), np.uint32))
            a = L.args(base, chunk)
            a.src, a.soff, a.snum, a.sstride = bsrc.ptr.value, bso.ptr.value, 2, nr * N
            if not fwd:
                a.es, a.ess = bes.ptr.value, bess.ptr.value
            assert abi.call("ntt_fwd" if fwd else "ntt_inv", a, stream, 16) == 0
            stream.sync()
            outs.append(base.download((nr, N))[L.roff])
        assert (outs[0] == outs[1]).all(), ("one pass == two passes", fwd)
        if fwd:
            want = oc.ntt_fwd(xs.copy(), list(L.ids))
        else:
            # es replaces N^-1: the oracle's inverse times N es
            inv = oc.ntt_inv(xs.copy(), list(L.ids)).astype(np.uint64)
            want = (inv * (N % P) % P * es[:, None] % P).astype(np.uint32)
        assert (outs[0] == want).all(), fwd
