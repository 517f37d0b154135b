"""Parity of the raise table entries (mod_raise, small_int, small_int1) with the oracle (oracle/bts.py, pinned by
tests/test_oracle_bts.py), word for word, through the kernel table's C-ABI, the tables from perseus_amd.bts. Each test
prints its case before the GPU runs.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import perseus_amd as pa
from oracle import bts as ob
from perseus_amd import abi, bts
from perseus_amd._lib import LIB

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    return pa.Stream()


_CTX = {}


def context(name):
    if name not in _CTX:
        ch = pa.preset(name)
        _CTX[name] = (ch, pa.Context(ch, k_rot=1))
    return _CTX[name]


def rand_cts(ch, K, rows, rng):
    x = np.zeros((K, 2, ch.rows, ch.n), np.uint32)
    for r in rows:
        x[:, :, r] = rng.integers(0, ch.primes[r], (K, 2, ch.n))
    return x


def run(name, args, st, logn):
    rc = abi.call(name, args, st, logn)
    assert rc == 0, f"{name} returned {rc}"
    st.sync()


@pytest.mark.parametrize("name,d,nparts", [("small31", 2, 2), ("small31", 3, 1), ("c3", 3, 2)])
def test_mod_raise(stream, name, d, nparts):
    say(f"[mod_raise] {name} d={d} nparts={nparts}")
    ch, ctx = context(name)
    rng = np.random.default_rng(d * 3 + nparts)
    K = 1 if name == "c3" else 2
    x = rand_cts(ch, K, range(ch.rows), rng)
    buf = pa.DevBuf.from_array(x)
    qhatinv, qhat = bts.mod_raise_consts(ch.primes, d)
    a = abi.ModRaiseArgs()
    a.x, a.pr = buf.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.ct_stride, a.part_stride = 2 * ch.rows * ch.n, ch.rows * ch.n
    for k in range(4):
        a.qhatinv[k] = qhatinv[k]
        for t in range(64):
            a.qhat[k][t] = qhat[k][t]
    a.K, a.d, a.r0, a.r1, a.nparts = K, d, d, ch.rows, nparts
    run("mod_raise", a, stream, ch.logn)
    got = buf.download(x.shape)
    for c in range(K):
        for part in range(2):
            if part < nparts:
                want = ob.mod_raise(ch.primes, x[c, part], d, d, ch.rows, qhatinv, qhat)
                assert (got[c, part, d:] == want).all(), (c, part)
                assert (got[c, part, :d] == x[c, part, :d]).all(), "sources untouched"
            else:
                assert (got[c, part] == x[c, part]).all(), "parts past nparts untouched"


def tab_buf(tab):
    return pa.DevBuf.from_array(np.frombuffer(bytes(tab), np.uint32))


@pytest.mark.parametrize("name,k,c,inplace", [("small31", 1, None, False), ("small31", 2, 1.0 / 3, False),
                                              ("small31", 3, 2.5e-7, True), ("small31", 4, 7.1e-12, False),
                                              ("c3", 3, 2.3167161361161844e-07 * 4096.0, False)])
def test_small_int(stream, name, k, c, inplace):
    say(f"[small_int] {name} k={k} c={c} inplace={inplace}")
    ch, ctx = context(name)
    rng = np.random.default_rng(k * 11 + inplace)
    K = 1 if name == "c3" else 2
    src = rand_cts(ch, K, range(k), rng)
    out_rows = list(range(ch.rows))[::-1]  # every prime id, written in descending order
    tab = bts.small_int_tab(ch.primes[:k], out_rows, [ch.primes[r] for r in out_rows], c)
    tb = tab_buf(tab)
    sbuf = pa.DevBuf.from_array(src)
    obuf = sbuf if inplace else pa.DevBuf(src.size)
    a = abi.SmallIntArgs()
    a.src, a.out, a.tab, a.pr = sbuf.ptr.value, obuf.ptr.value, tb.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.src_ct_stride = a.ct_stride = 2 * ch.rows * ch.n
    a.src_part_stride = a.part_stride = ch.rows * ch.n
    a.K, a.nparts = K, 2
    run("small_int", a, stream, ch.logn)
    got = obuf.download(src.shape)
    for cc in range(K):
        for part in range(2):
            want = ob.small_int(ch.primes[:k], src[cc, part, :k], ch.primes, None if c is None else list(tab.R))
            assert (got[cc, part] == want).all(), (cc, part)


def boundary_values(q_src, n, rng):
    """N integers in [0, Q): the ones where the CRT quotient sum_a y_a / q_a sits next to an integer (X near 0 and
    near Q), the centring boundary floor(Q / 2) and its neighbours, the CRT basis elements Q / q_a and their
    neighbours, thirds of Q; the rest uniform."""
    Q = 1
    for p in q_src:
        Q *= int(p)
    h = Q // 2
    vals = [0, 1, 2, 3, 1000, Q - 1, Q - 2, Q - 3, Q - 1000, h - 2, h - 1, h, h + 1, h + 2, Q // 3, 2 * Q // 3]
    for p in q_src:
        m = Q // int(p)
        vals += [m - 1, m, m + 1, Q - m, Q - m + 1]
    vals = [v % Q for v in vals]
    rest = [int(rng.integers(0, 1 << 62)) * (1 << 62) % Q + int(rng.integers(0, 1 << 62)) for _ in range(n - len(vals))]
    return vals + [v % Q for v in rest]


@pytest.mark.parametrize("k,c", [(1, None), (2, None), (3, 1.0 / 3), (4, None), (4, 7.1e-12)])
def test_small_int_boundaries(stream, k, c):
    """small_int on integers chosen where a CRT or centring step can go wrong (next to 0 and Q, at floor(Q / 2), at
    the basis elements Q / q_a), against the oracle's Garner reconstruction."""
    name = "small31"
    say(f"[small_int boundaries] {name} k={k} c={c}")
    ch, ctx = context(name)
    rng = np.random.default_rng(100 + k)
    X = boundary_values(ch.primes[:k], ch.n, rng)
    src = np.zeros((1, 2, ch.rows, ch.n), np.uint32)
    for a in range(k):
        src[0, 0, a] = [x % int(ch.primes[a]) for x in X]
        src[0, 1, a] = [(int(ch.primes[a]) - 1 - x) % int(ch.primes[a]) for x in X]
    out_rows = list(range(ch.rows))
    tab = bts.small_int_tab(ch.primes[:k], out_rows, [ch.primes[r] for r in out_rows], c)
    tb = tab_buf(tab)
    sbuf = pa.DevBuf.from_array(src)
    obuf = pa.DevBuf(src.size)
    a = abi.SmallIntArgs()
    a.src, a.out, a.tab, a.pr = sbuf.ptr.value, obuf.ptr.value, tb.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.src_ct_stride = a.ct_stride = 2 * ch.rows * ch.n
    a.src_part_stride = a.part_stride = ch.rows * ch.n
    a.K, a.nparts = 1, 2
    run("small_int", a, stream, ch.logn)
    got = obuf.download(src.shape)
    for part in range(2):
        want = ob.small_int(ch.primes[:k], src[0, part, :k], ch.primes, None if c is None else list(tab.R))
        bad = np.nonzero((got[0, part] != want).any(axis=0))[0]
        assert bad.size == 0, (part, bad[:8], [X[i] for i in bad[:4]])


@pytest.mark.parametrize("c,nparts", [(0.25, 2), (2.3167161361161844e-07 * 4096.0, 1), (3.0e-5, 2)])
def test_small_int1(stream, c, nparts):
    name = "small31"
    say(f"[small_int1] {name} c={c} nparts={nparts}")
    ch, ctx = context(name)
    rng = np.random.default_rng(int(c * 1e6) % 1000)
    K = 2
    x = rand_cts(ch, K, range(ch.rows), rng)
    buf = pa.DevBuf.from_array(x)
    mc, sh = bts.single_scale(c, ch.primes[0])
    a = abi.SmallInt1Args()
    a.x, a.pr = buf.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.ct_stride, a.part_stride, a.mc, a.sh = 2 * ch.rows * ch.n, ch.rows * ch.n, mc, sh
    a.nrows, a.K, a.nparts = ch.rows, K, nparts
    run("small_int1", a, stream, ch.logn)
    got = buf.download(x.shape)
    for cc in range(K):
        for part in range(2):
            if part < nparts:
                want = ob.small_int1(ch.primes[0], mc, sh, x[cc, part, 0], ch.primes)
                assert (got[cc, part] == want).all(), (cc, part)
            else:
                assert (got[cc, part] == x[cc, part]).all()
