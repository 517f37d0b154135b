"""Parity of the EvalMod / plaintext-product table entries and of the composite rescale with the oracle
(oracle/em.py, pinned by tests/test_oracle_em.py), word for word, through the kernel table's C-ABI: tensor,
tensor_y, tensor_sum, md_epilogue(_to), wsum, wsum_k, wsum_multi, add_const, mul_table, mul_add, mul_add_n,
rescale_combine(_to), ew_many, submul_many, rescale_coef (one and two primes, with the scalar fold) and rescale_fwd
(the corrections generated inside the forward NTT, the combine in its epilogue). Each test prints its case before the
GPU runs.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from oracle import em
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
        _CTX[name] = (ch, pa.Context(ch, k_rot=1), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum))
    return _CTX[name]


class Cts:
    """K ciphertexts [K][2][R][N] on the device, R = the chain's rows, with random residues on rows [0, n)."""

    def __init__(self, ch, K, n, rng, host=None):
        self.R, self.N, self.K = ch.rows, ch.n, K
        if host is None:
            host = np.zeros((K, 2, ch.rows, ch.n), np.uint32)
            for r in range(n):
                host[:, :, r] = rng.integers(0, ch.primes[r], (K, 2, ch.n))
        self.host = host
        self.buf = pa.DevBuf.from_array(host)

    def ref(self):
        return abi.PolyRef(self.buf.ptr.value, 2 * self.R * self.N, self.R * self.N)

    def get(self):
        return self.buf.download((self.K, 2, self.R, self.N))


def consts(ch, vals):
    """device per-prime-id words and their Shoup companions floor(w 2^32 / p)"""
    v = [int(x) % int(ch.primes[i]) for i, x in enumerate(vals)] + [0] * (ch.rows - len(vals))
    s = [(x << 32) // int(p) for x, p in zip(v, ch.primes)]
    return pa.DevBuf.from_array(np.array(v, np.uint32)), pa.DevBuf.from_array(np.array(s, np.uint32))


def raw(vals):
    return pa.DevBuf.from_array(np.array(vals, np.uint32))


def table(ch, n, rng):
    t = np.zeros((ch.rows, ch.n), np.uint32)
    for r in range(n):
        t[r] = rng.integers(0, ch.primes[r], ch.n)
    return t


def run(name, args, st, logn):
    rc = abi.call(name, args, st, logn)
    assert rc == 0, f"{name} returned {rc}"
    st.sync()


def pr_of(ctx):
    return LIB.pcx_ctx_primes(ctx.h)


# ----------------------------------------------------------------------------------------------- tensor
@pytest.mark.parametrize("case", ["one", "two_acc_dbl_coef", "y_add", "y_sub", "sum5", "alias"])
def test_tensor(stream, case):
    name = "small31"
    say(f"[tensor] {name} {case}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(sum(map(ord, case)))
    K, n, q = 2, 5, ch.primes
    np_ = {"one": 1, "sum5": 5}.get(case, 2)
    A = [Cts(ch, K, n, rng) for _ in range(np_)]
    B = [Cts(ch, K, n, rng) for _ in range(np_)]
    out, d2 = Cts(ch, K, n, rng), Cts(ch, K, n, rng)
    coef = pa.DevBuf(K * ch.rows * ch.n)
    acc = case in ("two_acc_dbl_coef", "sum5")
    acc_d2 = case == "two_acc_dbl_coef" or case == "sum5"
    dbl = case == "two_acc_dbl_coef"
    sl = lambda c: c.host[:, :, :n]
    pairs = [(sl(a), sl(b)) for a, b in zip(A, B)]
    y = Cts(ch, K, n, rng)
    yc = [int(rng.integers(0, p)) for p in q[:n]]
    yv, ys = consts(ch, yc)
    ysub = None if not case.startswith("y_") else case == "y_sub"
    if case == "alias":  # out is a0: every input word is read before the first store
        out = A[0]
    want = em.tensor(q, pairs, sl(out), d2.host[:, 1, :n], acc, acc_d2, dbl, None if ysub is None else sl(y), yc,
                     bool(ysub))
    if case == "sum5":
        a = abi.TensorSumArgs()
        a.out, a.d2 = out.ref(), d2.ref()
        for j in range(np_):
            a.a[j], a.b[j] = A[j].ref(), B[j].ref()
        a.pr, a.npairs, a.acc, a.n, a.K = pr_of(ctx), np_, 2, n, K
        run("tensor_sum", a, stream, ch.logn)
    else:
        t = abi.TensorArgs()
        t.out, t.d2, t.a0, t.b0 = out.ref(), d2.ref(), A[0].ref(), B[0].ref()
        if np_ == 2:
            t.a1, t.b1 = A[1].ref(), B[1].ref()
        t.pr, t.npairs, t.acc, t.n, t.K, t.dbl, t.acc_d2 = pr_of(ctx), np_, int(acc), n, K, int(dbl), int(acc_d2)
        if case == "two_acc_dbl_coef":
            t.coef, t.coef_ct_stride = coef.ptr.value, ch.rows * ch.n
        if ysub is not None:
            ya = abi.TensorYArgs()
            ya.t, ya.y, ya.c, ya.cs, ya.sub = t, y.ref(), yv.ptr.value, ys.ptr.value, int(ysub)
            run("tensor_y", ya, stream, ch.logn)
        else:
            run("tensor", t, stream, ch.logn)
    got, gd2 = out.get(), d2.get()
    assert (got[:, 0, :n] == want[0]).all() and (got[:, 1, :n] == want[1]).all()
    assert (gd2[:, 1, :n] == want[2]).all()
    assert (gd2[:, 0] == d2.host[:, 0]).all(), "part 0 of d2 is not an output"
    assert (got[:, :, n:] == out.host[:, :, n:]).all(), "rows past n untouched"
    if case == "two_acc_dbl_coef":
        assert (coef.download((K, ch.rows, ch.n))[:, :n] == want[2]).all()


# ----------------------------------------------------------------------------------------------- epilogues
@pytest.mark.parametrize("case", ["plain", "dbl_k", "to_add", "to_sub"])
def test_md_epilogue(stream, case):
    name = "small31"
    say(f"[md_epilogue] {name} {case}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(len(case) * 7)
    K, n, q = 2, 6, ch.primes
    dst, x, t, a = (Cts(ch, K, n, rng) for _ in range(4))
    binv = [int(rng.integers(1, p)) for p in q]
    bv, bs = consts(ch, binv)
    k = [int(p) + 3 if i % 2 else int(rng.integers(0, p)) for i, p in enumerate(q)]
    kb = raw(k)
    sl = lambda c: c.host[:, :, :n]
    m = abi.MdEpiArgs()
    m.dst, m.x, m.t, m.binv, m.binvs, m.pr, m.n, m.K = dst.ref(), x.ref(), t.ref(), bv.ptr.value, bs.ptr.value, \
        pr_of(ctx), n, K
    if case.startswith("to"):
        sub = case == "to_sub"
        want = em.md_epilogue_to(q, sl(a), sl(x), sl(t), binv, sub)
        b = abi.MdEpiToArgs()
        b.m, b.a, b.sub = m, a.ref(), int(sub)
        run("md_epilogue_to", b, stream, ch.logn)
    else:
        dbl = case == "dbl_k"
        want = em.md_epilogue(q, sl(dst), sl(x), sl(t), binv, k if dbl else None, dbl)
        m.dbl = int(dbl)
        if dbl:
            m.k = kb.ptr.value
        run("md_epilogue", m, stream, ch.logn)
    got = dst.get()
    assert (got[:, :, :n] == want).all()
    assert (got[:, :, n:] == dst.host[:, :, n:]).all()


# ----------------------------------------------------------------------------------------------- weighted sums
@pytest.mark.parametrize("case", ["wsum", "wsum_k", "multi"])
def test_wsum(stream, case):
    name = "small31"
    say(f"[wsum] {name} {case}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(len(case) * 13)
    K, n, q, ns = 2, 6, ch.primes, 7
    srcs = [Cts(ch, K, n, rng) for _ in range(ns)]
    rowstride = ch.rows + 3
    nout = 3 if case == "multi" else 1
    ws, wbufs, kbufs, ks, outs = [], [], [], [], []
    for m in range(nout):
        w = np.zeros((ns, rowstride), np.uint64)
        for j in range(ns):
            w[j, : ch.rows] = [int(rng.integers(0, p)) for p in q]
        wv = w.astype(np.uint32)
        wsh = np.zeros_like(wv)
        for j in range(ns):
            wsh[j, : ch.rows] = [(int(x) << 32) // int(p) for x, p in zip(wv[j, : ch.rows], q)]
        ws.append(wv)
        wbufs.append((pa.DevBuf.from_array(wv), pa.DevBuf.from_array(wsh)))
        k = [int(rng.integers(0, 2 * p)) for p in q]
        ks.append(k)
        kbufs.append(raw(k))
        outs.append(Cts(ch, K, n, rng))
    nrow = [n, n - 1, n - 3][:nout]
    if case == "multi":
        a = abi.WsumMultiArgs()
        for m in range(nout):
            a.out[m] = outs[m].ref()
            a.w[m], a.ws[m] = wbufs[m][0].ptr.value, wbufs[m][1].ptr.value
            a.k[m] = kbufs[m].ptr.value if m != 1 else None
            a.n[m] = nrow[m]
        for j in range(ns):
            a.src[j] = srcs[j].ref()
        a.pr, a.nout, a.nsrc, a.rowstride, a.K, a.nmax = pr_of(ctx), nout, ns, rowstride, K, n
        run("wsum_multi", a, stream, ch.logn)
    else:
        w = abi.WsumArgs()
        w.out = outs[0].ref()
        for j in range(ns):
            w.src[j] = srcs[j].ref()
        w.w, w.ws, w.pr, w.nsrc, w.rowstride, w.n, w.K = wbufs[0][0].ptr.value, wbufs[0][1].ptr.value, pr_of(ctx), \
            ns, rowstride, n, K
        if case == "wsum_k":
            wk = abi.WsumKArgs()
            wk.w, wk.k = w, kbufs[0].ptr.value
            run("wsum_k", wk, stream, ch.logn)
        else:
            run("wsum", w, stream, ch.logn)
    for m in range(nout):
        rows = nrow[m]
        withk = case == "wsum_k" or (case == "multi" and m != 1)
        want = em.wsum(q, [s.host[:, :, :rows] for s in srcs], [list(ws[m][j, :rows]) for j in range(ns)],
                       ks[m] if withk else None)
        got = outs[m].get()
        assert (got[:, :, :rows] == want).all(), f"output {m}"
        assert (got[:, :, rows:] == outs[m].host[:, :, rows:]).all()


def test_add_const(stream):
    name = "small31"
    say(f"[add_const] {name}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(3)
    K, n = 2, 7
    x = Cts(ch, K, n, rng)
    k = [int(rng.integers(0, 2 * p)) for p in ch.primes]
    kb = raw(k)
    want = em.add_const(ch.primes, x.host[:, :, :n], k)
    a = abi.AddConstArgs()
    a.x, a.k, a.pr, a.n, a.K = x.ref(), kb.ptr.value, pr_of(ctx), n, K
    run("add_const", a, stream, ch.logn)
    got = x.get()
    assert (got[:, :, :n] == want).all() and (got[:, :, n:] == x.host[:, :, n:]).all()


# ----------------------------------------------------------------------------------------------- plaintext tables
@pytest.mark.parametrize("case", ["table", "add", "sub", "rsub", "add_alias_y", "n8_y", "n3_lazy"])
def test_mul(stream, case):
    name = "small31"
    say(f"[mul] {name} {case}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(len(case) * 31)
    K, n, q = 2, 6, ch.primes
    sl = lambda c: c.host[:, :, :n]
    nterm = 8 if case == "n8_y" else 3 if case == "n3_lazy" else 1
    xs = [Cts(ch, K, n, rng) for _ in range(nterm)]
    ts = [table(ch, n, rng) for _ in range(nterm)]
    tb = [pa.DevBuf.from_array(t) for t in ts]
    y, out = Cts(ch, K, n, rng), Cts(ch, K, n, rng)
    mode = {"add": 0, "sub": 1, "rsub": 2, "add_alias_y": 0, "n8_y": 0}.get(case)
    want = em.mul_add_n(q, [(sl(x), t) for x, t in zip(xs, ts)], None if mode is None else sl(y), mode or 0)
    if case == "add_alias_y":
        out = y
    m = abi.MulTableArgs()
    m.out, m.in_, m.t, m.pr, m.n, m.K = out.ref(), xs[0].ref(), tb[0].ptr.value, pr_of(ctx), n, K
    if case == "table":
        run("mul_table", m, stream, ch.logn)
    elif nterm == 1:
        a = abi.MulAddArgs()
        a.m, a.y, a.sub = m, y.ref(), mode
        run("mul_add", a, stream, ch.logn)
    else:
        a = abi.MulAddNArgs()
        a.out = out.ref()
        if mode is not None:
            a.y = y.ref()
        for j in range(nterm):
            a.x[j], a.t[j] = xs[j].ref(), tb[j].ptr.value
        a.pr, a.n, a.K, a.nterm, a.lazy = pr_of(ctx), n, K, nterm, int(case == "n3_lazy")
        run("mul_add_n", a, stream, ch.logn)
    got = out.get()
    assert (got[:, :, :n] == want).all()
    assert (got[:, :, n:] == out.host[:, :, n:]).all()


@pytest.mark.parametrize("to", [False, True])
def test_rescale_combine(stream, to):
    name = "small31"
    say(f"[rescale_combine] {name} to={to}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(40 + to)
    K, n, q = 2, 5, ch.primes
    x, tmp, out = Cts(ch, K, n, rng), Cts(ch, K, n, rng), Cts(ch, K, n, rng)
    alpha = [int(rng.integers(0, p)) for p in q]
    av, as_ = consts(ch, alpha)
    want = em.combine(q, x.host[:, :, :n], tmp.host[:, :, :n], alpha)
    a = abi.RescaleCombineArgs()
    a.x, a.tmp, a.alpha, a.alphas, a.pr, a.n, a.K = x.ref(), tmp.ref(), av.ptr.value, as_.ptr.value, pr_of(ctx), n, K
    if to:
        b = abi.RescaleCombineToArgs()
        b.a, b.out = a, out.ref()
        run("rescale_combine_to", b, stream, ch.logn)
        assert (x.get() == x.host).all(), "x is read only"
        got = out.get()
        assert (got[:, :, n:] == out.host[:, :, n:]).all()
    else:
        run("rescale_combine", a, stream, ch.logn)
        got = x.get()
    assert (got[:, :, :n] == want).all()


def test_pointer_lists(stream):
    name = "small31"
    say(f"[ew_many / submul_many] {name}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(77)
    n, npoly, q = 6, 5, ch.primes
    rows = lambda: np.stack([rng.integers(0, ch.primes[r], ch.n) for r in range(n)]).astype(np.uint32)
    A = [rows() for _ in range(npoly)]
    B = [rows() for _ in range(npoly)]
    Cc = [rows() for _ in range(npoly)]
    t = rows()
    bufs = {k: [pa.DevBuf.from_array(v) for v in vs] for k, vs in (("a", A), ("b", B), ("c", Cc))}
    outs = [pa.DevBuf(n * ch.n) for _ in range(npoly)]
    tb = pa.DevBuf.from_array(t)
    a = abi.EwManyArgs()
    for j in range(npoly):
        a.out[j], a.a[j] = outs[j].ptr.value, bufs["a"][j].ptr.value
        a.b[j] = bufs["b"][j].ptr.value if j % 2 == 0 else None
        a.c[j] = bufs["c"][j].ptr.value if j % 3 == 0 else None
    a.pr, a.n, a.nrows = pr_of(ctx), npoly, n
    run("ew_many", a, stream, ch.logn)
    for j in range(npoly):
        want = em.ew_many(q, A[j], B[j] if j % 2 == 0 else None, Cc[j] if j % 3 == 0 else None)
        assert (outs[j].download((n, ch.n)) == want).all(), f"ew_many {j}"
    s = abi.SubMulManyArgs()
    for j in range(npoly):
        s.out[j], s.a[j], s.b[j] = outs[j].ptr.value, bufs["a"][j].ptr.value, bufs["b"][j].ptr.value
    s.t, s.pr, s.n, s.nrows = tb.ptr.value, pr_of(ctx), npoly, n
    run("submul_many", s, stream, ch.logn)
    for j in range(npoly):
        assert (outs[j].download((n, ch.n)) == em.submul_many(q, A[j], B[j], t)).all(), f"submul_many {j}"


# ----------------------------------------------------------------------------------------------- composite rescale
class RescaleTabs:
    def __init__(self, ch, top, ndrop, fold=None):
        c = em.rescale_consts(ch.primes, top, ndrop)
        alpha = list(c["alpha"])
        self.ca = self.cb = 1
        if fold is not None:
            self.ca, self.cb = fold[top] % ch.primes[top], fold[top - 1] % ch.primes[top - 1]
            alpha = [a * (fold[i] % ch.primes[i]) % ch.primes[i] for i, a in enumerate(alpha)]
        self.c = c
        self.A, self.As = consts(ch, c["A"])
        self.B, self.Bs = consts(ch, c["B"])
        self.al, self.als = consts(ch, alpha)
        self.qam, self.qbm = raw(c["qam"] + [0] * ch.rows), raw(c["qbm"] + [0] * ch.rows)

    def args(self, ctx, x, tmp, top, ndrop, K):
        r = abi.RescaleArgs()
        r.x, r.tmp = x.ref(), tmp.ref()
        r.A, r.As, r.B, r.Bs = self.A.ptr.value, self.As.ptr.value, self.B.ptr.value, self.Bs.ptr.value
        r.qam, r.qbm, r.pr = self.qam.ptr.value, self.qbm.ptr.value, pr_of(ctx)
        r.qinv_ab, r.C_ab, r.ca, r.cb = self.c["qinv_ab"], self.c["C_ab"], self.ca, self.cb
        r.top, r.nrows, r.K, r.ndrop = top, top + 1 - ndrop, K, ndrop
        return r


def coef_tops(oc, x, top):
    """x with its rows top - 1, top taken to coefficient form (what the rescale's first step, an INTT, leaves)"""
    y = x.copy()
    for k in range(x.shape[0]):
        for part in range(2):
            y[k, part, top - 1:top + 1] = oc.ntt_inv(x[k, part, top - 1:top + 1].copy(), [top - 1, top])
    return y


@pytest.mark.parametrize("name,ndrop,fold", [("small31", 1, False), ("small31", 2, False), ("small31", 2, True),
                                             ("small", 1, True)])
def test_rescale_coef(stream, name, ndrop, fold):
    say(f"[rescale_coef] {name} ndrop={ndrop} fold={fold}")
    ch, ctx, oc = contexts(name)
    rng = np.random.default_rng(ndrop * 10 + fold)
    K, top = 2, len(ch.q) - 1
    x = Cts(ch, K, top + 1, rng)
    xc = coef_tops(oc, x.host, top)
    x.buf.upload(xc)
    tmp = Cts(ch, K, 0, rng)
    f = [int(rng.integers(2, p)) for p in ch.primes] if fold else None
    T = RescaleTabs(ch, top, ndrop, f)
    run("rescale_coef", T.args(ctx, x, tmp, top, ndrop, K), stream, ch.logn)
    got = tmp.get()
    rows = top + 1 - ndrop
    for k in range(K):
        for part in range(2):
            want, _ = em.rescale_coef(ch.primes, xc[k, part, top], xc[k, part, top - 1], top, ndrop, T.c, T.ca, T.cb)
            assert (got[k, part, :rows] == want).all(), (k, part)


def ntt_args(ctx, ch, base, rows, K, epi_out=None, es=None):
    """NttArgs of the tmp rows (c, part, r < rows) of K ciphertexts, epilogue 3 onto epi_out (x) when given"""
    roff = [(c * 2 + part) * ch.rows + r for c in range(K) for part in range(2) for r in range(rows)]
    ids = [r for c in range(K) for part in range(2) for r in range(rows)]
    bo, bi = pa.DevBuf.from_array(np.array(roff, np.uint32)), pa.DevBuf.from_array(np.array(ids, np.int32).view(np.uint32))
    a = abi.NttArgs()
    a.base, a.roff, a.rprime = base.buf.ptr.value, bo.ptr.value, bi.ptr.value
    a.fw, a.fws, a.iw, a.iws = (LIB.pcx_ctx_twiddle(ctx.h, w) for w in range(4))
    a.ninv, a.ninvs = LIB.pcx_ctx_twiddle(ctx.h, 4), LIB.pcx_ctx_twiddle(ctx.h, 5)
    a.pr, a.nrows = pr_of(ctx), len(roff)
    a.lazy = int(max(ch.primes) < (1 << 30))
    if epi_out is not None:
        a.epi, a.eout, a.ex, a.xnum = 3, epi_out.buf.ptr.value, epi_out.buf.ptr.value, 1
        a.es, a.ess = es[0].ptr.value, es[1].ptr.value
    return a, (bo, bi)


@pytest.mark.parametrize("name,fold", [("small31", False), ("small", True), ("c3", False)])
def test_rescale_fwd(stream, name, fold):
    say(f"[rescale_fwd] {name} fold={fold}")
    ch, ctx, oc = contexts(name)
    rng = np.random.default_rng(5 + fold)
    K, top = (1 if name == "c3" else 2), len(ch.q) - 1
    x = Cts(ch, K, top + 1, rng)
    f = [int(rng.integers(2, p)) for p in ch.primes] if fold else None
    want = em.rescale(oc, ch.primes, x.host[:, :, : top + 1], top, 2, fold=f)
    x.buf.upload(coef_tops(oc, x.host, top))
    tmp = Cts(ch, K, 0, rng)
    T = RescaleTabs(ch, top, 2, f)
    nt, keep = ntt_args(ctx, ch, tmp, top - 1, K, x, (T.al, T.als))
    a = abi.RescaleNttArgs()
    a.rs, a.ntt = T.args(ctx, x, tmp, top, 2, K), nt
    run("rescale_fwd", a, stream, ch.logn)
    got = x.get()
    assert (got[:, :, : top - 1] == want).all()


# ----------------------------------------------------------------------------------------------- encryption
@pytest.mark.parametrize("name,with_m,with_c1,alias_e", [("small31", True, True, False), ("rej", False, True, True),
                                                        ("small", True, False, True), ("c3", False, True, True)])
def test_encrypt(stream, name, with_m, with_c1, alias_e):
    say(f"[encrypt] {name} m={with_m} c1={with_c1} e_in_c0={alias_e}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(len(name) + 2 * with_m + with_c1)
    nl, n = len(ch.q), ch.n
    rows = lambda: np.stack([rng.integers(0, ch.primes[r], n) for r in range(nl)]).astype(np.uint32)  # noqa: E731
    s, e, m = rows(), rows(), rows()
    seed = [int(v) for v in rng.integers(0, 1 << 32, 8, dtype=np.uint64)]
    nonce = 12345
    a_rows = np.stack([twin.expand_row(seed, nonce, ch.primes[r], n, twin.TAG_ENCA) for r in range(nl)])
    want = em.encrypt(ch.primes, a_rows, s, e, m if with_m else None)
    bs, bm, bseed = pa.DevBuf.from_array(s), pa.DevBuf.from_array(m), pa.DevBuf.from_array(np.array(seed, np.uint32))
    c0 = pa.DevBuf.from_array(e if alias_e else np.zeros_like(e))
    be = c0 if alias_e else pa.DevBuf.from_array(e)
    c1 = pa.DevBuf(nl * n)
    a = abi.EncryptArgs()
    a.c0, a.c1, a.s, a.e = c0.ptr.value, c1.ptr.value if with_c1 else None, bs.ptr.value, be.ptr.value
    a.m, a.seed, a.pr, a.nonce, a.nl = bm.ptr.value if with_m else None, bseed.ptr.value, pr_of(ctx), nonce, nl
    run("encrypt", a, stream, ch.logn)
    assert (c0.download((nl, n)) == want).all()
    if with_c1:
        assert (c1.download((nl, n)) == a_rows).all()


# ----------------------------------------------------------------------------------------------- BSGS plaintext dot
# the register form in groups of 4 or 8 baby steps (full, compact and masked diagonal indices, a last giant step
# short of diagonals): one group up to 8, two or three past it (a short last group; 16 babies x 4 giant steps, a
# SlotToCoeff stage's shape; K ciphertexts sharing the diagonals)
@pytest.mark.parametrize("name,enc,K,B,G,npts", [("small31", 0xFFFFFFFF, 2, 3, 2, 5), ("small31", 0x7F000003, 3, 3, 2, 5),
                                                ("small", 0x3FF, 1, 3, 2, 5), ("c3", 0xFFFFFFFF, 1, 3, 2, 5),
                                                ("small31", 0x7F000004, 2, 8, 3, 21), ("small31", 0xFFFFFFFF, 1, 7, 2, 14),
                                                ("small", 0x7F000001, 1, 6, 2, 9), ("small31", 0x7F000002, 1, 9, 2, 11),
                                                ("small31", 0xFFFFFFFF, 2, 16, 4, 63), ("small", 0x7F000003, 1, 16, 2, 25),
                                                ("small31", 0x1FF, 3, 24, 2, 40), ("c3", 0x7F000002, 1, 16, 4, 63)])
def test_pt_dot(stream, name, enc, K, B, G, npts):
    say(f"[pt_dot] {name} enc={enc:#x} K={K} B={B} G={G} npts={npts}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(enc % 1000 + K + B)
    top = len(ch.q) - 1 if name == "c3" else len(ch.q) - 2
    rows = list(range(top + 1)) + [len(ch.q) + j for j in range(len(ch.p))]
    n, R = len(rows), ch.rows
    # rotations (c, b): K x B extended ciphertexts [2][R][N] (rows of the row set filled); results K x G
    rot = np.zeros((K, B, 2, R, ch.n), np.uint32)
    for t in rows:
        rot[:, :, :, t] = rng.integers(0, ch.primes[t], (K, B, 2, ch.n))
    ptw = ch.n if enc == 0xFFFFFFFF else (ch.n >> (enc & 0xFF) if enc >> 24 == 0x7F else enc + 1)
    pt_prow = top + 1  # the special rows' diagonal rows follow the Q rows
    pts = [np.stack([rng.integers(0, ch.primes[t], ptw) for t in rows]).astype(np.uint32) for _ in range(npts)]
    pbufs = [pa.DevBuf.from_array(p) for p in pts]
    ptrs = pa.DevBuf.from_array(np.array([b.ptr.value for b in pbufs], np.uint64).view(np.uint32))
    brot = pa.DevBuf.from_array(rot)
    res = pa.DevBuf(K * G * 2 * R * ch.n)
    a = abi.PtDotArgs()
    a.rot = abi.PolyRef(brot.ptr.value, B * 2 * R * ch.n, R * ch.n)
    a.res = abi.PolyRef(res.ptr.value, G * 2 * R * ch.n, R * ch.n)
    a.rot_stride, a.res_stride = 2 * R * ch.n, 2 * R * ch.n
    a.pts, a.pr = ptrs.ptr.value, pr_of(ctx)
    a.rs = abi.RowSet(top + 1, len(ch.p), len(ch.q), 0)
    a.npts, a.bstep, a.gstep, a.K, a.ptw, a.pt_prow, a.enc = npts, B, G, K, ptw, pt_prow, enc
    run("pt_dot", a, stream, ch.logn)
    got = res.download((K, G, 2, R, ch.n))
    q = [ch.primes[t] for t in rows]
    want = em.pt_dot(q, rot[:, :, :, rows], pts, B, G, npts, enc, list(range(n)))
    assert (got[:, :, :, rows] == want).all()


# ----------------------------------------------------------------------------------------------- subring switch
@pytest.mark.parametrize("name,sub,K", [("small31", 4, 2), ("small", 16, 1), ("c3", 2, 1)])
def test_pack(stream, name, sub, K):
    say(f"[pack_split / pack_dot] {name} sub={sub} K={K}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(sub * 5 + K)
    nq = len(ch.q) - 1 if name == "c3" else 4
    kp = len(ch.p)
    rows = list(range(nq)) + [len(ch.q) + j for j in range(kp)]
    n, N = len(rows), ch.n
    # split: Q rows from one buffer, special rows from another
    xq = np.stack([np.stack([rng.integers(0, ch.primes[t], N) for t in rows[:nq]]) for _ in range(K)]).astype(np.uint32)
    xp = np.stack([np.stack([rng.integers(0, ch.primes[t], N) for t in rows[nq:]]) for _ in range(K)]).astype(np.uint32)
    bq, bp = pa.DevBuf.from_array(xq), pa.DevBuf.from_array(xp)
    dig = pa.DevBuf(K * sub * n * N)
    a = abi.PackSplitArgs()
    a.q, a.p, a.out = bq.ptr.value, bp.ptr.value, dig.ptr.value
    a.q_stride, a.p_stride, a.out_stride = nq * N, kp * N, sub * n * N
    a.K, a.sub, a.nq, a.nrows = K, sub, nq, n
    run("pack_split", a, stream, ch.logn)
    got = dig.download((K, sub, n, N))
    for c in range(K):
        assert (got[c] == em.pack_split(np.concatenate([xq[c], xp[c]]), sub)).all(), c
    # dot: the digits (taken as evaluation-form words) against a random pack key; c0 and outputs in prime-id rows
    q = [ch.primes[t] for t in rows]
    kb = np.stack([np.stack([rng.integers(0, p, N) for p in q]) for _ in range(sub)]).astype(np.uint32)
    ka = np.stack([np.stack([rng.integers(0, p, N) for p in q]) for _ in range(sub)]).astype(np.uint32)
    c0 = np.zeros((K, ch.rows, N), np.uint32)
    for t in range(ch.rows):
        c0[:, t] = rng.integers(0, ch.primes[t], (K, N))
    big_p = 1
    for x in ch.p:
        big_p *= int(x)
    pm = [big_p % int(p) for p in ch.primes]
    pmv, pms = consts(ch, pm)
    bkb, bka, bc0 = pa.DevBuf.from_array(kb), pa.DevBuf.from_array(ka), pa.DevBuf.from_array(c0)
    brows = pa.DevBuf.from_array(np.array(rows, np.uint32))
    o0, o1 = pa.DevBuf(K * ch.rows * N), pa.DevBuf(K * ch.rows * N)
    d = abi.PackDotArgs()
    d.dig, d.kb, d.ka, d.c0, d.out0, d.out1 = dig.ptr.value, bkb.ptr.value, bka.ptr.value, bc0.ptr.value, \
        o0.ptr.value, o1.ptr.value
    d.rows, d.pmod, d.pmods, d.pr = brows.ptr.value, pmv.ptr.value, pms.ptr.value, pr_of(ctx)
    d.dig_stride, d.ct_stride, d.out_ct_stride = sub * n * N, ch.rows * N, ch.rows * N
    d.K, d.sub, d.nq, d.nrows = K, sub, nq, n
    run("pack_dot", d, stream, ch.logn)
    g0, g1 = o0.download((K, ch.rows, N)), o1.download((K, ch.rows, N))
    for c in range(K):
        w0, w1 = em.pack_dot(q, got[c], kb, ka, c0[c][rows], [pm[t] for t in rows], nq)
        assert (g0[c][rows] == w0).all() and (g1[c][rows] == w1).all(), c


@pytest.mark.parametrize("nout,npairs,acc", [(3, 20, 0), (1, 32, 2), (4, 5, 1)])
def test_tensor_multi(stream, nout, npairs, acc):
    name = "small31"
    say(f"[tensor_multi] {name} nout={nout} npairs={npairs} acc={acc}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(nout * 100 + npairs + acc)
    K, n, q = 1, 4, ch.primes
    # a small pool of operands shared across the outputs' lists
    pool = [Cts(ch, K, n, rng) for _ in range(6)]
    pick = rng.integers(0, len(pool), (nout, npairs, 2))
    outs, d2s = [Cts(ch, K, n, rng) for _ in range(nout)], [Cts(ch, K, n, rng) for _ in range(nout)]
    a = abi.TensorMultiArgs()
    for o in range(nout):
        a.out[o], a.d2[o] = outs[o].ref(), d2s[o].ref()
        for j in range(npairs):
            a.a[o][j], a.b[o][j] = pool[pick[o, j, 0]].ref(), pool[pick[o, j, 1]].ref()
    a.pr, a.nout, a.npairs, a.acc, a.n, a.K = pr_of(ctx), nout, npairs, acc, n, K
    sl = lambda c: c.host[:, :, :n]  # noqa: E731
    want = [em.tensor(q, [(sl(pool[pick[o, j, 0]]), sl(pool[pick[o, j, 1]])) for j in range(npairs)], sl(outs[o]),
                      d2s[o].host[:, 1, :n], acc != 0, (acc & 2) != 0) for o in range(nout)]
    run("tensor_multi", a, stream, ch.logn)
    for o in range(nout):
        got, gd2 = outs[o].get(), d2s[o].get()
        assert (got[:, 0, :n] == want[o][0]).all() and (got[:, 1, :n] == want[o][1]).all(), o
        assert (gd2[:, 1, :n] == want[o][2]).all(), o


# ----------------------------------------------------------------------------------------------- coeff_sum
@pytest.mark.parametrize("name,nterm,L,acc,big", [("small", 3, 6, False, True), ("small31", 5, 9, True, False),
                                                  ("c3", 32, 36, False, False)])
def test_coeff_sum(stream, name, nterm, L, acc, big):
    """coeff_sum through the table: float32 weight rows rounded at a scale (ties, clamped values counted), NTT'd in the
    scratch (dense rows; 32 x 36 = 1152 rows of N = 2^16 take the one-pass transform), summed against the
    ciphertexts, onto the old output or not"""
    say(f"[coeff_sum] {name} n={nterm} L={L} acc={acc} clamp={big}")
    ch, ctx, oc = contexts(name)
    N, R = ch.n, ch.rows
    rng = np.random.default_rng(nterm * 7 + L)
    q = [int(p) for p in ch.primes[:L]]
    scale = 2.0 ** 20
    rows = (rng.normal(size=(nterm, N)) * 3e4).astype(np.float32)
    rows[0, :6] = [0.5 / scale, 1.5 / scale, 2.5 / scale, -0.5 / scale, -2.5 / scale, 7.0]
    if big:
        rows[1, :3] = [1e19, -3e30, 2e18]
    cts = [np.zeros((2, R, N), np.uint32) for _ in range(nterm)]
    for c in cts:
        for part in range(2):
            c[part, :L] = np.stack([rng.integers(0, p, N) for p in q])
    old = np.zeros((2, R, N), np.uint32)
    for part in range(2):
        old[part, :L] = np.stack([rng.integers(0, p, N) for p in q])
    bct = [pa.DevBuf.from_array(c) for c in cts]
    brow = [pa.DevBuf.from_array(r.view(np.uint32)) for r in rows]
    out = pa.DevBuf.from_array(old)
    scratch = pa.DevBuf(nterm * L * N)
    ovf = pa.DevBuf.from_array(np.zeros(2, np.uint32))
    a = abi.CoeffArgs()
    a.scratch, a.out = scratch.ptr.value, out.ptr.value
    a.fw, a.fws = LIB.pcx_ctx_twiddle(ctx.h, 0), LIB.pcx_ctx_twiddle(ctx.h, 1)
    a.pr, a.overflow = pr_of(ctx), ovf.ptr.value
    a.part_stride, a.scale, a.n, a.L, a.accumulate = R * N, scale, nterm, L, int(acc)
    for r in range(nterm):
        a.rows[r], a.ct[r] = brow[r].ptr.value, bct[r].ptr.value
    run("coeff_sum", a, stream, ch.logn)
    got = out.download((2, R, N))
    twin.set_threads(16)
    want, want_ovf = em.coeff_sum(q, rows, scale, [c[:, :L] for c in cts], oc.ntt_fwd,
                                  out=old[:, :L] if acc else None)
    assert (got[:, :L] == want).all()
    assert int(ovf.download().view(np.uint64)[0]) == want_ovf
    if not acc:
        assert (got[:, L:] == old[:, L:]).all(), "rows past L untouched"


# ----------------------------------------------------------------------------------------------- tensor_seeded
@pytest.mark.parametrize("name,nout,npairs,nq,packed,acc", [("small", 2, 3, 1, False, 0), ("small28", 5, 34, 2, True, 1),
                                                           ("c3", 1, 2, 1, False, 3)])
def test_tensor_seeded(stream, name, nout, npairs, nq, packed, acc):
    """tensor_seeded through the table: seeded first operands (c0 stored plain or as 28-bit streams, c1 drawn by the
    "CTSA" expander in the kernel), 5 outputs x 34 pairs cross the launcher's 4 x 32 chunks, two second-operand sets,
    accumulate modes"""
    say(f"[tensor_seeded] {name} nout={nout} npairs={npairs} nq={nq} packed={packed} acc={acc}")
    ch, ctx, _ = contexts(name)
    N, R = ch.n, ch.rows
    n = 4 if name == "c3" else len(ch.q)
    q = [int(p) for p in ch.primes]
    rng = np.random.default_rng(nout * 10 + npairs + acc)
    roww = (N * 28 + 31) // 32
    c0s, seeds, abufs = [], [], []
    for o in range(nout):
        rc, rs, rb = [], [], []
        for j in range(npairs):
            c0 = np.stack([rng.integers(0, min(q[r], 1 << 28), N) for r in range(n)]).astype(np.uint32)
            sd = rng.integers(0, 1 << 32, (n, 8), dtype=np.uint64).astype(np.uint32)
            body = em.pack28(c0) if packed else c0
            buf = np.concatenate([body.reshape(-1), sd.reshape(-1)])
            rc.append(c0)
            rs.append(sd)
            rb.append(pa.DevBuf.from_array(buf))
        c0s.append(rc)
        seeds.append(rs)
        abufs.append(rb)
    seed_off = n * (roww if packed else N)
    bsets = [[np.zeros((2, R, N), np.uint32) for _ in range(npairs)] for _ in range(nq)]
    for bs in bsets:
        for b in bs:
            for part in range(2):
                b[part, :n] = np.stack([rng.integers(0, q[r], N) for r in range(n)])
    bbufs = [[pa.DevBuf.from_array(b) for b in bs] for bs in bsets]
    M = nq * nout
    old = np.zeros((M, 2, R, N), np.uint32)
    for m in range(M):
        for part in range(2):
            old[m, part, :n] = np.stack([rng.integers(0, q[r], N) for r in range(n)])
    outb = pa.DevBuf.from_array(old)
    d2b = pa.DevBuf.from_array(old)  # d2 goes to part 1 of each d2 ciphertext
    a = abi.TensorSeededArgs()
    cw = 2 * R * N
    for m in range(M):
        a.out[m] = abi.PolyRef(outb.ptr.value + 4 * m * cw, cw, R * N)
        a.d2[m] = abi.PolyRef(d2b.ptr.value + 4 * m * cw, cw, R * N)
    for j in range(npairs):
        a.b[j] = abi.PolyRef(bbufs[0][j].ptr.value, cw, R * N)
        for qs in range(1, nq):
            a.bq[qs - 1][j] = bbufs[qs][j].ptr.value
        for o in range(nout):
            a.a[o][j] = abufs[o][j].ptr.value
    a.pr, a.seed_off = pr_of(ctx), seed_off
    a.nout, a.npairs, a.acc, a.n, a.packed, a.nq = nout, npairs, acc, n, int(packed), nq
    run("tensor_seeded", a, stream, ch.logn)
    got = outb.download((M, 2, R, N))
    got_d2 = d2b.download((M, 2, R, N))[:, 1]
    want, want_d2 = em.tensor_seeded(q, c0s, seeds, [[b[:, :n] for b in bs] for bs in bsets], acc=acc,
                                     old=old[:, :, :n], old_d2=old[:, 1, :n], cts_row=twin.cts_expand_row)
    assert (got[:, :, :n] == want).all()
    assert (got_d2[:, :n] == want_d2).all()
