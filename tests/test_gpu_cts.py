"""Parity of the fused CtS stage (hoisted baby rotations times the BSGS diagonals) with the oracle, word for word:
the driver's stage (ModUp + cts_fused_regen) and the kernel table's two entries called directly with the ABI structs
(crates/pc-kernels/kernels/cts.cuh; args.cuh CtsArgs / CtsRegenArgs). Each test prints its case before the GPU runs.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import abi
from perseus_amd._lib import LIB
from tests import twin

pytestmark = pytest.mark.gpu

FULL = 0xFFFFFFFF


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


def random_ct(ch, top, rng):
    ct = np.zeros((2, ch.rows, ch.n), np.uint32)
    for t in range(top + 1):
        ct[:, t] = rng.integers(0, ch.primes[t], (2, ch.n))
    return ct


def diagonals(ch, top, npts, ptw, rng):
    return [np.stack([rng.integers(0, ch.primes[t], ptw) for t in ext_rows(ch, top)]).astype(np.uint32)
            for _ in range(npts)]


def ptw_of(ch, enc):
    if enc == FULL:
        return ch.n
    if enc >> 24 == 0x7F:
        return ch.n >> (enc & 0xFF)
    return enc + 1


def dev_ptrs(bufs):
    """A device array of the buffers' device addresses (uint64), for the ABI's pointer arrays."""
    a = np.array([b.ptr.value for b in bufs], np.uint64)
    return pa.DevBuf.from_array(a.view(np.uint32))


def oracle_keys(oc, ch, steps, seed):
    g = twin.Prng([seed, 9, 8, 7, 6, 5, 4, 3], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
    gals = [twin.rotation_galois(r, ch.n) for r in steps]
    keys = [oc.rotation_key(g, s_eval, x) for x in gals]
    return gals, np.stack([k[0] for k in keys]), [k[1] for k in keys]


# ----------------------------------------------------------------------------------------------- driver stage
@pytest.mark.parametrize("name,B,G,npts,enc,top,bits", [
    ("small", 4, 2, 8, FULL, 5, 0),
    ("small", 3, 4, 10, 0x7F000003, 3, 0),    # four giant steps in one launch, the last two diagonals missing
    ("small31", 5, 3, 15, 0x7FF, 5, 31),      # packed b, periodic diagonals, a second launch for giant step 2
    ("c3", 5, 2, 10, FULL, 29, 0),            # the C3 chain at its full shape
    ("rej", 4, 2, 8, FULL, 5, 0),             # a third of the KSKA words rejected: the wave's redraw queue
    ("small28", 9, 4, 33, FULL, 5, 28),       # 28-bit primes, more than 8 baby steps: the reference's own regime
])
@pytest.mark.parametrize("route", ["fused", "hoisted"])
def test_cts_stage(stream, name, B, G, npts, enc, top, bits, route):
    """pcx_cts_stage (fused: the cts_fused_regen kernel) and pcx_cts_stage_hoisted (P ct, the babies' dots into a
    workspace of extended ciphertexts, pt_dot over the extended rows) against the oracle's fused stage; the hoisted
    route's results then through pcx_moddown_k (all G in one launch sequence) against the oracle's ModDown of each."""
    say(f"[cts stage] {route} {name} B={B} G={G} npts={npts} enc={enc:#x} top={top} bits={bits}")
    ch, ctx, oc = contexts(name)
    twin.set_threads(16)
    rng = np.random.default_rng(B * 31 + G)
    steps = [3 * i + 1 for i in range(1, B)]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=B + 10 * G)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=bits)
    ct = random_ct(ch, top, rng)
    ptw = ptw_of(ch, enc)
    pts = diagonals(ch, top, npts, ptw, rng)
    pbufs = [pa.DevBuf.from_array(p) for p in pts]
    ptrs = dev_ptrs(pbufs)
    dev = pa.DevBuf.from_array(ct)
    res = ctx.ct_buf(G)
    if route == "fused":
        ctx.cts_stage(keys, 0, B, G, ptrs, npts, ptw, enc, dev, top, res, stream)
    else:
        rot = ctx.ct_buf(B)
        ctx.cts_stage_hoisted(keys, 0, B, G, ptrs, npts, ptw, enc, dev, top, rot, res, stream)
    stream.sync()
    got = res.download((G, 2, ch.rows, ch.n))
    digits = oc.modup(ct[1], top)
    want = oc.cts_fused(ct[None], digits[None], top, B, G, pts, gals, seeds=seeds, bs=bs, enc=enc)[0]
    rs = ext_rows(ch, top)
    for j in range(G):
        assert (got[j][:, rs] == want[j][:, rs]).all(), j
    if route == "hoisted":
        out = ctx.ct_buf(G)
        ctx.moddown_k(res, top, out, G, stream)
        stream.sync()
        gq = out.download((G, 2, ch.rows, ch.n))
        for j in range(G):
            wq = oc.moddown(want[j].copy(), top)
            assert (gq[j][:, : top + 1] == wq[:, : top + 1]).all(), f"moddown {j}"


# ----------------------------------------------------------------------------------------------- table entries
class Tables:
    """Device tables of a chain the ABI structs point at: rows, digit_of, P mod q and its Shoup companion, primes."""

    def __init__(self, ch, ctx, top):
        nq, kp = len(ch.q), len(ch.p)
        alpha = ch.alpha
        self.rows = ext_rows(ch, top)
        big_p = 1
        for x in ch.p:
            big_p *= int(x)
        pm = [big_p % int(q) for q in ch.q] + [0] * kp
        pms = [(v << 32) // int(q) for v, q in zip(pm, ch.primes)]
        self.b_rows = pa.DevBuf.from_array(np.array(self.rows, np.uint32))
        self.b_dig = pa.DevBuf.from_array(np.array([t // alpha if t < nq else -1 for t in range(nq + kp)],
                                                   np.int32).view(np.uint32))
        self.b_pm = pa.DevBuf.from_array(np.array(pm, np.uint32))
        self.b_pms = pa.DevBuf.from_array(np.array(pms, np.uint32))
        self.pr = LIB.pcx_ctx_primes(ctx.h)

    def fill(self, a, ch, top):
        a.rows, a.digit_of = self.b_rows.ptr.value, self.b_dig.ptr.value
        a.pmod, a.pmods, a.pr = self.b_pm.ptr.value, self.b_pms.ptr.value, self.pr
        a.nq, a.nlive, a.nrows, a.pt_prow = len(ch.q), top + 1, len(self.rows), top + 1


def test_table_cts_fused_resident_keys(stream):
    """cts_fused: two ciphertexts (one group of 2), keys dense and resident (a and b read), periodic diagonals."""
    say("[cts table] cts_fused K=2 B=3 G=2 enc=0x3ff")
    ch, ctx, oc = contexts("small")
    rng = np.random.default_rng(41)
    top, K, B, G, npts, enc = 4, 2, 3, 2, 6, 0x3FF
    R, n = ch.rows, ch.n
    x = np.stack([random_ct(ch, top, rng) for _ in range(K)])
    digits = np.stack([oc.modup(x[c, 1], top) for c in range(K)])
    gals = [twin.rotation_galois(r, n) for r in (5, 17)]
    kb = [np.stack([np.stack([rng.integers(0, p, n) for p in ch.primes]) for _ in range(ch.dnum)]).astype(np.uint32)
          for _ in range(B - 1)]
    ka = [np.stack([np.stack([rng.integers(0, p, n) for p in ch.primes]) for _ in range(ch.dnum)]).astype(np.uint32)
          for _ in range(B - 1)]
    ptw = ptw_of(ch, enc)
    pts = diagonals(ch, top, npts, ptw, rng)
    T = Tables(ch, ctx, top)
    bx, bmu = pa.DevBuf.from_array(x), pa.DevBuf.from_array(digits)
    bres = pa.DevBuf(K * G * 2 * R * n)
    bkb, bka = [pa.DevBuf.from_array(k) for k in kb], [pa.DevBuf.from_array(k) for k in ka]
    pkb, pka = dev_ptrs(bkb), dev_ptrs(bka)
    bkinv = pa.DevBuf.from_array(np.array(gals, np.uint32))
    pbufs = [pa.DevBuf.from_array(p) for p in pts]
    ppts = dev_ptrs(pbufs)
    a = abi.CtsArgs()
    a.x, a.modup, a.res = bx.ptr.value, bmu.ptr.value, bres.ptr.value
    a.kb, a.ka, a.kinv, a.pts = pkb.ptr.value, pka.ptr.value, bkinv.ptr.value, ppts.ptr.value
    T.fill(a, ch, top)
    a.ct_stride, a.part_stride = 2 * R * n, R * n
    a.mu_ct_stride, a.mu_digit_stride, a.key_digit_stride = ch.dnum * R * n, R * n, R * n
    a.K, a.B, a.G, a.npts, a.ndig, a.ptw, a.enc, a.kmax = K, B, G, npts, oc.live_digits(top), ptw, enc, 2
    assert abi.call("cts_fused", a, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bres.download((K, G, 2, R, n))
    want = oc.cts_fused(x, digits, top, B, G, pts, gals, bs=kb, as_=ka, nregen=0, enc=enc)
    rs = T.rows
    assert (got[:, :, :, rs] == want[:, :, :, rs]).all()


@pytest.mark.parametrize("mode", ["x0_tail", "pairs_qtop"])
def test_table_cts_fused_regen(stream, mode):
    """cts_fused_regen. x0_tail: baby 0 taken as stored from x0, `a` regenerated for digit 0 only and read from the
    resident rows above it. pairs_qtop: four giant steps in the K = 1 pair layout (pair_cts), b stored in the compact
    slot order of a key made at limb top q_top (special prime j at slot q_top + 1 + j), block-constant diagonals."""
    say(f"[cts table] cts_fused_regen {mode}")
    ch, ctx, oc = contexts("small31")
    rng = np.random.default_rng(43 if mode == "x0_tail" else 47)
    R, n = ch.rows, ch.n
    if mode == "x0_tail":
        top, B, G, npts, enc, nregen, pair = 5, 4, 2, 8, FULL, 1, 0
    else:
        top, B, G, npts, enc, nregen, pair = 3, 3, 4, 11, 0x7F000002, 3, 5
    nd = oc.live_digits(top)
    x = random_ct(ch, top, rng)
    digits = oc.modup(x[1], top)
    steps = [7 * i for i in range(1, B)]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=77)
    as_ = []
    for i in range(B - 1):
        a_rows = np.zeros((ch.dnum, R, n), np.uint32)
        for d in range(ch.dnum):
            for t in range(R):
                a_rows[d, t] = twin.kska_row(seeds[i], d, ch.primes[t], n) if d < nregen else rng.integers(
                    0, ch.primes[t], n)
        as_.append(a_rows)
    x0 = None
    if mode == "x0_tail":
        x0 = np.stack([np.stack([rng.integers(0, p, n) for p in ch.primes]) for _ in range(2)]).astype(np.uint32)
    ptw = ptw_of(ch, enc)
    pts = diagonals(ch, top, npts, ptw, rng)
    T = Tables(ch, ctx, top)
    # b through the KeyTab: full layout, or compact slots at q_top = top
    if mode == "pairs_qtop":
        srows = top + 1 + len(ch.p)
        b_store = [np.ascontiguousarray(b[:, T.rows]) for b in bs]
        q_top = top
    else:
        srows, b_store, q_top = R, bs, -1
    bkb = [pa.DevBuf.from_array(b) for b in b_store]
    bka = [pa.DevBuf.from_array(a_) for a_ in as_]
    bseed = [pa.DevBuf.from_array(np.ascontiguousarray(s, np.uint32)) for s in seeds]
    pkb, pka, pseed = dev_ptrs(bkb), dev_ptrs(bka), dev_ptrs(bseed)
    bx = pa.DevBuf.from_array(x)
    bmu = pa.DevBuf.from_array(digits)
    bx0 = pa.DevBuf.from_array(x0) if x0 is not None else None
    nres = (G // 2) * pair + 2 if pair else G
    bres = pa.DevBuf(nres * 2 * R * n)
    bkinv = pa.DevBuf.from_array(np.array(gals, np.uint32))
    pbufs = [pa.DevBuf.from_array(p) for p in pts]
    ppts = dev_ptrs(pbufs)
    r = abi.CtsRegenArgs()
    a = r.cts
    a.x, a.modup, a.res = bx.ptr.value, bmu.ptr.value, bres.ptr.value
    a.ka, a.kinv, a.pts = pka.ptr.value, bkinv.ptr.value, ppts.ptr.value
    a.x0 = bx0.ptr.value if bx0 is not None else None
    T.fill(a, ch, top)
    a.ct_stride, a.part_stride = 2 * R * n, R * n
    a.mu_ct_stride, a.mu_digit_stride, a.key_digit_stride = ch.dnum * R * n, R * n, R * n
    a.K, a.B, a.G, a.npts, a.ndig, a.ptw, a.enc, a.kmax, a.pair_cts = 1, B, G, npts, nd, ptw, enc, 1, pair
    k = r.key
    k.kb, k.seed, k.row_words, k.bits = pkb.ptr.value, pseed.ptr.value, n, 0
    k.q_top, k.srows, k.nregen = q_top, srows, nregen
    assert abi.call("cts_fused_regen", r, stream, log_n=ch.logn) == 0
    stream.sync()
    got = bres.download((nres, 2, R, n))
    want = oc.cts_fused(x[None], digits[None], top, B, G, pts, gals, seeds=seeds, bs=bs, as_=as_, nregen=nregen,
                        enc=enc, x0=None if x0 is None else x0[None])[0]
    rs = T.rows
    for j in range(G):
        at = (j >> 1) * pair + (j & 1) if pair else j
        assert (got[at][:, rs] == want[j][:, rs]).all(), j
