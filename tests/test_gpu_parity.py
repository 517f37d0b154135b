"""Parity of the gfx950 path with the oracle, word for word, through the C-ABI (driver + kernel table).

Inputs are seeded; keys are the oracle's (seed of a + stored b), so the GPU regenerates a in-kernel from the same
seeds the twin expands. Each test prints the case it runs before touching the GPU.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import bootstrap as B
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


def contexts(name, k_rot=4, k_max=1):
    key = (name, k_rot, k_max)
    if key not in _CTX:
        ch = pa.preset(name)
        _CTX[key] = (ch, pa.Context(ch, k_rot=k_rot, k_max=k_max), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum))
    return _CTX[key]


def random_ct(ch, top, seed):
    rng = np.random.default_rng(seed)
    ct = np.zeros((2, ch.rows, ch.n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.primes[t], ch.n)
        ct[part, 0, :4] = [0, ch.primes[0] - 1, 1, ch.primes[0] - 1]
    return ct


def oracle_keys(oc, ch, steps, seed=7):
    g = twin.Prng([seed, 1, 2, 3, 4, 5, 6, 7], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
    gals = [twin.rotation_galois(r, ch.n) for r in steps]
    keys = [oc.rotation_key(g, s_eval, x) for x in gals]
    return gals, np.stack([k[0] for k in keys]), [k[1] for k in keys]


# ----------------------------------------------------------------------------------------------- NTT
@pytest.mark.parametrize("logn,bits,nrows", [(12, 30, 6), (13, 31, 5), (14, 30, 8), (15, 31, 4), (16, 31, 12)])
def test_ntt_rows(stream, logn, bits, nrows):
    say(f"[ntt] logn={logn} bits={bits} rows={nrows}")
    ps = twin.descending_primes(bits, 2 << logn, nrows)
    ch = pa.Chain(f"ntt{logn}", logn, ps[:-1], ps[-1:], 1)
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(logn, ps[:-1], ps[-1:], 1)
    n = 1 << logn
    rng = np.random.default_rng(logn)
    x = np.stack([rng.integers(0, p, n) for p in ps]).astype(np.uint32)
    x[0, :3] = [ps[0] - 1, 0, ps[0] - 1]
    x[1] = ps[1] - 1
    ids = list(range(nrows))
    rows = pa.Rows(ctx, ids, ids)
    buf = pa.DevBuf.from_array(x)
    rows.ntt(buf, 1, stream)
    stream.sync()
    y = buf.download((nrows, n))
    want = oc.ntt_fwd(x.copy(), ids)
    assert (y == want).all()
    rows.ntt(buf, -1, stream)
    stream.sync()
    assert (buf.download((nrows, n)) == x).all()
    # inverse of arbitrary words against the twin
    buf.upload(x)
    rows.ntt(buf, -1, stream)
    stream.sync()
    assert (buf.download((nrows, n)) == oc.ntt_inv(x.copy(), ids)).all()


def test_ntt_batch_c2(stream):
    """The C2 workload: 64 polynomials x 40 limbs at N = 2^16 (2560 row transforms), forward bit-exact against the
    twin and the round trip exact."""
    ch = pa.preset("c2")
    say("[ntt c2] 64 x 40 x 2^16")
    ctx = pa.Context(pa.Chain("c2k", 16, ch.q[:-1], ch.q[-1:], 1), k_rot=1)
    oc = twin.Ctx(16, ch.q, [], 1)
    twin.set_threads(16)
    npoly, L, n = 64, 40, 1 << 16
    rng = np.random.default_rng(2)
    qs = np.array(ch.q, np.uint64)
    x = (rng.integers(0, 1 << 62, (npoly, L, n), dtype=np.uint64) % qs[None, :, None]).astype(np.uint32)
    ids = [t for _ in range(npoly) for t in range(L)]
    rows = pa.Rows(ctx, list(range(npoly * L)), ids)
    buf = pa.DevBuf.from_array(x)
    rows.ntt(buf, 1, stream)
    stream.sync()
    y = buf.download((npoly, L, n))
    want = oc.ntt_fwd(x.reshape(-1, n).copy(), ids).reshape(npoly, L, n)
    assert (y == want).all()
    rows.ntt(buf, -1, stream)
    stream.sync()
    assert (buf.download((npoly, L, n)) == x).all()


# ----------------------------------------------------------------------------------------------- key switch stages
@pytest.mark.parametrize("name,top", [("small", 5), ("small", 2), ("small31", 5), ("c1", 11), ("c1", 6)])
def test_modup(stream, name, top):
    say(f"[modup] {name} top={top}")
    ch, ctx, oc = contexts(name)
    ct = random_ct(ch, top, 11 + top)
    dev = pa.DevBuf.from_array(ct)
    ctx.modup(dev, top, stream)
    got = ctx.modup_digits(stream)
    want = oc.modup(ct[1, : top + 1], top)
    nd = oc.live_digits(top)
    for d in range(nd):
        dl = [t for t in range(top + 1) if oc.digit_of(t) == d]
        tg = [t for t in range(top + 1) if t not in dl] + list(range(ch.rows - len(ch.p), ch.rows))
        assert (got[d, tg] == want[d, tg]).all(), d


@pytest.mark.parametrize("name,top,bits", [("small", 5, 0), ("small", 5, 30), ("small31", 4, 31), ("c1", 11, 0),
                                           ("c1", 11, 30), ("c1", 3, 30)])
def test_dot_and_moddown(stream, name, top, bits):
    say(f"[dot/moddown] {name} top={top} bits={bits}")
    ch, ctx, oc = contexts(name)
    gals, seeds, bs = oracle_keys(oc, ch, [1, 5])
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=bits)
    ct = random_ct(ch, top, 3)
    dev = pa.DevBuf.from_array(ct)
    ext = ctx.ct_buf()
    ext.zero()
    ctx.modup(dev, top, stream)
    ctx.dot(keys, 1, dev, top, ext, stream)
    stream.sync()
    got = ext.download((2, ch.rows, ch.n))
    digits = oc.modup(ct[1, : top + 1], top)
    want = oc.ks_dot(ct, digits, top, seeds[1], bs[1], twin.galois_inverse(gals[1], ch.n))
    live = list(range(top + 1)) + list(range(len(ch.q), ch.rows))
    assert (got[:, live] == want[:, live]).all()
    out = ctx.ct_buf()
    ctx.moddown(ext, top, out, stream)
    stream.sync()
    got_o = out.download((2, ch.rows, ch.n))
    want_o = oc.moddown(want, top)
    assert (got_o[:, : top + 1] == want_o[:, : top + 1]).all()


def test_moddown_table_path(stream, monkeypatch):
    """ModDown through the kernel table's separate stages (INTT, bconv, NTT with epilogue 1), the path the driver takes
    when the conversion cannot be fused into the NTT column pass (more than 6 special primes): same words as the fused
    path and the oracle."""
    say("[moddown table path] c3 top=29")
    monkeypatch.setenv("PCX_MD_FUSED", "0")
    ch = pa.preset("c3")
    ctx = pa.Context(ch, k_rot=1)
    _, _, oc = contexts("c3")
    top = len(ch.q) - 1
    rng = np.random.default_rng(11)
    ext_h = np.zeros((2, ch.rows, ch.n), np.uint32)
    for part in range(2):
        for t in list(range(top + 1)) + list(range(len(ch.q), ch.rows)):
            ext_h[part, t] = rng.integers(0, ch.primes[t], ch.n)
    ext = pa.DevBuf.from_array(ext_h)
    out = ctx.ct_buf()
    ctx.moddown(ext, top, out, stream)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.moddown(ext_h, top)
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


# ----------------------------------------------------------------------------------------------- rotations
def test_rotate_c1(stream):
    """C1: one rotation (r = 1) at N = 2^14, 12 limbs, dnum 3, 4 special primes, every output residue."""
    say("[rotate c1]")
    ch, ctx, oc = contexts("c1")
    gals, seeds, bs = oracle_keys(oc, ch, [1], seed=42)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=30)
    top = len(ch.q) - 1
    ct = random_ct(ch, top, 1)
    dev = pa.DevBuf.from_array(ct)
    out = ctx.ct_buf()
    ctx.rotate(keys, 0, dev, top, out, stream)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate(ct, top, seeds[0], bs[0], gals[0])
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


@pytest.mark.parametrize("name,steps,top", [("small", [1, 2, 3, 0, 7], 5), ("c3", [1, 2, 16, 1 << 15, 64], 29),
                                            ("c3", [3, 4], 13)])
def test_hoisted(stream, name, steps, top):
    say(f"[hoisted] {name} steps={steps} top={top}")
    ch, ctx, oc = contexts(name, k_rot=4)
    twin.set_threads(16)
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=5)
    bits = max(p.bit_length() for p in ch.primes)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=bits)
    ct = random_ct(ch, top, 9)
    dev = pa.DevBuf.from_array(ct)
    outs = ctx.ct_buf(len(steps))
    ctx.rotate_hoisted(keys, list(range(len(steps))), dev, top, outs, stream)
    stream.sync()
    got = outs.download((len(steps), 2, ch.rows, ch.n))
    want = oc.rotate_hoisted(ct, top, seeds, bs, gals)
    for j in range(len(steps)):
        assert (got[j, :, : top + 1] == want[j][:, : top + 1]).all(), steps[j]
    # the same outputs one rotation at a time (crates/pc-tools/src/word_seam.rs:312-317: hoisted == plain)
    one = ctx.ct_buf()
    for j in range(len(steps)):
        ctx.rotate(keys, j, dev, top, one, stream)
        stream.sync()
        assert (one.download((2, ch.rows, ch.n))[:, : top + 1] == got[j, :, : top + 1]).all()


def test_hoisted_dense_c3(stream):
    """The bench's configuration: C3 at the top with dense b, the fast dot reading the retry-value table."""
    say("[hoisted dense] c3 top=29")
    ch, ctx, oc = contexts("c3", k_rot=4)
    twin.set_threads(16)
    steps = [1, 5, 1 << 15, 256]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=6)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    assert keys.patch_bytes() > 0
    top = len(ch.q) - 1
    ct = random_ct(ch, top, 10)
    dev = pa.DevBuf.from_array(ct)
    outs = ctx.ct_buf(len(steps))
    ctx.rotate_hoisted(keys, list(range(len(steps))), dev, top, outs, stream)
    stream.sync()
    got = outs.download((len(steps), 2, ch.rows, ch.n))
    want = oc.rotate_hoisted(ct, top, seeds, bs, gals)
    for j in range(len(steps)):
        assert (got[j, :, : top + 1] == want[j][:, : top + 1]).all(), steps[j]


@pytest.mark.parametrize("mode", ["table", "redraw", "packed"])
def test_rejection_heavy(stream, monkeypatch, mode):
    """Primes just above 2^32 / 3, where a third of the KSKA words are rejected: the retry table (dense keys), the
    wave's redraw (dense keys with the table off) and the general dot (packed b), all against the oracle, including
    waves whose rejections overflow the queue."""
    say(f"[rejections] mode={mode}")
    if mode == "redraw":
        monkeypatch.setenv("PCX_KS_PATCH", "0")
    ch = pa.preset("rej")
    ctx = pa.Context(ch, k_rot=3)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    steps = [1, 3, 7]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=8)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=31 if mode == "packed" else 0)
    assert (keys.patch_bytes() > 0) == (mode == "table")
    top = len(ch.q) - 1
    ct = random_ct(ch, top, 12)
    dev = pa.DevBuf.from_array(ct)
    outs = ctx.ct_buf(len(steps))
    ctx.rotate_hoisted(keys, list(range(len(steps))), dev, top, outs, stream)
    stream.sync()
    got = outs.download((len(steps), 2, ch.rows, ch.n))
    want = oc.rotate_hoisted(ct, top, seeds, bs, gals)
    for j in range(len(steps)):
        assert (got[j, :, : top + 1] == want[j][:, : top + 1]).all(), steps[j]


# ----------------------------------------------------------------------------------------------- keys
@pytest.mark.parametrize("name,bits", [("small", 0), ("small", 30), ("c1", 30), ("small31", 31)])
def test_device_keygen(stream, name, bits):
    """ksk_gen on the device (a regenerated from the seed, b = e - a s_new + [digit] P s_old, packed) against the
    twin's ksk_gen on the same secret, errors and seeds."""
    say(f"[keygen] {name} bits={bits}")
    ch, ctx, oc = contexts(name)
    g = twin.Prng([3, 1, 4, 1, 5, 9, 2, 6], 0)
    s = g.sparse_ternary(ch.n, 64)
    s_eval = oc.secret_eval(s)
    gals = [twin.rotation_galois(r, ch.n) for r in (1, 3)]
    seeds = np.stack([g.ksk_seed() for _ in gals])
    errs = np.stack([np.stack([g.gaussian(ch.n) for _ in range(ch.dnum)]) for _ in gals])
    keys = pa.Keys(ctx, gals, seeds=seeds, bits=bits, secret=s, errors=errs)
    for r, gal in enumerate(gals):
        e = np.zeros((ch.dnum, ch.rows, ch.n), np.uint32)
        for d in range(ch.dnum):
            for t in range(ch.rows):
                e[d, t] = np.mod(errs[r, d], ch.primes[t])
        e = oc.ntt_fwd(e.reshape(-1, ch.n), [t for _ in range(ch.dnum) for t in range(ch.rows)]).reshape(e.shape)
        s_new = oc.automorph_rows(s_eval, twin.galois_inverse(gal, ch.n))
        want = oc.ksk_gen(s_new, s_eval, seeds[r], e)
        assert (keys.download_b(r) == want).all(), r


# ----------------------------------------------------------------------------------------------- summed rotations
@pytest.mark.parametrize("name,idx,mode", [("small", [0, 1, 2], "onto"), ("small", [2, 0], "plain"),
                                           ("small", [1, 3, 0, 2], "in_place"), ("c3", [0, 1, 2, 3], "onto")])
def test_rotate_sum(stream, name, idx, mode):
    """out = onto + ModDown(sum of the dots): runs of consecutive keys through the KS_SUM dot (later runs added with
    KS_ACC), one ModDown with the add-onto epilogue."""
    say(f"[rotate_sum] {name} keys={idx} {mode}")
    ch, ctx, oc = contexts(name, k_rot=4)
    twin.set_threads(16)
    steps = [1, 3, 2, 7]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=17)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    ct = random_ct(ch, top, 21)
    dev = pa.DevBuf.from_array(ct)
    if mode == "in_place":
        ctx.rotate_sum(keys, idx, dev, top, dev, stream, onto=dev)
        out = dev
    else:
        out = ctx.ct_buf()
        ctx.rotate_sum(keys, idx, dev, top, out, stream, onto=dev if mode == "onto" else None)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate_sum(ct, top, seeds[idx], [bs[i] for i in idx], [gals[i] for i in idx],
                         onto=None if mode == "plain" else ct)
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


@pytest.mark.parametrize("name,idx,mode", [("small", [0, 1, 2], "onto"), ("small", [2, 0], "plain"),
                                           ("small", [3, 1], "in_place"), ("small", [1, 2, 3], "table_only"),
                                           ("c3", [0, 1, 2, 3], "onto")])
def test_rotate_many(stream, name, idx, mode):
    """out = onto + ModDown(sum over j of the extended rotation of ct_j by key idx[j]): a ModUp per input, the dots
    added onto one extended sum (KS_ACC after the first), one ModDown with the add-onto epilogue."""
    say(f"[rotate_many] {name} keys={idx} {mode}")
    ch, ctx, oc = contexts(name, k_rot=4)
    twin.set_threads(16)
    steps = [1, 3, 2, 7]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=29)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    cts = [random_ct(ch, top, 31 + j) for j in range(len(idx))]
    base = random_ct(ch, top, 30)
    devs = [pa.DevBuf.from_array(x) for x in cts]
    onto = pa.DevBuf.from_array(base)
    if mode == "table_only":
        ctx.table_only(True)
    try:
        if mode == "in_place":
            ctx.rotate_many(keys, idx, devs, top, devs[0], stream, onto=devs[0])
            out = devs[0]
        else:
            out = ctx.ct_buf()
            ctx.rotate_many(keys, idx, devs, top, out, stream, onto=None if mode == "plain" else onto)
        stream.sync()
    finally:
        ctx.table_only(False)
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate_many(cts, top, seeds[idx], [bs[i] for i in idx], [gals[i] for i in idx],
                          onto={"plain": None, "in_place": cts[0]}.get(mode, base))
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


@pytest.mark.parametrize("name,idx,mode", [("small", [0, 1, 2], "onto"), ("small", [2, 0], "plain"),
                                           ("small", [3, 1], "in_place"), ("c3", [0, 1, 2, 3], "onto")])
def test_rotate_many_rescale(stream, name, idx, mode):
    """pcx_rotate_many with the two-prime rescale fused into its ModDown (one exact ModDown by P q_top q_{top-1}):
    word for word with the oracle on rows 0..top - 2."""
    say(f"[rotate_many_rescale] {name} keys={idx} {mode}")
    ch, ctx, oc = contexts(name, k_rot=4)
    twin.set_threads(16)
    gals, seeds, bs = oracle_keys(oc, ch, [1, 3, 2, 7], seed=37)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    cts = [random_ct(ch, top, 41 + j) for j in range(len(idx))]
    base = random_ct(ch, top, 40)
    devs = [pa.DevBuf.from_array(x) for x in cts]
    onto = pa.DevBuf.from_array(base)
    if mode == "in_place":
        ctx.rotate_many_rescale(keys, idx, devs, top, devs[0], stream, onto=devs[0])
        out = devs[0]
    else:
        out = ctx.ct_buf()
        ctx.rotate_many_rescale(keys, idx, devs, top, out, stream, onto=None if mode == "plain" else onto)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate_many(cts, top, seeds[idx], [bs[i] for i in idx], [gals[i] for i in idx],
                          onto={"plain": None, "in_place": cts[0]}.get(mode, base), rescale=True)
    assert (got[:, : top - 1] == want[:, : top - 1]).all()


@pytest.mark.parametrize("name,k_max,layout", [("small", 4, [0, 1, 2, 3]), ("small", 2, [0, 1, 2, 4]),
                                                ("small31", 3, [1, 2, 3, 0]), ("c3", 4, [0, 1, 2])])
def test_rotate_many_batched(stream, name, k_max, layout):
    """On a k_max > 1 context, inputs laid out ct_words apart share one ModUp launch sequence (runs of up to k_max;
    layout[j]: input j's slot in one buffer, so a gap or a backward step ends a run): the words equal the oracle's
    rotate_many with the rescale, as the one-ModUp-per-input path does."""
    say(f"[rotate_many batched] {name} k_max={k_max} slots={layout}")
    ch, ctx, oc = contexts(name, k_rot=1, k_max=k_max)
    twin.set_threads(16)
    idx = [0, 1, 2, 3][: len(layout)]
    gals, seeds, bs = oracle_keys(oc, ch, [1, 3, 2, 7], seed=43)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    cts = [random_ct(ch, top, 51 + j) for j in range(len(layout))]
    buf = pa.DevBuf((max(layout) + 1) * ctx.ct_words)
    for j, sl in enumerate(layout):
        buf.upload(cts[j], offset=sl * ctx.ct_words)
    views = [B.View(buf, sl * ctx.ct_words) for sl in layout]
    base = random_ct(ch, top, 50)
    onto = pa.DevBuf.from_array(base)
    out = ctx.ct_buf()
    ctx.rotate_many_rescale(keys, idx, views, top, out, stream, onto=onto)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate_many(cts, top, seeds[idx], [bs[i] for i in idx], [gals[i] for i in idx], onto=base,
                          rescale=True)
    assert (got[:, : top - 1] == want[:, : top - 1]).all()


@pytest.mark.parametrize("name,K,radix", [("small", 3, 2), ("small", 2, 1), ("c3", 4, 2), ("small31", 6, 3)])
def test_rotate_and_sum_batched(stream, name, K, radix):
    """The ladder over K consecutive ciphertexts (pcx_rotate_and_sum_k on a k_max = k_rot = K context): each output
    equals the one-ciphertext ladder's words (radix 1 takes the per-ciphertext fallback)."""
    say(f"[rotate_and_sum batched] {name} K={K} radix_bits={radix}")
    ch, ctx, oc = contexts(name, k_rot=4)
    ch2, ctxk, _ = contexts(name, k_rot=K, k_max=K)
    twin.set_threads(16)
    steps = [1, 2, 3, 4, 8, 12] if radix != 3 else [1, 2, 3, 4, 5, 6, 7, 8]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=19)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    keysk = pa.Keys(ctxk, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    cts = [random_ct(ch, top, 60 + j) for j in range(K)]
    stop = 16 if radix != 3 else 8
    want = []
    for x in cts:
        dev, out, tmp = pa.DevBuf.from_array(x), ctx.ct_buf(), ctx.ct_buf()
        ctx.rotate_and_sum(keys, dev, top, 1, stop, out, tmp, stream, radix_bits=radix)
        stream.sync()
        want.append(out.download((2, ch.rows, ch.n)))
    xb = pa.DevBuf.from_array(np.stack(cts))
    ob, tb = ctxk.ct_buf(K), ctxk.ct_buf(K)
    ctxk.rotate_and_sum(keysk, xb, top, 1, stop, ob, tb, stream, radix_bits=radix, K=K)
    stream.sync()
    got = ob.download((K, 2, ch.rows, ch.n))
    for j in range(K):
        assert (got[j][:, : top + 1] == want[j][:, : top + 1]).all(), f"ciphertext {j}"


@pytest.mark.parametrize("name,radix", [("small", 1), ("small", 2), ("c3", 2)])
def test_rotate_and_sum(stream, name, radix):
    say(f"[rotate_and_sum] {name} start=1 stop=16 radix_bits={radix}")
    ch, ctx, oc = contexts(name, k_rot=4)
    twin.set_threads(16)
    steps = [1, 2, 3, 4, 8, 12]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=19)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1 if name == "c3" else 5
    ct = random_ct(ch, top, 23)
    dev = pa.DevBuf.from_array(ct)
    out, tmp = ctx.ct_buf(), ctx.ct_buf()
    ctx.rotate_and_sum(keys, dev, top, 1, 16, out, tmp, stream, radix_bits=radix)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    want = oc.rotate_and_sum(ct, top, 1, 16, seeds, bs, gals, radix_bits=radix)
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


# ----------------------------------------------------------------------------------------------- graph capture
def test_graph_replay(stream):
    """The hoisted batch captured into a HIP graph (the launchers never allocate, synchronise or read device data on
    the host) and replayed three times, with eager work and a cleared output between replays: every replay equals the
    eager result word for word."""
    import ctypes as C

    say("[graph] small hoisted, 3 replays")
    ch, ctx, oc = contexts("small", k_rot=4)
    steps = [1, 2, 0, 5]
    gals, seeds, bs = oracle_keys(oc, ch, steps, seed=13)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=bs, bits=0)
    top = len(ch.q) - 1
    ct = random_ct(ch, top, 14)
    dev = pa.DevBuf.from_array(ct)
    idx = list(range(len(steps)))
    eager = ctx.ct_buf(len(steps))
    ctx.rotate_hoisted(keys, idx, dev, top, eager, stream)
    stream.sync()
    want = eager.download((len(steps), 2, ch.rows, ch.n))
    out = ctx.ct_buf(len(steps))
    graph, exe = C.c_void_p(), C.c_void_p()
    pa.check(pa.LIB.pc_hip_graph_begin_capture(stream.h), "begin_capture")
    ctx.rotate_hoisted(keys, idx, dev, top, out, stream)
    pa.check(pa.LIB.pc_hip_graph_end_capture(stream.h, C.byref(graph)), "end_capture")
    pa.check(pa.LIB.pc_hip_graph_instantiate(C.byref(exe), graph), "instantiate")
    try:
        for rep in range(3):
            out.zero()
            ctx.rotate_hoisted(keys, idx[::-1], dev, top, eager, stream)  # eager work between replays
            pa.check(pa.LIB.pc_hip_graph_launch(exe, stream.h), "graph_launch")
            stream.sync()
            got = out.download((len(steps), 2, ch.rows, ch.n))
            assert (got[:, :, : top + 1] == want[:, :, : top + 1]).all(), rep
    finally:
        pa.LIB.pc_hip_graph_exec_destroy(exe)
        pa.LIB.pc_hip_graph_destroy(graph)
