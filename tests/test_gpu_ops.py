"""Parity of the driver's composite operations with the oracle, word for word: the relinearization key (keygen with the
old secret squared), the relinearized product pcx_mul_relin (tensor, ModUp of d2, key dot, ModDown onto (c0, c1))
and the rescale pcx_rescale by one or two primes. The oracle composes its pinned pieces (tests/twin.py mul_relin,
rescale; pinned end to end by tests/test_oracle_em.py's decryption test). Each test prints its case before the GPU
runs.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
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
        _CTX[name] = (ch, pa.Context(ch, k_rot=2), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum))
    return _CTX[name]


_KEYS = {}


def relin_key(name, bits=0):
    """the relinearization key on the device, and its b and seed for the oracle"""
    if (name, bits) not in _KEYS:
        ch, ctx, oc = contexts(name)
        g = twin.Prng([1, 4, 1, 4, 2, 1, 3, 5], 0)
        s = g.sparse_ternary(ch.n, 192)
        seed = g.ksk_seed()
        errs = np.stack([g.gaussian(ch.n) for _ in range(ch.dnum)])
        keys = pa.Keys(ctx, [1], seeds=seed[None], bits=bits, secret=s, errors=errs[None], relin=True)
        _KEYS[(name, bits)] = (keys, s, seed, errs)
    return _KEYS[(name, bits)]


def random_ct(ch, top, rng):
    x = np.zeros((2, ch.rows, ch.n), np.uint32)
    for t in range(top + 1):
        x[:, t] = rng.integers(0, ch.primes[t], (2, ch.n))
    return x


@pytest.mark.parametrize("name,bits", [("small", 0), ("small31", 31)])
def test_relin_keygen(stream, name, bits):
    say(f"[relin keygen] {name} bits={bits}")
    ch, ctx, oc = contexts(name)
    keys, s, seed, errs = relin_key(name, bits)
    s_eval = oc.secret_eval(s)
    s2 = np.stack([(s_eval[t].astype(np.uint64) ** 2 % ch.primes[t]) for t in range(ch.rows)]).astype(np.uint32)
    e = np.zeros((ch.dnum, ch.rows, ch.n), np.uint32)
    for d in range(ch.dnum):
        for t in range(ch.rows):
            e[d, t] = np.mod(errs[d], ch.primes[t])
    e = oc.ntt_fwd(e.reshape(-1, ch.n), [t for _ in range(ch.dnum) for t in range(ch.rows)]).reshape(e.shape)
    assert (keys.download_b(0) == oc.ksk_gen(s_eval, s2, seed, e)).all()


@pytest.mark.parametrize("name,top,alias", [("small", 5, False), ("small", 3, True), ("small31", 5, False),
                                            ("c3", 29, False), ("c3", 17, True)])
def test_mul_relin(stream, name, top, alias):
    say(f"[mul_relin] {name} top={top} out=a:{alias}")
    ch, ctx, oc = contexts(name)
    keys, _, seed, _ = relin_key(name)
    rng = np.random.default_rng(top * 7 + alias)
    a, b = random_ct(ch, top, rng), random_ct(ch, top, rng)
    want = oc.mul_relin(a, b, top, seed, keys.download_b(0))
    ba, bb = pa.DevBuf.from_array(a), pa.DevBuf.from_array(b)
    out = ba if alias else ctx.ct_buf(1)
    ctx.mul_relin(keys, ba, bb, top, out, stream)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


@pytest.mark.parametrize("name,top,ndrop,inplace", [("small", 5, 2, False), ("small", 4, 1, True),
                                                    ("small31", 5, 1, False), ("small31", 3, 2, True),
                                                    ("c3", 29, 2, False), ("c3", 28, 1, False)])
def test_rescale(stream, name, top, ndrop, inplace):
    say(f"[rescale] {name} top={top} ndrop={ndrop} inplace={inplace}")
    ch, ctx, oc = contexts(name)
    rng = np.random.default_rng(top * 3 + ndrop)
    x = random_ct(ch, top, rng)
    want = oc.rescale(x, top, ndrop)
    bx = pa.DevBuf.from_array(x)
    out = bx if inplace else ctx.ct_buf(1)
    ctx.rescale(bx, top, ndrop, out, stream)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    rows = top + 1 - ndrop
    assert (got[:, :rows] == want[:, :rows]).all()
    if not inplace:
        assert (bx.download((2, ch.rows, ch.n)) == x).all(), "the source is read only"


def test_mul_relin_rescale_decrypts(stream):
    """The device chain encrypt -> mul_relin -> rescale decrypts to the product of the messages divided by the two
    dropped primes (the oracle's decryption test, on the GPU's words)."""
    say("[mul_relin + rescale] small decrypt")
    from tests.test_oracle_em import crt_centred, negacyclic
    from tests.test_oracle_ks import decrypt, encrypt
    ch, ctx, oc = contexts("small")
    keys, s, _, _ = relin_key("small")
    s_eval = oc.secret_eval(s)
    rng = np.random.default_rng(11)
    top = 5
    delta = 1 << 30
    ma, mb = np.zeros(ch.n, np.int64), rng.integers(-50, 50, ch.n) * delta
    ma[rng.choice(ch.n, 48, replace=False)] = rng.integers(-50, 50, 48) * delta  # sparse: the check's product is cheap
    ca, _ = encrypt(oc, s_eval, ma, rng, top)
    cb, _ = encrypt(oc, s_eval, mb, rng, top)
    ba, bb, out = pa.DevBuf.from_array(ca), pa.DevBuf.from_array(cb), ctx.ct_buf(1)
    ctx.mul_relin(keys, ba, bb, top, out, stream)
    ctx.rescale(out, top, 2, out, stream)
    stream.sync()
    got = crt_centred(decrypt(oc, s_eval, out.download((2, ch.rows, ch.n)), top - 2), ch.primes[: top - 1])
    div = int(ch.primes[top]) * int(ch.primes[top - 1])
    prod = negacyclic(ma, mb)
    assert max(abs(x - round(y / div)) for x, y in zip(got, prod)) < 1 << 8


@pytest.mark.parametrize("name,top,alias", [("small", 5, False), ("small", 3, True), ("small31", 5, False),
                                            ("c3", 29, False), ("c5", 46, True), ("c5", 20, False)])
def test_mul_relin_rescale(stream, name, top, alias):
    """The relinearized product and the two-prime rescale as one exact ModDown by P q_top q_{top-1}
    (pcx_mul_relin_rescale) against the oracle's composition, word for word on rows 0..top - 2."""
    say(f"[mul_relin_rescale] {name} top={top} out=a:{alias}")
    ch, ctx, oc = contexts(name)
    keys, _, seed, _ = relin_key(name)
    rng = np.random.default_rng(top * 11 + alias)
    a, b = random_ct(ch, top, rng), random_ct(ch, top, rng)
    want = oc.mul_relin_rescale(a, b, top, seed, keys.download_b(0))
    ba, bb = pa.DevBuf.from_array(a), pa.DevBuf.from_array(b)
    out = ba if alias else ctx.ct_buf(1)
    ctx.mul_relin_rescale(keys, ba, bb, top, out, stream)
    stream.sync()
    got = out.download((2, ch.rows, ch.n))
    assert (got[:, : top - 1] == want[:, : top - 1]).all()


_CTX2 = {}


def batched(name, k_max=2):
    """a k_max context of the preset and its relinearization key (the same secret, seed and errors as relin_key's)"""
    if (name, k_max) not in _CTX2:
        ch, _, _ = contexts(name)
        ctx2 = pa.Context(ch, k_rot=1, k_max=k_max)
        _, s, seed, errs = relin_key(name)
        _CTX2[name, k_max] = (ctx2, pa.Keys(ctx2, [1], seeds=seed[None], secret=s, errors=errs[None], relin=True))
    return _CTX2[name, k_max]


@pytest.mark.parametrize("name,top,K,twice", [("small", 5, 3, False), ("small31", 4, 6, True), ("c3", 29, 5, True)])
def test_product_list(stream, name, top, K, twice):
    """pcx_mul_relin_rescale_list on a k_max 6 context: K pairs at their own addresses (operands drawn with repeats
    from four ciphertexts of one buffer), one tensor launch and the batched key switch (key dots four ciphertexts at a
    time): each product's words equal the K = 1 call's; more pairs than k_max are refused."""
    say(f"[product list] {name} top={top} K={K} twice={twice}")
    from perseus_amd import bootstrap as B

    ch, ctx, _ = contexts(name)
    keys, _, _, _ = relin_key(name)
    ctxk, keysk = batched(name, 6)
    rng = np.random.default_rng(top * 11 + K)
    pool = np.stack([random_ct(ch, top, rng) for _ in range(4)])
    ia, ib = rng.integers(0, 4, K), rng.integers(0, 4, K)
    want = []
    for j in range(K):
        ba, bb, o = pa.DevBuf.from_array(pool[ia[j]]), pa.DevBuf.from_array(pool[ib[j]]), ctx.ct_buf(1)
        ctx.mul_relin_rescale(keys, ba, bb, top, o, stream, K=1, twice=twice)
        stream.sync()
        want.append(o.download((2, ch.rows, ch.n)))
    buf = pa.DevBuf.from_array(pool)
    views = lambda idx: [B.View(buf, int(i) * ctxk.ct_words) for i in idx]
    out = ctxk.ct_buf(K)
    ctxk.mul_relin_rescale_list(keysk, views(ia), views(ib), top, out, stream, twice=twice)
    stream.sync()
    got = out.download((K, 2, ch.rows, ch.n))
    for j in range(K):
        assert (got[j][:, : top - 1] == want[j][:, : top - 1]).all(), f"product {j} ({ia[j]} x {ib[j]})"
    with pytest.raises(pa.HipError):
        ctxk.mul_relin_rescale_list(keysk, views([0] * 7), views([1] * 7), top, ctxk.ct_buf(7), stream)
    # aliasing: slot j in place over pair j's own operand is allowed (the words of the out-of-place call) ...
    inplace = pa.DevBuf.from_array(pool[:2])
    both = [B.View(inplace, j * ctxk.ct_words) for j in range(2)]
    ctxk.mul_relin_rescale_list(keysk, both, views(ib[:2]), top, both[0], stream, twice=twice)
    stream.sync()
    got = inplace.download((2, 2, ch.rows, ch.n))
    out2 = ctxk.ct_buf(2)
    ctxk.mul_relin_rescale_list(keysk, views([0, 1]), views(ib[:2]), top, out2, stream, twice=twice)
    stream.sync()
    want2 = out2.download((2, 2, ch.rows, ch.n))
    for j in range(2):
        assert (got[j][:, : top - 1] == want2[j][:, : top - 1]).all(), f"in place, product {j}"
    # ... a slot over another pair's operand is refused, before anything is launched
    shifted = pa.DevBuf.from_array(pool[:3])
    tri = [B.View(shifted, j * ctxk.ct_words) for j in range(3)]
    with pytest.raises(pa.HipError):
        ctxk.mul_relin_rescale_list(keysk, tri[1:], tri[1:], top, tri[0], stream)
    assert (shifted.download((3, 2, ch.rows, ch.n)) == pool[:3]).all()


@pytest.mark.parametrize("name,top,sizes", [("small", 5, (1, 2, 3)), ("small31", 4, (3, 1)), ("c3", 29, (2, 2, 1)),
                                            ("c5", 30, (4, 4))])
def test_product_sums(stream, name, top, sizes):
    """pcx_mul_sum_relin_rescale_list on a k_max 6 context: product j the sum of sizes[j] pairs (operands drawn
    with repeats from four ciphertexts of one buffer), its tensors summed and relinearized and rescaled once: each
    product's words equal the oracle's (the tensor of all its pairs, ModUp of d2, the key dot, the exact ModDown by
    P q_top q_top-1 with (d0, d1) onto it); more than 8 pairs, an empty group and an out slot over an operand are
    refused before anything is launched. The same products with addends (one added, one subtracted, one without),
    then doubled with an addend times a multiplier, equal the oracle's with the addend folded into (d0, d1) before
    the key switch."""
    say(f"[product sums] {name} top={top} sizes={sizes}")
    from perseus_amd import bootstrap as B

    ch, _, oc = contexts(name)
    _, _, seed, _ = relin_key(name)
    ctxk, keysk = batched(name, 6)
    rng = np.random.default_rng(top * 7 + len(sizes))
    pool = np.stack([random_ct(ch, top, rng) for _ in range(4)])
    groups = [[(int(rng.integers(0, 4)), int(rng.integers(0, 4))) for _ in range(m)] for m in sizes]
    buf = pa.DevBuf.from_array(pool)
    view = lambda i: B.View(buf, i * ctxk.ct_words)
    out = ctxk.ct_buf(len(sizes))
    ctxk.mul_sum_relin_rescale_list(keysk, [[(view(i), view(j)) for i, j in g] for g in groups], top, out, stream)
    stream.sync()
    got = out.download((len(sizes), 2, ch.rows, ch.n))
    bkey = keysk.download_b(0)
    for j, g in enumerate(groups):
        want = oc.mul_sum_relin_rescale([(pool[a], pool[b]) for a, b in g], top, seed, bkey)
        assert (got[j][:, : top - 1] == want[:, : top - 1]).all(), f"product {j} ({g})"
    # addends: product 0 plus the pool's ciphertext 3, product 1 minus ciphertext 2, the last with none; against the
    # oracle's addend folded into (d0, d1) before the key switch
    adds = [3, 2] + [None] * (len(sizes) - 2)
    out2 = ctxk.ct_buf(len(sizes))
    ctxk.mul_sum_relin_rescale_list(keysk, [[(view(i), view(j)) for i, j in g] for g in groups], top, out2, stream,
                                    adds=[None if y is None else view(y) for y in adds], sub=0b10)
    stream.sync()
    got2 = out2.download((len(sizes), 2, ch.rows, ch.n))
    for j, g in enumerate(groups):
        y = None if adds[j] is None else pool[adds[j]]
        want = oc.mul_sum_relin_rescale([(pool[a], pool[b]) for a, b in g], top, seed, bkey, y, j == 1)
        assert (got2[j][:, : top - 1] == want[:, : top - 1]).all(), f"product {j} ({g}) with addend {adds[j]}"
        if adds[j] is None:
            assert (got2[j][:, : top - 1] == got[j][:, : top - 1]).all()
    # doubled tensors, addend 3 times an integer beyond every prime subtracted from product 0, addend 2 plain on 1
    k0 = (1 << 75) + 12345
    kr = np.array([k0 % int(p) for p in ch.primes], np.uint64)
    krows = pa.DevBuf.from_array(np.concatenate([kr, (kr << 32) // np.array(ch.primes, np.uint64)]).astype(np.uint32))
    out3 = ctxk.ct_buf(len(sizes))
    ctxk.mul_sum_relin_rescale_list(keysk, [[(view(i), view(j)) for i, j in g] for g in groups], top, out3, stream,
                                    adds=[None if y is None else view(y) for y in adds], sub=0b01,
                                    kmuls=[krows] + [None] * (len(sizes) - 1), twice=True)
    stream.sync()
    got3 = out3.download((len(sizes), 2, ch.rows, ch.n))
    for j, g in enumerate(groups):
        y = None if adds[j] is None else pool[adds[j]]
        want = oc.mul_sum_relin_rescale([(pool[a], pool[b]) for a, b in g], top, seed, bkey, y, j == 0,
                                        k0 if j == 0 else None, True)
        assert (got3[j][:, : top - 1] == want[:, : top - 1]).all(), f"doubled product {j} ({g}), addend {adds[j]}"
    o1 = ctxk.ct_buf(1)
    with pytest.raises(pa.HipError):  # an addend over the out slot
        ctxk.mul_sum_relin_rescale_list(keysk, [[(view(0), view(2))]], top, o1, stream, adds=[o1])
    with pytest.raises(pa.HipError):
        ctxk.mul_sum_relin_rescale_list(keysk, [[(view(0), view(1))] * 5, [(view(2), view(3))] * 4], top,
                                        ctxk.ct_buf(2), stream)
    with pytest.raises((pa.HipError, AssertionError)):
        ctxk.mul_sum_relin_rescale_list(keysk, [[(view(0), view(1))], []], top, ctxk.ct_buf(2), stream)
    with pytest.raises(pa.HipError):
        ctxk.mul_sum_relin_rescale_list(keysk, [[(view(1), view(2))]], top, view(1), stream)
    assert (buf.download((4, 2, ch.rows, ch.n)) == pool).all()


@pytest.mark.parametrize("name,top,alias", [("small", 5, False), ("small31", 4, True), ("c3", 29, True),
                                            ("c5", 30, False)])
def test_batched_product_and_rescale(stream, name, top, alias):
    """Two pairs in one launch sequence (pcx_mul_relin_rescale_k, K = 2, on a k_max 2 context): each product's words
    equal the K = 1 call's on a k_max 1 context (itself pinned to the oracle by test_mul_relin_rescale); the same for
    the two-prime rescale of two ciphertexts (pcx_rescale_k); K above k_max is refused."""
    say(f"[batched product / rescale] {name} top={top} K=2 out=a:{alias}")
    ch, ctx, _ = contexts(name)
    keys, _, _, _ = relin_key(name)
    ctx2, keys2 = batched(name)
    rng = np.random.default_rng(top * 7 + alias)
    a = np.stack([random_ct(ch, top, rng) for _ in range(2)])
    b = np.stack([random_ct(ch, top, rng) for _ in range(2)])
    want = []
    for k in range(2):
        ba, bb, o = pa.DevBuf.from_array(a[k]), pa.DevBuf.from_array(b[k]), ctx.ct_buf(1)
        ctx.mul_relin_rescale(keys, ba, bb, top, o, stream)
        stream.sync()
        want.append(o.download((2, ch.rows, ch.n)))
    ba, bb = pa.DevBuf.from_array(a), pa.DevBuf.from_array(b)
    out = ba if alias else ctx2.ct_buf(2)
    ctx2.mul_relin_rescale(keys2, ba, bb, top, out, stream, K=2)
    stream.sync()
    got = out.download((2, 2, ch.rows, ch.n))
    for k in range(2):
        assert (got[k][:, : top - 1] == want[k][:, : top - 1]).all(), f"product {k}"
    # the rescale: two ciphertexts at once against one at a time
    x = np.stack([random_ct(ch, top, rng) for _ in range(2)])
    wr = []
    for k in range(2):
        bx = pa.DevBuf.from_array(x[k])
        ctx.rescale(bx, top, 2, bx, stream)
        stream.sync()
        wr.append(bx.download((2, ch.rows, ch.n)))
    bx = pa.DevBuf.from_array(x)
    ro = ctx2.ct_buf(2)
    ctx2.rescale(bx, top, 2, ro, stream, K=2)
    stream.sync()
    gr = ro.download((2, 2, ch.rows, ch.n))
    for k in range(2):
        assert (gr[k][:, : top - 1] == wr[k][:, : top - 1]).all(), f"rescale {k}"
    with pytest.raises(pa.HipError):
        ctx2.rescale(bx, top, 2, ro, stream, K=3)
    with pytest.raises(pa.HipError):
        ctx.mul_relin_rescale(keys, ba, bb, top, out, stream, K=2)


@pytest.mark.parametrize("name,top,K", [("small", 5, 1), ("small31", 4, 2), ("c5", 24, 2)])
def test_product_twice(stream, name, top, K):
    """The doubling folded into the product (pcx_mul_relin_rescale_k with twice: the tensor's outputs doubled): the
    words of the oracle's product of 2a (mod q) and b, for each of K pairs."""
    say(f"[product twice] {name} top={top} K={K}")
    ch, _, oc = contexts(name)
    ctx2, keys2 = batched(name)
    _, _, seed, _ = relin_key(name)
    rng = np.random.default_rng(top + 17 * K)
    a = np.stack([random_ct(ch, top, rng) for _ in range(K)])
    b = np.stack([random_ct(ch, top, rng) for _ in range(K)])
    ba, bb, out = pa.DevBuf.from_array(a), pa.DevBuf.from_array(b), ctx2.ct_buf(K)
    ctx2.mul_relin_rescale(keys2, ba, bb, top, out, stream, K=K, twice=True)
    stream.sync()
    got = out.download((K, 2, ch.rows, ch.n))
    q = np.array(ch.primes[: top + 1], np.uint64)[None, :, None]
    for k in range(K):
        a2 = a[k].copy()
        a2[:, : top + 1] = (2 * a[k][:, : top + 1].astype(np.uint64) % q).astype(np.uint32)
        want = oc.mul_relin_rescale(a2, b[k], top, seed, keys2.download_b(0))
        assert (got[k][:, : top - 1] == want[:, : top - 1]).all(), f"pair {k}"


@pytest.mark.parametrize("name,top,K", [("small", 5, 3), ("c3", 29, 6)])
def test_mul_plain_k(stream, name, top, K):
    """pcx_mul_plain_k: K consecutive ciphertexts, each by its own plaintext, in one launch (also in place): each
    output equals pcx_mul_plain's (the table's mul_table) on that ciphertext."""
    say(f"[mul_plain_k] {name} top={top} K={K}")
    ch, ctx, _ = contexts(name)
    rng = np.random.default_rng(top + K)
    x = np.stack([random_ct(ch, top, rng) for _ in range(K)])
    pts = [np.stack([rng.integers(0, p, ch.n) for p in ch.primes]).astype(np.uint32) for _ in range(K)]
    bpts = [pa.DevBuf.from_array(p) for p in pts]
    want = []
    for j in range(K):
        bx, o = pa.DevBuf.from_array(x[j]), ctx.ct_buf(1)
        ctx.mul_plain(bx, bpts[j], top, o, stream)
        stream.sync()
        want.append(o.download((2, ch.rows, ch.n)))
    bx = pa.DevBuf.from_array(x)
    out = ctx.ct_buf(K)
    ctx.mul_plain_k(bx, bpts, top, out, stream)
    ctx.mul_plain_k(bx, bpts, top, bx, stream)  # in place
    stream.sync()
    got, got2 = out.download((K, 2, ch.rows, ch.n)), bx.download((K, 2, ch.rows, ch.n))
    for j in range(K):
        assert (got[j][:, : top + 1] == want[j][:, : top + 1]).all(), j
        assert (got2[j][:, : top + 1] == want[j][:, : top + 1]).all(), j
