"""Pins of the oracle's EvalMod / plaintext-product kernels and composite rescale (oracle/em.py), each against what the
mathematics fixes rather than against the formula restated:

- tensor / tensor_y / tensor_sum: decryption: c0 + c1 s + d2 s^2 = (a0 + a1 s)(b0 + b1 s) word by word in the
  evaluation domain (summed over the pairs), with the old words, the doubling and +- c y entering as the documented
  order says (a dropped cross term, a transposed operand or the doubling before the add fails it);
- mul_table: the evaluation-domain product is the negacyclic convolution of the coefficient rows (schoolbook, N = 64);
  mul_add / mul_add_n decrypt to y +- in t and y + sum_j x_j t_j;
- md_epilogue: with x = t + v b and binv = b^-1 the epilogue adds exactly v (then doubles, then adds k on part 0);
- wsum / add_const: decryption is linear: Dec(out) = sum_j w_j Dec(src_j) + k;
- ew_many / submul_many: the inverse operations undo them;
- composite rescale: in coefficient form each output coefficient is the exact integer (X - [X]_{q_a}) / q_a of the CRT
  value X (Python integers), twice for two primes; the fold equals scaling first.
"""
import numpy as np
import pytest

from oracle import em
from tests import twin
from tests.test_oracle_ks import small_chain

RNG = np.random.default_rng(2024)


def rand_ct(q, K, n, N, rng=RNG):
    x = np.zeros((K, 2, n, N), np.uint32)
    for r in range(n):
        x[:, :, r] = rng.integers(0, q[r], (K, 2, N))
    return x


def dec(q, c0, c1, s, d2=None):
    """c0 + c1 s (+ d2 s^2) per row, as Python-exact uint64 arithmetic mod q"""
    n = c0.shape[-2]
    qq = np.asarray(q[:n], np.uint64).reshape(n, 1)
    s = s.astype(np.uint64)
    v = (c0.astype(np.uint64) + (c1.astype(np.uint64) * s) % qq) % qq
    if d2 is not None:
        v = (v + (((d2.astype(np.uint64) * s) % qq) * s) % qq) % qq
    return v


def mulq(a, b, q):
    n = a.shape[-2]
    qq = np.asarray(q[:n], np.uint64).reshape(n, 1)
    return (a.astype(np.uint64) * b.astype(np.uint64)) % qq


def addq(a, b, q):
    n = a.shape[-2]
    qq = np.asarray(q[:n], np.uint64).reshape(n, 1)
    return (a.astype(np.uint64) + b.astype(np.uint64)) % qq


Q = twin.descending_primes(31, 1 << 13, 5)
N = 256


def secret(q, n, N):
    return np.stack([RNG.integers(0, q[r], N) for r in range(n)]).astype(np.uint64)


@pytest.mark.parametrize("npairs,acc,acc_d2,dbl,ysub", [(1, 0, 0, 0, None), (2, 1, 1, 1, None), (2, 0, 0, 1, 0),
                                                         (2, 1, 0, 0, 1), (7, 1, 1, 0, None)])
def test_tensor_decrypts_to_the_product(npairs, acc, acc_d2, dbl, ysub):
    K, n = 2, 4
    s = secret(Q, n, N)
    pairs = [(rand_ct(Q, K, n, N), rand_ct(Q, K, n, N)) for _ in range(npairs)]
    old, old_d2 = rand_ct(Q, K, n, N), rand_ct(Q, K, n, N)[:, 1]
    y, yc = rand_ct(Q, K, n, N), [int(RNG.integers(0, q)) for q in Q[:n]]
    c0, c1, d2 = em.tensor(Q, pairs, old, old_d2, acc, acc_d2, dbl, None if ysub is None else y, yc, bool(ysub))
    for k in range(K):
        want = np.zeros((n, N), np.uint64)
        for a, b in pairs:
            want = addq(want, mulq(dec(Q, a[k, 0], a[k, 1], s), dec(Q, b[k, 0], b[k, 1], s), Q), Q)
        if acc:
            want = addq(want, dec(Q, old[k, 0], old[k, 1], s), Q)
        if acc_d2:
            want = addq(want, mulq(mulq(old_d2[k], s, Q), s, Q), Q)
        if dbl:
            want = addq(want, want, Q)
        if ysub is not None:
            cy = mulq(dec(Q, y[k, 0], y[k, 1], s), np.array(yc, np.uint64).reshape(n, 1).repeat(N, 1), Q)
            qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
            want = (want + qq - cy) % qq if ysub else addq(want, cy, Q)
        assert (dec(Q, c0[k], c1[k], s, d2[k]) == want).all()


def test_mul_table_is_the_negacyclic_product():
    ctx = small_chain(logn=6, nq=3, kp=1, dnum=1, bits=30)
    n, N6 = 3, ctx.n
    q = ctx.q
    a = np.stack([RNG.integers(0, q[r], N6) for r in range(n)]).astype(np.uint32)
    t = np.stack([RNG.integers(0, q[r], N6) for r in range(n)]).astype(np.uint32)
    ids = list(range(n))
    ae, te = ctx.ntt_fwd(a.copy(), ids), ctx.ntt_fwd(t.copy(), ids)
    x = np.zeros((1, 2, n, N6), np.uint32)
    x[0, 0], x[0, 1] = ae, ae
    prod = em.mul_add_n(q, [(x, te)])
    got = ctx.ntt_inv(prod[0, 0], ids)
    for r in range(n):
        p = int(q[r])
        want = [0] * N6
        for i in range(N6):
            for j in range(N6):
                v = int(a[r, i]) * int(t[r, j])
                if i + j < N6:
                    want[i + j] += v
                else:
                    want[i + j - N6] -= v
        assert [w % p for w in want] == [int(v) for v in got[r]]


@pytest.mark.parametrize("mode", [None, 0, 1, 2])
def test_mul_add_decrypts(mode):
    K, n = 2, 3
    s = secret(Q, n, N)
    x, y = rand_ct(Q, K, n, N), rand_ct(Q, K, n, N)
    t = np.stack([RNG.integers(0, Q[r], N) for r in range(n)]).astype(np.uint32)
    out = em.mul_add_n(Q, [(x, t)], None if mode is None else y, mode or 0)
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    for k in range(K):
        m = mulq(dec(Q, x[k, 0], x[k, 1], s), t, Q)
        dy = dec(Q, y[k, 0], y[k, 1], s)
        want = m if mode is None else addq(dy, m, Q) if mode == 0 else (dy + qq - m) % qq if mode == 1 else (m + qq - dy) % qq
        assert (dec(Q, out[k, 0], out[k, 1], s) == want).all()


def test_mul_add_n_decrypts_to_the_sum():
    K, n, T = 1, 3, 8
    s = secret(Q, n, N)
    y = rand_ct(Q, K, n, N)
    terms = [(rand_ct(Q, K, n, N), np.stack([RNG.integers(0, Q[r], N) for r in range(n)]).astype(np.uint32))
             for _ in range(T)]
    out = em.mul_add_n(Q, terms, y, 0)
    want = dec(Q, y[0, 0], y[0, 1], s)
    for x, t in terms:
        want = addq(want, mulq(dec(Q, x[0, 0], x[0, 1], s), t, Q), Q)
    assert (dec(Q, out[0, 0], out[0, 1], s) == want).all()


@pytest.mark.parametrize("dbl,withk", [(0, 0), (1, 1), (0, 1)])
def test_md_epilogue_adds_v(dbl, withk):
    K, n = 2, 4
    dst, t, v = rand_ct(Q, K, n, N), rand_ct(Q, K, n, N), rand_ct(Q, K, n, N)
    b = [int(RNG.integers(1, q)) for q in Q[:n]]
    binv = [pow(bb, -1, int(q)) for bb, q in zip(b, Q)]
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    x = ((t.astype(np.uint64) + mulq(v, np.array(b, np.uint64).reshape(n, 1).repeat(N, 1), Q)) % qq).astype(np.uint32)
    k = [int(q) + 5 if i % 2 else int(RNG.integers(0, q)) for i, q in enumerate(Q[:n])]  # raw constants, some >= p
    got = em.md_epilogue(Q, dst, x, t, binv, k if withk else None, bool(dbl))
    want = addq(dst, v, Q)
    if dbl:
        want = addq(want, want, Q)
    if withk:
        want[:, 0] = addq(want[:, 0], np.array(k, np.uint64).reshape(n, 1) % qq, Q)
    assert (got == want).all()
    got_to = em.md_epilogue_to(Q, dst, x, t, binv, sub=True)
    assert (addq(got_to, v, Q) == dst).all()


def test_wsum_and_add_const_are_linear():
    K, n = 2, 4
    s = secret(Q, n, N)
    srcs = [rand_ct(Q, K, n, N) for _ in range(5)]
    w = [[int(RNG.integers(0, q)) for q in Q[:n]] for _ in srcs]
    k = [int(RNG.integers(0, 2 * q)) for q in Q[:n]]
    out = em.wsum(Q, srcs, w, k)
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    for c in range(K):
        want = np.array(k, np.uint64).reshape(n, 1) % qq + np.zeros((n, N), np.uint64)
        for j, x in enumerate(srcs):
            want = addq(want, mulq(dec(Q, x[c, 0], x[c, 1], s), np.array(w[j], np.uint64).reshape(n, 1).repeat(N, 1),
                                   Q), Q)
        assert (dec(Q, out[c, 0], out[c, 1], s) == want).all()
    x = srcs[0]
    got = em.add_const(Q, x, k)
    for c in range(K):
        want = addq(dec(Q, x[c, 0], x[c, 1], s), np.array(k, np.uint64).reshape(n, 1) % qq + np.zeros((n, N), np.uint64),
                    Q)
        assert (dec(Q, got[c, 0], got[c, 1], s) == want).all()


def test_ew_many_and_submul_many_invert():
    n = 4
    a, b, c = (rand_ct(Q, 1, n, N)[0, 0] for _ in range(3))
    t = np.stack([RNG.integers(1, Q[r], N) for r in range(n)]).astype(np.uint32)
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    s3 = em.ew_many(Q, a, b, c)
    assert (((s3.astype(np.uint64) + 2 * qq - b - c) % qq) == a).all()
    assert (em.ew_many(Q, a) == a).all()
    sm = em.submul_many(Q, a, b, t)
    tinv = np.vectorize(lambda v, p: pow(int(v), -1, int(p)), otypes=[object])(t, np.asarray(Q[:n]).reshape(n, 1))
    back = np.array([[(int(sm[r, i]) * int(tinv[r, i]) + int(b[r, i])) % int(Q[r]) for i in range(N)]
                     for r in range(n)], np.uint64)
    assert (back == a).all()


# ----------------------------------------------------------------------------------------------- composite rescale
def crt_values(q, rows):
    """the integers X in [0, prod q) of the coefficient rows [len(q)][N]"""
    big = 1
    for p in q:
        big *= int(p)
    out = []
    for i in range(rows.shape[1]):
        x = 0
        for r, p in enumerate(q):
            p = int(p)
            m = big // p
            x += int(rows[r, i]) * m * pow(m % p, -1, p)
        out.append(x % big)
    return out


def exact_rescale(vals, q_drop):
    out = []
    for x in vals:
        c = x % q_drop
        if c > q_drop // 2:
            c -= q_drop
        assert (x - c) % q_drop == 0
        out.append((x - c) // q_drop)
    return out


@pytest.mark.parametrize("ndrop", [1, 2])
def test_rescale_is_the_exact_division(ndrop):
    ctx = small_chain(logn=8, nq=6, kp=1, dnum=2, bits=30)
    q = ctx.q
    top = 5
    K = 2
    coef = np.zeros((K, 2, top + 1, ctx.n), np.uint32)
    for r in range(top + 1):
        coef[:, :, r] = RNG.integers(0, q[r], (K, 2, ctx.n))
    x = np.zeros_like(coef)
    for k in range(K):
        for part in range(2):
            x[k, part] = ctx.ntt_fwd(coef[k, part].copy(), list(range(top + 1)))
    out = em.rescale(ctx, q, x, top, ndrop)
    rows = top + 1 - ndrop
    for k in range(K):
        for part in range(2):
            got = ctx.ntt_inv(out[k, part], list(range(rows)))
            vals = crt_values(q[:top + 1], coef[k, part])
            vals = exact_rescale(vals, int(q[top]))
            if ndrop == 2:
                vals = exact_rescale(vals, int(q[top - 1]))
            want = np.array([[v % int(q[r]) for v in vals] for r in range(rows)], np.uint64)
            assert (got == want).all()


def test_composite_equals_two_single_drops_and_the_fold():
    ctx = small_chain(logn=8, nq=6, kp=1, dnum=2, bits=30)
    q = ctx.q
    top = 4
    x = rand_ct(q, 2, top + 1, ctx.n)
    two = em.rescale(ctx, q, x, top, 2)
    one = em.rescale(ctx, q, em.rescale(ctx, q, x, top, 1), top - 1, 1)
    assert (two == one).all()
    # fold c: rescale(c x) with the tops scaled and alpha_i c_i equals scaling every row first
    c = [int(RNG.integers(2, p)) for p in q]
    cx = x.copy()
    for r in range(top + 1):
        cx[:, :, r] = (x[:, :, r].astype(np.uint64) * c[r] % int(q[r])).astype(np.uint32)
    assert (em.rescale(ctx, q, x, top, 2, fold=c) == em.rescale(ctx, q, cx, top, 2)).all()


# ----------------------------------------------------------------------------------------------- encryption
def test_enca_lane_is_the_expander_rule():
    """The "ENCA" lane is the KSKA rule under another tag: with the KSKA tag it is the pinned KSKA row, and each ENCA
    word is the first accepted ChaCha12 word of (slot / 16 + t N / 16, nonce, p, "ENCA") at slot % 16, mod p."""
    n = 1 << 10
    seed = [int(v) for v in RNG.integers(0, 1 << 32, 8, dtype=np.uint64)]
    for p in (twin.descending_primes(31, 2 * n, 1)[0], 1431658497):  # the second rejects about a third of the words
        assert (twin.expand_row(seed, 2, p, n, twin.TAG_KSKA) == twin.kska_row(seed, 2, p, n)).all()
        row = twin.expand_row(seed, 77, p, n, twin.TAG_ENCA)
        bound = (0xFFFFFFFF // p) * p
        for s in range(0, n, 7):
            v = 0
            for t in range(16):
                v = int(twin.chacha_block(seed, s // 16 + t * (n // 16), 77, p, twin.TAG_ENCA, 12)[s % 16])
                if v < bound:
                    break
            assert int(row[s]) == v % p


def test_encryption_decrypts_to_e_plus_m():
    n, nl = 1 << 10, 4
    q = twin.descending_primes(31, 2 * n, nl)
    seed = [1, 2, 3, 4, 5, 6, 7, 8]
    a = np.stack([twin.expand_row(seed, 9, p, n, twin.TAG_ENCA) for p in q])
    s, e, m = (np.stack([RNG.integers(0, p, n) for p in q]).astype(np.uint32) for _ in range(3))
    c0 = em.encrypt(q, a, s, e, m)
    assert (addq(c0, mulq(a, s, q), q) == addq(e, m, q)).all()
    assert (addq(em.encrypt(q, a, s, e), mulq(a, s, q), q) == e).all()


# ----------------------------------------------------------------------------------------------- relinearized product
def crt_centred(rows, q):
    """the centred integers of coefficient rows [k][N] over the primes q"""
    big = 1
    for p in q:
        big *= int(p)
    vals = crt_values(q, rows)
    return [v - big if v > big // 2 else v for v in vals]


def negacyclic(a, b):
    n = len(a)
    out = [0] * n
    for i in range(n):
        ai = int(a[i])
        if ai == 0:
            continue
        for j in range(n):
            v = ai * int(b[j])
            if i + j < n:
                out[i + j] += v
            else:
                out[i + j - n] -= v
    return out


def test_mul_relin_then_rescale_decrypts_to_the_product():
    """Dec(mul_relin(ct_a, ct_b)) = m_a m_b (negacyclic, exact integers over Q) up to the encryption noise times the
    messages, with the relinearization key b = e - a s + P s^2 (ksk_gen with s_old = s^2); after a two-prime rescale
    the decryption is m_a m_b / (q_a q_b) up to a few units."""
    from tests.test_oracle_ks import decrypt, encrypt
    ctx = small_chain(logn=8, nq=6, kp=2, dnum=3, bits=30)
    top, n = 5, ctx.n
    g = twin.Prng([2, 7, 1, 8, 2, 8, 1, 8], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    s2 = np.stack([(s_eval[t].astype(np.uint64) ** 2 % ctx.primes[t]) for t in range(ctx.rows)]).astype(np.uint32)
    seed = g.ksk_seed()
    e = np.zeros((ctx.dnum, ctx.rows, n), np.uint32)
    for d in range(ctx.dnum):
        ed = g.gaussian(n)
        for t in range(ctx.rows):
            e[d, t] = np.mod(ed, ctx.primes[t])
    e = ctx.ntt_fwd(e.reshape(-1, n), [t for _ in range(ctx.dnum) for t in range(ctx.rows)]).reshape(e.shape)
    bkey = ctx.ksk_gen(s_eval, s2, seed, e)
    rng = np.random.default_rng(8)
    delta = 1 << 30
    ma, mb = rng.integers(-100, 100, n) * delta, rng.integers(-100, 100, n) * delta
    ca, _ = encrypt(ctx, s_eval, ma, rng, top)
    cb, _ = encrypt(ctx, s_eval, mb, rng, top)
    out = ctx.mul_relin(ca, cb, top, seed, bkey)
    prod = negacyclic(ma, mb)
    q = ctx.primes[: top + 1]
    got = crt_centred(decrypt(ctx, s_eval, out, top), q)
    assert max(abs(x - y) for x, y in zip(got, prod)) < delta << 20  # the product is ~ delta^2 2^20
    # without the relinearization term the decryption is far off (the key switch carries d2 s^2)
    plain = ctx.ct_zeros()
    from oracle import em as em_
    c0, c1, _ = em_.tensor(ctx.primes, [(ca[None, :, : top + 1], cb[None, :, : top + 1])])
    plain[0, : top + 1], plain[1, : top + 1] = c0[0], c1[0]
    bad = crt_centred(decrypt(ctx, s_eval, plain, top), q)
    assert max(abs(x - y) for x, y in zip(bad, prod)) > delta << 40
    # the rescale by the two top primes divides by q_4 q_5
    rs = ctx.rescale(out, top, 2)
    got = crt_centred(decrypt(ctx, s_eval, rs, top - 2), ctx.primes[: top - 1])
    div = int(ctx.primes[top]) * int(ctx.primes[top - 1])
    assert max(abs(x - round(y / div)) for x, y in zip(got, prod)) < 1 << 8


# ----------------------------------------------------------------------------------------------- BSGS plaintext dot
@pytest.mark.parametrize("enc", [0xFFFFFFFF, 0x7F000003, 0x1F])
def test_pt_dot_decrypts_to_the_diagonal_products(enc):
    """Dec(res_j) = sum_b Dec(rot_b) pt_{B j + b} word by word, diagonals past npts skipped; a compact diagonal read
    through enc equals its expansion to a full row read plainly."""
    K, B, G, n = 2, 3, 2, 4
    npts = 5
    s = secret(Q, n, N)
    rot = np.stack([np.stack([rand_ct(Q, 1, n, N)[0] for _ in range(B)]) for _ in range(K)])
    ptw = N if enc == 0xFFFFFFFF else (N >> 3 if enc >> 24 == 0x7F else enc + 1)
    pts = [np.stack([RNG.integers(0, Q[r], ptw) for r in range(n)]).astype(np.uint32) for _ in range(npts)]
    res = em.pt_dot(Q, rot, pts, B, G, npts, enc, list(range(n)))
    idx = em.ptidx(np.arange(N), enc).astype(np.int64)
    full = [p[:, idx] for p in pts]
    assert (em.pt_dot(Q, rot, full, B, G, npts, 0xFFFFFFFF, list(range(n))) == res).all()
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    for c in range(K):
        for j in range(G):
            want = np.zeros((n, N), np.uint64)
            for b in range(B):
                if B * j + b < npts:
                    want = addq(want, mulq(dec(Q, rot[c, b, 0], rot[c, b, 1], s), full[B * j + b], Q), Q)
            assert (dec(Q, res[c, j, 0], res[c, j, 1], s) == want % qq).all()


# ----------------------------------------------------------------------------------------------- subring switch
@pytest.mark.parametrize("sub", [2, 4, 16])
def test_pack_split_partitions_the_coefficients(sub):
    """The digits sum back to the row, and digit j vanishes off the exponents = j mod sub."""
    x = rand_ct(Q, 1, 4, N)[0, 0]
    d = em.pack_split(x, sub)
    assert (d.astype(np.uint64).sum(0) == x).all()
    for j in range(sub):
        off = (np.arange(N) % sub) != j
        assert (d[j][:, off] == 0).all()


def test_pack_dot_decrypts_to_the_errors():
    """With a pack key b_j = e_j - a_j s, Dec(s0, s1) = s0 + s1 s = sum_j D_j e_j + pmod c0 on the Q rows (and without
    the c0 term on the others): a swapped a / b or a dropped digit breaks it."""
    n, sub, nq = 4, 4, 3
    s = secret(Q, n, N)
    qq = np.asarray(Q[:n], np.uint64).reshape(n, 1)
    dig = np.stack([rand_ct(Q, 1, n, N)[0, 0] for _ in range(sub)])
    ka = np.stack([rand_ct(Q, 1, n, N)[0, 0] for _ in range(sub)])
    e = RNG.integers(0, 8, (sub, n, N)).astype(np.uint64)
    kb = ((e + qq - mulq(ka, s, Q)) % qq).astype(np.uint32)
    c0 = rand_ct(Q, 1, n, N)[0, 0]
    pmod = [int(RNG.integers(0, q)) for q in Q[:n]]
    s0, s1 = em.pack_dot(Q, dig, kb, ka, c0, pmod, nq)
    want = np.zeros((n, N), np.uint64)
    for j in range(sub):
        want = addq(want, mulq(dig[j], e[j], Q), Q)
    want[:nq] = addq(want[:nq], mulq(c0[:nq], np.array(pmod[:nq], np.uint64).reshape(nq, 1).repeat(N, 1), Q), Q)
    assert (addq(s0, mulq(s1, s, Q), Q) == want).all()


# ----------------------------------------------------------------------------------------------- coeff_sum
def test_coeff_residues_against_python_integers():
    """round half to even of float32 * scale in float64, the +-2^62 clamp past 9.2e18 counted per limb, the residue
    of a negative value p - (|m| mod p)"""
    q = [1073479681, 2147352577, 97]
    f = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.0, -7.25, 1e19, -1e19, 123456.78, -0.0], np.float32)
    rng = np.random.default_rng(4)
    f = np.concatenate([f, rng.normal(size=200).astype(np.float32) * 1e6])
    for scale in (1.0, 2.0 ** 20, 3.7):
        got, ovf = em.coeff_residues(f[None], scale, q)
        n_big = 0
        for k, v in enumerate(f):
            x = float(v) * scale
            if abs(x) < 9.2e18:
                m = round(x)
            else:
                m = -(1 << 62) if x < 0 else 1 << 62
                n_big += 1
            assert [int(got[t, 0, k]) for t in range(len(q))] == [m % p for p in q], (scale, k, v)
        assert ovf == n_big * len(q)


def test_coeff_sum_against_the_schoolbook_product():
    """INTT(out) = sum_r INTT(ct_r) * m_r (negacyclic, mod p) with m_r = round(rows_r scale), plus the old out"""
    oc = small_chain(logn=6, nq=3, kp=0, dnum=1)
    n_terms, N = 3, oc.n
    q = [int(p) for p in oc.primes]
    rng = np.random.default_rng(8)
    rows = (rng.normal(size=(n_terms, N)) * 40).astype(np.float32)
    cts = [np.stack([np.stack([rng.integers(0, p, N) for p in q]) for _ in range(2)]).astype(np.uint32)
           for _ in range(n_terms)]
    old = np.stack([np.stack([rng.integers(0, p, N) for p in q]) for _ in range(2)]).astype(np.uint32)
    out, ovf = em.coeff_sum(q, rows, 3.0, cts, oc.ntt_fwd, out=old)
    assert ovf == 0
    ids = list(range(len(q)))
    for part in range(2):
        got = oc.ntt_inv(out[part].copy(), ids)
        want = oc.ntt_inv(old[part].copy(), ids).astype(object)
        for r in range(n_terms):
            c = oc.ntt_inv(cts[r][part].copy(), ids)
            m = [round(float(v) * 3.0) for v in rows[r]]
            for t, p in enumerate(q):
                want[t] = (want[t] + np.array(negacyclic([int(x) for x in c[t]], m), dtype=object)) % p
        assert (got.astype(object) == want).all(), part


# ----------------------------------------------------------------------------------------------- tensor_seeded
def test_tensor_seeded_is_the_tensor_of_the_expanded_ciphertexts():
    """tensor_seeded's oracle equals the (pinned) tensor of full ciphertexts whose c1 rows are the (pinned) CTSA rows
    of their seeds, for every second-operand set; the 28-bit packing round-trips"""
    q = [268369921, 268361729, 268271617]
    n, N = 3, 64
    rng = np.random.default_rng(12)
    nout, npairs = 2, 3
    c0s = [[np.stack([rng.integers(0, p, N) for p in q]).astype(np.uint32) for _ in range(npairs)] for _ in range(nout)]
    seeds = [[rng.integers(0, 1 << 32, (n, 8), dtype=np.uint64).astype(np.uint32) for _ in range(npairs)]
             for _ in range(nout)]
    bsets = [[np.stack([np.stack([rng.integers(0, p, N) for p in q]) for _ in range(2)]).astype(np.uint32)
              for _ in range(npairs)] for _ in range(2)]
    old = rng.integers(0, 1 << 27, (4, 2, n, N)).astype(np.uint32)
    old_d2 = rng.integers(0, 1 << 27, (4, n, N)).astype(np.uint32)
    out, d2 = em.tensor_seeded(q, c0s, seeds, bsets, acc=3, old=old, old_d2=old_d2, cts_row=twin.cts_expand_row)
    m = 0
    for bs in bsets:
        for o in range(nout):
            pairs = []
            for j in range(npairs):
                c1 = np.stack([twin.cts_expand_row(seeds[o][j][r], q[r], N) for r in range(n)])
                pairs.append((np.stack([c0s[o][j], c1])[None], bs[j][None]))
            w0, w1, w2 = em.tensor(q, pairs, old=old[m][None], old_d2=old_d2[m][None], acc=True, acc_d2=True)
            assert (out[m, 0] == w0[0]).all() and (out[m, 1] == w1[0]).all() and (d2[m] == w2[0]).all()
            m += 1
    vals = rng.integers(0, 1 << 28, (2, 40)).astype(np.uint32)
    pk = em.pack28(vals)
    assert pk.shape == (2, (40 * 28 + 31) // 32)
    for r in range(2):
        stream = int.from_bytes(pk[r].tobytes(), "little")
        assert [(stream >> (28 * i)) & ((1 << 28) - 1) for i in range(40)] == [int(v) for v in vals[r]]
