"""Pins of the oracle's key switch: what the mathematics fixes, independent of how the twin orders its work.

- the switch relation of a generated key (crates/pc-gpu/src/keys/hostref.rs:109-158): INTT(b + a s_new -
  [t in digit d] (P mod q_t) s_old) is the small Gaussian error;
- the eval-form automorphism equals the coefficient-form map X -> X^g (crates/pc-core/src/galois.rs:84-148);
- decryption commutes with rotation: Dec(rot(ct, r)) = sigma_g(Dec(ct)) + a small key-switch error, the same integer
  on every limb (crates/pc-tools/src/word_seam.rs:31-34 asks >= 28 bits below the message);
- ModUp + ModDown of a key switch with b = 0 and a = 0 is the identity on P c0 / P = c0.
"""
import numpy as np
import pytest

from tests import twin

M17 = 1 << 17


def small_chain(logn=10, nq=6, kp=2, dnum=3, bits=30):
    m = 2 << logn
    ps = twin.descending_primes(bits, m, nq + kp)
    return twin.Ctx(logn, ps[:nq], ps[nq:], dnum)


def centred(x, p):
    x = np.asarray(x, np.int64)
    return np.where(x > p // 2, x - p, x)


def coeff_automorph(c, g, n):
    """sigma_g on signed coefficients: X^i -> X^(i g mod 2N), X^N = -1 (galois.rs:114-131)."""
    out = np.zeros(n, np.int64)
    for i, v in enumerate(c):
        e = (i * g) % (2 * n)
        if e < n:
            out[e] = v
        else:
            out[e - n] = -v
    return out


def encrypt(ctx, s_eval, m_coef, rng, top):
    """Secret-key encryption at limbs 0..top: c1 = a uniform, c0 = -a s + NTT(m + e) (eval form)."""
    n = ctx.n
    ct = ctx.ct_zeros()
    e = np.round(rng.normal(0, 3.19, n)).astype(np.int64)
    me = m_coef + e
    ids = list(range(top + 1))
    rows = np.stack([np.mod(me, ctx.primes[t]) for t in ids]).astype(np.uint32)
    rows = ctx.ntt_fwd(rows, ids)
    for t in ids:
        p = ctx.primes[t]
        a = rng.integers(0, p, n, dtype=np.int64)
        ct[1, t] = a
        ct[0, t] = (rows[t].astype(np.int64) - (a * s_eval[t].astype(np.int64)) % p) % p
    return ct, me


def decrypt(ctx, s_eval, ct, top):
    ids = list(range(top + 1))
    rows = np.stack([(ct[0, t].astype(np.int64) + (ct[1, t].astype(np.int64) * s_eval[t]) % ctx.primes[t])
                     % ctx.primes[t] for t in ids]).astype(np.uint32)
    return ctx.ntt_inv(rows, ids)


def test_automorphism_eval_vs_coeff():
    ctx = small_chain(logn=8, nq=2, kp=0, dnum=1)
    n, p = ctx.n, ctx.primes[0]
    rng = np.random.default_rng(2)
    a = rng.integers(-1000, 1000, n)
    for g in [5, 25, 2 * n - 1, twin.rotation_galois(7, n)]:
        lhs = ctx.ntt_fwd(np.mod(coeff_automorph(a, g, n), p)[None, :].astype(np.uint32), [0])
        rhs = ctx.automorph_rows(ctx.ntt_fwd(np.mod(a, p)[None, :].astype(np.uint32), [0]), g)
        assert (lhs == rhs).all()


def test_switch_relation():
    ctx = small_chain()
    g = twin.Prng([11, 22, 33, 44, 55, 66, 77, 88], 0)
    s = g.sparse_ternary(ctx.n, 64)
    s_eval = ctx.secret_eval(s)
    gal = twin.rotation_galois(1, ctx.n)
    seed, b = ctx.rotation_key(g, s_eval, gal)
    s_new = ctx.automorph_rows(s_eval, twin.galois_inverse(gal, ctx.n))
    # a regenerated from the seed (KSKA lane), the relation undone, the error recovered in coefficient form
    for d in range(ctx.dnum):
        for t in range(ctx.rows):
            p = ctx.primes[t]
            a = twin.kska_row(seed, d, p, ctx.n).astype(np.int64)
            v = (b[d, t].astype(np.int64) + a * s_new[t] % p) % p
            if t < ctx.nq and ctx.digit_of(t) == d:
                pm = 1
                for q in ctx.p:
                    pm = pm * q % p
                v = (v - pm * s_eval[t].astype(np.int64) % p) % p
            e = centred(ctx.ntt_inv(v.astype(np.uint32)[None, :], [t])[0], p)
            assert 0 < np.abs(e).max() <= 45, (d, t)


@pytest.mark.parametrize("top", [5, 3, 0])
def test_rotation_decrypts_to_rotated_message(top):
    ctx = small_chain()
    n = ctx.n
    g = twin.Prng([1, 2, 3, 4, 5, 6, 7, 8], 9)
    s = g.sparse_ternary(n, 64)
    s_eval = ctx.secret_eval(s)
    rng = np.random.default_rng(top)
    m = rng.integers(-(1 << 24), 1 << 24, n)
    ct, me = encrypt(ctx, s_eval, m, rng, top)
    for r in [1, 3, -1]:
        gal = twin.rotation_galois(r, n)
        seed, b = ctx.rotation_key(g, s_eval, gal)
        out = ctx.rotate(ct, top, seed, b, gal)
        dec = decrypt(ctx, s_eval, out, top)
        want = coeff_automorph(me, gal, n)
        errs = [centred((dec[t].astype(np.int64) - want) % ctx.primes[t], ctx.primes[t]) for t in range(top + 1)]
        for e in errs[1:]:
            assert (e == errs[0]).all()  # one integer error polynomial, the same on every limb
        assert np.abs(errs[0]).max() < (1 << 20)  # >= 28 bits below the message's 2^48-scale CRT range


def test_moddown_of_p_c0_is_c0():
    """With b = 0 and a = 0 the dot leaves (P c0, 0) and the ModDown divides it back: out = c0 exactly (P c0 is a
    multiple of P, so the conversion from its P rows is zero and no rounding remains)."""
    ctx = small_chain()
    top = 4
    rng = np.random.default_rng(5)
    ct = ctx.ct_zeros()
    for t in range(top + 1):
        ct[0, t] = rng.integers(0, ctx.primes[t], ctx.n)
        ct[1, t] = rng.integers(0, ctx.primes[t], ctx.n)
    digits = ctx.modup(ct[1, : top + 1], top)
    ext = ctx.ct_zeros()
    for t in range(top + 1):
        pm = 1
        for q in ctx.p:
            pm = pm * q % ctx.primes[t]
        ext[0, t] = (ct[0, t].astype(np.int64) * pm) % ctx.primes[t]
    out = ctx.moddown(ext, top)
    assert (out[0, : top + 1] == ct[0, : top + 1]).all()
    assert (out[1, : top + 1] == 0).all()
    assert digits.shape == (ctx.dnum, ctx.rows, ctx.n)


def test_hoisted_batch_matches_single_rotations():
    ctx = small_chain()
    g = twin.Prng([5] * 8, 1)
    s_eval = ctx.secret_eval(g.sparse_ternary(ctx.n, 64))
    rng = np.random.default_rng(9)
    top = 5
    ct = ctx.ct_zeros()
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ctx.primes[t], ctx.n)
    gals = [twin.rotation_galois(r, ctx.n) for r in [1, 2, 0, 5]]
    keys = [ctx.rotation_key(g, s_eval, x) for x in gals]
    outs = ctx.rotate_hoisted(ct, top, np.stack([k[0] for k in keys]), [k[1] for k in keys], gals)
    for (seed, b), x, o in zip(keys, gals, outs):
        assert (o[:, : top + 1] == ctx.rotate(ct, top, seed, b, x)[:, : top + 1]).all()
    assert (outs[2][:, : top + 1] == ct[:, : top + 1]).all()  # step 0: g = 1, a copy
