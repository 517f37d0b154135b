"""Pins of the oracle's summed rotations (crates/pc-gpu/src/rotate.rs:692-776 rotate_sum_core) and of the
rotate-and-sum ladder (rotate.rs:924-992).

- one key: the summed path is the single rotation's sequence (ModUp, dot, ModDown), so it equals the oracle's
  rotation word for word;
- decryption: Dec(x + sum_s rot(x, s)) = m + sum_s sigma_s(m) up to one small integer error on every limb (the sum is
  ModDowned once, so it carries one rounding, not one per rotation);
- the ladder rung by rung is its own composition of single rotations and additions, restated here from the oracle's
  rotate; with radix rungs it decrypts to the same slot sums.
"""
import numpy as np
import pytest

from tests import twin
from tests.test_oracle_ks import centred, coeff_automorph, decrypt, encrypt, small_chain


def keys_for(ctx, g, s_eval, steps):
    gals = [twin.rotation_galois(r, ctx.n) for r in steps]
    ks = [ctx.rotation_key(g, s_eval, x) for x in gals]
    return gals, np.stack([k[0] for k in ks]), [k[1] for k in ks]


def add_q(ctx, a, b, top):
    out = ctx.ct_zeros()
    for t in range(top + 1):
        out[:, t] = (a[:, t].astype(np.int64) + b[:, t]) % ctx.primes[t]
    return out


def test_one_key_is_the_rotation():
    ctx = small_chain()
    top = 4
    g = twin.Prng([3, 1, 4, 1, 5, 9, 2, 6], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(ctx.n, 64))
    rng = np.random.default_rng(1)
    ct, _ = encrypt(ctx, s_eval, rng.integers(-1000, 1000, ctx.n), rng, top)
    gals, seeds, bs = keys_for(ctx, g, s_eval, [3])
    got = ctx.rotate_sum(ct, top, seeds, bs, gals)
    want = ctx.rotate(ct, top, seeds[0], bs[0], gals[0])
    assert (got[:, : top + 1] == want[:, : top + 1]).all()
    onto = ctx.rotate_sum(ct, top, seeds, bs, gals, onto=ct)
    assert (onto[:, : top + 1] == add_q(ctx, ct, want, top)[:, : top + 1]).all()
    with pytest.raises(ValueError):
        ctx.rotate_sum(ct, top, seeds, bs, [1])  # no identity in a sum group


@pytest.mark.parametrize("steps", [[1, 2, 3], [4, -1]])
def test_sum_decrypts_to_the_rotated_sum(steps):
    ctx = small_chain()
    n, top = ctx.n, 5
    g = twin.Prng([2, 7, 1, 8, 2, 8, 1, 8], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    rng = np.random.default_rng(len(steps))
    m = rng.integers(-(1 << 22), 1 << 22, n)
    ct, me = encrypt(ctx, s_eval, m, rng, top)
    gals, seeds, bs = keys_for(ctx, g, s_eval, steps)
    out = ctx.rotate_sum(ct, top, seeds, bs, gals, onto=ct)
    dec = decrypt(ctx, s_eval, out, top)
    want = me + sum(coeff_automorph(me, x, n) for x in gals)
    errs = [centred((dec[t].astype(np.int64) - want) % ctx.primes[t], ctx.primes[t]) for t in range(top + 1)]
    for e in errs[1:]:
        assert (e == errs[0]).all()
    assert np.abs(errs[0]).max() < (1 << 20)


def test_ladder_rung_by_rung_and_radix():
    ctx = small_chain()
    n, top = ctx.n, 4
    g = twin.Prng([1, 4, 1, 4, 2, 1, 3, 5], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    rng = np.random.default_rng(9)
    m = rng.integers(-(1 << 20), 1 << 20, n)
    ct, me = encrypt(ctx, s_eval, m, rng, top)
    steps = [1, 2, 3, 4, 8, 12]  # every step the ladders below take: gaps 1, 2, 4, 8 and radix-4 rungs {1,2,3}, {4,8,12}
    gals, seeds, bs = keys_for(ctx, g, s_eval, steps)
    out = ctx.rotate_and_sum(ct, top, 1, 16, seeds, bs, gals)
    # rung by rung: out = x; for gap in 1, 2, 4, 8: out += rot(out, gap)
    key = {s: i for i, s in enumerate(steps)}
    acc = ct.copy()
    for gap in (1, 2, 4, 8):
        i = key[gap]
        acc = add_q(ctx, acc, ctx.rotate(acc, top, seeds[i], bs[i], gals[i]), top)
    assert (out[:, : top + 1] == acc[:, : top + 1]).all()
    # both ladders decrypt to the sum of the 16 rotations of the message (one error per ModDown)
    want = sum(coeff_automorph(me, twin.rotation_galois(r, n), n) for r in range(16))
    for radix in (1, 2):
        o = ctx.rotate_and_sum(ct, top, 1, 16, seeds, bs, gals, radix_bits=radix)
        dec = decrypt(ctx, s_eval, o, top)
        errs = [centred((dec[t].astype(np.int64) - want) % ctx.primes[t], ctx.primes[t]) for t in range(top + 1)]
        for e in errs[1:]:
            assert (e == errs[0]).all()
        assert np.abs(errs[0]).max() < (1 << 24)
    with pytest.raises(ValueError):
        ctx.rotate_and_sum(ct, top, 1, 64, seeds, bs, gals)  # gap 16 has no key


def test_sum_is_one_moddown_of_the_summed_dots():
    """The InModDown form: the extended rotations (the pinned dot, scattered by g^-1) summed word by word, then ONE
    ModDown, then the add. The sum of separately ModDowned rotations gives other words (each ModDown rounds), so the
    check tells the two forms apart."""
    ctx = small_chain()
    n, top = ctx.n, 4
    g = twin.Prng([6, 6, 2, 6, 0, 7, 0, 1], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    rng = np.random.default_rng(4)
    ct, _ = encrypt(ctx, s_eval, rng.integers(-1000, 1000, n), rng, top)
    gals, seeds, bs = keys_for(ctx, g, s_eval, [1, 5, 2])
    got = ctx.rotate_sum(ct, top, seeds, bs, gals, onto=ct)
    digits = ctx.modup(ct[1, : top + 1], top)
    rows = list(range(top + 1)) + [ctx.nq + j for j in range(ctx.kp)]
    ext = ctx.ct_zeros()
    for r, x in enumerate(gals):
        e = ctx.ks_dot(ct, digits, top, seeds[r], bs[r], twin.galois_inverse(x, n))
        for t in rows:
            ext[:, t] = (ext[:, t].astype(np.int64) + e[:, t]) % ctx.primes[t]
    want = add_q(ctx, ct, ctx.moddown(ext, top), top)
    assert (got[:, : top + 1] == want[:, : top + 1]).all()
    separate = ct.copy()
    for r, x in enumerate(gals):
        separate = add_q(ctx, separate, ctx.rotate(ct, top, seeds[r], bs[r], x), top)
    assert not (got[:, : top + 1] == separate[:, : top + 1]).all()


def test_rotate_many_pins():
    """The giant-step sum over distinct inputs: with every input the same ciphertext it is the summed rotation (one
    ModUp reused there, one per input here: the same digits); with one input, the single rotation; with distinct
    inputs it decrypts to the sum of their rotated messages up to one small error shared by every limb."""
    ctx = small_chain()
    n, top = ctx.n, 5
    g = twin.Prng([1, 6, 1, 8, 0, 3, 3, 9], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    rng = np.random.default_rng(7)
    ms = [rng.integers(-(1 << 22), 1 << 22, n) for _ in range(3)]
    enc = [encrypt(ctx, s_eval, m, rng, top) for m in ms]
    cts = [c for c, _ in enc]
    gals, seeds, bs = keys_for(ctx, g, s_eval, [1, 2, 5])
    same = ctx.rotate_many([cts[0]] * 3, top, seeds, bs, gals, onto=cts[1])
    want = ctx.rotate_sum(cts[0], top, seeds, bs, gals, onto=cts[1])
    assert (same[:, : top + 1] == want[:, : top + 1]).all()
    one = ctx.rotate_many([cts[2]], top, seeds[1:2], bs[1:2], gals[1:2])
    assert (one[:, : top + 1] == ctx.rotate(cts[2], top, seeds[1], bs[1], gals[1])[:, : top + 1]).all()
    out = ctx.rotate_many(cts, top, seeds, bs, gals, onto=cts[0])
    dec = decrypt(ctx, s_eval, out, top)
    me = [e for _, e in enc]
    want = me[0] + sum(coeff_automorph(e, x, n) for e, x in zip(me, gals))
    errs = [centred((dec[t].astype(np.int64) - want) % ctx.primes[t], ctx.primes[t]) for t in range(top + 1)]
    for e in errs[1:]:
        assert (e == errs[0]).all()
    assert np.abs(errs[0]).max() < (1 << 20)
    with pytest.raises(ValueError):
        ctx.rotate_many(cts[:1], top, seeds[:1], bs[:1], [1])
