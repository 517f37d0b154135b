"""Pins of the oracle's fused ModDown-rescale (crates/pc-gpu/src/bts/cts.rs:740-751, LtEnd::FusedRescale: one exact
ModDown by B = P q_top q_{top-1}):

- against big integers: with X the CRT lift of all top + 1 + kp residues of x = ext + P onto (coefficient form, in
  [0, Q_top P)), the output's CRT value over q_0..q_{top-2} is round(X / B), coefficient by coefficient. A wrong source
  order, pre factor, conversion matrix, B mod q, B^-1, onto scale or rounding constant moves it;
- the same summed rotations through or_rotate_many with and without the fusion decrypt to the same message up to a
  few units (the sequential ModDown and rescale each round once, the fusion once).
"""
import numpy as np
import pytest

from tests import twin
from tests.test_oracle_ks import small_chain


def crt(rows, primes):
    """integers of the residue rows [k][n] over primes (in [0, prod))"""
    M = 1
    for p in primes:
        M *= int(p)
    acc = [0] * rows.shape[1]
    for r, p in zip(rows, primes):
        p = int(p)
        Mi = M // p
        f = Mi * pow(Mi % p, -1, p)
        for i, v in enumerate(r):
            acc[i] += int(v) * f
    return [a % M for a in acc], M


@pytest.mark.parametrize("with_onto", [False, True])
def test_moddown_rescale_is_round_x_over_b(with_onto):
    ctx = small_chain(logn=10, nq=6, kp=2)
    n, R, nq, top = ctx.n, ctx.rows, len(ctx.primes) - 2, 5
    primes = [int(p) for p in ctx.primes]
    rng = np.random.default_rng(3 + with_onto)
    ext = np.zeros((2, R, n), np.uint32)
    onto = np.zeros((2, R, n), np.uint32)
    live = list(range(top + 1)) + list(range(nq, R))
    for part in range(2):
        for t in live:
            ext[part, t] = rng.integers(0, primes[t], n, dtype=np.uint64).astype(np.uint32)
            if t <= top:
                onto[part, t] = rng.integers(0, primes[t], n, dtype=np.uint64).astype(np.uint32)
    out = ctx.moddown_rescale(ext, top, onto if with_onto else None)
    P = 1
    for j in range(nq, R):
        P *= primes[j]
    B = P * primes[top] * primes[top - 1]
    for part in range(2):
        x = ext[part].astype(np.uint64).copy()
        if with_onto:
            for t in range(top + 1):
                x[t] = (x[t] + onto[part, t].astype(np.uint64) * (P % primes[t])) % primes[t]
        coef = np.stack([ctx.ntt_inv(x[t][None].astype(np.uint32).copy(), [t])[0] for t in live])
        X, _ = crt(coef, [primes[t] for t in live])
        want = [(2 * v + B) // (2 * B) for v in X]  # round(X / B), halves up
        oc = np.stack([ctx.ntt_inv(out[part, t][None].copy(), [t])[0] for t in range(top - 1)])
        got, Mo = crt(oc, primes[: top - 1])
        assert all(g == w % Mo for g, w in zip(got, want))


def test_rotate_many_fused_decrypts_like_sequential():
    from tests.test_oracle_ks import centred, decrypt, encrypt
    from tests.test_oracle_rotsum import keys_for

    ctx = small_chain()
    n, top = ctx.n, 5
    g = twin.Prng([5, 3, 5, 8, 9, 7, 9, 3], 0)
    s_eval = ctx.secret_eval(g.sparse_ternary(n, 64))
    rng = np.random.default_rng(21)
    ms = [rng.integers(-(1 << 22), 1 << 22, n) for _ in range(3)]
    enc = [encrypt(ctx, s_eval, m, rng, top) for m in ms]
    cts = [c for c, _ in enc]
    gals, seeds, bs = keys_for(ctx, g, s_eval, [1, 2])
    seq = ctx.rotate_many(cts[1:], top, seeds, bs, gals, onto=cts[0])
    seq = ctx.rescale(seq, top, 2)
    fused = ctx.rotate_many(cts[1:], top, seeds, bs, gals, onto=cts[0], rescale=True)
    d1 = decrypt(ctx, s_eval, seq, top - 2)
    d2 = decrypt(ctx, s_eval, fused, top - 2)
    for t in range(top - 1):
        diff = centred((d1[t].astype(np.int64) - d2[t]) % ctx.primes[t], ctx.primes[t])
        assert np.abs(diff).max() <= 64
