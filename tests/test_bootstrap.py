"""The bootstrap composite (perseus_amd/bootstrap.py) on the CPU: the route's stage plans (the reference's factors,
pinned in tests/test_bts_setup.py) composing to the CoeffToSlot / SlotToCoeff maps, the float simulation of the whole
algorithm, and the homomorphic composite run on the oracle's operations at N = 2^12: the decrypted output equals the
input's message.
"""
import numpy as np
import pytest

from perseus_amd import bootstrap as B
from perseus_amd.encoding import decode, encode
from tests import special_fft as SF
from tests import twin
from tests.bts_ops import OracleOps
from tests.test_oracle_ks import decrypt, encrypt


def test_route_stages_compose_to_the_transforms():
    """the route's stage plans (the reference's factors in FIDESlib's layout): the CtS stages take the decoding of a
    coefficient vector to n times its bit-reversed coefficients up to the layout's rotation, and the StC stages after
    them give n times the input back (the accumulated rotation paid by the last StC stage)"""
    for logn in (6, 9):
        N, n = 1 << logn, 1 << (logn - 1)
        cts, stc, gain = B.lt_plans(N, B.Params(logn).budget)
        assert gain == n
        rng = np.random.default_rng(logn)
        m = rng.normal(size=N)
        z = decode(m, N, 1.0)
        y = z
        for p in cts:
            y = p.apply(y)
        coeffs = (m[:n] + 1j * m[n:])[SF.bitrev(n)] * n
        assert min(np.abs(np.roll(y, r) - coeffs).max() for r in range(n)) < 1e-8, "CtS: rotated coefficients"
        for p in stc:
            y = p.apply(y)
        assert np.abs(y - n * z).max() < 1e-8 * n, "StC undoes CtS"


def test_residues_exact():
    rng = np.random.default_rng(3)
    f = np.concatenate([rng.normal(size=50) * 2.0 ** 70, rng.normal(size=50) * 1e6, [2.0 ** 84, -2.0 ** 84, 0.5, -1.5]])
    ps = [1073479681, 1073184769, 3]
    got = B.residues(f, ps)
    for r, p in enumerate(ps):
        assert [int(v) for v in got[r]] == [int(round(x)) % p if abs(x) < 2 ** 53 else int(x) % p for x in f]


def test_simulated_bootstrap():
    logn = 10
    N = 1 << logn
    par = B.Params(logn)
    rng = np.random.default_rng(3)
    m = rng.uniform(-1, 1, N) * 2.0 ** -12
    out = B.simulate(m + rng.integers(-20, 21, N), par)
    want = decode(m, N, 1.0)
    assert np.abs(out - want).max() / np.abs(want).max() < 1e-5


def setup_oracle(logn=12, seed=5, fused=True, chain=None):
    """a chain with the bootstrap's levels plus one spare (three limbs out), or the given chain (q, p, dnum), oracle
    keys, the composite (fused: the levels' babies in the extended basis; "cts": the CtS levels' only)"""
    par = B.Params(logn)
    if chain is None:
        nq = 1 + 2 * par.levels_used() + 2
        dnum = 3
        kp = -(-nq // dnum)
        ps = [int(p) for p in twin.descending_primes(30, 2 << logn, nq + kp)]
        q, p = ps[:nq], ps[nq:]
    else:
        q, p, dnum = [int(x) for x in chain[0]], [int(x) for x in chain[1]], chain[2]
    oc = twin.Ctx(logn, q, p, dnum)
    g = twin.Prng([seed, 2, 7, 1, 8, 2, 8, 1], 0)
    s = g.sparse_ternary(1 << logn, 192)
    s_eval = oc.secret_eval(s)
    boot = B.Bootstrap(None, par, q, special=p if fused else None, fuse_stc=fused != "cts")
    gal, levels, conj = B.key_plan(boot)
    keys = [oc.rotation_key(g, s_eval, x) for x in gal]
    seeds = np.stack([k[0] for k in keys])
    bs = [k[1] for k in keys]
    rseed = g.ksk_seed()
    e = np.zeros((dnum, oc.rows, 1 << logn), np.uint32)
    errs = [g.gaussian(1 << logn) for _ in range(dnum)]
    for d in range(dnum):
        for t in range(oc.rows):
            e[d, t] = np.mod(errs[d], oc.primes[t])
    e = oc.ntt_fwd(e.reshape(-1, 1 << logn), [t for _ in range(dnum) for t in range(oc.rows)]).reshape(e.shape)
    s2 = np.stack([(s_eval[t].astype(np.uint64) ** 2 % oc.primes[t]) for t in range(oc.rows)]).astype(np.uint32)
    rb = oc.ksk_gen(s_eval, s2, rseed, e)
    ops = OracleOps(oc, q, seeds, bs, levels, conj, rseed, rb)
    ops.set_galois(gal)
    boot.ops = boot.ev.ops = ops
    return dict(par=par, oc=oc, s=s, s_eval=s_eval, boot=boot, ops=ops, q=q, p=p, gal=gal, seeds=seeds, bs=bs,
                levels=levels, conj=conj, rseed=rseed, rb=rb, errs=errs, fused=fused)


def input_ct(S, rng):
    par, oc = S["par"], S["oc"]
    z = rng.uniform(-1, 1, par.n) + 1j * rng.uniform(-1, 1, par.n)
    m = np.rint(encode(z, par.N, par.delta_in)).astype(np.int64)
    ct, me = encrypt(oc, S["s_eval"], m, rng, 0)
    return z, ct, me


def decrypt_slots(S, ct, top, scale):
    from perseus_amd.encoding import from_residues

    oc = S["oc"]
    coef = from_residues(decrypt(oc, S["s_eval"], ct, top), oc.primes[: top + 1])
    return decode(coef, S["par"].N, scale)


@pytest.mark.parametrize("fused", [True, False, "cts"])
def test_bootstrap_on_the_oracle(fused):
    S = setup_oracle(fused=fused)
    boot, ops = S["boot"], S["ops"]
    rng = np.random.default_rng(9)
    z, ct, me = input_ct(S, rng)
    boot.prepare()
    out = boot.run((ct[None], 0))
    assert out.top == boot.top_out
    got = decrypt_slots(S, OracleOps.get(out.h), out.top, out.scale)
    ref = decode(me.astype(np.float64), S["par"].N, S["par"].delta_in)  # the input's message with its noise
    err = np.abs(got - ref).max()
    print(f"bootstrap error vs the input's decryption: {err:.3g} (vs the plaintext: {np.abs(got - z).max():.3g})")
    assert err < 1e-3


def test_compact_diagonals():
    """A polynomial in X^(2^s) has evaluation rows constant on aligned blocks of 2^s words (the transforms'
    bit-reversed order: slot i evaluates at psi^(2 brev(i) + 1), and the low s bits of i only move that exponent by
    multiples of 2N / 2^s after the power 2^s), so the plaintext dot on its compact rows at index i >> s gives the
    full rows' words; one odd coefficient makes the shift 0 and the rows no longer compact."""
    from oracle import em

    logn, N = 10, 1 << 10
    q = [int(p) for p in twin.descending_primes(30, 2 << logn, 3)]
    oc = twin.Ctx(logn, q, [int(p) for p in twin.descending_primes(31, 2 << logn, 1)], 1)
    rng = np.random.default_rng(3)
    for s in (0, 1, 4, 7):
        coef = np.zeros((3, N), np.uint32)
        coef[:, :: 1 << s] = rng.integers(0, 1 << 20, (1, N >> s))
        coef %= np.array(q, np.uint32)[:, None]
        assert B.compact_shift(coef) == s
        ev = oc.ntt_fwd(coef.copy(), [0, 1, 2])
        c = B.compact_rows(ev, s)
        assert c.shape == (3, N >> s)
        assert (np.repeat(c, 1 << s, axis=1) == ev).all()
        rot = rng.integers(0, q[-1], (1, 2, 2, 3, N)).astype(np.uint32)
        full = em.pt_dot(q, rot, [ev, ev], 2, 1, 2, 0xFFFFFFFF, [0, 1, 2])
        enc = (0x7F000000 | s) if s else 0xFFFFFFFF
        assert (em.pt_dot(q, rot, [c, c], 2, 1, 2, enc, [0, 1, 2]) == full).all()
        if s:
            coef[:, 1] = 1
            assert B.compact_shift(coef) == 0
            with pytest.raises(ValueError):
                B.compact_rows(oc.ntt_fwd(coef.copy(), [0, 1, 2]), s)
    assert B.compact_shift(np.zeros((2, N), np.uint32)) == 12
