"""The table's `encode` entry (device slot encoding) against the oracle (oracle/encode.py):
- the coefficients it leaves in its c workspace agree with the oracle's within the double error of a radix-2 transform,
  log2(N) ulps of the largest coefficient (the reference observes about 1e-5 coefficient units between its host and
  device encoders, encode_dev.rs:1-9);
- its residue rows equal the oracle's scatter of those same coefficients word for word (split, rounding half away
  from zero, deg_factor, 2^split), including a scale that forces OpenFHE's 2^61 split;
- against the oracle's own coefficients, words differ only where the two transforms' errors straddle a half, and
  there by one;
- the rows, taken through the forward NTT and decoded, give back the slots.
Each test prints its case before the GPU runs."""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from oracle import encode as oe
from perseus_amd import abi
from perseus_amd._lib import LIB

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_encode(ctx, ch, z, scale, nl, deg_factor, st):
    n = ch.n
    v = np.zeros((n // 2, 2), np.float64)
    v[:, 0], v[:, 1] = z.real, z.imag
    bv = pa.DevBuf.from_array(v.view(np.uint32))
    ba, bb = pa.DevBuf(4 * n), pa.DevBuf(4 * n)
    bc, bm = pa.DevBuf(2 * n), pa.DevBuf(2)
    bo = pa.DevBuf(nl * n)
    bd = pa.DevBuf.from_array(np.array(deg_factor, np.uint32))
    a = abi.EncodeArgs()
    a.v, a.a, a.b, a.c, a.cmax, a.out = bv.ptr.value, ba.ptr.value, bb.ptr.value, bc.ptr.value, bm.ptr.value, \
        bo.ptr.value
    a.deg_factor, a.pr, a.scale, a.nl = bd.ptr.value, LIB.pcx_ctx_primes(ctx.h), scale, nl
    assert abi.call("encode", a, st, log_n=ch.logn) == 0
    st.sync()
    c = bc.download().view(np.float64)
    cmax = bm.download().view(np.float64)[0]
    return c, cmax, bo.download((nl, n))


@pytest.mark.parametrize("name,logscale,deg", [("small", 40, 1), ("c4", 40, 1), ("c4", 40, 2), ("small", 75, 1)])
def test_device_encode(name, logscale, deg):
    say(f"[encode] {name} scale 2^{logscale} degree {deg}")
    ch = pa.preset(name)
    ctx = pa.Context(ch, k_rot=1)
    st = pa.Stream()
    n = ch.n
    rng = np.random.default_rng(logscale + n + deg)
    z = rng.uniform(-1, 1, n // 2) + 1j * rng.uniform(-1, 1, n // 2)
    scale = 2.0 ** logscale
    nl = len(ch.q)
    df = [int(round(scale)) % p if deg == 2 else 1 for p in ch.q]
    c, cmax, out = run_encode(ctx, ch, z, scale, nl, df, st)
    ref = oe.coefficients(z, n, scale)
    # a radix-2 transform's rounding grows with its stage count: log2(N) ulps of the largest coefficient (at scale
    # 2^40, N = 2^16 about 6e-5 units; the reference observes ~1e-5 between its two encoders)
    tol = ch.logn * 2.0 ** -52 * float(np.abs(ref).max())
    err = float(np.abs(c - ref).max())
    say(f"[encode] max |c_device - c_oracle| = {err:.3g} coefficient units (tolerance {tol:.3g}), "
        f"max |c| = 2^{np.log2(np.abs(ref).max()):.1f}")
    assert err <= tol
    assert cmax == float(np.abs(c).max())
    want, split = oe.scatter(c, ch.q, df)
    assert (out == want).all(), "the scatter of the device's own coefficients, word for word"
    if logscale > 61:
        assert split > 0
    else:
        assert split == 0
        # against the oracle's own coefficients: only half-straddling coefficients may differ, by one
        wo, _ = oe.scatter(ref, ch.q, df)
        diff = np.nonzero((out != wo).any(axis=0))[0]
        for k in diff:
            assert abs(abs(ref[k] - np.trunc(ref[k])) - 0.5) <= tol, k
            for l, p in enumerate(ch.q):
                d = (int(out[l, k]) - int(wo[l, k])) % p
                assert d in (df[l] % p, (p - df[l]) % p), (k, l)
        say(f"[encode] {len(diff)} of {n} coefficients straddle a half")
    if deg == 1 and logscale <= 61:
        # the rows through the forward NTT, decrypted-as-plaintext: CRT, decode, the slots back
        from perseus_amd.encoding import decode, from_residues
        rows = pa.DevBuf.from_array(out)
        pa.Rows(ctx, list(range(nl)), list(range(nl))).ntt(rows, 1, st)
        pa.Rows(ctx, list(range(nl)), list(range(nl))).ntt(rows, -1, st)
        st.sync()
        back = decode(from_residues(rows.download((nl, n)), ch.q), n, scale)
        assert np.abs(back - z).max() < 1e-6
