"""Decryption on the device (pcx_decryptor / pcx_decrypt_rows, crates/pc-gpu/src/decrypt.rs): the coefficient rows of
c0 + c1 s over the bottom d rows of K ciphertexts, word for word against the oracle's decryption (c0 + c1 s on the
host, then its inverse NTT), for the dense and the sparse secret; an encryption of a known message decrypts to it plus
the encryption's own error, exactly; arguments outside the range are refused."""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from tests import twin
from tests.test_oracle_ks import decrypt, encrypt

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    return pa.Stream()


def secrets(oc, ch, seed):
    g = twin.Prng([seed, 9, 8, 7, 6, 5, 4, 3], 0)
    return oc.secret_eval(g.sparse_ternary(ch.n, 192)), oc.secret_eval(g.sparse_ternary(ch.n, 32))


@pytest.mark.parametrize("name,d,K,top", [("small", 1, 1, 5), ("small", 2, 3, 4), ("c3", 2, 2, 29),
                                          ("c5", 1, 4, 12), ("c5", 3, 1, 46)])
def test_decrypt_rows_against_the_oracle(stream, name, d, K, top):
    say(f"[decrypt] {name} d={d} K={K} top={top}")
    ch = pa.preset(name)
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    dense, sparse = secrets(oc, ch, d * 10 + K)
    dec = pa.Decryptor(ctx, d, k_max=4)
    dec.load_secret(np.stack([dense[:d], sparse[:d]]), stream)
    rng = np.random.default_rng(top + K)
    cts = np.zeros((K, 2, ch.rows, ch.n), np.uint32)
    for c in range(K):
        for part in range(2):
            for t in range(top + 1):
                cts[c, part, t] = rng.integers(0, ch.primes[t], ch.n)
    cts[0, :, 0, :3] = [[0, ch.primes[0] - 1, 1], [ch.primes[0] - 1, ch.primes[0] - 1, 0]]
    buf = pa.DevBuf.from_array(cts)
    for which, s_eval in ((0, dense), (1, sparse)):
        got = dec.decrypt_rows(buf, top, stream, K=K, which=which)
        for c in range(K):
            want = decrypt(oc, s_eval, cts[c], d - 1)
            assert (got[c] == want[:d]).all(), (which, c)


def test_decrypt_recovers_the_message(stream):
    say("[decrypt] small: an encryption decrypts to m + e exactly")
    ch = pa.preset("small")
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    dense, _ = secrets(oc, ch, 5)
    dec = pa.Decryptor(ctx, 2)
    dec.load_secret(dense[:2], stream)
    rng = np.random.default_rng(4)
    m = rng.integers(-(1 << 20), 1 << 20, ch.n)
    ct, me = encrypt(oc, dense, m, rng, 4)
    got = dec.decrypt_rows(pa.DevBuf.from_array(ct), 4, stream)[0]
    for r in range(2):
        assert (got[r] == np.mod(me, ch.primes[r])).all(), r


def test_decrypt_refuses_out_of_range(stream):
    say("[decrypt] argument checks")
    ch = pa.preset("small")
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    dense, _ = secrets(oc, ch, 6)
    dec = pa.Decryptor(ctx, 2, k_max=2)
    buf = ctx.ct_buf(3)
    with pytest.raises(pa.HipError):  # no secret loaded
        dec.decrypt_rows(buf, 3, stream)
    dec.load_secret(dense[:2], stream)
    with pytest.raises(pa.HipError):  # the sparse secret was not loaded
        dec.decrypt_rows(buf, 3, stream, which=1)
    with pytest.raises(pa.HipError):  # K > k_max
        dec.decrypt_rows(buf, 3, stream, K=3)
    with pytest.raises(pa.HipError):  # top below the bottom level
        dec.decrypt_rows(buf, 0, stream)
    bad = dense[:2].copy()
    bad[0, 0] = ch.primes[0]
    with pytest.raises(pa.HipError):  # a word not below its prime
        dec.load_secret(bad, stream)
